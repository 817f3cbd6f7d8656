// CPU check of det::host::CopyPool (mind_amd/csrc/det_copy_pool.h), the
// host-pointer entry points' threaded host copy: lengths on both sides of
// the split and part thresholds and random ones, at odd source and
// destination offsets, from several caller threads at once, with guard
// bytes around every destination, and the pool stopped and restarted
// between rounds.  Prints "bad=0" and exits 0 when every copy is exact.
// Built plainly and under ThreadSanitizer by tests/test_copy_pool.py.
#include "../../mind_amd/csrc/det_copy_pool.h"

#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <thread>
#include <vector>

int main(int argc, char **argv) {
    using det::host::COPY_PART;
    using det::host::COPY_SPLIT;
    const int rounds = argc > 1 ? atoi(argv[1]) : 3;
    const int per_caller = argc > 2 ? atoi(argv[2]) : 24;
    constexpr size_t MAXB = 5u << 20, GUARD = 16;
    det::host::CopyPool pool;
    std::atomic<long> bad{0}, copies{0};
    for (int r = 0; r < rounds; ++r) {
        std::vector<std::thread> callers;
        for (int t = 0; t < 3; ++t)
            callers.emplace_back([&, t, r] {
                std::mt19937_64 rng(1000u * (unsigned)r + (unsigned)t);
                std::vector<unsigned char> src(MAXB + 64), dst(MAXB + 64 + 2 * GUARD);
                for (auto &c : src) c = (unsigned char)rng();
                const size_t edges[] = {0, 1, 4095, COPY_PART - 1, COPY_PART, COPY_SPLIT - 1, COPY_SPLIT,
                                        COPY_SPLIT + 1, 4 * COPY_PART + 3, MAXB};
                for (int i = 0; i < per_caller; ++i) {
                    const size_t n = i < 10 ? edges[i] : (size_t)(rng() % MAXB);
                    const size_t so = rng() % 17, doff = GUARD + rng() % 13;
                    memset(dst.data(), 0xEE, dst.size());
                    pool.copy(dst.data() + doff, src.data() + so, n);
                    copies++;
                    if (memcmp(dst.data() + doff, src.data() + so, n) != 0) bad++;
                    for (size_t g = 0; g < doff; ++g)
                        if (dst[g] != 0xEE) { bad++; break; }
                    for (size_t g = 0; g < GUARD; ++g)
                        if (dst[doff + n + g] != 0xEE) { bad++; break; }
                }
            });
        for (auto &c : callers) c.join();
        pool.stop();   // the next round's first large copy starts the workers again
    }
    printf("copies=%ld bad=%ld\n", copies.load(), bad.load());
    return bad.load() != 0;
}
