// det_harness.cpp -- seeded input generators of the reference bench harness,
// exported from libmind_det_hip.so so the bench and the tests create the same
// inputs the reference benches draw (benches/det_matmul_q16.rs:196-219,
// benches/det_matmul_i8.rs:221-226, benches/det_matmul_i16.rs:194-208,
// benches/det_gemv_q16_mt.rs:167-177).
//
// The reference LCG  s <- s*1664525 + 1013904223 (mod 2^64), sample
// u32 = s >> 16, is sequential; these generators split the stream into
// contiguous chunks and start each worker thread at its chunk with an O(log n)
// jump-ahead (composition of the affine map), so the output is the same
// sequence as a single sequential walk.
#include <stdint.h>

#include <algorithm>
#include <thread>
#include <vector>

namespace {

constexpr uint64_t LCG_A = 1664525ull, LCG_C = 1013904223ull;

// State after `n` steps from `s`.
uint64_t lcg_jump(uint64_t s, uint64_t n) {
    uint64_t a = LCG_A, c = LCG_C;        // map for 2^i steps
    uint64_t ra = 1, rc = 0;              // accumulated map
    while (n) {
        if (n & 1) {
            ra = a * ra;
            rc = a * rc + c;
        }
        c = a * c + c;
        a = a * a;
        n >>= 1;
    }
    return ra * s + rc;
}

inline uint32_t next_u32(uint64_t &s) {
    s = s * LCG_A + LCG_C;
    return (uint32_t)(s >> 16);
}

// Fill `count` elements, each consuming exactly `draws` LCG steps, starting
// `skip` steps into the stream of `seed`.
template <typename F>
void parallel_fill(uint64_t seed, uint64_t skip, int64_t count, int draws, F &&f) {
    if (count <= 0) return;
    unsigned nt = std::max(1u, std::min(64u, std::thread::hardware_concurrency()));
    if (count < (1 << 16)) nt = 1;
    const int64_t chunk = (count + nt - 1) / nt;
    std::vector<std::thread> th;
    for (unsigned t = 0; t < nt; ++t) {
        const int64_t lo = (int64_t)t * chunk, hi = std::min(count, lo + chunk);
        if (lo >= hi) break;
        th.emplace_back([=, &f]() {
            uint64_t s = lcg_jump(seed, skip + (uint64_t)lo * draws);
            for (int64_t i = lo; i < hi; ++i) f(i, s);
        });
    }
    for (auto &t : th) t.join();
}

}  // namespace

extern "C" {

// A (na) then B (nb), sample (i8)(u32 >> 16).
void det_gen_i8(uint64_t seed, int8_t *a, int64_t na, int8_t *b, int64_t nb) {
    parallel_fill(seed, 0, na, 1, [a](int64_t i, uint64_t &s) { a[i] = (int8_t)(next_u32(s) >> 16); });
    parallel_fill(seed, (uint64_t)na, nb, 1, [b](int64_t i, uint64_t &s) { b[i] = (int8_t)(next_u32(s) >> 16); });
}

// A then B, sample (i16)(u32 >> 16).
void det_gen_i16(uint64_t seed, int16_t *a, int64_t na, int16_t *b, int64_t nb) {
    parallel_fill(seed, 0, na, 1, [a](int64_t i, uint64_t &s) { a[i] = (int16_t)(next_u32(s) >> 16); });
    parallel_fill(seed, (uint64_t)na, nb, 1, [b](int64_t i, uint64_t &s) { b[i] = (int16_t)(next_u32(s) >> 16); });
}

// A then B, sample ((float)u32 / (float)UINT32_MAX) * 2 - 1 in [-1, 1]
// (the reference f32 canary generator, cross_substrate_identity.rs
// make_pair_f32 / make_matvec_f32).
void det_gen_f32_unit(uint64_t seed, float *a, int64_t na, float *b, int64_t nb) {
    auto f = [](uint64_t &s) {
        const float q = (float)next_u32(s) / (float)UINT32_MAX;
        const float t = q * 2.0f;
        return t - 1.0f;
    };
    parallel_fill(seed, 0, na, 1, [a, f](int64_t i, uint64_t &s) { a[i] = f(s); });
    parallel_fill(seed, (uint64_t)na, nb, 1, [b, f](int64_t i, uint64_t &s) { b[i] = f(s); });
}

// A then B, sample (int32)u32 >> shift (12: +-8.0, 13: +-4.0, 15: +-1.0).
void det_gen_q16(uint64_t seed, int shift, int32_t *a, int64_t na, int32_t *b, int64_t nb) {
    parallel_fill(seed, 0, na, 1, [a, shift](int64_t i, uint64_t &s) { a[i] = ((int32_t)next_u32(s)) >> shift; });
    parallel_fill(seed, (uint64_t)na, nb, 1,
                  [b, shift](int64_t i, uint64_t &s) { b[i] = ((int32_t)next_u32(s)) >> shift; });
}

// Q16 GEMM config: value (int32)u32 >> shift, then one more draw r; when
// r % 100 == 0 the value becomes +-(2^31-1), negative when bit 31 of r is set.
void det_gen_q16_sat(uint64_t seed, int shift, int32_t *a, int64_t na, int32_t *b, int64_t nb) {
    auto draw = [shift](uint64_t &s) {
        int32_t v = ((int32_t)next_u32(s)) >> shift;
        const uint32_t r = next_u32(s);
        if (r % 100u == 0u) v = (r >> 31) ? -2147483647 : 2147483647;
        return v;
    };
    parallel_fill(seed, 0, na, 2, [a, draw](int64_t i, uint64_t &s) { a[i] = draw(s); });
    parallel_fill(seed, 2 * (uint64_t)na, nb, 2, [b, draw](int64_t i, uint64_t &s) { b[i] = draw(s); });
}

// MLP activations: integer Irwin-Hall(12) Gaussian with sigma 32, clipped to
// [-127, 127]: x = clamp(floor((2 * sum_12(u32 >> 16) - 12 * 65535) / 4096)).
void det_gen_i8_gauss(uint64_t seed, int8_t *x, int64_t n) {
    parallel_fill(seed, 0, n, 12, [x](int64_t i, uint64_t &s) {
        int64_t acc = 0;
        for (int j = 0; j < 12; ++j) acc += (int64_t)(next_u32(s) >> 16);
        int64_t t = 2 * acc - 12 * 65535;
        int64_t q = t >= 0 ? t / 4096 : -((-t + 4095) / 4096);
        x[i] = (int8_t)std::max<int64_t>(-127, std::min<int64_t>(127, q));
    });
}

// MLP weights: (i8)(u32 >> 16) redrawn while -128 (uniform on [-127, 127]).
// Rejection consumes a variable number of draws, so this walk is sequential.
void det_gen_i8_sym127(uint64_t seed, int8_t *w, int64_t n) {
    uint64_t s = seed;
    for (int64_t i = 0; i < n; ++i) {
        int8_t v;
        do v = (int8_t)(next_u32(s) >> 16);
        while (v == -128);
        w[i] = v;
    }
}

}  // extern "C"
