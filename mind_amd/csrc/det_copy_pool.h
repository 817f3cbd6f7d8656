// det_copy_pool.h -- the host-side copy pool of the host-pointer entry
// points (det_abi.hip): large copies between the caller's pageable buffers
// and the library's pinned memory, split over the calling thread and a few
// worker threads.  Host-only C++17 (no HIP), so the CPU tests compile it
// alone, under ThreadSanitizer too.
#pragma once
#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstddef>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

namespace det {
namespace host {

constexpr int COPY_THREADS = 4;
// Host copies of at least COPY_SPLIT bytes are split, in parts of at least
// COPY_PART (measured: a 512 KiB copy in two parts was slower than one
// memcpy by the calling thread, whose caches often hold the caller's
// buffer; 1 MiB in four parts faster than in two).
constexpr size_t COPY_SPLIT = 1u << 20, COPY_PART = 256u << 10;

// The caller and COPY_THREADS - 1 workers share each host copy.  Workers
// start on first use and stop at teardown or unload; one copy runs at a
// time (the caller of another waits).  After a copy the workers poll for the
// next one for SPIN_US before sleeping: the copies of one call (inputs, then
// outputs; a ring transfer's pieces) come within that, and waking a
// sleeping thread cost more than the copy it was to share (measured: Q16
// 512^3 host call 168 -> 156 us, int8 512^3 87 -> 81 us).
class CopyPool {
  public:
    ~CopyPool() { stop(); }
    void copy(void *dst, const void *src, size_t bytes) {
        if (bytes < COPY_SPLIT) {
            memcpy(dst, src, bytes);
            return;
        }
        std::lock_guard<std::mutex> job(job_mu_);
        std::unique_lock<std::mutex> lk(mu_);
        if (workers_.empty()) start();
        const size_t parts = std::min<size_t>(workers_.size() + 1, (bytes + COPY_PART - 1) / COPY_PART);
        dst_ = (char *)dst;
        src_ = (const char *)src;
        bytes_ = bytes;
        piece_ = ((bytes + parts - 1) / parts + 4095) & ~(size_t)4095;
        npieces_ = (bytes + piece_ - 1) / piece_;
        next_ = 0;
        pending_ = npieces_;
        jobs_.fetch_add(1, std::memory_order_release);
        work_cv_.notify_all();
        while (next_ < npieces_) run_one(lk);
        done_cv_.wait(lk, [&] { return pending_ == 0; });
    }
    void stop() {
        std::lock_guard<std::mutex> job(job_mu_);
        {
            std::lock_guard<std::mutex> lk(mu_);
            quit_ = true;
            jobs_.fetch_add(1, std::memory_order_release);
        }
        work_cv_.notify_all();
        for (auto &t : workers_) t.join();
        workers_.clear();
        quit_ = false;
    }

  private:
    // called with mu_ held; copies piece next_ with mu_ released
    void run_one(std::unique_lock<std::mutex> &lk) {
        const size_t i = next_++, o = i * piece_;
        char *d = dst_ + o;
        const char *sp = src_ + o;
        const size_t n = std::min(piece_, bytes_ - o);
        lk.unlock();
        memcpy(d, sp, n);
        lk.lock();
        if (--pending_ == 0) done_cv_.notify_all();
    }
    void start() {   // mu_ held; a thread that cannot start leaves the copy to fewer
        for (int t = 1; t < COPY_THREADS; ++t) {
            try {
                workers_.emplace_back([this] {
                    unsigned seen = jobs_.load(std::memory_order_acquire);
                    for (;;) {
                        // a new copy usually follows within a call: poll for it
                        // for a while before sleeping (a wake-up costs tens of us)
                        const auto t0 = std::chrono::steady_clock::now();
                        while (jobs_.load(std::memory_order_acquire) == seen &&
                               std::chrono::steady_clock::now() - t0 < std::chrono::microseconds(SPIN_US))
                            std::this_thread::yield();
                        std::unique_lock<std::mutex> lk(mu_);
                        work_cv_.wait(lk, [&] { return quit_ || next_ < npieces_; });
                        if (quit_) return;
                        seen = jobs_.load(std::memory_order_acquire);
                        while (next_ < npieces_) run_one(lk);
                    }
                });
            } catch (...) {
                break;
            }
        }
    }
    std::mutex job_mu_, mu_;
    std::condition_variable work_cv_, done_cv_;
    std::vector<std::thread> workers_;
    char *dst_ = nullptr;
    const char *src_ = nullptr;
    size_t bytes_ = 0, piece_ = 0, npieces_ = 0, next_ = 0, pending_ = 0;
    bool quit_ = false;
    std::atomic<unsigned> jobs_{0};
    static constexpr int SPIN_US = 200;
};
}  // namespace host
}  // namespace det
