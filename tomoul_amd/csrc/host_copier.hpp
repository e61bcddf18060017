// host_copier.hpp -- parallel host memcpy for the host-pointer entry points
// (runtime.hip): copies between the caller's pageable memory and the pinned
// staging buffers, split over a few worker threads.  Plain C++ (no HIP), so
// tests/c/test_host_copier.cpp can run it under ThreadSanitizer.
#pragma once

#include <algorithm>
#include <condition_variable>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

namespace tml {

// Host copies between the caller's pageable memory and the pinned staging,
// split over a few worker threads.  On MI355X hosts PCIe moves 50+ GB/s from
// pinned memory, while one thread copies a small fraction of that, and the
// runtime's own pageable path reaches 32 GB/s up and 17 GB/s down (8 MiB).
// Copies below 512 KiB stay on the calling thread.  One copy at a time.
class HostCopier {
  public:
    static HostCopier &get() {
        static HostCopier h;
        return h;
    }
    void copy(void *dst, const void *src, size_t n) {
        constexpr size_t kMinPart = (size_t)256 << 10;
        if (n == 0) return;  // (memcpy's pointers must be valid even for no bytes)
        if (n < 2 * kMinPart) {
            std::memcpy(dst, src, n);
            return;
        }
        std::lock_guard<std::mutex> job(job_mu_);
        start_threads();
        const size_t parts = std::min<size_t>(threads_.size() + 1, n / kMinPart);
        if (parts <= 1) {
            std::memcpy(dst, src, n);
            return;
        }
        {
            std::lock_guard<std::mutex> lk(mu_);
            dst_ = (char *)dst;
            src_ = (const char *)src;
            n_ = n;
            part_ = (n / parts + 63) & ~(size_t)63;
            nparts_ = (n + part_ - 1) / part_;
            next_ = 0;
            done_ = 0;
            ++gen_;
        }
        cv_.notify_all();
        work();
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [&] { return done_ == nparts_; });
    }
    ~HostCopier() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto &t : threads_) t.join();
    }

  private:
    void start_threads() {
        if (!threads_.empty()) return;
        const unsigned hw = std::thread::hardware_concurrency();
        const unsigned n = std::min(7u, hw > 1 ? hw - 1 : 0u);
        for (unsigned i = 0; i < n; ++i) threads_.emplace_back([this] { worker(); });
    }
    // Claims parts of the current job (under the lock, so a thread that
    // wakes late never sees a job half set up) until none is left.  A job
    // ends only when every claimed part has been copied.
    void work() {
        for (;;) {
            char *d;
            const char *s;
            size_t len;
            {
                std::lock_guard<std::mutex> lk(mu_);
                if (next_ >= nparts_) return;
                const size_t off = next_++ * part_;
                d = dst_ + off;
                s = src_ + off;
                len = std::min(part_, n_ - off);
            }
            std::memcpy(d, s, len);
            std::lock_guard<std::mutex> lk(mu_);
            if (++done_ == nparts_) done_cv_.notify_all();
        }
    }
    void worker() {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return stop_ || gen_ != seen; });
                if (stop_) return;
                seen = gen_;
            }
            work();
        }
    }
    std::mutex job_mu_, mu_;
    std::condition_variable cv_, done_cv_;
    std::vector<std::thread> threads_;
    char *dst_ = nullptr;
    const char *src_ = nullptr;
    size_t n_ = 0, part_ = 0, nparts_ = 0, next_ = 0, done_ = 0;
    uint64_t gen_ = 0;
    bool stop_ = false;
};

}  // namespace tml
