// Host -> HBM weight upload through a ring of pinned staging slots.  Worker
// threads copy source rows (from caller memory or a file mapping, assembling
// concatenations and row interleaves on the way) into one slot while the DMA
// engine drains the others, so page-cache reads, the layout work and the PCIe
// transfer overlap instead of running one after another.
#pragma once
#include <condition_variable>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include "model.h"

class Stager {
public:
    explicit Stager(hipStream_t st) : st_(st) {}
    ~Stager();
    int init();
    // dst row (r * n_src + s) <- row r of srcs[s], rows of row_bytes, r < rows:
    // n_src = 1 is a plain copy, 2 the gate/up row interleave
    int upload_rows(void *dst, const void *const *srcs, int n_src, int64_t rows, size_t row_bytes);
    int upload(void *dst, const void *src, size_t bytes) {
        return bytes ? upload_rows(dst, &src, 1, 1, bytes) : QASR_OK;
    }
    int finish();   // waits for every staged transfer

private:
    static constexpr int kSlots = 3;
    static constexpr size_t kSlotBytes = 32u << 20;
    hipStream_t st_;
    char *slot_[kSlots] = {};
    hipEvent_t ev_[kSlots] = {};
    bool used_[kSlots] = {};
    int next_ = 0;
    // worker pool: run(job) calls job(part, n_parts) on every worker and the caller
    std::vector<std::thread> th_;
    std::mutex m_;
    std::condition_variable cv_, done_;
    std::function<void(int, int)> job_;
    unsigned long gen_ = 0;
    int pending_ = 0, n_parts_ = 1;
    bool stop_ = false;
    void run(const std::function<void(int, int)> &job);
    void worker(int part);
    int stage(void *dst, size_t bytes, const std::function<void(char *, int, int)> &fill);
};
