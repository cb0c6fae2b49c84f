#include "upload.h"

#include <cstdlib>
#include <cstring>

Stager::~Stager() {
    if (!th_.empty()) {
        {
            std::lock_guard<std::mutex> g(m_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto &t : th_) t.join();
    }
    for (int k = 0; k < kSlots; k++) {
        if (ev_[k]) {
            (void)hipEventSynchronize(ev_[k]);
            (void)hipEventDestroy(ev_[k]);
        }
        if (slot_[k]) (void)hipHostFree(slot_[k]);
    }
}

int Stager::init() {
    for (int k = 0; k < kSlots; k++) {
        if (hipHostMalloc(reinterpret_cast<void **>(&slot_[k]), kSlotBytes, hipHostMallocDefault) != hipSuccess) {
            slot_[k] = nullptr;
            return qasr_fail(QASR_ERR_NOMEM, "upload: pinned staging allocation failed");
        }
        HIPCHK(hipEventCreateWithFlags(&ev_[k], hipEventDisableTiming));
    }
    // copy threads: QASR_UPLOAD_THREADS, else up to 8 of the host's cores
    const unsigned hw = std::thread::hardware_concurrency();
    static const int forced = [] { const char *e = getenv("QASR_UPLOAD_THREADS"); return e ? atoi(e) : 0; }();
    n_parts_ = forced > 0 ? std::min(forced, 64) : (int)std::max(1u, std::min(8u, hw ? hw : 1u));
    for (int p = 1; p < n_parts_; p++) th_.emplace_back(&Stager::worker, this, p);
    return QASR_OK;
}

void Stager::worker(int part) {
    unsigned long seen = 0;
    for (;;) {
        std::function<void(int, int)> job;
        {
            std::unique_lock<std::mutex> g(m_);
            cv_.wait(g, [&] { return stop_ || gen_ != seen; });
            if (stop_) return;
            seen = gen_;
            job = job_;
        }
        job(part, n_parts_);
        std::lock_guard<std::mutex> g(m_);
        if (--pending_ == 0) done_.notify_one();
    }
}

void Stager::run(const std::function<void(int, int)> &job) {
    {
        std::lock_guard<std::mutex> g(m_);
        job_ = job;
        pending_ = n_parts_ - 1;
        gen_++;
    }
    cv_.notify_all();
    job(0, n_parts_);
    std::unique_lock<std::mutex> g(m_);
    done_.wait(g, [&] { return pending_ == 0; });
}

// fill(slot, part, n_parts) writes this part's share of `bytes` staged bytes;
// the slot then drains to dst on the stream
int Stager::stage(void *dst, size_t bytes, const std::function<void(char *, int, int)> &fill) {
    const int k = next_;
    next_ = (next_ + 1) % kSlots;
    if (used_[k]) HIPCHK(hipEventSynchronize(ev_[k]));   // the slot's previous transfer has landed
    char *s = slot_[k];
    run([&](int part, int n) { fill(s, part, n); });
    HIPCHK(hipMemcpyAsync(dst, s, bytes, hipMemcpyHostToDevice, st_));
    HIPCHK(hipEventRecord(ev_[k], st_));
    used_[k] = true;
    return QASR_OK;
}

int Stager::upload_rows(void *dst, const void *const *srcs, int n_src, int64_t rows, size_t row_bytes) {
    char *d = reinterpret_cast<char *>(dst);
    if (n_src == 1) {
        // one contiguous run of rows * row_bytes bytes, split into slot-sized chunks
        const char *src = reinterpret_cast<const char *>(srcs[0]);
        const size_t total = (size_t)rows * row_bytes;
        for (size_t off = 0; off < total; off += kSlotBytes) {
            const size_t len = std::min(kSlotBytes, total - off);
            int rc = stage(d + off, len, [&](char *s, int part, int n) {
                const size_t a = len * part / n / 64 * 64, b = part + 1 == n ? len : len * (part + 1) / n / 64 * 64;
                if (b > a) std::memcpy(s + a, src + off + a, b - a);
            });
            if (rc != QASR_OK) return rc;
        }
        return QASR_OK;
    }
    const size_t group = (size_t)n_src * row_bytes;
    if (group > kSlotBytes) return qasr_fail(QASR_ERR_INVALID, "upload: interleaved row group exceeds a staging slot");
    const int64_t per = (int64_t)(kSlotBytes / group);
    for (int64_t r0 = 0; r0 < rows; r0 += per) {
        const int64_t nr = std::min(per, rows - r0);
        int rc = stage(d + (size_t)r0 * group, (size_t)nr * group, [&](char *s, int part, int n) {
            const int64_t a = nr * part / n, b = nr * (part + 1) / n;
            for (int64_t r = a; r < b; r++)
                for (int k = 0; k < n_src; k++)
                    std::memcpy(s + (size_t)r * group + (size_t)k * row_bytes,
                                reinterpret_cast<const char *>(srcs[k]) + (size_t)(r0 + r) * row_bytes, row_bytes);
        });
        if (rc != QASR_OK) return rc;
    }
    return QASR_OK;
}

int Stager::finish() {
    for (int k = 0; k < kSlots; k++)
        if (used_[k]) HIPCHK(hipEventSynchronize(ev_[k]));
    return QASR_OK;
}
