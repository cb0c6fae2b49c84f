// Internal host-side definitions shared by the C-ABI translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <algorithm>
#include <string>
#include <vector>
#include "qasr_hip.h"
#include "kernels.h"

// scratch area of a handle: argmax partials, attention partials
#define QASR_SCRATCH_BYTES (8u << 20)
#define QASR_ARGMAX_MAX_BLOCKS 4096
#define QASR_COUNTERS 1024
#define QASR_CTR_ARGMAX 0
#define QASR_CTR_ATTN 64
#define QASR_CTR_ATTN_N 256
// kernel kinds of qasr_hip_decoder_profile
#define QASR_PROFILE_KINDS 8

struct qasr_hip {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    void *scratch = nullptr;       // QASR_SCRATCH_BYTES
    unsigned *counters = nullptr;  // QASR_COUNTERS, zero between kernels
};

int qasr_fail(int code, const std::string &msg);

// Device buffer owned by a model object and kept between calls: an entry point
// calls hipMalloc only when it needs more bytes than any earlier call on the
// same object (dbuf_ensure waits for the streams that use the buffer, st and
// st2 when given, before it frees the smaller one), so repeated calls of one
// shape allocate nothing.
struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
    template <typename T> T *as() const { return reinterpret_cast<T *>(p); }
};
int dbuf_ensure(DevBuf &b, size_t bytes, hipStream_t st, hipStream_t st2 = nullptr);
void dbuf_release(DevBuf &b);
// Pinned host buffer with the same grow-only rule (device-to-host copies that
// return without waiting land here).
struct HostBuf {
    void *p = nullptr;
    size_t cap = 0;
    template <typename T> T *as() const { return reinterpret_cast<T *>(p); }
};
int hbuf_ensure(HostBuf &b, size_t bytes, hipStream_t st, hipStream_t st2 = nullptr);
void hbuf_release(HostBuf &b);

// Resolves the allocation-free argmax's device scratch address on the current
// device (qasr_hip_create calls it at set-up).
int noalloc_init_device();

// The stream's next push prefills every row instead of reusing the rows its
// previous push left in the decoder's KV cache (another caller has written
// that cache since).
void stream_drop_prefix(qasr_stream *s);
// Replaces the stream's settings (already validated by the caller).
void stream_set_config(qasr_stream *s, const qasr_stream_config &c);

// The id rows of transcribe_segment's prompt around the audio rows
// (transcribe.rs:97-169), each checked to lie in [0, vocab).
int prompt_id_rows(const qasr_prompt *p, const int32_t *past, int64_t n_past, int32_t vocab,
                   std::vector<int32_t> &head, std::vector<int32_t> &tail);

// Multi-stream batch internals used by the streaming driver: chunk prefills
// from device rows into stream KV slots at positions [start, start + n) (one
// slot, or several in one call), the per-stream capacity and the stream count.
int batch_prefill_dev(qasr_batch *b, int32_t stream, const float *rows, int64_t start, int64_t n);
int batch_prefill_segments(qasr_batch *b, int n, const int32_t *slots, const float *const *rows,
                           const int64_t *starts, const int64_t *counts);
int64_t batch_max_seq(const qasr_batch *b);
int32_t batch_streams(const qasr_batch *b);

#define CHECK_H(h)                                                                   \
    do {                                                                             \
        if (!(h)) return qasr_fail(QASR_ERR_INVALID, "handle is null");              \
        hipError_t e_ = hipSetDevice((h)->device);                                   \
        if (e_ != hipSuccess) return qasr_fail(QASR_ERR_HIP, hipGetErrorString(e_)); \
    } while (0)

#define HIPCHK(x)                                                                                    \
    do {                                                                                             \
        hipError_t e_ = (x);                                                                         \
        if (e_ != hipSuccess) return qasr_fail(QASR_ERR_HIP, std::string(#x) + ": " + hipGetErrorString(e_)); \
    } while (0)

#define LAUNCHCHK(x, what)                                                                          \
    do {                                                                                             \
        hipError_t e_ = (x);                                                                         \
        if (e_ == hipErrorInvalidValue) return qasr_fail(QASR_ERR_INVALID, std::string(what) + ": unsupported shape"); \
        if (e_ != hipSuccess) return qasr_fail(QASR_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e_)); \
    } while (0)

// number of context splits of the decode attention for a context of `len`
// positions: about 256 positions per split, at least min(16, len) splits, at
// most 64 (the attention kernel's limit)
static inline int attn_splits_for(int64_t len) {
    int64_t s = std::max<int64_t>((len + 255) / 256, std::min<int64_t>(16, len));
    return (int)std::min<int64_t>(64, std::max<int64_t>(1, s));
}

// o_proj merges the split-attention partials itself for the 16-query-head /
// 8-KV-head shapes (hidden of attention output 2048) at 1, 2, 4, 8 or 16 splits
static inline bool oproj_merges(const qasr_dec_config &c, int n_split) {
    return c.n_kv_heads == 8 && c.n_heads == 16 && c.head_dim == 128 && c.hidden % 4 == 0 &&
           (n_split == 1 || n_split == 2 || n_split == 4 || n_split == 8 || n_split == 16);
}

// Context splits of the decode attention for a context bucket of `cap`
// positions.  Measured on the 0.6B decoder (16 query / 8 KV heads, 4 waves
// per block): 8 splits merged in the o_proj prologue are fastest up to a
// 1024-position bucket (2-4 groups of 8 positions per wave; 16 splits cost
// 1.4 us more in the o_proj merge than they save in the attention), 16 up to
// 2048; longer contexts use about cap / 64 splits (<= 64) merged by the
// attention kernel's last block per KV head.
static inline int attn_splits_auto(const qasr_dec_config &c, int64_t cap) {
    if (oproj_merges(c, 8)) {
        if (cap <= 1024) return 8;
        if (cap <= 2048) return 16;
    }
    return (int)std::min<int64_t>(64, std::max<int64_t>(1, (cap + 63) / 64));
}

// groups per wave of k_attn_step (4 waves per block, each holding its whole
// share of the block's run): 1-4, or 0 when a block's run is longer than 16
// groups (contexts past 8192 positions), where k_attn_decode takes over.
// Measured on the 0.6B decode at contexts 780-980 (1024-position bucket, 16
// groups per block): 666 us/token with k_attn_step (fused with the qkv
// matvec) against 702 us with k_attn_decode.
static inline int attn_step_gpw(int64_t gpb) {
    return gpb <= QASR_STEP_MAX_GPB ? (int)std::max<int64_t>(1, (gpb + 3) / 4) : 0;
}

// blocks of the LM-head argmax grid (4 waves of 4-row groups each): 1024
// blocks (4 per CU) stream the 0.6B LM head in 24.6 us against 26.2 us at
// 512, 26.2 at 1536 and 26.1 at 2048; the merge pass costs 0.3 us more than
// at 512 (measured; 8-row groups were slower at 1024 blocks)
static inline int argmax_blocks(int64_t rows) {
    int64_t groups = (rows + 3) / 4;
    int64_t b = (groups + 3) / 4;
    return (int)std::max<int64_t>(1, std::min<int64_t>(b, 1024));
}
