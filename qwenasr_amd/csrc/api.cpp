// C-ABI of the qasr_hip library: handles, op-level entry points and the
// device-resident Qwen3 decoder.  See include/qasr_hip.h for the contract.
#include "qasr_hip.h"
#include "kernels.h"
#include "model.h"

#include <cmath>
#include <climits>
#include <cstring>
#include <string>
#include <vector>

using namespace qasr;

static thread_local std::string g_err;

int qasr_fail(int code, const std::string &msg) {
    g_err = msg;
    return code;
}

extern "C" const char *qasr_hip_last_error(void) { return g_err.c_str(); }

// waits for the streams whose queued work may still use a buffer about to be freed
static int sync_users(hipStream_t st, hipStream_t st2) {
    HIPCHK(hipStreamSynchronize(st));
    if (st2 && st2 != st) HIPCHK(hipStreamSynchronize(st2));
    return QASR_OK;
}

int dbuf_ensure(DevBuf &b, size_t bytes, hipStream_t st, hipStream_t st2) {
    if (bytes <= b.cap) return QASR_OK;
    if (b.p) {
        int rc = sync_users(st, st2);   // work queued on the old buffer has finished
        if (rc != QASR_OK) return rc;
        (void)hipFree(b.p);
    }
    b.p = nullptr;
    b.cap = 0;
    const size_t want = std::max<size_t>((bytes + 255) / 256 * 256, 4096);
    if (hipMalloc(&b.p, want) != hipSuccess) {
        b.p = nullptr;
        return qasr_fail(QASR_ERR_NOMEM, "device allocation of " + std::to_string(want) + " bytes failed");
    }
    b.cap = want;
    return QASR_OK;
}

void dbuf_release(DevBuf &b) {
    if (b.p) (void)hipFree(b.p);
    b.p = nullptr;
    b.cap = 0;
}

int hbuf_ensure(HostBuf &b, size_t bytes, hipStream_t st, hipStream_t st2) {
    if (bytes <= b.cap) return QASR_OK;
    if (b.p) {
        int rc = sync_users(st, st2);   // copies queued into the old buffer have finished
        if (rc != QASR_OK) return rc;
        (void)hipHostFree(b.p);
    }
    b.p = nullptr;
    b.cap = 0;
    const size_t want = std::max<size_t>((bytes + 255) / 256 * 256, 4096);
    if (hipHostMalloc(&b.p, want, hipHostMallocDefault) != hipSuccess) {
        b.p = nullptr;
        return qasr_fail(QASR_ERR_NOMEM, "pinned host allocation of " + std::to_string(want) + " bytes failed");
    }
    b.cap = want;
    return QASR_OK;
}

void hbuf_release(HostBuf &b) {
    if (b.p) (void)hipHostFree(b.p);
    b.p = nullptr;
    b.cap = 0;
}

extern "C" int qasr_hip_device_count(int *n) {
    if (!n) return qasr_fail(QASR_ERR_INVALID, "n is null");
    HIPCHK(hipGetDeviceCount(n));
    return QASR_OK;
}

extern "C" int qasr_hip_create(int device, qasr_hip **out) {
    if (!out) return qasr_fail(QASR_ERR_INVALID, "out is null");
    *out = nullptr;
    int n = 0;
    HIPCHK(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return qasr_fail(QASR_ERR_INVALID, "device index out of range");
    HIPCHK(hipSetDevice(device));
    qasr_hip *h = new qasr_hip();
    h->device = device;
    hipError_t e = hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreate(&h->ev0);
    if (e == hipSuccess) e = hipEventCreate(&h->ev1);
    if (e == hipSuccess) e = hipMalloc(&h->scratch, QASR_SCRATCH_BYTES);
    if (e == hipSuccess) e = hipMalloc((void **)&h->counters, QASR_COUNTERS * sizeof(unsigned));
    if (e == hipSuccess) e = hipMemset(h->counters, 0, QASR_COUNTERS * sizeof(unsigned));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        qasr_hip_destroy(h);
        return qasr_fail(QASR_ERR_HIP, std::string("qasr_hip_create: ") + hipGetErrorString(e));
    }
    const int rc = noalloc_init_device();
    if (rc != QASR_OK) {
        qasr_hip_destroy(h);
        return rc;
    }
    *out = h;
    return QASR_OK;
}

extern "C" void qasr_hip_destroy(qasr_hip *h) {
    if (!h) return;
    (void)hipSetDevice(h->device);
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    if (h->scratch) (void)hipFree(h->scratch);
    if (h->counters) (void)hipFree(h->counters);
    if (h->ev0) (void)hipEventDestroy(h->ev0);
    if (h->ev1) (void)hipEventDestroy(h->ev1);
    if (h->stream) (void)hipStreamDestroy(h->stream);
    delete h;
}

extern "C" int qasr_hip_synchronize(qasr_hip *h) {
    CHECK_H(h);
    HIPCHK(hipStreamSynchronize(h->stream));
    return QASR_OK;
}

extern "C" void *qasr_hip_stream(qasr_hip *h) { return h ? (void *)h->stream : nullptr; }

extern "C" int qasr_hip_malloc(qasr_hip *h, size_t bytes, void **dptr) {
    CHECK_H(h);
    if (!dptr) return qasr_fail(QASR_ERR_INVALID, "dptr is null");
    hipError_t e = hipMalloc(dptr, bytes ? bytes : 1);
    if (e != hipSuccess) return qasr_fail(QASR_ERR_NOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
    return QASR_OK;
}

extern "C" int qasr_hip_free(qasr_hip *h, void *dptr) {
    CHECK_H(h);
    if (dptr) HIPCHK(hipFree(dptr));
    return QASR_OK;
}

extern "C" int qasr_hip_upload(qasr_hip *h, void *dst, const void *src, size_t bytes) {
    CHECK_H(h);
    if (!bytes) return QASR_OK;
    if (!dst || !src) return qasr_fail(QASR_ERR_INVALID, "null pointer");
    HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, h->stream));
    HIPCHK(hipStreamSynchronize(h->stream));
    return QASR_OK;
}

extern "C" int qasr_hip_download(qasr_hip *h, void *dst, const void *src, size_t bytes) {
    CHECK_H(h);
    if (!bytes) return QASR_OK;
    if (!dst || !src) return qasr_fail(QASR_ERR_INVALID, "null pointer");
    HIPCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, h->stream));
    HIPCHK(hipStreamSynchronize(h->stream));
    return QASR_OK;
}

extern "C" int qasr_hip_memset(qasr_hip *h, void *dst, int value, size_t bytes) {
    CHECK_H(h);
    if (!bytes) return QASR_OK;
    HIPCHK(hipMemsetAsync(dst, value, bytes, h->stream));
    return QASR_OK;
}

extern "C" int qasr_hip_copy(qasr_hip *h, void *dst, const void *src, size_t bytes) {
    CHECK_H(h);
    if ((!dst || !src) && bytes) return qasr_fail(QASR_ERR_INVALID, "copy: null pointer");
    LAUNCHCHK(launch_copy(dst, src, (int64_t)bytes, h->stream), "copy");
    return QASR_OK;
}

extern "C" int qasr_hip_timer_start(qasr_hip *h) {
    CHECK_H(h);
    HIPCHK(hipEventRecord(h->ev0, h->stream));
    return QASR_OK;
}

extern "C" int qasr_hip_timer_stop(qasr_hip *h, float *ms) {
    CHECK_H(h);
    HIPCHK(hipEventRecord(h->ev1, h->stream));
    HIPCHK(hipEventSynchronize(h->ev1));
    float t = 0.0f;
    HIPCHK(hipEventElapsedTime(&t, h->ev0, h->ev1));
    if (ms) *ms = t;
    return QASR_OK;
}

extern "C" int qasr_hip_timer_hold(qasr_hip *h, int us) {
    CHECK_H(h);
    if (us < 0 || us > 100000) return qasr_fail(QASR_ERR_INVALID, "timer_hold: us must be in [0, 100000]");
    LAUNCHCHK(launch_delay(us, h->stream), "timer_hold");
    return QASR_OK;
}

// ---------------------------------------------------------------------------
// op level
// ---------------------------------------------------------------------------

extern "C" int qasr_hip_pack_int8_rows(qasr_hip *h, const uint16_t *w, int64_t n, int64_t k,
                                       int mode, int8_t *q, float *scales) {
    CHECK_H(h);
    if (!w || !q || !scales || n <= 0 || k <= 0 || k > (1 << 24))
        return qasr_fail(QASR_ERR_INVALID, "pack_int8_rows: bad arguments");
    if (mode != QASR_ROUND_HALF_AWAY && mode != QASR_TRUNC)
        return qasr_fail(QASR_ERR_INVALID, "pack_int8_rows: unknown round_mode");
    LAUNCHCHK(launch_pack_int8(w, n, (int)k, mode, q, scales, h->stream), "pack_int8_rows");
    return QASR_OK;
}

extern "C" int qasr_hip_quantize_act(qasr_hip *h, const float *x, int64_t k, int8_t *q, float *scale) {
    CHECK_H(h);
    if (!x || !q || !scale || k <= 0 || k > (1 << 24))
        return qasr_fail(QASR_ERR_INVALID, "quantize_act: bad arguments");
    LAUNCHCHK(launch_quant_act(x, (int)k, q, scale, h->stream), "quantize_act");
    return QASR_OK;
}

// rows per wave: largest of 4/2/1 dividing every segment that still leaves >= 1024 waves
static int pick_rows(int64_t total, std::initializer_list<int64_t> segs, int min_r) {
    for (int r : {4, 2, 1}) {
        if (r < min_r) break;
        bool ok = true;
        for (int64_t s : segs) ok = ok && (s % r == 0);
        if (ok && (total / r >= 1024 || r == min_r)) return r;
    }
    return 0;
}

static int check_mv(int64_t in_dim, bool norm) {
    if (in_dim <= 0 || in_dim % 64 != 0 || in_dim > (norm ? 4096 : 6144))
        return qasr_fail(QASR_ERR_INVALID, "in_dim must be a positive multiple of 64 and <= " +
                                               std::to_string(norm ? 4096 : 6144));
    return QASR_OK;
}

static int mv_common(qasr_hip *h, MvArgs &a, int mode, bool norm, int r, const char *what) {
    if (r == 0) return qasr_fail(QASR_ERR_INVALID, std::string(what) + ": row counts must be multiples of the rows per wave");
    LAUNCHCHK(launch_w8a8(a, mode, norm, false, r, h->stream), what);
    return QASR_OK;
}

extern "C" int qasr_hip_linear_int8(qasr_hip *h, float *y, const float *x, const int8_t *w,
                                    const float *ws, const float *bias, int64_t in_dim,
                                    int64_t out_dim) {
    CHECK_H(h);
    if (int rc = check_mv(in_dim, false)) return rc;
    if (!y || !x || !w || !ws || out_dim <= 0 || out_dim > (1 << 30))
        return qasr_fail(QASR_ERR_INVALID, "linear_int8: bad arguments");
    MvArgs a{};
    a.x = x; a.K = (int)in_dim; a.bias = bias;
    a.seg[0] = {w, ws, y, (int)out_dim};
    a.n_total = (int)out_dim;
    return mv_common(h, a, bias ? MV_BIAS : MV_PLAIN, false, pick_rows(out_dim, {out_dim}, 1), "linear_int8");
}

static int qkv_impl(qasr_hip *h, float *q, float *k, float *v, const float *x, const float *norm_w,
                    float eps, const int8_t *wq, const float *sq, const int8_t *wk, const float *sk,
                    const int8_t *wv, const float *sv, int64_t in_dim, int64_t q_dim, int64_t kv_dim) {
    CHECK_H(h);
    const bool norm = norm_w != nullptr;
    if (int rc = check_mv(in_dim, norm)) return rc;
    if (!q || !k || !v || !x || !wq || !sq || !wk || !sk || !wv || !sv || q_dim <= 0 || kv_dim <= 0)
        return qasr_fail(QASR_ERR_INVALID, "linear_int8_qkv: bad arguments");
    MvArgs a{};
    a.x = x; a.K = (int)in_dim; a.norm_w = norm_w; a.eps = eps;
    a.seg[0] = {wq, sq, q, (int)q_dim};
    a.seg[1] = {wk, sk, k, (int)kv_dim};
    a.seg[2] = {wv, sv, v, (int)kv_dim};
    a.n_total = (int)(q_dim + 2 * kv_dim);
    return mv_common(h, a, MV_PLAIN, norm, pick_rows(a.n_total, {q_dim, kv_dim}, 1), "linear_int8_qkv");
}

extern "C" int qasr_hip_linear_int8_qkv(qasr_hip *h, float *q, float *k, float *v, const float *x,
                                        const int8_t *wq, const float *sq, const int8_t *wk,
                                        const float *sk, const int8_t *wv, const float *sv,
                                        int64_t in_dim, int64_t q_dim, int64_t kv_dim) {
    return qkv_impl(h, q, k, v, x, nullptr, 0.0f, wq, sq, wk, sk, wv, sv, in_dim, q_dim, kv_dim);
}

extern "C" int qasr_hip_rmsnorm_linear_int8_qkv(qasr_hip *h, float *q, float *k, float *v,
                                                const float *x, const float *norm_w, float eps,
                                                const int8_t *wq, const float *sq, const int8_t *wk,
                                                const float *sk, const int8_t *wv, const float *sv,
                                                int64_t in_dim, int64_t q_dim, int64_t kv_dim) {
    if (!norm_w) return qasr_fail(QASR_ERR_INVALID, "norm_w is null");
    return qkv_impl(h, q, k, v, x, norm_w, eps, wq, sq, wk, sk, wv, sv, in_dim, q_dim, kv_dim);
}

static int swiglu_impl(qasr_hip *h, float *ffn, const float *x, const float *norm_w, float eps,
                       const int8_t *w, const float *ws, int64_t in_dim, int64_t inter) {
    CHECK_H(h);
    const bool norm = norm_w != nullptr;
    if (int rc = check_mv(in_dim, norm)) return rc;
    if (!ffn || !x || !w || !ws || inter <= 0 || inter > (1 << 28))
        return qasr_fail(QASR_ERR_INVALID, "linear_int8_swiglu: bad arguments");
    MvArgs a{};
    a.x = x; a.K = (int)in_dim; a.norm_w = norm_w; a.eps = eps;
    a.seg[0] = {w, ws, ffn, (int)(2 * inter)};
    a.n_total = (int)(2 * inter);
    return mv_common(h, a, MV_SWIGLU, norm, pick_rows(2 * inter, {2 * inter}, 2), "linear_int8_swiglu");
}

extern "C" int qasr_hip_linear_int8_swiglu(qasr_hip *h, float *ffn, const float *x, const int8_t *w,
                                           const float *ws, int64_t in_dim, int64_t inter) {
    return swiglu_impl(h, ffn, x, nullptr, 0.0f, w, ws, in_dim, inter);
}

extern "C" int qasr_hip_rmsnorm_linear_int8_swiglu(qasr_hip *h, float *ffn, const float *x,
                                                   const float *norm_w, float eps, const int8_t *w,
                                                   const float *ws, int64_t in_dim, int64_t inter) {
    if (!norm_w) return qasr_fail(QASR_ERR_INVALID, "norm_w is null");
    return swiglu_impl(h, ffn, x, norm_w, eps, w, ws, in_dim, inter);
}

extern "C" int qasr_hip_linear_int8_addto(qasr_hip *h, float *y, const float *x, const int8_t *w,
                                          const float *ws, int64_t in_dim, int64_t out_dim) {
    CHECK_H(h);
    if (int rc = check_mv(in_dim, false)) return rc;
    if (!y || !x || !w || !ws || out_dim <= 0 || out_dim > (1 << 30))
        return qasr_fail(QASR_ERR_INVALID, "linear_int8_addto: bad arguments");
    MvArgs a{};
    a.x = x; a.K = (int)in_dim;
    a.seg[0] = {w, ws, y, (int)out_dim};
    a.n_total = (int)out_dim;
    return mv_common(h, a, MV_ADDTO, false, pick_rows(out_dim, {out_dim}, 1), "linear_int8_addto");
}

static int argmax_impl(qasr_hip *h, const float *x, const float *norm_w, float eps, const int8_t *w,
                       const float *ws, int64_t in_dim, int64_t out_dim, int32_t *idx) {
    CHECK_H(h);
    const bool norm = norm_w != nullptr;
    if (in_dim <= 0 || in_dim % 64 != 0 || in_dim > 4096)
        return qasr_fail(QASR_ERR_INVALID, "argmax_int8: in_dim must be a positive multiple of 64 and <= 4096");
    if (!x || !w || !ws || !idx || out_dim <= 0 || out_dim > (1 << 30))
        return qasr_fail(QASR_ERR_INVALID, "argmax_int8: bad arguments");
    ArgmaxArgs a{};
    a.x = x; a.norm_w = norm_w; a.eps = eps; a.K = (int)in_dim; a.N = (int)out_dim;
    a.w = w; a.ws = ws;
    const int blocks = argmax_blocks(out_dim);
    a.part_val = reinterpret_cast<float *>(h->scratch);
    a.part_idx = reinterpret_cast<int *>(reinterpret_cast<char *>(h->scratch) + QASR_ARGMAX_MAX_BLOCKS * 4);
    a.out_idx = idx;
    LAUNCHCHK(launch_argmax(a, norm, blocks, h->stream), "argmax_int8");
    return QASR_OK;
}

extern "C" int qasr_hip_argmax_int8(qasr_hip *h, const float *x, const int8_t *w, const float *ws,
                                    int64_t in_dim, int64_t out_dim, int32_t *idx) {
    return argmax_impl(h, x, nullptr, 0.0f, w, ws, in_dim, out_dim, idx);
}

extern "C" int qasr_hip_rmsnorm_argmax_int8(qasr_hip *h, const float *x, const float *norm_w,
                                            float eps, const int8_t *w, const float *ws,
                                            int64_t in_dim, int64_t out_dim, int32_t *idx) {
    if (!norm_w) return qasr_fail(QASR_ERR_INVALID, "norm_w is null");
    return argmax_impl(h, x, norm_w, eps, w, ws, in_dim, out_dim, idx);
}

extern "C" int qasr_hip_argmax_f32_rows(qasr_hip *h, const float *x, int64_t ld, int64_t rows, int64_t cols,
                                        int32_t *idx) {
    CHECK_H(h);
    if (!x || !idx || rows < 0 || cols <= 0 || ld < cols || rows > INT32_MAX)
        return qasr_fail(QASR_ERR_INVALID, "argmax_f32_rows: bad arguments");
    LAUNCHCHK(launch_argmax_f32_rows(x, ld, rows, cols, idx, h->stream), "argmax_f32_rows");
    return QASR_OK;
}

extern "C" int qasr_hip_rms_norm(qasr_hip *h, float *out, const float *x, const float *w, int64_t seq,
                                 int64_t hidden, float eps) {
    CHECK_H(h);
    if (!out || !x || !w || seq < 0 || hidden <= 0 || hidden % 64 != 0 || hidden > 4096)
        return qasr_fail(QASR_ERR_INVALID, "rms_norm: hidden must be a positive multiple of 64 and <= 4096");
    if (seq == 0) return QASR_OK;
    LAUNCHCHK(launch_rms_norm_rows(out, x, w, seq, (int)hidden, eps, h->stream), "rms_norm");
    return QASR_OK;
}

extern "C" int qasr_hip_rms_norm_per_head(qasr_hip *h, float *x, const float *w, int64_t seq,
                                          int64_t n_heads, int64_t hd, float eps) {
    CHECK_H(h);
    if (!x || !w || seq < 0 || n_heads <= 0 || hd != 128)
        return qasr_fail(QASR_ERR_INVALID, "rms_norm_per_head: head_dim must be 128");
    if (seq == 0) return QASR_OK;
    LAUNCHCHK(launch_head_norm_rope(x, w, nullptr, nullptr, seq, (int)n_heads, (int)hd, eps, 1, 0, h->stream),
              "rms_norm_per_head");
    return QASR_OK;
}

extern "C" int qasr_hip_apply_rope_neox(qasr_hip *h, float *x, const float *c, const float *s,
                                        int64_t seq, int64_t n_heads, int64_t hd) {
    CHECK_H(h);
    if (!x || !c || !s || seq < 0 || n_heads <= 0 || hd != 128)
        return qasr_fail(QASR_ERR_INVALID, "apply_rope_neox: head_dim must be 128");
    if (seq == 0) return QASR_OK;
    LAUNCHCHK(launch_head_norm_rope(x, nullptr, c, s, seq, (int)n_heads, (int)hd, 0.0f, 0, 1, h->stream),
              "apply_rope_neox");
    return QASR_OK;
}

extern "C" int qasr_hip_causal_attention(qasr_hip *h, float *out, const float *q, const float *k_base,
                                         const float *v_base, int64_t head_stride, int64_t seq_q,
                                         int64_t seq_k, int64_t n_heads, int64_t n_kv_heads,
                                         int64_t hd, float scale, int64_t q_offset) {
    CHECK_H(h);
    if (!out || !q || !k_base || !v_base || seq_q <= 0 || hd != 128 || n_kv_heads <= 0 ||
        n_heads != 2 * n_kv_heads || seq_k < 0 || q_offset < 0 || head_stride < hd || seq_k > (1 << 24))
        return qasr_fail(QASR_ERR_INVALID,
                         "causal_attention: supported shape is head_dim 128, n_heads == 2 * n_kv_heads");
    if (seq_q > 1) {
        AttnRowsArgs a{};
        a.q = q; a.q_rs = n_heads * hd;
        a.k = k_base; a.v = v_base; a.k_hs = head_stride; a.k_rs = hd;
        a.out = out; a.o_rs = n_heads * hd;
        a.n_q = (int)seq_q; a.n_k = (int)seq_k; a.G = (int)(n_heads / n_kv_heads);
        a.q_offset = (int)q_offset; a.window = 0; a.scale = scale;
        LAUNCHCHK(launch_attn_rows(a, (int)n_kv_heads, (int)hd, h->stream), "causal_attention");
        return QASR_OK;
    }
    const int64_t k_end = std::min(q_offset + 1, seq_k);
    if (k_end == 0) {
        HIPCHK(hipMemsetAsync(out, 0, sizeof(float) * n_heads * hd, h->stream));
        return QASR_OK;
    }
    AttnDecodeArgs a{};
    a.qkv = q;
    a.pos = (int)(k_end - 1);
    a.kcache = const_cast<float *>(k_base);
    a.vcache = const_cast<float *>(v_base);
    a.head_stride = head_stride;
    a.n_split = attn_splits_for(k_end);
    const size_t need = (size_t)n_kv_heads * a.n_split * 2 * (hd + 2) * sizeof(float);
    if (need > QASR_SCRATCH_BYTES || n_kv_heads > QASR_CTR_ATTN_N || a.n_split > 64)
        return qasr_fail(QASR_ERR_INVALID, "causal_attention: context too long for the scratch area");
    a.part = reinterpret_cast<float *>(h->scratch);
    a.counters = h->counters + QASR_CTR_ATTN;
    a.out = out;
    a.scale = scale;
    LAUNCHCHK(launch_attn_decode(a, (int)n_heads, (int)n_kv_heads, (int)hd, 0, h->stream), "causal_attention");
    return QASR_OK;
}

extern "C" int qasr_hip_causal_attention_bf16kv(qasr_hip *h, float *out, const float *q, const uint16_t *k_base,
                                                const uint16_t *v_base, int64_t head_stride, int64_t seq_k,
                                                int64_t n_heads, int64_t n_kv_heads, int64_t hd, float scale,
                                                int64_t q_offset) {
    CHECK_H(h);
    if (!out || !q || !k_base || !v_base || hd != 128 || n_kv_heads <= 0 || n_heads != 2 * n_kv_heads ||
        seq_k < 0 || q_offset < 0 || head_stride < hd || seq_k > (1 << 24))
        return qasr_fail(QASR_ERR_INVALID,
                         "causal_attention_bf16kv: supported shape is head_dim 128, n_heads == 2 * n_kv_heads");
    const int64_t k_end = std::min(q_offset + 1, seq_k);
    if (k_end == 0) {
        HIPCHK(hipMemsetAsync(out, 0, sizeof(float) * n_heads * hd, h->stream));
        return QASR_OK;
    }
    AttnDecodeArgs a{};
    a.qkv = q;
    a.pos = (int)(k_end - 1);
    a.kcache = const_cast<uint16_t *>(k_base);
    a.vcache = const_cast<uint16_t *>(v_base);
    a.head_stride = head_stride;
    a.n_split = attn_splits_for(k_end);
    const size_t need = (size_t)n_kv_heads * a.n_split * 2 * (hd + 2) * sizeof(float);
    if (need > QASR_SCRATCH_BYTES || n_kv_heads > QASR_CTR_ATTN_N || a.n_split > 64)
        return qasr_fail(QASR_ERR_INVALID, "causal_attention_bf16kv: context too long for the scratch area");
    a.part = reinterpret_cast<float *>(h->scratch);
    a.counters = h->counters + QASR_CTR_ATTN;
    a.out = out;
    a.scale = scale;
    LAUNCHCHK(launch_attn_decode(a, (int)n_heads, (int)n_kv_heads, (int)hd, 1, h->stream), "causal_attention_bf16kv");
    return QASR_OK;
}

extern "C" int qasr_hip_bidirectional_attention(qasr_hip *h, float *out, const float *q, const float *k,
                                                const float *v, int64_t seq, int64_t n_heads, int64_t hd,
                                                float scale, int64_t window) {
    CHECK_H(h);
    if (!out || !q || !k || !v || seq <= 0 || n_heads <= 0 || (hd != 64 && hd != 128) || window <= 0 ||
        seq > (1 << 24))
        return qasr_fail(QASR_ERR_INVALID, "bidirectional_attention: bad arguments (head_dim 64 or 128)");
    AttnRowsArgs a{};
    a.q = q; a.q_rs = n_heads * hd;
    a.k = k; a.v = v; a.k_hs = hd; a.k_rs = n_heads * hd;
    a.out = out; a.o_rs = n_heads * hd;
    a.n_q = (int)seq; a.n_k = (int)seq; a.G = 1; a.q_offset = 0; a.window = (int)window; a.scale = scale;
    LAUNCHCHK(launch_attn_rows(a, (int)n_heads, (int)hd, h->stream), "bidirectional_attention");
    return QASR_OK;
}

extern "C" int qasr_hip_linear_bf16w(qasr_hip *h, float *y, const float *x, const uint16_t *w,
                                     const float *bias, int64_t seq, int64_t in_dim, int64_t out_dim,
                                     int accumulate) {
    CHECK_H(h);
    if (!y || !x || !w || seq <= 0 || in_dim <= 0 || out_dim <= 0 || seq > (1 << 28) || in_dim > (1 << 24) ||
        out_dim > (1 << 28))
        return qasr_fail(QASR_ERR_INVALID, "linear_bf16w: bad arguments");
    GemmArgs g{};
    g.M = (int)seq; g.N = (int)out_dim; g.K = (int)in_dim;
    g.A = x; g.lda = in_dim; g.B = w; g.ldb = in_dim; g.C = y; g.ldc = out_dim; g.bias = bias;
    g.ws = reinterpret_cast<float *>(h->scratch); g.ws_bytes = QASR_SCRATCH_BYTES;   // split-K partials
    LAUNCHCHK(launch_gemm(g, A_F32_SPLIT, B_BF16, accumulate ? EPI_ACCUM : EPI_NONE, h->stream), "linear_bf16w");
    return QASR_OK;
}

extern "C" int qasr_hip_gemm_w8_bf16(qasr_hip *h, float *y, const uint16_t *a, const int8_t *w,
                                     const float *scales, int64_t M, int64_t N, int64_t K) {
    CHECK_H(h);
    if (!y || !a || !w || !scales || M <= 0 || N <= 0 || K <= 0 || M > (1 << 28) || N > (1 << 28) ||
        K > (1 << 24))
        return qasr_fail(QASR_ERR_INVALID, "gemm_w8_bf16: bad arguments");
    GemmArgs g{};
    g.M = (int)M; g.N = (int)N; g.K = (int)K;
    g.A = a; g.lda = K; g.B = w; g.ldb = K; g.C = y; g.ldc = N; g.scale = scales;
    g.ws = reinterpret_cast<float *>(h->scratch); g.ws_bytes = QASR_SCRATCH_BYTES;   // split-K partials
    LAUNCHCHK(launch_gemm(g, A_BF16, B_I8, EPI_SCALE, h->stream), "gemm_w8_bf16");
    return QASR_OK;
}

extern "C" int qasr_hip_layer_norm(qasr_hip *h, float *out, const float *x, const float *w, const float *b,
                                   int64_t seq, int64_t hidden, float eps) {
    CHECK_H(h);
    if (!out || !x || !w || !b || seq < 0 || hidden <= 0 || hidden % 16 != 0 || hidden > 4096)
        return qasr_fail(QASR_ERR_INVALID, "layer_norm: hidden must be a positive multiple of 16 and <= 4096");
    if (seq == 0) return QASR_OK;
    LAUNCHCHK(launch_layer_norm_rows(out, x, w, b, seq, (int)hidden, eps, h->stream), "layer_norm");
    return QASR_OK;
}
