// decoder_prefill (decoder.rs:455-547) on the device: f32-class MFMA GEMMs on
// the bf16 weights (as the reference's cblas_sgemm on bf16->f32 weights),
// exact-order RMSNorm rows, per-head norm + RoPE, KV scatter, causal GQA
// attention and the AVX-order SwiGLU.
#include <cmath>

#include "decoder.h"
#include "upload.h"

using namespace qasr;

void decoder_free_prefill(qasr_decoder *d) {
    PrefillBufs &p = d->pf;
    for (float *b : {p.x, p.xn, p.qkv, p.att, p.gu, p.g})
        if (b) (void)hipFree(b);
    p = PrefillBufs{};
}

static int ensure_prefill(qasr_decoder *d, int64_t S) {
    if (S <= d->pf.cap) return QASR_OK;
    HIPCHK(hipStreamSynchronize(d->h->stream));
    decoder_free_prefill(d);
    const qasr_dec_config &c = d->c;
    const int64_t H = c.hidden, qd = (int64_t)c.n_heads * c.head_dim, kvd = (int64_t)c.n_kv_heads * c.head_dim;
    const int64_t I = c.intermediate, cap = std::max<int64_t>(64, S);
    PrefillBufs &p = d->pf;
    struct { float **ptr; int64_t n; } bufs[] = {
        {&p.x, cap * H}, {&p.xn, cap * H}, {&p.qkv, cap * (qd + 2 * kvd)}, {&p.att, cap * qd},
        {&p.gu, cap * 2 * I}, {&p.g, cap * I}};
    for (auto &b : bufs) {
        hipError_t e = hipMalloc(b.ptr, sizeof(float) * b.n);
        if (e != hipSuccess) {
            decoder_free_prefill(d);
            return qasr_fail(QASR_ERR_NOMEM, "decoder_prefill: buffer allocation failed");
        }
    }
    p.cap = cap;
    return QASR_OK;
}

// The prefill GEMMs split K by the shape alone (split_by_shape), so that a
// row's result is the same whether its sequence is prefilled alone or with
// others; their partials live in the decoder's grow-only workspace.
static int gemm(qasr_decoder *d, const float *A, int64_t lda, const uint16_t *B, int64_t ldb, float *C,
                int64_t ldc, int M, int N, int K, int epi) {
    GemmArgs g{};
    g.M = M; g.N = N; g.K = K;
    g.A = A; g.lda = lda; g.B = B; g.ldb = ldb; g.C = C; g.ldc = ldc;
    g.ws = d->gemm_ws.as<float>(); g.ws_bytes = (int64_t)d->gemm_ws.cap;   // split-K partials
    g.split_by_shape = 1;
    LAUNCHCHK(launch_gemm(g, A_F32_SPLIT, B_BF16, epi, d->h->stream), "prefill gemm");
    return QASR_OK;
}

#define TRY(x)                  \
    do {                        \
        int rc_ = (x);          \
        if (rc_ != QASR_OK) {   \
            return rc_;         \
        }                       \
    } while (0)

int decoder_prefill_segments(qasr_decoder *d, const PrefillSeg *segs, int n_seg) {
    const qasr_dec_config &c = d->c;
    if (d->kv_bf16) return qasr_fail(QASR_ERR_INVALID, "decoder_prefill: needs an f32 KV cache");
    int64_t S = 0;
    for (int i = 0; i < n_seg; i++) {
        const PrefillSeg &g = segs[i];
        if (g.n < 0 || g.start < 0 || (g.n > 0 && (!g.rows || !g.kc || !g.vc)))
            return qasr_fail(QASR_ERR_INVALID, "decoder_prefill: bad sequence");
        if (g.start + g.n > g.cap) return qasr_fail(QASR_ERR_INVALID, "decoder_prefill: KV cache capacity exceeded");
        S += g.n;
    }
    if (S <= 0) return QASR_OK;
    if (S > (1 << 30) / 8) return qasr_fail(QASR_ERR_INVALID, "decoder_prefill: too many rows");
    TRY(ensure_prefill(d, S));
    TRY(dbuf_ensure(d->gemm_ws, sizeof(float) * 2 * (size_t)S * 1024, d->h->stream));
    hipStream_t st = d->h->stream;
    PrefillBufs &p = d->pf;
    const int H = c.hidden, hd = c.head_dim, qd = c.n_heads * hd, kvd = c.n_kv_heads * hd;
    const int I = c.intermediate, nqkv = qd + 2 * kvd;
    const int M = (int)S;
    const float scale = 1.0f / sqrtf((float)hd);
    // one launch for every sequence's q/k post-processing and attention when
    // there are several (at most 32, the decoder's 128-dim heads with two
    // query heads per KV head, one head stride: the attention reads it from
    // the shared arguments)
    int n_live = 0;
    int64_t segs_head_stride = -1;
    bool same_stride = true;
    for (int i = 0; i < n_seg; i++)
        if (segs[i].n > 0) {
            n_live++;
            if (segs_head_stride < 0) segs_head_stride = segs[i].head_stride;
            same_stride = same_stride && segs[i].head_stride == segs_head_stride && segs[i].head_stride % 4 == 0 &&
                          segs[i].layer_elems % 4 == 0 && (uintptr_t)segs[i].kc % 16 == 0 &&
                          (uintptr_t)segs[i].vc % 16 == 0;   // the MFMA form's float4 K/V loads
        }
    const bool multi = n_live > 1 && n_live <= QASR_ATTN_MAX_SEQ && hd == 128 && c.n_heads == 2 * c.n_kv_heads &&
                       same_stride;
    {
        int64_t off = 0;
        for (int i = 0; i < n_seg; i++) {
            if (segs[i].n > 0)
                HIPCHK(hipMemcpyAsync(p.x + off * H, segs[i].rows, sizeof(float) * segs[i].n * H,
                                      hipMemcpyDeviceToDevice, st));
            off += segs[i].n;
        }
    }
    for (int l = 0; l < c.n_layers; l++) {
        const DecLayerDev &L = d->L[l];
        LAUNCHCHK(launch_rms_norm_rows(p.xn, p.x, L.in_norm, S, H, c.eps, st), "prefill rms_norm");
        TRY(gemm(d, p.xn, H, L.bqkv, H, p.qkv, nqkv, M, nqkv, H, EPI_NONE));
        if (multi) {
            // every sequence's q/k norm, RoPE and KV write, then its causal
            // attention, one launch each (each sequence's rows get the bits of
            // its own launches)
            PrefillPostSeqArgs pp{};
            pp.base.qkv = p.qkv; pp.base.row_stride = nqkv; pp.base.Hq = c.n_heads; pp.base.Hkv = c.n_kv_heads;
            pp.base.q_norm = L.q_norm; pp.base.k_norm = L.k_norm; pp.base.cos_t = d->rc; pp.base.sin_t = d->rs;
            pp.base.eps = c.eps;
            AttnSeqArgs as{};
            as.base.q = p.qkv; as.base.q_rs = nqkv; as.base.k_hs = 0; as.base.k_rs = hd;
            as.base.out = p.att; as.base.o_rs = qd;
            as.base.G = c.n_heads / c.n_kv_heads; as.base.window = 0; as.base.scale = scale;
            int64_t off = 0;
            for (int i = 0; i < n_seg; i++) {
                const PrefillSeg &g = segs[i];
                if (g.n == 0) continue;
                const int j = pp.n++;
                pp.row[j] = off;
                pp.start[j] = g.start;
                pp.head_stride[j] = g.head_stride;
                pp.kc[j] = g.kc + l * g.layer_elems;
                pp.vc[j] = g.vc + l * g.layer_elems;
                as.row[j] = off;
                as.k[j] = pp.kc[j];
                as.v[j] = pp.vc[j];
                as.n_q[j] = (int)g.n;
                as.n_k[j] = (int)(g.start + g.n);
                as.q_offset[j] = (int)g.start;
                off += g.n;
            }
            pp.row[pp.n] = off;
            as.n = pp.n;
            as.base.k_hs = segs_head_stride;
            LAUNCHCHK(launch_prefill_qkv_post_seqs(pp, st), "prefill q/k norm, rope and kv write");
            LAUNCHCHK(launch_attn_rows_seqs(as, c.n_kv_heads, hd, st), "prefill attention");
        }
        int64_t off = 0;
        for (int i = 0; i < n_seg && !multi; i++) {
            const PrefillSeg &g = segs[i];
            if (g.n == 0) continue;
            float *kc = g.kc + l * g.layer_elems;
            float *vc = g.vc + l * g.layer_elems;
            PrefillPostArgs pp{};
            pp.qkv = p.qkv + off * nqkv; pp.row_stride = nqkv; pp.S = g.n; pp.Hq = c.n_heads; pp.Hkv = c.n_kv_heads;
            pp.q_norm = L.q_norm; pp.k_norm = L.k_norm; pp.cos_t = d->rc + g.start * hd; pp.sin_t = d->rs + g.start * hd;
            pp.kc = kc; pp.vc = vc; pp.head_stride = g.head_stride; pp.start = g.start; pp.eps = c.eps;
            LAUNCHCHK(launch_prefill_qkv_post(pp, st), "prefill q/k norm, rope and kv write");
            AttnRowsArgs a{};
            a.q = p.qkv + off * nqkv; a.q_rs = nqkv;
            a.k = kc; a.v = vc; a.k_hs = g.head_stride; a.k_rs = hd;
            a.out = p.att + off * qd; a.o_rs = qd;
            a.n_q = (int)g.n; a.n_k = (int)(g.start + g.n);
            a.G = c.n_heads / c.n_kv_heads; a.q_offset = (int)g.start; a.window = 0; a.scale = scale;
            LAUNCHCHK(launch_attn_rows(a, c.n_kv_heads, hd, st), "prefill attention");
            off += g.n;
        }
        TRY(gemm(d, p.att, qd, L.bo, qd, p.x, H, M, H, qd, EPI_ACCUM));
        LAUNCHCHK(launch_rms_norm_rows(p.xn, p.x, L.post_norm, S, H, c.eps, st), "prefill rms_norm");
        // gate_up with the SwiGLU in its epilogue (interleaved gate / up rows)
        TRY(gemm(d, p.xn, H, L.bgu, H, p.g, I, M, 2 * I, H, EPI_SWIGLU));
        TRY(gemm(d, p.g, I, L.bdown, I, p.x, H, M, H, I, EPI_ACCUM));
    }
    return QASR_OK;
}

int decoder_prefill_dev(qasr_decoder *d, const float *emb_dev, int64_t S) {
    const qasr_dec_config &c = d->c;
    if (S <= 0) return QASR_OK;
    PrefillSeg g;
    g.rows = emb_dev;
    g.n = S;
    g.start = d->len;
    g.kc = reinterpret_cast<float *>(d->kc);
    g.vc = reinterpret_cast<float *>(d->vc);
    g.head_stride = d->max_seq * c.head_dim;
    g.layer_elems = d->kv_layer_stride ? d->kv_layer_stride : (int64_t)c.n_kv_heads * g.head_stride;
    g.cap = d->max_seq;
    TRY(decoder_prefill_segments(d, &g, 1));
    d->len = g.start + S;
    return QASR_OK;
}

extern "C" int qasr_hip_decoder_prefill(qasr_decoder *d, const float *embeds, int64_t seq_len) {
    if (!d) return qasr_fail(QASR_ERR_INVALID, "decoder is null");
    CHECK_H(d->h);
    if (seq_len < 0 || (seq_len > 0 && !embeds)) return qasr_fail(QASR_ERR_INVALID, "decoder_prefill: bad arguments");
    if (seq_len == 0) return QASR_OK;
    TRY(decoder_reserve(d, d->len + seq_len));
    TRY(ensure_prefill(d, seq_len));
    // stage the host rows in the layer-norm buffer, then run from device memory
    HIPCHK(hipMemcpyAsync(d->pf.xn, embeds, sizeof(float) * seq_len * d->c.hidden, hipMemcpyHostToDevice,
                          d->h->stream));
    TRY(decoder_prefill_dev(d, d->pf.xn, seq_len));
    HIPCHK(hipStreamSynchronize(d->h->stream));
    return QASR_OK;
}

int decoder_prefill_hidden(qasr_decoder *d, float *host_out, int64_t seq_len) {
    HIPCHK(hipMemcpyAsync(host_out, d->pf.x, sizeof(float) * seq_len * d->c.hidden, hipMemcpyDeviceToHost,
                          d->h->stream));
    HIPCHK(hipStreamSynchronize(d->h->stream));
    return QASR_OK;
}

// The bf16 LM head decoder_prefill_logits projects onto (decoder.lm_head_bf16,
// decoder.rs:143, 671): w [out_dim][hidden] host bf16, copied to the device;
// null restores the tied embedding.
extern "C" int qasr_hip_decoder_set_lm_head(qasr_decoder *d, const uint16_t *w, int64_t out_dim) {
    if (!d) return qasr_fail(QASR_ERR_INVALID, "decoder is null");
    CHECK_H(d->h);
    HIPCHK(hipStreamSynchronize(d->h->stream));
    if (d->lm_bf16) (void)hipFree(d->lm_bf16);
    d->lm_bf16 = nullptr;
    d->lm_rows = 0;
    if (!w) return QASR_OK;
    if (out_dim <= 0) return qasr_fail(QASR_ERR_INVALID, "set_lm_head: out_dim must be positive");
    const size_t bytes = sizeof(uint16_t) * out_dim * d->c.hidden;
    if (hipMalloc(&d->lm_bf16, bytes) != hipSuccess) {
        d->lm_bf16 = nullptr;
        return qasr_fail(QASR_ERR_NOMEM, "set_lm_head: device allocation failed");
    }
    // one synchronous copy from the caller's memory (the form whose GPU tests
    // pass; the checkpoint loader no longer hands its mapping to this call)
    if (hipMemcpy(d->lm_bf16, w, bytes, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(d->lm_bf16);
        d->lm_bf16 = nullptr;
        return qasr_fail(QASR_ERR_HIP, "set_lm_head: upload failed");
    }
    d->lm_rows = out_dim;
    return QASR_OK;
}

extern "C" int64_t qasr_hip_decoder_head_rows(const qasr_decoder *d) { return d ? d->lm_i8_rows : -1; }

extern "C" int64_t qasr_hip_decoder_logits_dim(const qasr_decoder *d) {
    return d ? (d->lm_rows ? d->lm_rows : d->c.vocab) : -1;
}

// decoder_prefill_logits (decoder.rs:649-681) on the device: the prefill,
// then the final RMSNorm and the bf16 LM head (f32-class MFMA GEMM, as the
// reference's linear_nobias_bf16 f32 sgemm) over the prefill rows `rows` (host,
// nullptr: all seq_len rows in order; each row's logits depend on that row
// alone, so a subset computes exactly those rows).  Downloads the logits
// [n][out_dim] when `logits` is set and the aligner's per-row argmax
// (align.rs:312-321) when `idx` is set.
static int prefill_head_rows(qasr_decoder *d, const float *embeds, int64_t seq_len, const int32_t *rows, int64_t n,
                             float *logits, int32_t *idx) {
    if (!d) return qasr_fail(QASR_ERR_INVALID, "decoder is null");
    CHECK_H(d->h);
    if (seq_len <= 0 || !embeds) return qasr_fail(QASR_ERR_INVALID, "prefill_logits: bad arguments");
    if (d->kv_bf16) return qasr_fail(QASR_ERR_INVALID, "prefill_logits: needs an f32 KV cache");
    TRY(decoder_reserve(d, d->len + seq_len));
    if (rows)
        for (int64_t k = 0; k < n; k++)
            if (rows[k] < 0 || rows[k] >= seq_len) return qasr_fail(QASR_ERR_INVALID, "prefill_argmax: row out of range");
    const int64_t H = d->c.hidden, out_dim = qasr_hip_decoder_logits_dim(d);
    if (rows && 2 * (int64_t)d->c.intermediate < H)
        return qasr_fail(QASR_ERR_INVALID, "prefill_argmax: unsupported shape (intermediate < hidden / 2)");
    const uint16_t *w = d->lm_bf16 ? d->lm_bf16 : d->embed;
    TRY(ensure_prefill(d, seq_len));
    hipStream_t st = d->h->stream;
    // one device block: logits [n][out_dim], row list [n], argmax [n]
    const size_t y_bytes = (sizeof(float) * n * out_dim + 255) / 256 * 256;
    if (n > 0) TRY(dbuf_ensure(d->head_out, y_bytes + 2 * sizeof(int32_t) * n, d->h->stream));
    char *buf = d->head_out.as<char>();
    float *y = reinterpret_cast<float *>(buf);
    int32_t *rows_dev = reinterpret_cast<int32_t *>(buf + y_bytes), *idx_dev = rows_dev + n;
    auto body = [&]() -> int {
        HIPCHK(hipMemcpyAsync(d->pf.xn, embeds, sizeof(float) * seq_len * H, hipMemcpyHostToDevice, st));
        TRY(decoder_prefill_dev(d, d->pf.xn, seq_len));
        if (n == 0) return QASR_OK;
        const float *src = d->pf.x;
        if (rows) {
            HIPCHK(hipMemcpyAsync(rows_dev, rows, sizeof(int32_t) * n, hipMemcpyHostToDevice, st));
            LAUNCHCHK(launch_gather_rows(d->pf.gu, d->pf.x, rows_dev, n, H, st), "logits row gather");
            src = d->pf.gu;
        }
        LAUNCHCHK(launch_rms_norm_rows(d->pf.xn, src, d->norm, n, (int)H, d->c.eps, st), "logits rms_norm");
        TRY(gemm(d, d->pf.xn, H, w, H, y, out_dim, (int)n, (int)out_dim, (int)H, EPI_NONE));
        if (logits)
            HIPCHK(hipMemcpyAsync(logits, y, sizeof(float) * n * out_dim, hipMemcpyDeviceToHost, st));
        if (idx) {
            LAUNCHCHK(launch_argmax_f32_rows(y, out_dim, n, out_dim, idx_dev, st), "logits argmax");
            HIPCHK(hipMemcpyAsync(idx, idx_dev, sizeof(int32_t) * n, hipMemcpyDeviceToHost, st));
        }
        return QASR_OK;
    };
    int rc = body();
    const hipError_t e = hipStreamSynchronize(st);
    if (rc != QASR_OK) return rc;
    if (e != hipSuccess) return qasr_fail(QASR_ERR_HIP, "prefill_logits: stream failed");
    return QASR_OK;
}

extern "C" int qasr_hip_decoder_prefill_logits(qasr_decoder *d, const float *embeds, int64_t seq_len,
                                               float *logits) {
    if (!logits) return qasr_fail(QASR_ERR_INVALID, "prefill_logits: logits is null");
    return prefill_head_rows(d, embeds, seq_len, nullptr, seq_len, logits, nullptr);
}

extern "C" int qasr_hip_decoder_prefill_argmax(qasr_decoder *d, const float *embeds, int64_t seq_len,
                                               const int32_t *rows, int64_t n_rows, int32_t *idx) {
    if (n_rows < 0 || (n_rows > 0 && (!rows || !idx)))
        return qasr_fail(QASR_ERR_INVALID, "prefill_argmax: bad row list");
    return prefill_head_rows(d, embeds, seq_len, rows, n_rows, nullptr, idx);
}
