/*
 * qasr_oracle — CPU restatement of huanglizhuo/QwenASR's int8 inference path.
 * TEST INFRASTRUCTURE ONLY (the parity checker; never part of the product).
 *
 * Built with -ffp-contract=off: every fused multiply-add below is an explicit
 * fmaf() placed where the reference calls _mm256_fmadd_ps / vfmaq_f32.
 * Citations are relative to crates/qwen-asr/src/ of the reference.
 */
#include "qasr_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <omp.h>

/* Thread count the reference's pool would use (MAX_THREADS, kernels/mod.rs:184).
 * Only gelu()'s per-thread chunking depends on it (mod.rs:1255-1275). */
#define REF_THREADS 16

static int g_threads = 8;
void or_set_threads(int n) { g_threads = n < 1 ? 1 : n; omp_set_num_threads(g_threads); }
int or_get_threads(void) { return g_threads; }

static inline float bf16f(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void or_bf16_to_f32(float *dst, const uint16_t *src, int64_t n) {   /* avx.rs:7-23 */
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) dst[i] = bf16f(src[i]);
}

/* ======================================================================= */
/* int8                                                                     */
/* ======================================================================= */

static inline int8_t sat_i8_from_i32(int32_t v) {   /* vqmovn_s32 then vqmovn_s16 */
    if (v > 32767) v = 32767;
    if (v < -32768) v = -32768;
    if (v > 127) v = 127;
    if (v < -128) v = -128;
    return (int8_t)v;
}

static inline int32_t cvt_trunc_sat_i32(float f) {  /* vcvtq_s32_f32 */
    if (f != f) return 0;
    if (f >= 2147483648.0f) return 2147483647;
    if (f <= -2147483648.0f) return (-2147483647 - 1);
    return (int32_t)f;
}

static inline int8_t round_clamp_i8(float f) {      /* (v).round().clamp(-127,127) as i8 */
    float r = roundf(f);
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    return (int8_t)r;
}

/* quantize_bf16_weights_to_int8: generic/x86 (kernels/mod.rs:1805-1829) and
 * NEON quantize_bf16_to_int8 (kernels/neon.rs:637-694). */
void or_quantize_bf16_rows(const uint16_t *w, int64_t n, int64_t k, int mode,
                           int8_t *q, float *scales) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n; r++) {
        const uint16_t *row = w + r * k;
        float max_abs = 0.0f;
        for (int64_t i = 0; i < k; i++) {
            float v = fabsf(bf16f(row[i]));
            if (v > max_abs) max_abs = v;
        }
        float scale = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
        float inv = 127.0f / fmaxf(max_abs, 1e-10f);
        scales[r] = scale;
        int8_t *dst = q + r * k;
        int64_t vec_end = mode == OR_TRUNC ? k - (k % 8) : 0;
        for (int64_t i = 0; i < vec_end; i++)            /* neon.rs:673-683 */
            dst[i] = sat_i8_from_i32(cvt_trunc_sat_i32(bf16f(row[i]) * inv));
        for (int64_t i = vec_end; i < k; i++)            /* mod.rs:1821-1824, neon.rs:685-690 */
            dst[i] = round_clamp_i8(bf16f(row[i]) * inv);
    }
}

/* quantize_f32_to_int8 (kernels/mod.rs:1795-1802) */
float or_quantize_act(const float *x, int64_t k, int8_t *q) {
    float max_abs = 0.0f;
    for (int64_t i = 0; i < k; i++) max_abs = fmaxf(max_abs, fabsf(x[i]));
    float scale = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
    float inv = 127.0f / fmaxf(max_abs, 1e-10f);
    for (int64_t i = 0; i < k; i++) q[i] = round_clamp_i8(x[i] * inv);
    return scale;
}

/* int32 dot of the 16-element blocks (neon.rs:723-749).  The sum is an exact
 * integer, so any order gives the same value; x86 SIMD restates the NEON SDOT
 * loop.  a is the quantized activation (|a| <= 127): |a| (u8) times b with a's
 * sign moved onto it is a*b, and a pair of such products is at most
 * 2 * 127 * 127 < 2^15, so maddubs never saturates.  AVX-512 VNNI when the
 * host has it, else AVX2 (the build's baseline). */
#include <immintrin.h>

__attribute__((target("avx512f,avx512bw,avx512vnni")))
static int32_t dot_i8_vnni512(const int8_t *a, const int8_t *b, int64_t k16) {
    __m512i acc = _mm512_setzero_si512();
    int64_t i = 0;
    for (; i + 64 <= k16; i += 64) {
        const __m512i va = _mm512_loadu_si512((const void *)(a + i));
        const __m512i vb = _mm512_loadu_si512((const void *)(b + i));
        const __mmask64 neg = _mm512_movepi8_mask(va);
        const __m512i sb = _mm512_mask_sub_epi8(vb, neg, _mm512_setzero_si512(), vb);
        acc = _mm512_dpbusd_epi32(acc, _mm512_abs_epi8(va), sb);
    }
    int32_t s = _mm512_reduce_add_epi32(acc);
    for (; i < k16; i++) s += (int32_t)a[i] * (int32_t)b[i];
    return s;
}

__attribute__((target("avx2")))
static int32_t dot_i8_avx2(const int8_t *a, const int8_t *b, int64_t k16) {
    __m256i acc = _mm256_setzero_si256();
    const __m256i ones = _mm256_set1_epi16(1);
    int64_t i = 0;
    for (; i + 32 <= k16; i += 32) {
        const __m256i va = _mm256_loadu_si256((const __m256i *)(a + i));
        const __m256i vb = _mm256_loadu_si256((const __m256i *)(b + i));
        const __m256i p = _mm256_maddubs_epi16(_mm256_abs_epi8(va), _mm256_sign_epi8(vb, va));
        acc = _mm256_add_epi32(acc, _mm256_madd_epi16(p, ones));
    }
    __m128i h = _mm_add_epi32(_mm256_castsi256_si128(acc), _mm256_extracti128_si256(acc, 1));
    h = _mm_add_epi32(h, _mm_shuffle_epi32(h, 0x4E));
    h = _mm_add_epi32(h, _mm_shuffle_epi32(h, 0xB1));
    int32_t s = _mm_cvtsi128_si32(h);
    for (; i < k16; i++) s += (int32_t)a[i] * (int32_t)b[i];
    return s;
}

static int g_vnni512 = -1;

static inline int32_t dot_i8_blocks(const int8_t *a, const int8_t *b, int64_t k16) {
    if (g_vnni512 < 0)
        g_vnni512 = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
                    __builtin_cpu_supports("avx512vnni");
    return g_vnni512 ? dot_i8_vnni512(a, b, k16) : dot_i8_avx2(a, b, k16);
}

/* 0: AVX2, 1: AVX-512 VNNI when the host has it (tests run both) */
void or_set_int8_dot(int vnni512) {
    g_vnni512 = vnni512 && __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
                __builtin_cpu_supports("avx512vnni");
}

/* which int8 dot the host runs (reported with the CPU baseline) */
const char *or_int8_dot_kind(void) {
    dot_i8_blocks(NULL, NULL, 0);
    return g_vnni512 ? "avx512-vnni vpdpbusd" : "avx2 vpmaddubsw";
}

/* neon::matvec_int8 (kernels/neon.rs:716-793) */
void or_matvec_w8a8(float *y, const int8_t *xq, float xs, const int8_t *w,
                    const float *ws, const float *bias, int64_t k, int64_t n) {
    int64_t k16 = k - (k % 16);
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < n; o++) {
        const int8_t *row = w + o * k;
        int32_t acc = dot_i8_blocks(xq, row, k16);
        float v = (float)acc * xs * ws[o];
        for (int64_t i = k16; i < k; i++)                /* scalar tail, neon.rs:754-760 */
            v += (float)xq[i] * (float)row[i] * xs * ws[o];
        if (bias) v += bias[o];
        y[o] = v;
    }
}

/* int8_matvec_threaded (kernels/mod.rs:839-880) */
void or_linear_int8(float *y, const float *x, const int8_t *w, const float *ws,
                    const float *bias, int64_t k, int64_t n) {
    int8_t *xq = (int8_t *)malloc((size_t)k);
    float xs = or_quantize_act(x, k, xq);
    or_matvec_w8a8(y, xq, xs, w, ws, bias, k, n);
    free(xq);
}

/* linear_nobias_int8_qkv (kernels/mod.rs:884-967): one activation quant, three matvecs */
void or_linear_int8_qkv(float *q, float *kk, float *v, const float *x,
                        const int8_t *wq, const float *sq, const int8_t *wk, const float *sk,
                        const int8_t *wv, const float *sv, int64_t in_dim, int64_t q_dim,
                        int64_t kv_dim) {
    int8_t *xq = (int8_t *)malloc((size_t)in_dim);
    float xs = or_quantize_act(x, in_dim, xq);
    or_matvec_w8a8(q, xq, xs, wq, sq, NULL, in_dim, q_dim);
    or_matvec_w8a8(kk, xq, xs, wk, sk, NULL, in_dim, kv_dim);
    or_matvec_w8a8(v, xq, xs, wv, sv, NULL, in_dim, kv_dim);
    free(xq);
}

/* linear_nobias_int8_swiglu (kernels/mod.rs:970-1027): rows 2j / 2j+1 = gate / up,
 * ffn[j] = g / (1 + expf(-g)) * u with libm expf. */
void or_linear_int8_swiglu(float *ffn, const float *x, const int8_t *w, const float *ws,
                           int64_t in_dim, int64_t inter) {
    int8_t *xq = (int8_t *)malloc((size_t)in_dim);
    float *gu = (float *)malloc(sizeof(float) * 2 * inter);
    float xs = or_quantize_act(x, in_dim, xq);
    or_matvec_w8a8(gu, xq, xs, w, ws, NULL, in_dim, 2 * inter);
    for (int64_t j = 0; j < inter; j++) {
        float g = gu[2 * j], u = gu[2 * j + 1];
        ffn[j] = g / (1.0f + expf(-g)) * u;
    }
    free(gu);
    free(xq);
}

/* linear_nobias_int8_addto (kernels/mod.rs:1030-1034): y doubles as the bias,
 * read before it is written. */
void or_linear_int8_addto(float *y, const float *x, const int8_t *w, const float *ws,
                          int64_t in_dim, int64_t out_dim) {
    or_linear_int8(y, x, w, ws, y, in_dim, out_dim);
}

/* argmax_matvec_int8 (kernels/mod.rs:1832-1893) + neon::argmax_int8_range
 * (neon.rs:802-849): max value, lowest index on ties.  Also reports the
 * second-largest value (over all other rows) for margin bookkeeping. */
int64_t or_argmax_int8(const float *x, const int8_t *w, const float *ws, int64_t in_dim,
                       int64_t out_dim, float *best_val_out, float *second_val_out) {
    int8_t *xq = (int8_t *)malloc((size_t)in_dim);
    float xs = or_quantize_act(x, in_dim, xq);
    int64_t k16 = in_dim - (in_dim % 16);
    /* REF_THREADS contiguous ranges (mod.rs:1854-1866), scanned in parallel and
     * merged in range order with strict > (mod.rs:1876-1883). */
    const int T = REF_THREADS;
    int64_t bi[REF_THREADS];
    float bv[REF_THREADS], sv[REF_THREADS];
    int64_t chunk = (out_dim + T - 1) / T;
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++) {
        int64_t start = t * chunk, end = start + chunk < out_dim ? start + chunk : out_dim;
        int64_t best = start;
        float best_val = -1e30f, second = -1e30f;
        for (int64_t o = start; o < end; o++) {
            const int8_t *row = w + o * in_dim;
            int32_t acc = dot_i8_blocks(xq, row, k16);
            float val = (float)acc * xs * ws[o];
            int32_t tail = 0;
            for (int64_t i = k16; i < in_dim; i++) tail += (int32_t)xq[i] * (int32_t)row[i];
            val = val + (float)tail * xs * ws[o];
            if (val > best_val) { second = best_val; best_val = val; best = o; }
            else if (val > second) second = val;
        }
        bi[t] = start < end ? best : 0;
        bv[t] = start < end ? best_val : -1e30f;
        sv[t] = second;
    }
    int64_t best = bi[0];
    float best_val = bv[0], second = sv[0];
    for (int t = 1; t < T; t++) {                        /* merge in thread order, strict > */
        if (bv[t] > best_val) { second = fmaxf(best_val, sv[t]); best_val = bv[t]; best = bi[t]; }
        else second = fmaxf(second, bv[t]);
    }
    if (best_val_out) *best_val_out = best_val;
    if (second_val_out) *second_val_out = second;
    free(xq);
    return best;
}

/* ======================================================================= */
/* float ops                                                                */
/* ======================================================================= */

/* hsum_ps (kernels/avx.rs:37-51): (v0+v4 + v1+v5) + (v2+v6 + v3+v7) */
float or_hsum8(const float v[8]) {
    float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
    return (s0 + s1) + (s2 + s3);
}

/* avx::dot_f32 (kernels/avx.rs:247-297) */
float or_dot_f32(const float *a, const float *b, int64_t n) {
    float acc[4][8] = {{0}};
    int64_t i = 0;
    for (; i + 32 <= n; i += 32)
        for (int r = 0; r < 4; r++)
            for (int l = 0; l < 8; l++)
                acc[r][l] = fmaf(a[i + 8 * r + l], b[i + 8 * r + l], acc[r][l]);
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) acc[0][l] = fmaf(a[i + l], b[i + l], acc[0][l]);
    float t[8];
    for (int l = 0; l < 8; l++) t[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
    float sum = or_hsum8(t);
    for (; i < n; i++) sum += a[i] * b[i];
    return sum;
}

/* avx::rms_norm_row (kernels/avx.rs:377-415) via rms_norm (mod.rs:1191-1212) */
void or_rms_norm(float *out, const float *x_all, const float *w, int64_t seq, int64_t hidden,
                 float eps) {
#pragma omp parallel for schedule(static) if (seq > 1)
    for (int64_t s = 0; s < seq; s++) {
        const float *x = x_all + s * hidden;
        float *o = out + s * hidden;
        float a0[8] = {0}, a1[8] = {0};
        int64_t i = 0;
        for (; i + 16 <= hidden; i += 16)
            for (int l = 0; l < 8; l++) {
                a0[l] = fmaf(x[i + l], x[i + l], a0[l]);
                a1[l] = fmaf(x[i + 8 + l], x[i + 8 + l], a1[l]);
            }
        for (; i + 8 <= hidden; i += 8)
            for (int l = 0; l < 8; l++) a0[l] = fmaf(x[i + l], x[i + l], a0[l]);
        float t[8];
        for (int l = 0; l < 8; l++) t[l] = a0[l] + a1[l];
        float ss = or_hsum8(t);
        for (; i < hidden; i++) ss += x[i] * x[i];
        float r = 1.0f / sqrtf(ss / (float)hidden + eps);
        for (int64_t j = 0; j < hidden; j++) o[j] = x[j] * r * w[j];
    }
}

/* rms_norm_per_head, non-aarch64 branch (kernels/mod.rs:1214-1238) */
void or_rms_norm_per_head(float *x, const float *w, int64_t seq, int64_t heads, int64_t hd,
                          float eps) {
    for (int64_t s = 0; s < seq; s++)
        for (int64_t h = 0; h < heads; h++) {
            float *v = x + (s * heads + h) * hd;
            float ss = 0.0f;
            for (int64_t d = 0; d < hd; d++) ss += v[d] * v[d];
            float r = 1.0f / sqrtf(ss / (float)hd + eps);
            for (int64_t d = 0; d < hd; d++) v[d] = v[d] * r * w[d];
        }
}

/* RopeCache::ensure (decoder.rs:301-338): table [pos][hd], cos/sin in both halves */
void or_rope_table(float *cos_t, float *sin_t, int64_t n_pos, int64_t hd, float theta) {
    int64_t half = hd / 2;
    float *inv = (float *)malloc(sizeof(float) * half);
    for (int64_t d = 0; d < half; d++) inv[d] = 1.0f / powf(theta, (float)(2 * d) / (float)hd);
    for (int64_t p = 0; p < n_pos; p++) {
        float pf = (float)p;
        for (int64_t d = 0; d < half; d++) {
            float a = pf * inv[d];
            float c = cosf(a), s = sinf(a);
            cos_t[p * hd + d] = c; cos_t[p * hd + half + d] = c;
            sin_t[p * hd + d] = s; sin_t[p * hd + half + d] = s;
        }
    }
    free(inv);
}

/* apply_rope_neox, non-aarch64 branch (kernels/mod.rs:1738-1791, 1780-1788) */
void or_apply_rope(float *x, const float *cos_t, const float *sin_t, int64_t seq,
                   int64_t heads, int64_t hd) {
    int64_t half = hd / 2;
    for (int64_t s = 0; s < seq; s++) {
        const float *c = cos_t + s * hd, *sn = sin_t + s * hd;
        for (int64_t h = 0; h < heads; h++) {
            float *v = x + (s * heads + h) * hd;
            for (int64_t d = 0; d < half; d++) {
                float x1 = v[d], x2 = v[half + d];
                v[d] = x1 * c[d] + (-x2) * sn[d];
                v[half + d] = x2 * c[half + d] + x1 * sn[half + d];
            }
        }
    }
}

/* avx::vec_scale_add / vec_axpy_inplace / vec_scale_inplace (avx.rs:301-372) */
static void vec_scale_add(float *dst, const float *src, float c, int64_t n) {
    int64_t nv = n - (n % 8);
    for (int64_t i = 0; i < nv; i++) dst[i] = fmaf(dst[i], c, src[i]);
    for (int64_t i = nv; i < n; i++) dst[i] = dst[i] * c + src[i];
}
static void vec_axpy(float *dst, const float *src, float a, int64_t n) {
    int64_t nv = n - (n % 8);
    for (int64_t i = 0; i < nv; i++) dst[i] = fmaf(src[i], a, dst[i]);
    for (int64_t i = nv; i < n; i++) dst[i] += a * src[i];
}
static void vec_scale(float *dst, float s, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] *= s;
}

/* Online-softmax row (mod.rs:1508-1535, 1413-1430): one query against keys [j0, j1). */
static void online_softmax_row(float *o, const float *q, const float *kbase, const float *vbase,
                               int64_t kstride, int64_t j0, int64_t j1, int64_t hd, float scale) {
    float mx = -1e30f, sum = 0.0f;
    for (int64_t d = 0; d < hd; d++) o[d] = 0.0f;
    for (int64_t j = j0; j < j1; j++) {
        const float *kr = kbase + j * kstride, *vr = vbase + j * kstride;
        float score = or_dot_f32(q, kr, hd) * scale;
        if (score > mx) {
            float corr = expf(mx - score);
            sum = sum * corr + 1.0f;
            vec_scale_add(o, vr, corr, hd);
            mx = score;
        } else {
            float wt = expf(score - mx);
            sum += wt;
            vec_axpy(o, vr, wt, hd);
        }
    }
    if (sum > 0.0f) vec_scale(o, 1.0f / sum, hd);
}

/* causal_attention (kernels/mod.rs:1663-1698) with the BLAS build's
 * causal_attention_heads (mod.rs:1482-1608): seq_q == 1 is the online-softmax
 * scan; seq_q > 1 is the 3-pass scores / softmax / V^T p. */
void or_causal_attention(float *out, const float *q, const float *k_base, const float *v_base,
                         int64_t head_stride, int64_t seq_q, int64_t seq_k, int64_t n_heads,
                         int64_t n_kv_heads, int64_t hd, float scale, int64_t q_offset) {
    int64_t per_kv = n_heads / n_kv_heads;
    int64_t qh = n_heads * hd;
    if (seq_q == 1) {
#pragma omp parallel for schedule(static)
        for (int64_t h = 0; h < n_heads; h++) {
            int64_t kvh = h / per_kv;
            int64_t k_end = q_offset + 1 < seq_k ? q_offset + 1 : seq_k;
            float *o = out + h * hd;
            if (k_end == 0) { for (int64_t d = 0; d < hd; d++) o[d] = 0.0f; continue; }
            online_softmax_row(o, q + h * hd, k_base + kvh * head_stride,
                               v_base + kvh * head_stride, hd, 0, k_end, hd, scale);
        }
        return;
    }
#pragma omp parallel
    {
        float *scores = (float *)malloc(sizeof(float) * (seq_k > 0 ? seq_k : 1));
#pragma omp for schedule(static) collapse(2)
        for (int64_t h = 0; h < n_heads; h++)
            for (int64_t i = 0; i < seq_q; i++) {
                int64_t kvh = h / per_kv;
                const float *kh = k_base + kvh * head_stride, *vh = v_base + kvh * head_stride;
                const float *qr = q + i * qh + h * hd;
                float *o = out + i * qh + h * hd;
                int64_t gp = q_offset + i;
                int64_t k_end = gp + 1 < seq_k ? gp + 1 : seq_k;
                if (k_end == 0) { for (int64_t d = 0; d < hd; d++) o[d] = 0.0f; continue; }
                /* pass 1: scores = scale * K q  (sgemm with alpha = scale; order unpinned) */
                for (int64_t j = 0; j < k_end; j++) {
                    float acc = 0.0f;
                    for (int64_t d = 0; d < hd; d++) acc = fmaf(kh[j * hd + d], qr[d], acc);
                    scores[j] = scale * acc;
                }
                /* pass 2: softmax with libm expf (mod.rs:1574-1591) */
                float mx = scores[0];
                for (int64_t j = 1; j < k_end; j++) if (scores[j] > mx) mx = scores[j];
                for (int64_t j = 0; j < k_end; j++) scores[j] -= mx;
                for (int64_t j = 0; j < k_end; j++) scores[j] = expf(scores[j]);
                float sum = 0.0f;
                for (int64_t j = 0; j < k_end; j++) sum += scores[j];
                if (sum > 0.0f) {
                    float inv = 1.0f / sum;
                    for (int64_t j = 0; j < k_end; j++) scores[j] *= inv;
                }
                /* pass 3: out = V^T p  (sgemm; order unpinned) */
                for (int64_t d = 0; d < hd; d++) {
                    float acc = 0.0f;
                    for (int64_t j = 0; j < k_end; j++) acc = fmaf(vh[j * hd + d], scores[j], acc);
                    o[d] = acc;
                }
            }
        free(scores);
    }
}

/* bidirectional_attention (kernels/mod.rs:1386-1471): windows of full attention */
void or_bidir_attention(float *out, const float *q, const float *k, const float *v,
                        int64_t seq, int64_t n_heads, int64_t hd, float scale,
                        const int32_t *ws, int64_t n_windows) {
    int64_t hidden = n_heads * hd;
    (void)seq;
#pragma omp parallel for schedule(dynamic) collapse(2)
    for (int64_t h = 0; h < n_heads; h++)
        for (int64_t w = 0; w < n_windows; w++)
            for (int64_t i = ws[w]; i < ws[w + 1]; i++)
                online_softmax_row(out + i * hidden + h * hd, q + i * hidden + h * hd,
                                   k + h * hd, v + h * hd, hidden, ws[w], ws[w + 1], hd, scale);
}

/* avx::fast_exp_avx (kernels/avx.rs:487-514); _mm256_cvtps_epi32 rounds to nearest even */
float or_fast_exp(float x) {
    float val = x * 1.442695041f;
    val = val < 126.0f ? val : 126.0f;          /* _mm256_min_ps(val, 126) */
    val = val > -126.0f ? val : -126.0f;        /* _mm256_max_ps(val, -126) */
    int32_t ip = (int32_t)nearbyintf(val);
    float fp = val - (float)ip;
    uint32_t eb = (uint32_t)(ip + 127) << 23;
    float ei;
    memcpy(&ei, &eb, 4);
    float f = fp * 0.6931471806f;
    float p = fmaf(1.0f / 120.0f, f, 1.0f / 24.0f);
    p = fmaf(p, f, 1.0f / 6.0f);
    p = fmaf(p, f, 0.5f);
    p = fmaf(p, f, 1.0f);
    p = fmaf(p, f, 1.0f);
    return ei * p;
}

/* swiglu_multiply (mod.rs:1291-1341) -> avx::swiglu_interleaved (avx.rs:568-599) */
void or_swiglu_rows(float *out, const float *gate_up, int64_t seq, int64_t inter) {
    int64_t nv = inter - (inter % 8);
#pragma omp parallel for schedule(static)
    for (int64_t s = 0; s < seq; s++) {
        const float *gu = gate_up + s * 2 * inter;
        float *o = out + s * inter;
        for (int64_t j = 0; j < nv; j++) {
            float g = gu[2 * j], u = gu[2 * j + 1];
            float e = or_fast_exp(0.0f - g);
            o[j] = (g / (1.0f + e)) * u;
        }
        for (int64_t j = nv; j < inter; j++) {
            float g = gu[2 * j], u = gu[2 * j + 1];
            o[j] = (g / (1.0f + expf(-g))) * u;
        }
    }
}

/* avx::gelu_inplace (avx.rs:536-563) over one thread's chunk */
static void gelu_chunk(float *x, int64_t n) {
    int64_t nv = n - (n % 8);
    for (int64_t i = 0; i < nv; i++) {
        float v = x[i];
        float v3 = (v * v) * v;
        float inner = 0.7978845608028654f * fmaf(0.044715f, v3, v);
        float e2 = or_fast_exp(2.0f * inner);
        float t = 1.0f - 2.0f / (e2 + 1.0f);
        x[i] = 0.5f * (v * (1.0f + t));
    }
    for (int64_t i = nv; i < n; i++) {
        float v = x[i];
        float x3 = v * v * v;
        float inner = 0.7978845608028654f * (v + 0.044715f * x3);
        x[i] = 0.5f * v * (1.0f + tanhf(inner));
    }
}

/* gelu (kernels/mod.rs:1250-1289): chunks of ceil(n / threads) when n > 4096 */
void or_gelu(float *x, int64_t n) {
    if (n > 4096) {
        int64_t chunk = (n + REF_THREADS - 1) / REF_THREADS;
#pragma omp parallel for schedule(static)
        for (int t = 0; t < REF_THREADS; t++) {
            int64_t s = t * chunk, e = s + chunk < n ? s + chunk : n;
            if (s < e) gelu_chunk(x + s, e - s);
        }
        return;
    }
    gelu_chunk(x, n);
}

/* avx::layer_norm_row (avx.rs:420-481) via layer_norm (mod.rs:1160-1189) */
void or_layer_norm(float *out, const float *x_all, const float *w, const float *b,
                   int64_t seq, int64_t hidden, float eps) {
    int64_t nv = hidden - (hidden % 8);
#pragma omp parallel for schedule(static) if (seq > 1)
    for (int64_t s = 0; s < seq; s++) {
        const float *x = x_all + s * hidden;
        float *o = out + s * hidden;
        float s0[8] = {0}, s1[8] = {0};
        int64_t i = 0;
        for (; i + 16 <= hidden; i += 16)
            for (int l = 0; l < 8; l++) { s0[l] += x[i + l]; s1[l] += x[i + 8 + l]; }
        for (; i + 8 <= hidden; i += 8)
            for (int l = 0; l < 8; l++) s0[l] += x[i + l];
        float t[8];
        for (int l = 0; l < 8; l++) t[l] = s0[l] + s1[l];
        float mean = or_hsum8(t);
        for (; i < hidden; i++) mean += x[i];
        mean /= (float)hidden;
        float v0[8] = {0}, v1[8] = {0};
        i = 0;
        for (; i + 16 <= hidden; i += 16)
            for (int l = 0; l < 8; l++) {
                float d0 = x[i + l] - mean, d1 = x[i + 8 + l] - mean;
                v0[l] = fmaf(d0, d0, v0[l]);
                v1[l] = fmaf(d1, d1, v1[l]);
            }
        for (; i + 8 <= hidden; i += 8)
            for (int l = 0; l < 8; l++) { float d = x[i + l] - mean; v0[l] = fmaf(d, d, v0[l]); }
        for (int l = 0; l < 8; l++) t[l] = v0[l] + v1[l];
        float var = or_hsum8(t);
        for (; i < hidden; i++) { float d = x[i] - mean; var += d * d; }
        float inv = 1.0f / sqrtf(var / (float)hidden + eps);
        for (int64_t j = 0; j < nv; j++) o[j] = fmaf((x[j] - mean) * inv, w[j], b[j]);
        for (int64_t j = nv; j < hidden; j++) o[j] = (x[j] - mean) * inv * w[j] + b[j];
    }
}

/* sinusoidal_pe (kernels/mod.rs:1704-1717) */
void or_sinusoidal_pe(float *pe, int64_t n_pos, int64_t d_model) {
    int64_t half = d_model / 2;
    float lt = logf(10000.0f) / (float)(half - 1);
    for (int64_t p = 0; p < n_pos; p++)
        for (int64_t d = 0; d < half; d++) {
            float inv_ts = expf(-(float)d * lt);
            float a = (float)p * inv_ts;
            pe[p * d_model + d] = sinf(a);
            pe[p * d_model + half + d] = cosf(a);
        }
}

/* ======================================================================= */
/* GEMM call sites                                                          */
/* ======================================================================= */

/* linear (kernels/mod.rs:550-584), BLAS branch: sgemm then a separate bias loop */
void or_linear(float *y, const float *x, const float *w, const float *b, int64_t seq,
               int64_t in_dim, int64_t out_dim) {
    or_sgemm_nt(seq, out_dim, in_dim, x, in_dim, w, in_dim, y, out_dim, 0);
    if (b) {
#pragma omp parallel for schedule(static)
        for (int64_t s = 0; s < seq; s++)
            for (int64_t o = 0; o < out_dim; o++) y[s * out_dim + o] += b[o];
    }
}

/* linear_accumulate (kernels/mod.rs:591-628), BLAS branch: y += b, then y += x W^T */
void or_linear_accumulate(float *y, const float *x, const float *w, const float *b,
                          int64_t seq, int64_t in_dim, int64_t out_dim) {
    if (b) {
#pragma omp parallel for schedule(static)
        for (int64_t s = 0; s < seq; s++)
            for (int64_t o = 0; o < out_dim; o++) y[s * out_dim + o] += b[o];
    }
    or_sgemm_nt(seq, out_dim, in_dim, x, in_dim, w, in_dim, y, out_dim, 1);
}

/* conv2d (kernels/mod.rs:1077-1154): im2col, sgemm W[c_out, patch] x cols, then bias */
void or_conv2d(float *out, const float *in, const float *w, const float *b, int64_t c_in,
               int64_t c_out, int64_t h_in, int64_t w_in, int64_t kh, int64_t kw,
               int64_t stride, int64_t pad) {
    int64_t h_out = (h_in + 2 * pad - kh) / stride + 1;
    int64_t w_out = (w_in + 2 * pad - kw) / stride + 1;
    int64_t patch = c_in * kh * kw, sp = h_out * w_out;
    /* cols^T: [sp][patch] so the product is an NT GEMM */
    float *colsT = (float *)malloc(sizeof(float) * (size_t)(patch * sp));
#pragma omp parallel for schedule(static)
    for (int64_t s = 0; s < sp; s++) {
        int64_t oh = s / w_out, ow = s % w_out;
        for (int64_t cr = 0; cr < patch; cr++) {
            int64_t ic = cr / (kh * kw), rem = cr % (kh * kw), ki = rem / kw, kj = rem % kw;
            int64_t ih = oh * stride + ki - pad, iw = ow * stride + kj - pad;
            colsT[s * patch + cr] = (ih >= 0 && ih < h_in && iw >= 0 && iw < w_in)
                                        ? in[ic * h_in * w_in + ih * w_in + iw] : 0.0f;
        }
    }
    or_sgemm_nt(c_out, sp, patch, w, patch, colsT, patch, out, sp, 0);
    free(colsT);
    if (b) {
#pragma omp parallel for schedule(static)
        for (int64_t oc = 0; oc < c_out; oc++)
            for (int64_t s = 0; s < sp; s++) out[oc * sp + s] += b[oc];
    }
}

/* ======================================================================= */
/* mel (audio.rs:202-372)                                                   */
/* ======================================================================= */

#define MEL_BINS 128
#define N_FFT 400
#define N_FREQ 201
#define HOP 160
#define PI_F 3.14159265358979323846264338327950288f

static float hz_to_mel(float f) {                     /* audio.rs:202-212 */
    float logstep = 27.0f / logf(6.4f);
    float mels = 3.0f * f / 200.0f;
    return f >= 1000.0f ? 15.0f + logf(f / 1000.0f) * logstep : mels;
}
static float mel_to_hz(float m) {                     /* audio.rs:214-223 */
    float logstep = logf(6.4f) / 27.0f;
    return m >= 15.0f ? 1000.0f * expf(logstep * (m - 15.0f)) : 200.0f * m / 3.0f;
}

static void build_mel_filters(float *filters) {       /* audio.rs:225-262 */
    float fft_freqs[N_FREQ], ff[MEL_BINS + 2], fd[MEL_BINS + 1];
    for (int i = 0; i < N_FREQ; i++) fft_freqs[i] = (float)i * (16000.0f / 2.0f) / (float)(N_FREQ - 1);
    float mmin = hz_to_mel(0.0f), mmax = hz_to_mel(16000.0f / 2.0f);
    for (int i = 0; i < MEL_BINS + 2; i++)
        ff[i] = mel_to_hz(mmin + (mmax - mmin) * (float)i / (float)(MEL_BINS + 1));
    for (int i = 0; i < MEL_BINS + 1; i++) {
        fd[i] = ff[i + 1] - ff[i];
        if (fd[i] == 0.0f) fd[i] = 1e-6f;
    }
    for (int m = 0; m < MEL_BINS; m++) {
        float enorm = 2.0f / (ff[m + 2] - ff[m]);
        for (int f = 0; f < N_FREQ; f++) {
            float down = (fft_freqs[f] - ff[m]) / fd[m];
            float up = (ff[m + 2] - fft_freqs[f]) / fd[m + 1];
            float v = fmaxf(fminf(down, up), 0.0f);
            filters[m * N_FREQ + f] = v * enorm;
        }
    }
}

int64_t or_mel_frames(int64_t n) {
    int64_t padded = n + 2 * (N_FFT / 2);
    if (padded < N_FFT) return 0;
    return (padded - N_FFT) / HOP + 1 - 1;
}

/* mel_spectrogram (audio.rs:273-372): out [128][frames] */
int64_t or_mel(const float *samples, int64_t n, float *mel_out) {
    int64_t pad = N_FFT / 2, plen = n + 2 * pad;
    int64_t nf = or_mel_frames(n);
    if (nf <= 0) return 0;
    float *padded = (float *)malloc(sizeof(float) * plen);
    for (int64_t i = 0; i < pad; i++) { int64_t s = pad - i; padded[i] = s < n ? samples[s] : 0.0f; }
    memcpy(padded + pad, samples, sizeof(float) * n);
    for (int64_t i = 0; i < pad; i++) { int64_t s = n - 2 - i; padded[pad + n + i] = s >= 0 ? samples[s] : 0.0f; }
    float window[N_FFT];
    for (int i = 0; i < N_FFT; i++) window[i] = 0.5f * (1.0f - cosf(2.0f * PI_F * (float)i / (float)N_FFT));
    float *ct = (float *)malloc(sizeof(float) * N_FREQ * N_FFT);
    float *st = (float *)malloc(sizeof(float) * N_FREQ * N_FFT);
    for (int k = 0; k < N_FREQ; k++)
        for (int i = 0; i < N_FFT; i++) {
            float a = 2.0f * PI_F * (float)k * (float)i / (float)N_FFT;
            ct[k * N_FFT + i] = cosf(a);
            st[k * N_FFT + i] = sinf(a);
        }
    /* frames [t][n] = windowed^T so the DFT is an NT GEMM */
    float *fr = (float *)malloc(sizeof(float) * nf * N_FFT);
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < nf; t++)
        for (int i = 0; i < N_FFT; i++) fr[t * N_FFT + i] = padded[t * HOP + i] * window[i];
    float *re = (float *)malloc(sizeof(float) * N_FREQ * nf);
    float *im = (float *)malloc(sizeof(float) * N_FREQ * nf);
    or_sgemm_nt(N_FREQ, nf, N_FFT, ct, N_FFT, fr, N_FFT, re, nf, 0);
    or_sgemm_nt(N_FREQ, nf, N_FFT, st, N_FFT, fr, N_FFT, im, nf, 0);
    /* power^T [t][k] */
    float *pT = (float *)malloc(sizeof(float) * N_FREQ * nf);
#pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < N_FREQ; k++)
        for (int64_t t = 0; t < nf; t++) {
            float r = re[k * nf + t], m = im[k * nf + t];
            pT[t * N_FREQ + k] = r * r + m * m;
        }
    float *filters = (float *)malloc(sizeof(float) * MEL_BINS * N_FREQ);
    build_mel_filters(filters);
    or_sgemm_nt(MEL_BINS, nf, N_FREQ, filters, N_FREQ, pT, N_FREQ, mel_out, nf, 0);
    float gmax = -1e30f;
    for (int64_t i = 0; i < MEL_BINS * nf; i++) {
        float v = log10f(fmaxf(mel_out[i], 1e-10f));
        mel_out[i] = v;
        if (v > gmax) gmax = v;
    }
    float mn = gmax - 8.0f;
    for (int64_t i = 0; i < MEL_BINS * nf; i++) mel_out[i] = (fmaxf(mel_out[i], mn) + 4.0f) / 4.0f;
    free(padded); free(ct); free(st); free(fr); free(re); free(im); free(pT); free(filters);
    return nf;
}

/* ======================================================================= */
/* decoder (decoder.rs)                                                     */
/* ======================================================================= */

typedef struct {
    int8_t *wq, *wk, *wv, *wo, *gu, *down;
    float *sq, *sk, *sv, *so, *sgu, *sdown;
    uint16_t *gu_bf16;                 /* interleaved gate/up rows (decoder.rs:91-104) */
} or_dec_packed;

struct or_decoder {
    or_dec_config c;
    or_dec_weights w;
    or_dec_packed *p;
    int8_t *lm; float *lm_s;
    int64_t max_seq, len;
    int kv_bf16;                       /* store K/V rows rounded to bf16 (this build's config-3 cache) */
    float *k, *v;                      /* [layer][kvh][max_seq][hd] */
    float *rc, *rs;                    /* rope [max_seq][hd] */
    float *x, *xn, *q, *kk, *vv, *att, *ffn;
    float *scratch;                    /* bf16 -> f32 weight scratch (mod.rs:693-703) */
};

or_decoder *or_decoder_create(const or_dec_config *cfg, const or_dec_weights *w,
                              int pack_mode, int64_t max_seq) {
    or_decoder *d = (or_decoder *)calloc(1, sizeof(or_decoder));
    d->c = *cfg;
    d->w = *w;
    int64_t H = cfg->hidden, qd = (int64_t)cfg->n_heads * cfg->head_dim;
    int64_t kvd = (int64_t)cfg->n_kv_heads * cfg->head_dim, I = cfg->intermediate;
    d->p = (or_dec_packed *)calloc(cfg->n_layers, sizeof(or_dec_packed));
    for (int l = 0; l < cfg->n_layers; l++) {            /* decoder.rs:106-118 */
        const or_dec_layer *L = &w->layers[l];
        or_dec_packed *P = &d->p[l];
        P->gu_bf16 = (uint16_t *)malloc(sizeof(uint16_t) * 2 * I * H);
        for (int64_t r = 0; r < I; r++) {
            memcpy(P->gu_bf16 + 2 * r * H, L->gate + r * H, sizeof(uint16_t) * H);
            memcpy(P->gu_bf16 + (2 * r + 1) * H, L->up + r * H, sizeof(uint16_t) * H);
        }
#define PACK(dst, sc, src, n, k) do { dst = (int8_t *)malloc((size_t)((n) * (k))); \
        sc = (float *)malloc(sizeof(float) * (n)); or_quantize_bf16_rows(src, n, k, pack_mode, dst, sc); } while (0)
        PACK(P->wq, P->sq, L->wq, qd, H);
        PACK(P->wk, P->sk, L->wk, kvd, H);
        PACK(P->wv, P->sv, L->wv, kvd, H);
        PACK(P->wo, P->so, L->wo, H, qd);
        PACK(P->gu, P->sgu, P->gu_bf16, 2 * I, H);
        PACK(P->down, P->sdown, L->down, H, I);
    }
    PACK(d->lm, d->lm_s, w->embed, (int64_t)cfg->vocab, H);   /* decoder.rs:154-157 */
#undef PACK
    d->max_seq = max_seq;
    size_t kvn = (size_t)cfg->n_layers * cfg->n_kv_heads * max_seq * cfg->head_dim;
    d->k = (float *)calloc(kvn, sizeof(float));
    d->v = (float *)calloc(kvn, sizeof(float));
    d->rc = (float *)malloc(sizeof(float) * max_seq * cfg->head_dim);
    d->rs = (float *)malloc(sizeof(float) * max_seq * cfg->head_dim);
    or_rope_table(d->rc, d->rs, max_seq, cfg->head_dim, cfg->theta);
    d->x = (float *)malloc(sizeof(float) * H);
    d->xn = (float *)malloc(sizeof(float) * H);
    d->q = (float *)malloc(sizeof(float) * qd);
    d->kk = (float *)malloc(sizeof(float) * kvd);
    d->vv = (float *)malloc(sizeof(float) * kvd);
    d->att = (float *)malloc(sizeof(float) * qd);
    d->ffn = (float *)malloc(sizeof(float) * I);
    int64_t mw = 2 * I * H;
    if (qd * H > mw) mw = qd * H;
    d->scratch = (float *)malloc(sizeof(float) * mw);
    return d;
}

void or_decoder_destroy(or_decoder *d) {
    if (!d) return;
    for (int l = 0; l < d->c.n_layers; l++) {
        or_dec_packed *P = &d->p[l];
        free(P->wq); free(P->wk); free(P->wv); free(P->wo); free(P->gu); free(P->down);
        free(P->sq); free(P->sk); free(P->sv); free(P->so); free(P->sgu); free(P->sdown);
        free(P->gu_bf16);
    }
    free(d->p); free(d->lm); free(d->lm_s); free(d->k); free(d->v); free(d->rc); free(d->rs);
    free(d->x); free(d->xn); free(d->q); free(d->kk); free(d->vv); free(d->att); free(d->ffn);
    free(d->scratch);
    free(d);
}

const int8_t *or_decoder_packed(const or_decoder *d, int layer, int which, const float **scales) {
    if (layer < 0) { if (scales) *scales = d->lm_s; return d->lm; }
    const or_dec_packed *P = &d->p[layer];
    const int8_t *r[6] = {P->wq, P->wk, P->wv, P->wo, P->gu, P->down};
    const float *s[6] = {P->sq, P->sk, P->sv, P->so, P->sgu, P->sdown};
    if (scales) *scales = s[which];
    return r[which];
}

void or_decoder_set_len(or_decoder *d, int64_t len) { d->len = len; }
int64_t or_decoder_len(const or_decoder *d) { return d->len; }
const float *or_decoder_kv(const or_decoder *d, int which) { return which ? d->v : d->k; }

void or_embed_token(const or_decoder *d, int32_t token, float *out) {   /* decoder.rs:687-690 */
    const uint16_t *row = d->w.embed + (int64_t)token * d->c.hidden;
    for (int64_t i = 0; i < d->c.hidden; i++) out[i] = bf16f(row[i]);
}

/* f32 -> bf16 round-to-nearest-even -> f32 (finite values) */
static float bf16_round(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    u &= 0xFFFF0000u;
    memcpy(&f, &u, 4);
    return f;
}

static void kv_write(or_decoder *d, int layer, int64_t pos, const float *k, const float *v) {
    int64_t hd = d->c.head_dim, hs = d->max_seq * hd;   /* decoder.rs:233-253 */
    for (int h = 0; h < d->c.n_kv_heads; h++) {
        int64_t off = ((int64_t)layer * d->c.n_kv_heads + h) * hs + pos * hd;
        memcpy(d->k + off, k + h * hd, sizeof(float) * hd);
        memcpy(d->v + off, v + h * hd, sizeof(float) * hd);
        if (d->kv_bf16)
            for (int64_t i = 0; i < hd; i++) {
                d->k[off + i] = bf16_round(d->k[off + i]);
                d->v[off + i] = bf16_round(d->v[off + i]);
            }
    }
}

/* Not in the reference (its cache is f32, decoder.rs:186-197): K/V rows
 * stored rounded to bf16, as the GPU's bf16 cache holds them; attention then
 * reads the rounded rows, the new position's included. */
void or_decoder_set_kv_bf16(or_decoder *d, int on) { d->kv_bf16 = on ? 1 : 0; }

/* linear_nobias_bf16_scratch (kernels/mod.rs:693-703): convert, then sgemm */
static void linear_bf16(or_decoder *d, float *y, const float *x, const uint16_t *w, int64_t seq,
                        int64_t in_dim, int64_t out_dim) {
    or_bf16_to_f32(d->scratch, w, in_dim * out_dim);
    or_linear(y, x, d->scratch, NULL, seq, in_dim, out_dim);
}

/* decoder_prefill (decoder.rs:455-547); hidden_out (nullable) receives the
 * last layer's output rows [S][H] (pref_x before the final norm) */
static void dec_prefill(or_decoder *d, const float *embeds, int64_t S, float *hidden_out);
void or_decoder_prefill(or_decoder *d, const float *embeds, int64_t S) { dec_prefill(d, embeds, S, NULL); }
void or_decoder_prefill_hidden(or_decoder *d, const float *embeds, int64_t S, float *hidden) {
    dec_prefill(d, embeds, S, hidden);
}

/* decoder_prefill_logits (decoder.rs:649-681): prefill, the final RMSNorm of
 * every row, then the bf16 LM head (lm_bf16 [out_dim][H]; NULL: the tied
 * embedding, out_dim = vocab) through linear_nobias_bf16 (f32 sgemm) */
void or_decoder_prefill_logits(or_decoder *d, const float *embeds, int64_t S, const uint16_t *lm_bf16,
                               int64_t out_dim, float *logits) {
    const int64_t H = d->c.hidden;
    float *x = (float *)malloc(sizeof(float) * S * H), *xn = (float *)malloc(sizeof(float) * S * H);
    dec_prefill(d, embeds, S, x);
    or_rms_norm(xn, x, d->w.norm, S, H, d->c.eps);
    float *wf = (float *)malloc(sizeof(float) * out_dim * H);
    or_bf16_to_f32(wf, lm_bf16 ? lm_bf16 : d->w.embed, out_dim * H);
    or_linear(logits, xn, wf, NULL, S, H, out_dim);
    free(wf);
    free(x);
    free(xn);
}

/* forced_align's timestamp readout (align.rs:312-321): per row, a scan from
 * column 0 that moves on only for a strictly greater value */
void or_argmax_f32_rows(const float *x, int64_t rows, int64_t cols, int32_t *idx) {
    for (int64_t r = 0; r < rows; r++) {
        const float *row = x + r * cols;
        int64_t best = 0;
        float best_val = row[0];
        for (int64_t j = 1; j < cols; j++)
            if (row[j] > best_val) {
                best_val = row[j];
                best = j;
            }
        idx[r] = (int32_t)best;
    }
}

static void dec_prefill(or_decoder *d, const float *embeds, int64_t S, float *hidden_out) {
    const or_dec_config *c = &d->c;
    int64_t H = c->hidden, hd = c->head_dim, qd = (int64_t)c->n_heads * hd;
    int64_t kvd = (int64_t)c->n_kv_heads * hd, I = c->intermediate;
    int64_t start = d->len;
    float *x = (float *)malloc(sizeof(float) * S * H);
    float *xn = (float *)malloc(sizeof(float) * S * H);
    float *q = (float *)malloc(sizeof(float) * S * qd);
    float *k = (float *)malloc(sizeof(float) * S * kvd);
    float *v = (float *)malloc(sizeof(float) * S * kvd);
    float *att = (float *)malloc(sizeof(float) * S * qd);
    float *proj = (float *)malloc(sizeof(float) * S * H);
    float *gu = (float *)malloc(sizeof(float) * S * 2 * I);
    float *g = (float *)malloc(sizeof(float) * S * I);
    memcpy(x, embeds, sizeof(float) * S * H);
    const float *rc = d->rc + start * hd, *rs = d->rs + start * hd;
    float scale = 1.0f / sqrtf((float)hd);
    for (int l = 0; l < c->n_layers; l++) {
        const or_dec_layer *L = &d->w.layers[l];
        or_rms_norm(xn, x, L->input_norm, S, H, c->eps);
        linear_bf16(d, q, xn, L->wq, S, H, qd);
        linear_bf16(d, k, xn, L->wk, S, H, kvd);
        linear_bf16(d, v, xn, L->wv, S, H, kvd);
        or_rms_norm_per_head(q, L->q_norm, S, c->n_heads, hd, c->eps);
        or_rms_norm_per_head(k, L->k_norm, S, c->n_kv_heads, hd, c->eps);
        or_apply_rope(q, rc, rs, S, c->n_heads, hd);
        or_apply_rope(k, rc, rs, S, c->n_kv_heads, hd);
        for (int64_t s = 0; s < S; s++) kv_write(d, l, start + s, k + s * kvd, v + s * kvd);
        int64_t lo = (int64_t)l * c->n_kv_heads * d->max_seq * hd;
        or_causal_attention(att, q, d->k + lo, d->v + lo, d->max_seq * hd, S, start + S,
                            c->n_heads, c->n_kv_heads, hd, scale, start);
        linear_bf16(d, proj, att, L->wo, S, qd, H);
        for (int64_t i = 0; i < S * H; i++) x[i] += proj[i];          /* add_inplace */
        or_rms_norm(xn, x, L->post_attn_norm, S, H, c->eps);
        linear_bf16(d, gu, xn, d->p[l].gu_bf16, S, H, 2 * I);
        or_swiglu_rows(g, gu, S, I);
        linear_bf16(d, proj, g, L->down, S, I, H);
        for (int64_t i = 0; i < S * H; i++) x[i] += proj[i];
    }
    d->len = start + S;
    if (hidden_out) memcpy(hidden_out, x, sizeof(float) * S * H);
    free(x); free(xn); free(q); free(k); free(v); free(att); free(proj); free(gu); free(g);
}

/* decoder_forward (decoder.rs:550-645) */
int32_t or_decoder_forward(or_decoder *d, const float *embed, float *best_val, float *second_val,
                           float *hidden_out) {
    const or_dec_config *c = &d->c;
    int64_t H = c->hidden, hd = c->head_dim, qd = (int64_t)c->n_heads * hd;
    int64_t kvd = (int64_t)c->n_kv_heads * hd, I = c->intermediate;
    int64_t pos = d->len;
    memcpy(d->x, embed, sizeof(float) * H);
    const float *rc = d->rc + pos * hd, *rs = d->rs + pos * hd;
    float scale = 1.0f / sqrtf((float)hd);
    for (int l = 0; l < c->n_layers; l++) {
        const or_dec_layer *L = &d->w.layers[l];
        const or_dec_packed *P = &d->p[l];
        or_rms_norm(d->xn, d->x, L->input_norm, 1, H, c->eps);
        or_linear_int8_qkv(d->q, d->kk, d->vv, d->xn, P->wq, P->sq, P->wk, P->sk, P->wv, P->sv,
                           H, qd, kvd);
        or_rms_norm_per_head(d->q, L->q_norm, 1, c->n_heads, hd, c->eps);
        or_rms_norm_per_head(d->kk, L->k_norm, 1, c->n_kv_heads, hd, c->eps);
        or_apply_rope(d->q, rc, rs, 1, c->n_heads, hd);
        or_apply_rope(d->kk, rc, rs, 1, c->n_kv_heads, hd);
        kv_write(d, l, pos, d->kk, d->vv);
        int64_t lo = (int64_t)l * c->n_kv_heads * d->max_seq * hd;
        or_causal_attention(d->att, d->q, d->k + lo, d->v + lo, d->max_seq * hd, 1, pos + 1,
                            c->n_heads, c->n_kv_heads, hd, scale, pos);
        or_linear_int8_addto(d->x, d->att, P->wo, P->so, qd, H);
        or_rms_norm(d->xn, d->x, L->post_attn_norm, 1, H, c->eps);
        or_linear_int8_swiglu(d->ffn, d->xn, P->gu, P->sgu, H, I);
        or_linear_int8_addto(d->x, d->ffn, P->down, P->sdown, I, H);
    }
    d->len = pos + 1;
    or_rms_norm(d->xn, d->x, d->w.norm, 1, H, c->eps);
    if (hidden_out) memcpy(hidden_out, d->xn, sizeof(float) * H);
    return (int32_t)or_argmax_int8(d->xn, d->lm, d->lm_s, H, c->vocab, best_val, second_val);
}

/* ======================================================================= */
/* encoder (encoder.rs)                                                     */
/* ======================================================================= */

typedef struct {
    float *wq, *wk, *wv, *wo, *fc1, *fc2;
} or_enc_f32;

struct or_encoder {
    or_enc_config c;
    or_enc_weights w;
    or_enc_f32 *L;
    float *c1, *c2, *c3, *cout, *p1, *p2;
};

static float *bf16_dup(const uint16_t *src, int64_t n) {   /* encoder.rs:106-120 */
    float *f = (float *)malloc(sizeof(float) * n);
    or_bf16_to_f32(f, src, n);
    return f;
}

or_encoder *or_encoder_create(const or_enc_config *cfg, const or_enc_weights *w) {
    or_encoder *e = (or_encoder *)calloc(1, sizeof(or_encoder));
    e->c = *cfg;
    e->w = *w;
    int64_t D = cfg->d_model, F = cfg->ffn_dim, C = cfg->conv_hidden;
    e->L = (or_enc_f32 *)calloc(cfg->n_layers, sizeof(or_enc_f32));
    for (int l = 0; l < cfg->n_layers; l++) {
        const or_enc_layer *s = &w->layers[l];
        e->L[l].wq = bf16_dup(s->wq, D * D);
        e->L[l].wk = bf16_dup(s->wk, D * D);
        e->L[l].wv = bf16_dup(s->wv, D * D);
        e->L[l].wo = bf16_dup(s->wo, D * D);
        e->L[l].fc1 = bf16_dup(s->fc1, F * D);
        e->L[l].fc2 = bf16_dup(s->fc2, D * F);
    }
    e->c1 = bf16_dup(w->conv1_w, C * 9);
    e->c2 = bf16_dup(w->conv2_w, C * C * 9);
    e->c3 = bf16_dup(w->conv3_w, C * C * 9);
    int64_t h3 = ((((128 + 2 - 3) / 2 + 1) + 2 - 3) / 2 + 1 + 2 - 3) / 2 + 1;
    e->cout = bf16_dup(w->conv_out_w, D * C * h3);
    e->p1 = bf16_dup(w->proj1_w, D * D);
    e->p2 = bf16_dup(w->proj2_w, (int64_t)cfg->output_dim * D);
    return e;
}

void or_encoder_destroy(or_encoder *e) {
    if (!e) return;
    for (int l = 0; l < e->c.n_layers; l++) {
        free(e->L[l].wq); free(e->L[l].wk); free(e->L[l].wv); free(e->L[l].wo);
        free(e->L[l].fc1); free(e->L[l].fc2);
    }
    free(e->L); free(e->c1); free(e->c2); free(e->c3); free(e->cout); free(e->p1); free(e->p2);
    free(e);
}

static int64_t conv_out_len(int64_t n) { return (n + 2 - 3) / 2 + 1; }

int64_t or_encoder_tokens(const or_encoder *e, int64_t frames) {
    int64_t cs = e->c.chunk_size, tot = 0;
    for (int64_t s = 0; s < frames; s += cs) {
        int64_t w = frames - s < cs ? frames - s : cs;
        tot += conv_out_len(conv_out_len(conv_out_len(w)));
    }
    return tot;
}

/* Encoder::forward (encoder.rs:186-358); out [tokens][output_dim] */
int64_t or_encoder_forward(or_encoder *e, const float *mel, int64_t frames, float *out) {
    const or_enc_config *c = &e->c;
    int64_t D = c->d_model, F = c->ffn_dim, C = c->conv_hidden, cs = c->chunk_size;
    int64_t T = or_encoder_tokens(e, frames);
    int64_t tpc = conv_out_len(conv_out_len(conv_out_len(cs)));
    float *x = (float *)calloc((size_t)(T * D), sizeof(float));
    int64_t h1 = conv_out_len(128), h2 = conv_out_len(h1), h3 = conv_out_len(h2);
    int64_t off = 0;
    for (int64_t st = 0; st < frames; st += cs) {
        int64_t cw = frames - st < cs ? frames - st : cs;
        int64_t w1 = conv_out_len(cw), w2 = conv_out_len(w1), w3 = conv_out_len(w2);
        float *cm = (float *)malloc(sizeof(float) * 128 * cw);
        for (int m = 0; m < 128; m++) memcpy(cm + m * cw, mel + m * frames + st, sizeof(float) * cw);
        float *a1 = (float *)malloc(sizeof(float) * C * h1 * w1);
        or_conv2d(a1, cm, e->c1, e->w.conv1_b, 1, C, 128, cw, 3, 3, 2, 1);
        or_gelu(a1, C * h1 * w1);
        float *a2 = (float *)malloc(sizeof(float) * C * h2 * w2);
        or_conv2d(a2, a1, e->c2, e->w.conv2_b, C, C, h1, w1, 3, 3, 2, 1);
        or_gelu(a2, C * h2 * w2);
        float *a3 = (float *)malloc(sizeof(float) * C * h3 * w3);
        or_conv2d(a3, a2, e->c3, e->w.conv3_b, C, C, h2, w2, 3, 3, 2, 1);
        or_gelu(a3, C * h3 * w3);
        int64_t pd = C * h3;                               /* encoder.rs:265-277 */
        float *rs = (float *)malloc(sizeof(float) * w3 * pd);
        for (int64_t ch = 0; ch < C; ch++)
            for (int64_t f = 0; f < h3; f++)
                for (int64_t t = 0; t < w3; t++) rs[t * pd + ch * h3 + f] = a3[ch * h3 * w3 + f * w3 + t];
        float *pr = x + off * D;
        or_linear(pr, rs, e->cout, NULL, w3, pd, D);
        float *pe = (float *)malloc(sizeof(float) * w3 * D);
        or_sinusoidal_pe(pe, w3, D);
        for (int64_t i = 0; i < w3 * D; i++) pr[i] += pe[i];
        off += w3;
        free(cm); free(a1); free(a2); free(a3); free(rs); free(pe);
    }
    int64_t wts = tpc * (c->n_window_infer / cs);          /* encoder.rs:291-298 */
    int64_t nw = (T + wts - 1) / wts;
    int32_t *ws = (int32_t *)malloc(sizeof(int32_t) * (nw + 1));
    for (int64_t w = 0; w < nw; w++) ws[w] = (int32_t)(w * wts);
    ws[nw] = (int32_t)T;
    float *xn = (float *)malloc(sizeof(float) * T * D);
    float *q = (float *)malloc(sizeof(float) * T * D);
    float *k = (float *)malloc(sizeof(float) * T * D);
    float *v = (float *)malloc(sizeof(float) * T * D);
    float *att = (float *)malloc(sizeof(float) * T * D);
    float *mid = (float *)malloc(sizeof(float) * T * F);
    float scale = 1.0f / sqrtf((float)c->head_dim);
    for (int l = 0; l < c->n_layers; l++) {
        const or_enc_layer *s = &e->w.layers[l];
        const or_enc_f32 *L = &e->L[l];
        or_layer_norm(xn, x, s->ln1_w, s->ln1_b, T, D, 1e-5f);
        or_linear(q, xn, L->wq, s->bq, T, D, D);
        or_linear(k, xn, L->wk, s->bk, T, D, D);
        or_linear(v, xn, L->wv, s->bv, T, D, D);
        or_bidir_attention(att, q, k, v, T, c->n_heads, c->head_dim, scale, ws, nw);
        or_linear_accumulate(x, att, L->wo, s->bo, T, D, D);
        or_layer_norm(xn, x, s->ln2_w, s->ln2_b, T, D, 1e-5f);
        or_linear(mid, xn, L->fc1, s->b1, T, D, F);
        or_gelu(mid, T * F);
        or_linear_accumulate(x, mid, L->fc2, s->b2, T, F, D);
    }
    or_layer_norm(xn, x, e->w.ln_post_w, e->w.ln_post_b, T, D, 1e-5f);
    memcpy(x, xn, sizeof(float) * T * D);
    or_linear(q, x, e->p1, e->w.proj1_b, T, D, D);
    or_gelu(q, T * D);
    or_linear(out, q, e->p2, e->w.proj2_b, T, D, c->output_dim);
    free(x); free(ws); free(xn); free(q); free(k); free(v); free(att); free(mid);
    return T;
}

/* ======================================================================= */
/* offline driver (transcribe.rs:63-247) with a forced step count          */
/* ======================================================================= */

static const int32_t PREFIX_HEAD[] = {151644, 8948, 198};
static const int32_t PREFIX_TAIL[] = {151645, 198, 151644, 872, 198, 151669};
static const int32_t SUFFIX_BASE[] = {151670, 151645, 198, 151644, 77091, 198};

static double now_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec * 1e-6;
}

int64_t or_prompt_ids(const int32_t *prompt, int64_t n_prompt, const int32_t *force, int64_t n_force,
                      const int32_t *past, int64_t n_past, int32_t *head, int64_t *n_head, int32_t *tail,
                      int64_t *n_tail) {
    /* transcribe.rs:97-169: PREFIX_HEAD | prompt | PREFIX_TAIL before the audio
     * rows; SUFFIX_BASE | force | past | <asr_text> (the last two only when
     * there are past tokens) after them */
    int64_t h = 0, t = 0;
    for (int i = 0; i < 3; i++) head[h++] = PREFIX_HEAD[i];
    for (int64_t i = 0; i < n_prompt; i++) head[h++] = prompt[i];
    for (int i = 0; i < 6; i++) head[h++] = PREFIX_TAIL[i];
    for (int i = 0; i < 6; i++) tail[t++] = SUFFIX_BASE[i];
    for (int64_t i = 0; i < n_force; i++) tail[t++] = force[i];
    for (int64_t i = 0; i < n_past; i++) tail[t++] = past[i];
    if (n_past > 0) tail[t++] = 151704;   /* TOKEN_ASR_TEXT */
    *n_head = h;
    *n_tail = t;
    return h + t;
}

int64_t or_transcribe_prompt(or_decoder *d, or_encoder *e, const float *samples, int64_t n_samples,
                             const int32_t *prompt, int64_t n_prompt, const int32_t *force, int64_t n_force,
                             const int32_t *past, int64_t n_past, int32_t n_steps, int32_t *tokens,
                             float *margins, double *times_ms) {
    int64_t H = d->c.hidden;
    double t0 = now_ms();
    int64_t nf = or_mel_frames(n_samples);
    float *mel = (float *)malloc(sizeof(float) * 128 * (nf > 0 ? nf : 1));
    or_mel(samples, n_samples, mel);
    double t1 = now_ms();
    int64_t T = or_encoder_tokens(e, nf);
    float *enc = (float *)malloc(sizeof(float) * T * H);
    or_encoder_forward(e, mel, nf, enc);
    double t2 = now_ms();
    int32_t *head = (int32_t *)malloc(sizeof(int32_t) * (9 + n_prompt));
    int32_t *tail = (int32_t *)malloc(sizeof(int32_t) * (7 + n_force + n_past));
    int64_t nh = 0, ns = 0;
    or_prompt_ids(prompt, n_prompt, force, n_force, past, n_past, head, &nh, tail, &ns);
    int64_t total = nh + T + ns;
    float *emb = (float *)malloc(sizeof(float) * total * H);
    int64_t o = 0;
    for (int64_t i = 0; i < nh; i++) or_embed_token(d, head[i], emb + (o++) * H);
    memcpy(emb + o * H, enc, sizeof(float) * T * H);
    o += T;
    for (int64_t i = 0; i < ns; i++) or_embed_token(d, tail[i], emb + (o++) * H);
    free(head);
    free(tail);
    d->len = 0;
    or_decoder_prefill(d, emb, total - 1);
    float bv, sv;
    int32_t tok = or_decoder_forward(d, emb + (total - 1) * H, &bv, &sv, NULL);
    double t3 = now_ms();
    float *te = (float *)malloc(sizeof(float) * H);
    for (int32_t s = 0; s < n_steps; s++) {
        tokens[s] = tok;
        if (margins) margins[s] = bv - sv;
        if (s + 1 == n_steps) break;
        or_embed_token(d, tok, te);
        tok = or_decoder_forward(d, te, &bv, &sv, NULL);
    }
    double t4 = now_ms();
    if (times_ms) { times_ms[0] = t1 - t0; times_ms[1] = t2 - t1; times_ms[2] = t3 - t2; times_ms[3] = t4 - t3; }
    free(mel); free(enc); free(emb); free(te);
    return total;
}

int64_t or_transcribe_forced(or_decoder *d, or_encoder *e, const float *samples,
                             int64_t n_samples, int32_t n_steps, int32_t *tokens,
                             float *margins, double *times_ms) {
    return or_transcribe_prompt(d, e, samples, n_samples, NULL, 0, NULL, 0, NULL, 0, n_steps, tokens, margins,
                                times_ms);
}

/* ======================================================================= */
/* segmentation of long audio (transcribe.rs:252-277, 323-341)              */
/* ======================================================================= */

/* Rust's `f32 as usize`: truncation toward zero, negative and NaN to 0 */
static int64_t f32_to_count(float v) {
    if (!(v > 0.0f)) return 0;
    if (v >= 9.2e18f) return INT64_MAX;
    return (int64_t)v;
}

/* find_split_point (transcribe.rs:252-277): the center of the 100 ms window
 * (1600 samples, hop 800) of least mean energy inside target +- search_sec;
 * the first of equal minima; target itself when no window fits */
int64_t or_find_split_point(const float *x, int64_t n, int64_t target, float search_sec) {
    const int64_t half = f32_to_count(search_sec * 16000.0f);
    const int64_t lo = target > half ? target - half : 0;
    const int64_t hi = target + half < n ? target + half : n;
    const int64_t win = 1600;
    float best = 1e30f;
    int64_t center = target;
    for (int64_t pos = lo; pos + win <= hi; pos += win / 2) {
        const int64_t end = pos + win < n ? pos + win : n;
        float energy = 0.0f;
        for (int64_t i = pos; i < end; i++) energy += x[i] * x[i];
        energy /= (float)(end - pos);
        if (energy < best) {
            best = energy;
            center = pos + (end - pos) / 2;
        }
    }
    return center;
}

/* transcribe_audio's split points (transcribe.rs:323-341): 0, then one split
 * near every segment_sec until the rest fits in one segment plus the search
 * margin, at most 127 in all.  Returns the count; writes min(count, cap). */
int64_t or_segment_splits(const float *x, int64_t n, float segment_sec, float search_sec, int64_t *splits,
                          int64_t cap) {
    const int64_t target = f32_to_count(segment_sec * 16000.0f);
    const float half_seg = segment_sec / 2.0f;
    /* f32::min: a NaN operand yields the other one */
    const float search = isnan(half_seg) ? search_sec : (search_sec < half_seg ? search_sec : half_seg);
    const int64_t margin = f32_to_count(search * 16000.0f);
    int64_t k = 0;
    if (cap > 0) splits[0] = 0;
    k = 1;
    if (segment_sec <= 0.0f || n <= target + margin) return k;
    int64_t pos = 0;
    while (pos + target + margin < n) {
        const int64_t s = or_find_split_point(x, n, pos + target, search);
        if (k < cap) splits[k] = s;
        k++;
        pos = s;
        if (k >= 127) break;
    }
    return k;
}
