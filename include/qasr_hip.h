/*
 * qasr_hip — MI355X (gfx950) HIP backend for the int8 inference hot path of
 * huanglizhuo/QwenASR.
 *
 * A plain C ABI: no C++ or torch types, device memory passed as raw pointers,
 * sizes as int64_t, status as int (0 = ok, < 0 = error; the message of the
 * last failure on the calling thread is returned by qasr_hip_last_error()).
 * Nothing throws across this boundary.
 *
 * Each entry point cites the reference function it replaces
 * (crates/qwen-asr/src/...:line).  The reference binds native code the same
 * way it binds BLAS today (kernels/mod.rs:11-59, build.rs:1-18); the Rust
 * binding a maintainer would add is shown in INTEGRATION.md.
 *
 * Threading: one handle per host thread (the handle owns one HIP stream and a
 * small scratch area).  Op-level calls take device pointers, enqueue work on
 * the handle's stream and return without synchronising.  Model-level calls
 * take host pointers where the reference passes host slices and synchronise
 * only where a host result is returned.
 */
#ifndef QASR_HIP_H
#define QASR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QASR_OK 0
#define QASR_ERR_INVALID (-1)      /* bad argument or unsupported shape */
#define QASR_ERR_HIP (-2)          /* HIP runtime failure */
#define QASR_ERR_NOMEM (-3)        /* device allocation failed */

/* weight-packer rounding: x86/generic branch (kernels/mod.rs:1819-1825) or
 * the NEON branch (kernels/neon.rs:673-690) */
#define QASR_ROUND_HALF_AWAY 0
#define QASR_TRUNC 1

typedef struct qasr_hip qasr_hip;

/* ---- lifecycle ---------------------------------------------------------- */
int qasr_hip_create(int device, qasr_hip **out);
void qasr_hip_destroy(qasr_hip *h);
const char *qasr_hip_last_error(void);
int qasr_hip_device_count(int *n);
int qasr_hip_synchronize(qasr_hip *h);
void *qasr_hip_stream(qasr_hip *h);                 /* the handle's hipStream_t */

/* ---- device memory helpers (for callers without an allocator of their own) */
int qasr_hip_malloc(qasr_hip *h, size_t bytes, void **dptr);
int qasr_hip_free(qasr_hip *h, void *dptr);
int qasr_hip_upload(qasr_hip *h, void *dst, const void *src, size_t bytes);     /* synchronous */
int qasr_hip_download(qasr_hip *h, void *dst, const void *src, size_t bytes);   /* synchronous */
int qasr_hip_memset(qasr_hip *h, void *dst, int value, size_t bytes);

/* ---- timing on the handle's stream (HIP events) ------------------------- */
int qasr_hip_timer_start(qasr_hip *h);
int qasr_hip_timer_stop(qasr_hip *h, float *ms);    /* synchronises */

/* ---- A1: weight packer --------------------------------------------------
 * Replaces kernels::quantize_bf16_weights_to_int8 (kernels/mod.rs:1805-1829,
 * neon.rs:637-694).  w_bf16 [n, k] row-major -> q int8 [n, k], scales f32 [n]. */
int qasr_hip_pack_int8_rows(qasr_hip *h, const uint16_t *w_bf16, int64_t n, int64_t k,
                            int round_mode, int8_t *q, float *scales);

/* ---- A2: activation quantizer (kernels::quantize_f32_to_int8, mod.rs:1795) */
int qasr_hip_quantize_act(qasr_hip *h, const float *x, int64_t k, int8_t *q, float *scale);

/* ---- A3-A7: W8A8 decode matvecs (x f32, quantized on the fly) ----------
 * in_dim % 64 == 0, in_dim <= 6144. */
/* int8_matvec_threaded with optional bias (kernels/mod.rs:839-880) */
int qasr_hip_linear_int8(qasr_hip *h, float *y, const float *x, const int8_t *w, const float *ws,
                         const float *bias, int64_t in_dim, int64_t out_dim);
/* linear_nobias_int8_qkv (kernels/mod.rs:884-967) */
int qasr_hip_linear_int8_qkv(qasr_hip *h, float *q, float *k, float *v, const float *x,
                             const int8_t *wq, const float *sq, const int8_t *wk, const float *sk,
                             const int8_t *wv, const float *sv, int64_t in_dim, int64_t q_dim,
                             int64_t kv_dim);
/* linear_nobias_int8_swiglu (kernels/mod.rs:970-1027); w holds interleaved gate/up rows */
int qasr_hip_linear_int8_swiglu(qasr_hip *h, float *ffn_out, const float *x, const int8_t *w,
                                const float *ws, int64_t in_dim, int64_t intermediate);
/* linear_nobias_int8_addto (kernels/mod.rs:1030-1034): y += W x */
int qasr_hip_linear_int8_addto(qasr_hip *h, float *y, const float *x, const int8_t *w,
                               const float *ws, int64_t in_dim, int64_t out_dim);
/* argmax_matvec_int8 (kernels/mod.rs:1832-1893): writes the index to *idx (device) */
int qasr_hip_argmax_int8(qasr_hip *h, const float *x, const int8_t *w, const float *ws,
                         int64_t in_dim, int64_t out_dim, int32_t *idx);

/* Fused forms used by the decode step: rms_norm (mod.rs:1191) of x with gain
 * norm_w feeding the int8 op, exactly as decoder.rs:583-593 / 619-625 / 634-641
 * chain them.  in_dim % 64 == 0, in_dim <= 4096. */
int qasr_hip_rmsnorm_linear_int8_qkv(qasr_hip *h, float *q, float *k, float *v, const float *x,
                                     const float *norm_w, float eps, const int8_t *wq,
                                     const float *sq, const int8_t *wk, const float *sk,
                                     const int8_t *wv, const float *sv, int64_t in_dim,
                                     int64_t q_dim, int64_t kv_dim);
int qasr_hip_rmsnorm_linear_int8_swiglu(qasr_hip *h, float *ffn_out, const float *x,
                                        const float *norm_w, float eps, const int8_t *w,
                                        const float *ws, int64_t in_dim, int64_t intermediate);
int qasr_hip_rmsnorm_argmax_int8(qasr_hip *h, const float *x, const float *norm_w, float eps,
                                 const int8_t *w, const float *ws, int64_t in_dim, int64_t out_dim,
                                 int32_t *idx);

/* ---- A8-A12: norms, RoPE, attention (f32, device pointers) -------------- */
/* rms_norm (kernels/mod.rs:1191-1212); hidden % 64 == 0, hidden <= 4096 */
int qasr_hip_rms_norm(qasr_hip *h, float *out, const float *x, const float *w, int64_t seq,
                      int64_t hidden, float eps);
/* rms_norm_per_head (kernels/mod.rs:1214-1238); head_dim == 128 */
int qasr_hip_rms_norm_per_head(qasr_hip *h, float *x, const float *w, int64_t seq, int64_t n_heads,
                               int64_t head_dim, float eps);
/* apply_rope_neox (kernels/mod.rs:1738-1791); cos/sin hold seq rows of head_dim */
int qasr_hip_apply_rope_neox(qasr_hip *h, float *x, const float *cos_vals, const float *sin_vals,
                             int64_t seq, int64_t n_heads, int64_t head_dim);
/* causal_attention (kernels/mod.rs:1663-1698); K/V layout [kv_head][pos][head_dim]
 * with head_stride elements between heads, as KvCache (decoder.rs:174-271).
 * seq_q == 1 only in this build; head_dim == 128, n_heads == 2 * n_kv_heads. */
int qasr_hip_causal_attention(qasr_hip *h, float *out, const float *q, const float *k_base,
                              const float *v_base, int64_t head_stride, int64_t seq_q,
                              int64_t seq_k, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                              float scale, int64_t q_offset);

/* ---- model level: the Qwen3 decoder (decoder.rs) ------------------------ */
typedef struct {
    int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, intermediate, vocab;
    float eps, theta;                                   /* QwenConfig, config.rs:27-55 */
} qasr_dec_config;

typedef struct {                                        /* DecLayer, decoder.rs:7-34 */
    const uint16_t *wq, *wk, *wv, *wo, *gate, *up, *down;     /* host bf16 [out, in] */
    const float *q_norm, *k_norm, *input_norm, *post_attn_norm;
} qasr_dec_layer;

typedef struct {                                        /* Decoder, decoder.rs:39-48 */
    const uint16_t *embed;          /* host bf16 [vocab, hidden]; tied LM head */
    const float *norm;              /* [hidden] */
    const qasr_dec_layer *layers;   /* [n_layers] */
} qasr_dec_weights;

typedef struct qasr_decoder qasr_decoder;

/* Decoder::load (decoder.rs:70-167): uploads the bf16 weights, packs every
 * projection and the LM head to int8 on the GPU, allocates a device-resident
 * KV cache of max_seq positions (f32, or bf16 when kv_bf16 != 0) and the RoPE
 * table (decoder.rs:301-338, computed on the host with libm and uploaded). */
int qasr_hip_decoder_load(qasr_hip *h, const qasr_dec_config *cfg, const qasr_dec_weights *w,
                          int round_mode, int64_t max_seq, int kv_bf16, qasr_decoder **out);
void qasr_hip_decoder_free(qasr_decoder *d);
/* decoder_prefill (decoder.rs:455-547): host f32 embeddings [seq_len, hidden] */
int qasr_hip_decoder_prefill(qasr_decoder *d, const float *embeds, int64_t seq_len);
/* decoder_forward (decoder.rs:550-645): embed is a host f32 row, or NULL to use
 * token_in's embedding row (tok_embed_bf16_to_f32, decoder.rs:687).  Returns the
 * greedy token in *token_out. */
int qasr_hip_decoder_forward(qasr_decoder *d, const float *embed, int32_t token_in,
                             int32_t *token_out);
/* n_steps greedy steps with no host round trip in between (the decode loop of
 * transcribe.rs:194-226 with a forced step count): the first step consumes
 * first_embed (host f32 row, or NULL to embed first_token), each later step
 * embeds the previous token on the device.  tokens_out gets n_steps ids. */
int qasr_hip_decoder_generate(qasr_decoder *d, const float *first_embed, int32_t first_token,
                              int32_t n_steps, int32_t *tokens_out);
/* kv_cache.len accessors (transcribe.rs:173, 1106) */
int qasr_hip_decoder_set_len(qasr_decoder *d, int64_t len);
int64_t qasr_hip_decoder_len(const qasr_decoder *d);
/* test hooks: the packed int8 rows / scales of layer `layer` (-1 = LM head),
 * which = 0 q, 1 k, 2 v, 3 o, 4 gate_up (interleaved), 5 down; and the KV cache
 * in the reference layout [layer][kv_head][max_seq][head_dim] as f32 */
int qasr_hip_decoder_packed(qasr_decoder *d, int layer, int which, int8_t *q_host,
                            float *scales_host);
int qasr_hip_decoder_kv_upload(qasr_decoder *d, const float *k_host, const float *v_host);
int qasr_hip_decoder_kv_download(qasr_decoder *d, float *k_host, float *v_host);
/* decode-step tuning: attention context splits (default chosen from max_seq)
 * and whether steps replay a captured HIP graph (default 1) */
int qasr_hip_decoder_set_options(qasr_decoder *d, int attn_splits, int use_graph);

#ifdef __cplusplus
}
#endif
#endif
