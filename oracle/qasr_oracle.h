/*
 * qasr_oracle — CPU restatement of huanglizhuo/QwenASR's int8 inference path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path in qwenasr_amd/.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product never links, imports or calls it.
 *
 * Semantics (every function cites the reference file:line it restates; paths
 * are relative to crates/qwen-asr/src/ of the reference):
 *   - int8 paths: exact integer arithmetic, so the result does not depend on
 *     summation order (NEON SDOT algorithm, kernels/neon.rs).
 *   - float paths: the x86_64 AVX2+FMA order the Linux build runs
 *     (kernels/avx.rs), with explicit fmaf() exactly where the reference uses
 *     _mm256_fmadd_ps, and no other contraction (built with -ffp-contract=off).
 *   - libm: glibc expf/powf/cosf/sinf/logf/log10f/tanhf, the functions Rust's
 *     std calls on Linux.
 *   - cblas_sgemm (OpenBLAS in the reference's Linux build) is restated as a
 *     blocked f32 GEMM; BLAS summation order is not pinned by anything the
 *     reference ships, so GEMM outputs are compared with a tolerance.
 *
 * Pinning (what checks each function; see tests/test_oracle_*.py):
 *   quantizers, matvec, argmax  : closed-form KATs, brute force in numpy int64,
 *                                 tie/ordering KATs
 *   rms_norm, per-head norm     : numpy float64 restatement + exact-order KAT
 *   rope                        : numpy float64 rotation; norm preservation
 *   attention                   : numpy float64 softmax attention (GQA map)
 *   swiglu / fast_exp / gelu    : numpy float64 formulas; fast_exp error bound
 *   layer_norm                  : numpy float64 mean/var
 *   sgemm                       : numpy float64 matmul
 *   mel                         : numpy float64 STFT + Slaney filterbank
 *   decoder / encoder / prompt  : an independent float64 restatement of the
 *                                 compositions (tests/ref64.py) with planted
 *                                 mistakes that fail it; the prompt ids around
 *                                 the audio rows likewise
 *   segmentation                : float64 brute force and known answers
 *   stream                      : tail-repeat KATs; one finalizing chunk equals
 *                                 the offline driver (also with prompt ids);
 *                                 the text-start rules on a planted model that
 *                                 emits <asr_text> at every step
 *   The Rust binary itself is unbuildable here (no Rust toolchain).
 */
#ifndef QASR_ORACLE_H
#define QASR_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* weight packer rounding: generic/x86 branch (mod.rs:1819-1825) or NEON (neon.rs:673-690) */
#define OR_ROUND_HALF_AWAY 0
#define OR_TRUNC 1

/* ---- int8 ---------------------------------------------------------------- */
void or_quantize_bf16_rows(const uint16_t *w, int64_t n, int64_t k, int mode,
                           int8_t *q, float *scales);
float or_quantize_act(const float *x, int64_t k, int8_t *q);
void or_matvec_w8a8(float *y, const int8_t *xq, float xs, const int8_t *w,
                    const float *ws, const float *bias, int64_t k, int64_t n);
void or_linear_int8(float *y, const float *x, const int8_t *w, const float *ws,
                    const float *bias, int64_t k, int64_t n);
void or_linear_int8_qkv(float *q, float *kk, float *v, const float *x,
                        const int8_t *wq, const float *sq, const int8_t *wk, const float *sk,
                        const int8_t *wv, const float *sv, int64_t in_dim, int64_t q_dim,
                        int64_t kv_dim);
void or_linear_int8_swiglu(float *ffn, const float *x, const int8_t *w, const float *ws,
                           int64_t in_dim, int64_t inter);
void or_linear_int8_addto(float *y, const float *x, const int8_t *w, const float *ws,
                          int64_t in_dim, int64_t out_dim);
int64_t or_argmax_int8(const float *x, const int8_t *w, const float *ws, int64_t in_dim,
                       int64_t out_dim, float *best_val, float *second_val);

/* ---- float ops ----------------------------------------------------------- */
float or_hsum8(const float v[8]);
float or_dot_f32(const float *a, const float *b, int64_t n);
void or_rms_norm(float *out, const float *x, const float *w, int64_t seq, int64_t hidden, float eps);
void or_rms_norm_per_head(float *x, const float *w, int64_t seq, int64_t heads, int64_t hd, float eps);
void or_rope_table(float *cos_t, float *sin_t, int64_t n_pos, int64_t hd, float theta);
void or_apply_rope(float *x, const float *cos_t, const float *sin_t, int64_t seq,
                   int64_t heads, int64_t hd);
void or_causal_attention(float *out, const float *q, const float *k_base, const float *v_base,
                         int64_t head_stride, int64_t seq_q, int64_t seq_k, int64_t n_heads,
                         int64_t n_kv_heads, int64_t hd, float scale, int64_t q_offset);
void or_bidir_attention(float *out, const float *q, const float *k, const float *v,
                        int64_t seq, int64_t n_heads, int64_t hd, float scale,
                        const int32_t *window_starts, int64_t n_windows);
float or_fast_exp(float x);
void or_swiglu_rows(float *out, const float *gate_up, int64_t seq, int64_t inter);
void or_gelu(float *x, int64_t n);
void or_layer_norm(float *out, const float *x, const float *w, const float *b,
                   int64_t seq, int64_t hidden, float eps);
void or_sinusoidal_pe(float *pe, int64_t n_pos, int64_t d_model);

/* ---- GEMM (restates cblas_sgemm call sites) ----------------------------- */
/* C[m,n] = (beta_one ? C[m,n] : 0) + sum_k A[m,k] * B[n,k] */
void or_sgemm_nt(int64_t M, int64_t N, int64_t K, const float *A, int64_t lda,
                 const float *B, int64_t ldb, float *C, int64_t ldc, int beta_one);
void or_linear(float *y, const float *x, const float *w, const float *b, int64_t seq,
               int64_t in_dim, int64_t out_dim);
void or_linear_accumulate(float *y, const float *x, const float *w, const float *b,
                          int64_t seq, int64_t in_dim, int64_t out_dim);
void or_conv2d(float *out, const float *in, const float *w, const float *b, int64_t c_in,
               int64_t c_out, int64_t h_in, int64_t w_in, int64_t kh, int64_t kw,
               int64_t stride, int64_t pad);
void or_bf16_to_f32(float *dst, const uint16_t *src, int64_t n);

/* ---- mel ----------------------------------------------------------------- */
int64_t or_mel_frames(int64_t n_samples);
int64_t or_mel(const float *samples, int64_t n_samples, float *mel_out);

/* ---- models -------------------------------------------------------------- */
typedef struct {
    int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, intermediate, vocab;
    float eps, theta;
} or_dec_config;

typedef struct {
    const uint16_t *wq, *wk, *wv, *wo, *gate, *up, *down;     /* bf16 [out, in] */
    const float *q_norm, *k_norm, *input_norm, *post_attn_norm;
} or_dec_layer;

typedef struct {
    const uint16_t *embed;          /* bf16 [vocab, hidden]; tied LM head */
    const float *norm;              /* [hidden] */
    const or_dec_layer *layers;     /* [n_layers] */
} or_dec_weights;

typedef struct {
    int32_t d_model, n_layers, n_heads, head_dim, ffn_dim, output_dim;
    int32_t chunk_size, n_window_infer, conv_hidden;
} or_enc_config;

typedef struct {
    const uint16_t *wq, *wk, *wv, *wo, *fc1, *fc2;          /* bf16 [out, in] */
    const float *bq, *bk, *bv, *bo, *b1, *b2;
    const float *ln1_w, *ln1_b, *ln2_w, *ln2_b;
} or_enc_layer;

typedef struct {
    const uint16_t *conv1_w, *conv2_w, *conv3_w, *conv_out_w;   /* bf16 */
    const float *conv1_b, *conv2_b, *conv3_b;
    const or_enc_layer *layers;
    const float *ln_post_w, *ln_post_b;
    const uint16_t *proj1_w, *proj2_w;
    const float *proj1_b, *proj2_b;
} or_enc_weights;

typedef struct or_decoder or_decoder;
typedef struct or_encoder or_encoder;

or_decoder *or_decoder_create(const or_dec_config *cfg, const or_dec_weights *w,
                              int pack_mode, int64_t max_seq);
void or_decoder_destroy(or_decoder *d);
const int8_t *or_decoder_packed(const or_decoder *d, int layer, int which, const float **scales);
void or_decoder_set_len(or_decoder *d, int64_t len);
void or_decoder_set_kv_bf16(or_decoder *d, int on);
int64_t or_decoder_len(const or_decoder *d);
void or_decoder_prefill(or_decoder *d, const float *embeds, int64_t seq_len);
void or_decoder_prefill_hidden(or_decoder *d, const float *embeds, int64_t seq_len, float *hidden);
void or_decoder_prefill_logits(or_decoder *d, const float *embeds, int64_t seq_len, const uint16_t *lm_bf16,
                               int64_t out_dim, float *logits);
void or_argmax_f32_rows(const float *x, int64_t rows, int64_t cols, int32_t *idx);
int32_t or_decoder_forward(or_decoder *d, const float *embed, float *best_val, float *second_val,
                           float *hidden_out);
void or_embed_token(const or_decoder *d, int32_t token, float *out);
const float *or_decoder_kv(const or_decoder *d, int which);   /* 0: K, 1: V */

or_encoder *or_encoder_create(const or_enc_config *cfg, const or_enc_weights *w);
void or_encoder_destroy(or_encoder *e);
int64_t or_encoder_tokens(const or_encoder *e, int64_t mel_frames);
int64_t or_encoder_forward(or_encoder *e, const float *mel, int64_t frames, float *out);

/* Offline transcription with a forced number of decode steps (transcribe.rs:63-247):
 * mel -> encoder -> prompt -> prefill(total-1) -> n_steps forwards.  Returns the
 * prompt length; tokens/margins get n_steps entries; times_ms[4] = mel, enc,
 * prefill(+first forward), decode. */
int64_t or_transcribe_forced(or_decoder *d, or_encoder *e, const float *samples,
                             int64_t n_samples, int32_t n_steps, int32_t *tokens,
                             float *margins, double *times_ms);
/* The same with transcribe_segment's optional prompt ids (transcribe.rs:97-169):
 * prompt between PREFIX_HEAD and PREFIX_TAIL, force (the language ids and
 * <asr_text>) after SUFFIX_BASE, then past and <asr_text> when n_past > 0. */
int64_t or_transcribe_prompt(or_decoder *d, or_encoder *e, const float *samples, int64_t n_samples,
                             const int32_t *prompt, int64_t n_prompt, const int32_t *force, int64_t n_force,
                             const int32_t *past, int64_t n_past, int32_t n_steps, int32_t *tokens,
                             float *margins, double *times_ms);
/* the id rows of that layout: head [9 + n_prompt] before the audio rows,
 * tail [6 + n_force + n_past + (n_past > 0)] after them; returns their sum */
int64_t or_prompt_ids(const int32_t *prompt, int64_t n_prompt, const int32_t *force, int64_t n_force,
                      const int32_t *past, int64_t n_past, int32_t *head, int64_t *n_head, int32_t *tail,
                      int64_t *n_tail);
/* find_split_point (transcribe.rs:252-277) and transcribe_audio's split list
 * (transcribe.rs:323-341; returns the count, writes min(count, cap)) */
int64_t or_find_split_point(const float *x, int64_t n, int64_t target, float search_sec);
int64_t or_segment_splits(const float *x, int64_t n, float segment_sec, float search_sec, int64_t *splits,
                          int64_t cap);

/* Threads used by the oracle's OpenMP loops; results do not depend on it. */
/* streaming (stream_push_audio, transcribe.rs:902-1304), oracle_stream.c */
typedef struct {
    float chunk_sec;
    int32_t rollback, unfixed_chunks, max_new_tokens, past_text_conditioning;
    int32_t stop_tokens[2];
} or_stream_config;
typedef struct or_stream or_stream;
void or_stream_default_config(or_stream_config *c);
or_stream *or_stream_create(or_decoder *d, or_encoder *e, const or_stream_config *cfg, int64_t hidden);
void or_stream_destroy(or_stream *s);
int64_t or_stream_push(or_stream *s, const float *samples, int64_t n, int finalize, int32_t *out, int64_t cap);
int64_t or_stream_tokens(const or_stream *s, int32_t *out, int64_t cap);
/* QwenCtx::prompt_tokens / force_prompt_tokens for the following chunks
 * (transcribe.rs:1037-1089); n = 0 clears */
void or_stream_set_prompt(or_stream *s, const int32_t *prompt, int64_t n_prompt, const int32_t *force,
                          int64_t n_force);
void or_stream_stats(const or_stream *s, int64_t *stats);
int64_t or_tail_repeat_blocks(const int32_t *t, int64_t n, int64_t max_period, int64_t *period);

void or_set_threads(int n);
const char *or_int8_dot_kind(void);
void or_set_int8_dot(int vnni512);
int or_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
