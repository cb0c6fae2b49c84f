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
 * binding a maintainer would add is generated from this header by
 * `python -m qwenasr_amd.ffi_rust`.
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
void qasr_hip_destroy(qasr_hip *h);   /* free every decoder / encoder / allocation made on h first */
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
/* device-to-device copy on the handle's stream with the library's own copy
 * kernel (asynchronous; also the known-size kernel that calibrates HBM
 * traffic counters) */
int qasr_hip_copy(qasr_hip *h, void *dst, const void *src, size_t bytes);

/* ---- timing on the handle's stream (HIP events) ------------------------- */
int qasr_hip_timer_start(qasr_hip *h);
int qasr_hip_timer_stop(qasr_hip *h, float *ms);    /* synchronises */
/* queues a wait of `us` microseconds (0..100000) on the handle's stream:
 * launches enqueued while it runs start back to back when it ends, so a timer
 * started behind it measures the GPU rather than the host's launch rate (no
 * counterpart in the reference, whose kernels run on the calling thread) */
int qasr_hip_timer_hold(qasr_hip *h, int us);

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
/* No counterpart in the reference.  qasr_hip_argmax_int8 (norm_w null) or
 * qasr_hip_rmsnorm_argmax_int8 (norm_w set) for callers that cannot allocate
 * (code under HIP graph capture, serving loops that forbid hipMalloc): no
 * handle, no device allocation.  Runs on `stream` (a hipStream_t; null: the
 * null stream) of the current device; the block partials live in a 32 KiB
 * device array each GPU holds until the process ends, so calls that overlap
 * on one GPU race (order them on one stream).  in_dim a multiple of 64, at
 * most 4096; every pointer is device memory. */
int qasr_hip_argmax_int8_noalloc(void *stream, const float *x, const float *norm_w, float eps,
                                 const int8_t *w, const float *ws, int64_t in_dim, int64_t out_dim,
                                 int32_t *idx);

/* The aligner's per-row argmax (align.rs:312-321) over device logits
 * x [rows][ld] (cols <= ld used): idx (device [rows]) = lowest column of the
 * row maximum, NaN values skipped, 0 when column 0 is NaN. */
int qasr_hip_argmax_f32_rows(qasr_hip *h, const float *x, int64_t ld, int64_t rows, int64_t cols, int32_t *idx);

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
 * head_dim == 128, n_heads == 2 * n_kv_heads; seq_q > 1 uses the multi-row kernel. */
int qasr_hip_causal_attention(qasr_hip *h, float *out, const float *q, const float *k_base,
                              const float *v_base, int64_t head_stride, int64_t seq_q,
                              int64_t seq_k, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                              float scale, int64_t q_offset);
/* the same single-query (decode) attention over a bf16 KV cache (the config-3
 * layout; no counterpart in the reference, whose KV cache is f32): seq_q must
 * be 1; k_base / v_base hold bf16 [kv_head][pos][head_dim] */
int qasr_hip_causal_attention_bf16kv(qasr_hip *h, float *out, const float *q, const uint16_t *k_base,
                                     const uint16_t *v_base, int64_t head_stride, int64_t seq_k,
                                     int64_t n_heads, int64_t n_kv_heads, int64_t hd, float scale,
                                     int64_t q_offset);

/* ---- A15/A16: dense GEMMs (MFMA) ----------------------------------------
 * linear (kernels/mod.rs:550-584) / linear_accumulate (mod.rs:591-628) on
 * bf16-valued weights, as the reference runs them through cblas_sgemm after
 * bf16->f32 conversion: y[seq, out] = x W^T (+ bias), or with accumulate != 0
 * y = (y + bias) + x W^T.  x f32 is split into three bf16 terms so every
 * product is exact and accumulation is f32 (f32-class accuracy). */
int qasr_hip_linear_bf16w(qasr_hip *h, float *y, const float *x, const uint16_t *w_bf16,
                          const float *bias, int64_t seq, int64_t in_dim, int64_t out_dim,
                          int accumulate);
/* int8 weights x bf16 activations (the prefill / encoder GEMM of the int8 path):
 * y[M, N] = (sum_k a[m, k] * q[n, k]) * scales[n]; q and scales as packed by
 * qasr_hip_pack_int8_rows.  MFMA bf16 with exact int8->bf16 dequantisation. */
int qasr_hip_gemm_w8_bf16(qasr_hip *h, float *y, const uint16_t *a_bf16, const int8_t *w,
                          const float *scales, int64_t M, int64_t N, int64_t K);
/* layer_norm (kernels/mod.rs:1160-1189, AVX order); hidden % 16 == 0, <= 4096 */
int qasr_hip_layer_norm(qasr_hip *h, float *out, const float *x, const float *w, const float *b,
                        int64_t seq, int64_t hidden, float eps);
/* bidirectional_attention (kernels/mod.rs:1386-1471) over windows of window_tokens
 * (every window full except the last); q/k/v/out [seq][n_heads * head_dim], head_dim 64 or 128 */
int qasr_hip_bidirectional_attention(qasr_hip *h, float *out, const float *q, const float *k,
                                     const float *v, int64_t seq, int64_t n_heads, int64_t head_dim,
                                     float scale, int64_t window_tokens);

/* ---- checkpoints: safetensors (safetensors.rs) ---------------------------
 * A read-only mapping of one checkpoint file or of a directory's shards.
 * Tensor data stays in the mapping (no host copy); the *_load_st loaders
 * stream it through pinned staging buffers into HBM and pack on the GPU.
 * Free the qasr_st after the loads that read it. */
typedef struct qasr_st qasr_st;
#define QASR_ST_UNKNOWN 0
#define QASR_ST_F32 1
#define QASR_ST_F16 2
#define QASR_ST_BF16 3
#define QASR_ST_I32 4
#define QASR_ST_I64 5
#define QASR_ST_BOOL 6
#define QASR_ST_MAX_DIMS 8
/* MultiSafetensors::open (safetensors.rs:212-250): <dir>/model.safetensors
 * when it opens, else every <dir>/model-*.safetensors in byte order of names */
int qasr_hip_st_open(const char *model_dir, qasr_st **out);
/* SafetensorsFile::open (safetensors.rs:73-140); headers are validated (UTF-8
 * JSON, offsets inside the data section and consistent with dtype x shape) */
int qasr_hip_st_open_file(const char *path, qasr_st **out);
void qasr_hip_st_free(qasr_st *st);
int64_t qasr_hip_st_count(const qasr_st *st);           /* distinct tensor names */
int64_t qasr_hip_st_shards(const qasr_st *st);
const char *qasr_hip_st_name(const qasr_st *st, int64_t i);   /* shard order, then header order */
/* MultiSafetensors::find (safetensors.rs:254-262): the first shard holding
 * name; dtype QASR_ST_*, shape [QASR_ST_MAX_DIMS], data points into the
 * mapping; each output pointer may be null.  QASR_ERR_INVALID when absent. */
int qasr_hip_st_find(const qasr_st *st, const char *name, int *dtype, int *ndim, int64_t *shape,
                     const void **data, int64_t *bytes);

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
 * table (decoder.rs:301-338, computed on the host with libm and uploaded).
 * max_seq is the initial capacity: a prefill, forward, generate or
 * transcription that needs more positions doubles the cache first
 * (KvCache::grow, decoder.rs:199-231; at least to what the call needs, in
 * whole 256-position buckets, at most 2^20 positions), keeping every row.
 * The attention shape must be that of both Qwen3-ASR decoders: 16 query
 * heads and 8 KV heads of head_dim 128 (QASR_ERR_INVALID otherwise); hidden
 * and intermediate multiples of 64, hidden <= 4096, intermediate <= 6144. */
int qasr_hip_decoder_load(qasr_hip *h, const qasr_dec_config *cfg, const qasr_dec_weights *w,
                          int round_mode, int64_t max_seq, int kv_bf16, qasr_decoder **out);
/* Decoder::load (decoder.rs:70-167) from a checkpoint: the reference's tensor
 * names; matrices BF16 (shapes checked against cfg), norms F32 or BF16.  A
 * thinker.lm_head.weight [rows, hidden] of any row count (vocab, or the forced
 * aligner's classify_num, config.rs:86-88, 145-150) is packed as the int8
 * decode head, whose argmax then ranges over those rows, and becomes the
 * prefill-logits head (as qasr_hip_decoder_set_lm_head) (decoder.rs:143-157);
 * without it both heads are the tied embedding. */
int qasr_hip_decoder_load_st(qasr_hip *h, const qasr_st *st, const qasr_dec_config *cfg, int round_mode,
                             int64_t max_seq, int kv_bf16, qasr_decoder **out);
/* Rows of the int8 decode head (cfg.lm_head_dim(), config.rs:86-88): vocab for
 * a tied head, the separate head's rows otherwise; -1 for a null decoder. */
int64_t qasr_hip_decoder_head_rows(const qasr_decoder *d);
void qasr_hip_decoder_free(qasr_decoder *d);
/* decoder_prefill (decoder.rs:455-547): host f32 embeddings [seq_len, hidden] */
int qasr_hip_decoder_prefill(qasr_decoder *d, const float *embeds, int64_t seq_len);
/* decoder_prefill_logits (decoder.rs:649-681), the forced aligner's path:
 * prefill of seq_len rows, then the final RMSNorm of every row and the bf16
 * LM head (f32-class GEMM); logits host [seq_len][qasr_hip_decoder_logits_dim].
 * The head is the tied embedding unless qasr_hip_decoder_set_lm_head gave a
 * separate one (decoder.lm_head_bf16, decoder.rs:143: host bf16 [out_dim][hidden],
 * copied; null restores the tied embedding). */
int qasr_hip_decoder_set_lm_head(qasr_decoder *d, const uint16_t *w_bf16, int64_t out_dim);
int64_t qasr_hip_decoder_logits_dim(const qasr_decoder *d);
int qasr_hip_decoder_prefill_logits(qasr_decoder *d, const float *embeds, int64_t seq_len, float *logits);
/* The forced aligner's use of those logits (align.rs:300-321): the same
 * prefill, then the head and a per-row argmax only for the n_rows prefill rows
 * listed in rows (host, each in [0, seq_len): the <timestamp> positions),
 * written to idx (host [n_rows]).  The argmax is the reference's left scan:
 * lowest column of the row maximum, NaN values skipped, 0 when column 0 is NaN.
 * The logits stay on the device; only the indices come back. */
int qasr_hip_decoder_prefill_argmax(qasr_decoder *d, const float *embeds, int64_t seq_len, const int32_t *rows,
                                    int64_t n_rows, int32_t *idx);
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
/* Inspection hook with no counterpart in the reference (whose argmax_matvec_int8
 * returns the index only): the winning logit of the last decode step's LM-head
 * argmax (the value the returned token was chosen by), for callers and tests
 * that check a step beyond its token id. */
int qasr_hip_decoder_last_logit(qasr_decoder *d, float *best);
/* kv_cache.len accessors (transcribe.rs:173, 1106); set_len stays within the
 * current capacity */
int qasr_hip_decoder_set_len(qasr_decoder *d, int64_t len);
int64_t qasr_hip_decoder_len(const qasr_decoder *d);
/* kv_cache.max_seq (decoder.rs:174-231): the positions the cache holds now
 * (the max_seq of the kv_upload / kv_download layout); -1 for a null decoder */
int64_t qasr_hip_decoder_capacity(const qasr_decoder *d);
/* test hooks: the packed int8 rows / scales of layer `layer` (-1 = LM head),
 * which = 0 q, 1 k, 2 v, 3 o, 4 gate_up (interleaved), 5 down; and the KV cache
 * in the reference layout [layer][kv_head][max_seq][head_dim] as f32 (a bf16
 * cache is rounded to nearest even on upload and widened exactly on download) */
int qasr_hip_decoder_packed(qasr_decoder *d, int layer, int which, int8_t *q_host,
                            float *scales_host);
int qasr_hip_decoder_kv_upload(qasr_decoder *d, const float *k_host, const float *v_host);
int qasr_hip_decoder_kv_download(qasr_decoder *d, float *k_host, float *v_host);
/* the same for positions [start, start + n) only: host [layer][kv_head][n][head_dim] */
int qasr_hip_decoder_kv_upload_rows(qasr_decoder *d, int64_t start, int64_t n, const float *k_host,
                                    const float *v_host);
int qasr_hip_decoder_kv_download_rows(qasr_decoder *d, int64_t start, int64_t n, float *k_host, float *v_host);
/* decode-step tuning: attention context splits, 1..64 (0 keeps the current
 * value, -1 restores the automatic choice per context bucket of 256
 * positions: 8 up to 1024 positions, 16 up to 2048, then about one per 64).
 * At 1, 2, 4, 8 or 16 splits with 16 query / 8 KV heads the o_proj kernel
 * merges the split partials in its prologue; otherwise the attention kernel's
 * last block per KV head merges them.  use_graph: steps replay a captured HIP
 * graph, one per context bucket (default 1). */
int qasr_hip_decoder_set_options(qasr_decoder *d, int attn_splits, int use_graph);
/* Profiling hook with no counterpart in the reference: in the profiling build
 * (libqasr_hip_stamps.so, `make stamps`) the decode step's fused qkv +
 * attention, o_proj, gate_up and down launches of every layer write the 100 MHz
 * real-time counter at their phase boundaries into dev ([4 kinds][n_layers]
 * [2048 blocks][16] uint64; a launch uses its first gridDim.x blocks); null
 * stops.  The product library returns QASR_ERR_INVALID. */
int qasr_hip_decoder_set_stamps(qasr_decoder *d, void *dev, int64_t bytes);
/* No counterpart in the reference (the decode step's launch shape, for tuning
 * and tests).  fuse_qkv_attention = 1 (default): each layer's RMSNorm + qkv
 * matvec and its decode attention run as one launch, the qkv rows handed to
 * the attention blocks as (tag, value) pairs; 0: two launches.  Tokens and
 * KV rows are bit-identical either way. */
int qasr_hip_decoder_set_fusion(qasr_decoder *d, int fuse_qkv_attention);
/* per-kernel timing over n_steps real decode steps from the current KV length
 * (no graph).  After each step every kernel kind is launched once per layer
 * (the LM head n_layers times) back to back between two HIP events on the
 * handle's stream, from the step's input state.  Kinds: 0 norm+qkv (with the
 * fused launch: norm+qkv+attention), 1 attention (with the fused launch:
 * nothing), 2 o_proj, 3 norm+gate_up+swiglu, 4 down, 5 norm+LM-head argmax
 * streaming pass, 6 argmax merge (+ step-state update), 7 norm+qkv as its own
 * launch (not part of a fused step: launches_per_step 0).  Outputs average us
 * per launch, algorithmic bytes per launch and launches per step (8 entries
 * each).  The KV length is restored afterwards. */
int qasr_hip_decoder_profile(qasr_decoder *d, int32_t n_steps, float *us_per_launch,
                             double *bytes_per_launch, int32_t *launches_per_step);

/* ---- model level: audio front end (audio.rs:273-372, encoder.rs) ---------- */
typedef struct {
    int32_t d_model, n_layers, n_heads, head_dim, ffn_dim, output_dim;
    int32_t chunk_size, n_window_infer, conv_hidden;        /* QwenConfig enc_*, config.rs:29-39 */
} qasr_enc_config;

typedef struct {                                        /* EncLayer, encoder.rs:7-24 */
    const uint16_t *wq, *wk, *wv, *wo, *fc1, *fc2;      /* host bf16 [out, in] */
    const float *bq, *bk, *bv, *bo, *b1, *b2;
    const float *ln1_w, *ln1_b, *ln2_w, *ln2_b;
} qasr_enc_layer;

typedef struct {                                        /* Encoder, encoder.rs:78-93 */
    const uint16_t *conv1_w, *conv2_w, *conv3_w, *conv_out_w;   /* bf16 [out, in*3*3] / [d, 480*16] */
    const float *conv1_b, *conv2_b, *conv3_b;
    const qasr_enc_layer *layers;
    const float *ln_post_w, *ln_post_b;
    const uint16_t *proj1_w, *proj2_w;
    const float *proj1_b, *proj2_b;
} qasr_enc_weights;

typedef struct qasr_encoder qasr_encoder;

/* Encoder::load (encoder.rs:123-182) plus the mel tables (audio.rs:225-330) */
int qasr_hip_encoder_load(qasr_hip *h, const qasr_enc_config *cfg, const qasr_enc_weights *w,
                          qasr_encoder **out);
/* Encoder::load (encoder.rs:123-182) from a checkpoint: weight matrices (the
 * convolutions included) BF16, biases and norms F32 or BF16 */
int qasr_hip_encoder_load_st(qasr_hip *h, const qasr_st *st, const qasr_enc_config *cfg, qasr_encoder **out);
void qasr_hip_encoder_free(qasr_encoder *e);
int64_t qasr_hip_encoder_tokens(const qasr_encoder *e, int64_t mel_frames);
/* mel_spectrogram (audio.rs:273): host samples -> host mel [128][frames]
 * (mel_out NULL: only report *frames) */
int qasr_hip_mel(qasr_encoder *e, const float *samples, int64_t n_samples, float *mel_out,
                 int64_t *frames);
/* Encoder::forward (encoder.rs:186): host mel [128][frames] -> host [tokens][output_dim] */
int qasr_hip_encoder_forward(qasr_encoder *e, const float *mel, int64_t frames, float *out,
                             int64_t *n_tokens);
/* Encoder::forward of n (1..64) mels in one pass (no counterpart in the
 * reference, which encodes one mel per call): mels[j] host [128][frames[j]];
 * each sequence's rows equal those of qasr_hip_encoder_forward on its own
 * mel bit for bit (its attention windows restart at its first row), and they
 * follow one another in out (host [sum tokens][output_dim]); tokens[j] = the
 * row count of sequence j.  The streaming drivers' stream batch encodes all
 * of a round's encoder windows this way. */
int qasr_hip_encoder_forward_batch(qasr_encoder *e, int32_t n, const float *const *mels, const int64_t *frames,
                                   float *out, int64_t *tokens);
/* transcribe_segment (transcribe.rs:63-247) with a forced decode length and no
 * text prompt: mel -> encoder -> prompt -> prefill(total - 1) -> n_steps greedy
 * forwards, all device-resident.  times_ms (optional, 4 entries): mel, encoder,
 * prefill + first forward, remaining decode. */
int qasr_hip_transcribe_forced(qasr_decoder *d, qasr_encoder *e, const float *samples,
                               int64_t n_samples, int32_t n_steps, int32_t *tokens_out,
                               double *times_ms);

/* transcribe_segment (transcribe.rs:63-247) with its own stop rule: the same
 * pipeline as qasr_hip_transcribe_forced, then greedy forwards until one
 * yields a stop token (151643 endoftext, 151645 im_end) or max_tokens tokens
 * have been produced (the reference's max_tokens is 2048).  tokens_out
 * (capacity max_tokens) receives every token produced, the stop included;
 * *n_out their count. */
int qasr_hip_transcribe(qasr_decoder *d, qasr_encoder *e, const float *samples, int64_t n_samples,
                        int32_t max_tokens, int32_t *tokens_out, int64_t *n_out, double *times_ms);
/* The ids transcribe_segment turns into text (transcribe.rs:196-214): those
 * after the first <asr_text> (151704) and before the first stop token, in
 * order; written to out (nullable: count only).  Returns the count (-1 for a
 * null raw).  Host only. */
int64_t qasr_hip_text_tokens(const int32_t *raw, int64_t n, int32_t *out);
/* The optional ids of transcribe_segment's prompt (transcribe.rs:97-169), as
 * QwenCtx::prepare_prompt_tokens (context.rs:197-230) leaves them:
 *   prompt: QwenCtx::prompt_tokens, the tokenizer's ids of the text prompt,
 *           placed between PREFIX_HEAD and PREFIX_TAIL;
 *   force:  QwenCtx::force_prompt_tokens, the ids of "language <Name>"
 *           followed by <asr_text> (151704), placed after SUFFIX_BASE.
 * A null pointer with a zero count leaves that part out. */
typedef struct {
    const int32_t *prompt;
    int64_t n_prompt;
    const int32_t *force;
    int64_t n_force;
} qasr_prompt;
/* transcribe_segment (transcribe.rs:63-247) with its whole prompt: PREFIX_HEAD,
 * prompt, PREFIX_TAIL, the audio rows, SUFFIX_BASE, force, and when n_past > 0
 * the previous segments' text ids (past) followed by <asr_text>; then the
 * decode loop of qasr_hip_transcribe.  prompt may be null.  Every id must lie
 * in [0, vocab). */
int qasr_hip_transcribe_prompt(qasr_decoder *d, qasr_encoder *e, const float *samples, int64_t n_samples,
                               const qasr_prompt *prompt, const int32_t *past, int64_t n_past,
                               int32_t max_tokens, int32_t *tokens_out, int64_t *n_out, double *times_ms);
/* qasr_hip_text_tokens with the text region open from the first token when
 * text_open != 0, as transcribe_segment starts when its prompt holds
 * forced-language or past-text ids (past_asr_text, transcribe.rs:196); a
 * later <asr_text> is skipped, not counted.  Host only. */
int64_t qasr_hip_text_tokens_from(const int32_t *raw, int64_t n, int text_open, int32_t *out);
/* transcribe_audio's segment starts (transcribe.rs:323-341): 0, then, while
 * the audio after the last start is longer than segment_sec plus the search
 * margin, the center of the quietest 100 ms window (1600 samples, hop 800,
 * least mean square, the first of equal minima) within +-search of that start
 * + segment_sec (find_split_point, transcribe.rs:252-277), where search =
 * min(search_sec, segment_sec / 2); at most 127 starts.  segment_sec <= 0 or
 * short audio: the one start 0.  Returns the count (-1 on bad arguments) and
 * writes min(count, cap) starts.  Host only. */
int64_t qasr_hip_segment_splits(const float *samples, int64_t n_samples, float segment_sec, float search_sec,
                                int64_t *splits_out, int64_t cap);

/* ---- the reference's C API (c_api.rs) at token level -------------------------
 * Text is token ids; turning them into bytes is the caller's tokenizer
 * (tokenizer.rs).  One engine = one handle, the checkpoint mapping, the
 * encoder and the decoder (QwenCtx::load, context.rs:86-150). */
typedef struct qasr_engine qasr_engine;
typedef struct qasr_engine_stream qasr_engine_stream;
/* QwenConfig::detect (config.rs:108-156) from tensor shapes: decoder hidden
 * and vocab from embed_tokens, intermediate from layer 0's gate_proj, the
 * large encoder when audio_tower layer 18 exists; layer counts are those the
 * checkpoint holds (the reference's 28 / 24 / 18 for its checkpoints). */
int qasr_hip_engine_detect(const qasr_st *st, qasr_dec_config *dc, qasr_enc_config *ec);
/* qwen_asr_load_model (c_api.rs:20-46): the model directory's safetensors on
 * GPU `device`; the KV cache holds max_seq positions (0: 8192). */
int qasr_hip_engine_load(const char *model_dir, int device, int64_t max_seq, qasr_engine **out);
void qasr_hip_engine_free(qasr_engine *g);                          /* qwen_asr_free */
int qasr_hip_engine_config(const qasr_engine *g, qasr_dec_config *dc, qasr_enc_config *ec);
/* qwen_asr_transcribe_pcm (c_api.rs:75-95), no segmentation (segment_sec 0,
 * the default): the text token ids of the transcription (up to cap written;
 * *n_out = their count). */
int qasr_hip_engine_transcribe_pcm(qasr_engine *g, const float *samples, int64_t n_samples, int32_t *tokens_out,
                                   int64_t cap, int64_t *n_out);
/* every token of the last transcription, the stop included (segments one
 * after another) */
int qasr_hip_engine_last_raw_tokens(const qasr_engine *g, int32_t *tokens_out, int64_t cap, int64_t *n);
/* the segments of the last transcribe_pcm, [n][4] int64: first sample, end
 * sample, index of the segment's first text id in transcribe_pcm's output,
 * its count of text ids (0: transcribe_audio skips the segment's empty text,
 * transcribe.rs:382).  The caller's text step joins the segments' texts with
 * a space where should_insert_boundary_space (transcribe.rs:279-286) asks. */
int qasr_hip_engine_last_segments(const qasr_engine *g, int64_t *bounds, int64_t cap, int64_t *n);
/* qwen_asr_set_segment_sec (c_api.rs:123-129): transcribe_pcm cuts audio longer
 * than sec plus the search margin at qasr_hip_segment_splits and transcribes
 * the segments one after another, each cut one zero-padded to 0.5 s at least
 * (transcribe.rs:343-372); 0 (the default): one segment */
void qasr_hip_engine_set_segment_sec(qasr_engine *g, float sec);
/* QwenCtx::search_sec (context.rs:145; default 3.0): the split search radius */
void qasr_hip_engine_set_search_sec(qasr_engine *g, float sec);
/* qwen_asr_set_language (c_api.rs:131-148) at token level: ids = the caller's
 * tokenizer encoding of "language " + the normalized language name
 * (set_force_language, context.rs:177-195); the engine appends <asr_text> as
 * prepare_prompt_tokens does (context.rs:215-221).  n = 0: automatic language
 * (the reference's empty string).  Used by transcribe_pcm and by every
 * stream's next push.  Ids outside the vocabulary: QASR_ERR_INVALID, the
 * setting unchanged. */
int qasr_hip_engine_set_language_tokens(qasr_engine *g, const int32_t *ids, int64_t n);
/* QwenCtx::set_prompt (context.rs:165-175) at token level: the encoded text
 * prompt for transcribe_pcm and every stream's next push; n = 0 clears */
int qasr_hip_engine_set_prompt_tokens(qasr_engine *g, const int32_t *ids, int64_t n);
/* qwen_asr_stream_new / _free / _reset (c_api.rs:179-202).  Streams borrow
 * the engine's decoder and encoder; several may be alive and interleave their
 * pushes with each other and with transcribe_pcm (a push after another
 * caller's work prefills every row instead of reusing the KV cache's rows,
 * where the reference's shared cache would hold the other caller's rows).
 * qasr_hip_engine_free releases the device state of streams still alive;
 * they then accept only qasr_hip_engine_stream_free. */
int qasr_hip_engine_stream_new(qasr_engine *g, qasr_engine_stream **out);
void qasr_hip_engine_stream_free(qasr_engine_stream *s);
int qasr_hip_engine_stream_reset(qasr_engine_stream *s);
/* qwen_asr_stream_push (c_api.rs:212-248): append n_samples new samples (16 kHz
 * mono f32), run stream_push_audio over the stream's audio so far with the
 * engine's current stream settings; the newly
 * committed text token ids go to tokens_out (*n_out = their count) */
int qasr_hip_engine_stream_push(qasr_engine_stream *s, const float *samples, int64_t n_samples, int finalize,
                                int32_t *tokens_out, int64_t cap, int64_t *n_out);
/* qwen_asr_stream_get_result (c_api.rs:250-267): every committed text token */
int qasr_hip_engine_stream_get_result(const qasr_engine_stream *s, int32_t *tokens_out, int64_t cap, int64_t *n);
/* qwen_asr_stream_set_* (c_api.rs:269-299): the settings every stream of the
 * engine uses from its next push on (the reference reads them from its
 * context on every push); out-of-range values are ignored */
void qasr_hip_engine_stream_set_chunk_sec(qasr_engine *g, float sec);
void qasr_hip_engine_stream_set_rollback(qasr_engine *g, int32_t tokens);
void qasr_hip_engine_stream_set_unfixed_chunks(qasr_engine *g, int32_t chunks);
void qasr_hip_engine_stream_set_max_new_tokens(qasr_engine *g, int32_t tokens);

/* ---- multi-stream decode (no counterpart in the reference,
 * whose streaming is batch 1 per QwenCtx) ----
 * Up to 32 independent streams share a loaded decoder's weights; each owns a
 * KV region of max_seq positions (<= the decoder's max_seq) and steps together
 * with the others: M = streams int8 MFMA projections, attention over every
 * stream's own cache.  Integer dots are exact, so a stream's tokens equal
 * those of the single-stream decoder run with the same attention split count
 * (e.g. 1 for both).  Creating a batch switches the decoder's own decode
 * steps to the multi-stream attention arithmetic (the lone decoder uses a
 * latency-optimised kernel whose f32 rounding differs), so solo runs on that
 * decoder stay bit-identical to its streams. */
typedef struct qasr_batch qasr_batch;
int qasr_hip_batch_create(qasr_decoder *d, int32_t n_streams, int64_t max_seq, int64_t max_steps,
                          qasr_batch **out);
void qasr_hip_batch_free(qasr_batch *b);
/* decoder_prefill of one stream (host f32 [seq_len][hidden]) */
int qasr_hip_batch_prefill(qasr_batch *b, int32_t stream, const float *embeds, int64_t seq_len);
int qasr_hip_batch_set_len(qasr_batch *b, int32_t stream, int64_t len);
int64_t qasr_hip_batch_len(const qasr_batch *b, int32_t stream);
/* attn_splits: 1, 2, 4, 8, 16 (-1: automatic per context bucket); use_graph as the decoder's */
int qasr_hip_batch_set_options(qasr_batch *b, int attn_splits, int use_graph);
/* n_steps greedy steps of every stream; first_tokens [streams] (each stream's
 * first input token); tokens_out [streams][n_steps] */
int qasr_hip_batch_generate(qasr_batch *b, const int32_t *first_tokens, int32_t n_steps, int32_t *tokens_out);
/* HIP-event timing per kernel kind of a step, us per launch (QASR_BATCH_PROFILE_KINDS
 * entries: embed, in-norm+quant, qkv, q/k prep, attention, merge+quant, o_proj,
 * post-norm+quant, gate_up+swiglu, ffn quant, down, final norm+quant, LM head,
 * argmax finish); launches_per_step (nullable) likewise.  Lengths are restored. */
#define QASR_BATCH_PROFILE_KINDS 14
int qasr_hip_batch_profile(qasr_batch *b, const int32_t *first_tokens, int32_t n_steps, float *us_per_launch,
                           int32_t *launches_per_step);

/* ---- A20: incremental streaming (stream_push_audio, transcribe.rs:902-1304) ----
 * A stream borrows a decoder (its KV cache and step state) and an encoder; one
 * stream per decoder at a time.  Text comes out as token ids (the caller's
 * tokenizer turns them into bytes).  Defaults are QwenCtx's (context.rs:144-150). */
typedef struct qasr_stream qasr_stream;
typedef struct {
    float chunk_sec;                /* 2.0 */
    int32_t rollback;               /* 5 */
    int32_t unfixed_chunks;         /* 2 */
    int32_t max_new_tokens;         /* 32 */
    int32_t past_text_conditioning; /* 0 */
    int32_t stop_tokens[2];         /* TOKEN_ENDOFTEXT 151643, TOKEN_IM_END 151645 */
} qasr_stream_config;
#define QASR_STREAM_STATS 8
void qasr_hip_stream_default_config(qasr_stream_config *cfg);
int qasr_hip_stream_create(qasr_decoder *d, qasr_encoder *e, const qasr_stream_config *cfg, qasr_stream **out);
void qasr_hip_stream_free(qasr_stream *s);
/* StreamState::reset (transcribe.rs:865-883) */
int qasr_hip_stream_reset(qasr_stream *s);
/* samples: the whole audio of the stream so far (16 kHz mono f32); processes
 * every complete chunk past the cursor (and the rest when finalize != 0) and
 * writes the newly committed text token ids to tokens_out (capacity cap);
 * n_out = their count.  After a failed push the stream's position is not
 * defined: reset it before pushing again. */
int qasr_hip_stream_push(qasr_stream *s, const float *samples, int64_t n_samples, int finalize,
                         int32_t *tokens_out, int64_t cap, int64_t *n_out);
/* every committed text token so far (up to cap); n = the total count */
int qasr_hip_stream_tokens(const qasr_stream *s, int32_t *tokens_out, int64_t cap, int64_t *n);
/* QwenCtx::prompt_tokens / force_prompt_tokens (the qasr_prompt ids, copied)
 * for the stream's next chunks (transcribe.rs:1037-1089); null clears both.
 * With forced-language ids every decoded token of the tail is text
 * (transcribe.rs:1166-1172, 1257-1263).  Also for a stream batch's members. */
int qasr_hip_stream_set_prompt(qasr_stream *s, const qasr_prompt *prompt);
int64_t qasr_hip_stream_audio_cursor(const qasr_stream *s);
/* chunks processed, last chunk's reused prefill rows, prefill length, rows
 * prefilled, forwards, total forwards, encoder windows encoded, raw tokens */
int qasr_hip_stream_stats(const qasr_stream *s, int64_t *stats);

/* ---- many streams fed by the streaming pipeline, decoded as one batch -------
 * BASELINE config 4 from real audio: n_streams (1..32) streaming states over
 * one decoder and encoder; each chunk runs its encoder and prompt prefill
 * (with common-prefix reuse) into the stream's slot of a multi-stream batch
 * (max_seq positions each), then every stream with a chunk in that round takes
 * its greedy steps in one batched decode (M = n_streams per projection), each
 * stopping at its own stop token or max_new_tokens.  Per stream the sequence
 * of stream_push_audio operations (transcribe.rs:902-1304) is that of
 * qasr_hip_stream_push, and the decode is the lone decoder's arithmetic, so
 * every stream commits the tokens it would commit alone.  The states belong to
 * the batch: query them with qasr_hip_stream_tokens / _stats / _audio_cursor /
 * _reset through qasr_hip_stream_batch_stream; qasr_hip_stream_push and
 * qasr_hip_stream_free refuse or must not be used on them.  The decoder needs
 * the multi-stream batch's shape (qasr_hip_batch_create). */
typedef struct qasr_stream_batch qasr_stream_batch;
int qasr_hip_stream_batch_create(qasr_decoder *d, qasr_encoder *e, const qasr_stream_config *cfg, int32_t n_streams,
                                 int64_t max_seq, qasr_stream_batch **out);
void qasr_hip_stream_batch_free(qasr_stream_batch *g);
qasr_stream *qasr_hip_stream_batch_stream(qasr_stream_batch *g, int32_t i);
/* wall time of the last push's phases on the library stream, summed over its
 * rounds (HIP events; ms[4]): the encoder pass over every stream's new windows
 * and partial tails, the prompt rows and prefix comparison, the multi-stream
 * prefill, the batched decode */
int qasr_hip_stream_batch_times(const qasr_stream_batch *g, double *ms);
/* samples[i] / n_samples[i]: the whole audio of stream i so far; finalize
 * (nullable) per stream; stream i's newly committed text tokens go to
 * tokens_out + i * cap (nullable), n_out[i] = their count.  Streams advance
 * chunk by chunk in rounds until none has a complete chunk left (or, when
 * finalizing, any audio).  After a failed push the streams' positions are not
 * defined: reset them before pushing again. */
int qasr_hip_stream_batch_push(qasr_stream_batch *g, const float *const *samples, const int64_t *n_samples,
                               const int32_t *finalize, int32_t *tokens_out, int64_t cap, int64_t *n_out);

#ifdef __cplusplus
}
#endif
#endif
