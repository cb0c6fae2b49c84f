// Kernel argument blocks and launcher declarations shared by the qasr_hip
// translation units.  Host code includes this; device code adds common.h.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "common.h"

#define QASR_ROUND_HALF_AWAY_I 0
#define QASR_TRUNC 1

namespace qasr {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum { MV_PLAIN = 0, MV_ADDTO = 1, MV_SWIGLU = 2, MV_BIAS = 3 };

struct MvSeg {
    const int8_t *w;      // [n, K] row-major int8
    const float *ws;      // [n] per-row scales
    float *y;             // outputs (SwiGLU: [n / 2])
    int n;                // rows (multiple of the rows-per-wave)
};

struct MvArgs {
    const float *x;           // f32 [K] activation (unused when the input is an embedding row)
    const uint16_t *embed;    // bf16 embedding table [vocab, K] (EMBED mode)
    const int *state;         // decode-loop state {token, pos, step, flag} (EMBED mode)
    const float *norm_w;      // RMSNorm gain [K] (NORM mode)
    float eps;
    int K;
    MvSeg seg[3];
    int n_total;
    const float *bias;        // MV_BIAS
    float *resid_out;         // EMBED mode: block 0 stores the f32 embedding here
    unsigned long long *stamps;   // profiling build only: [layer][block][QASR_STAMP_SLOTS] (null: none)
    int layer;
};

struct ArgmaxArgs {
    const float *x;
    const float *norm_w;
    float eps;
    int K, N;
    const int8_t *w;
    const float *ws;
    float *part_val;          // [gridDim.x] per-block partials, merged by k_argmax_finish
    int *part_idx;            // [gridDim.x]
    int *out_idx;             // [1]
    float *out_val;           // nullable: [1] the winning logit
    int *state;               // nullable decode-loop state
    int *token_log;           // nullable
    const float *rope_cos, *rope_sin;   // decode loop: RoPE table [max_pos][128]
    float *rope_cur;          // nullable: receives the cos, sin rows of the next position
    int max_pos;
    int *epoch;               // nullable: advanced by one per decode step (the qkv + attention tags)
};

hipError_t launch_pack_int8(const uint16_t *w, int64_t n, int K, int mode, int8_t *q, float *s,
                            hipStream_t st);
hipError_t launch_quant_act(const float *x, int K, int8_t *q, float *xs, hipStream_t st);
hipError_t launch_w8a8(const MvArgs &a, int mode, bool norm, bool embed, int rows_per_wave,
                       hipStream_t st);
// stream: the per-block pass; finish: the one-block merge (and decode-state update)
hipError_t launch_argmax(const ArgmaxArgs &a, bool norm, int blocks, hipStream_t st, bool stream = true,
                         bool finish = true);
hipError_t launch_copy(void *dst, const void *src, int64_t bytes, hipStream_t st);

// ---- multi-stream decode (config 4) -----------------------------------------
struct BatchMvArgs {
    const int8_t *xq;         // [32][K] int8 activations (rows >= B zero)
    const float *xs;          // [B] activation scales
    const int8_t *w;          // [N][K] int8 weights
    const float *ws;          // [N] row scales
    float *y;                 // [B][ldy] outputs (SwiGLU: N / 2 per row)
    int64_t ldy;
    int K, N, B;
    float *part_val;          // argmax partials [blocks][32]
    int *part_idx;
};
hipError_t launch_embed_rows(float *x, const uint16_t *embed, const int *state, int B, int H, hipStream_t st);
hipError_t launch_quant_rows(const float *x, const float *norm_w, float eps, int K, int B, int8_t *xq, float *xs,
                             hipStream_t st);
hipError_t launch_w8a8_batch(const BatchMvArgs &a, int mode, hipStream_t st);
// gpb_table[pos] (nullable): the attention partition of a step at pos, copied to gpb_dev[stream]
hipError_t launch_argmax_batch(const BatchMvArgs &a, int blocks, int *state, int *token_log, int64_t log_stride,
                               const float *rope_cos, const float *rope_sin, float *rope_cur, int max_pos,
                               const int *gpb_table, int *gpb_dev, hipStream_t st, bool stream = true,
                               bool finish = true);
// split merge per stream + int8 quantization of the merged row (xq [B][2048], xs [B]);
// att nullable.  n_split 1, 2, 4, 8, 16: the o_proj prologue's merge (xq required);
// any other count <= 64: a sequential merge (xq nullable: att only)
hipError_t launch_attn_merge_rows(const float *part, int64_t part_stride, int n_split, float *att,
                                  int64_t att_stride, int8_t *xq, float *xs, int B, hipStream_t st);

// ---- attention / norms / rope ---------------------------------------------
// Position of o[split][e] (e = 128 h + d) among the attention partials of one
// step: after the 2 Hq S (max, sum) entries, split index fastest for the
// split counts the o_proj prologue merges (1, 2, 4, 8, 16: a thread loads
// its S values as one vector), split index slowest otherwise (the merge
// kernel's threads read consecutive e).
__host__ __device__ inline bool part_split_fastest(int S) { return S <= 16 && (S & (S - 1)) == 0; }
// o partial e (= 128 h + d) of `split`, split index slowest: every block's
// stores are contiguous (the multi-stream step always uses this layout)
__host__ __device__ inline int64_t part_o_index_slow(int S, int split, int Hq, int e) {
    return (int64_t)2 * Hq * S + (int64_t)split * Hq * 128 + e;
}
__host__ __device__ inline int64_t part_o_index(int S, int split, int Hq, int e) {
    return part_split_fastest(S) ? (int64_t)(2 * Hq + e) * S + split : part_o_index_slow(S, split, Hq, e);
}

// longest run (8-position groups per block) of the single-stream step form of
// the decode attention (k_attn_step: 4 waves of up to 4 groups)
#define QASR_STEP_MAX_GPB 16

struct AttnDecodeArgs {
    const float *qkv;         // raw projections: q [Hq*D] | k [Hkv*D] | v [Hkv*D]
    const float *q_norm, *k_norm;   // per-head RMSNorm gains [D] (nullable: skip norm+rope)
    const float *rope_cos, *rope_sin;   // [max_pos][D]
    const float *rope_cur;    // nullable: [2][D] cos, sin rows of the current position
    const int *state;         // decode state (pos = state[1]); nullable -> use pos
    int pos;
    void *kcache, *vcache;    // layer base, layout [Hkv][max_seq][D]
    int64_t head_stride;      // max_seq * D (elements)
    float *part;              // [Hkv][n_split][G][D + 2]
    unsigned *counters;       // [Hkv], zero-initialised; the merging block resets its counter
    float *out;               // [Hq * D]
    int n_split;
    int waves;                // waves per block: 4 or 8 (0: 8)
    int gpw;                  // decode step: > 0 selects the 2-dims-per-lane kernel with up to
                              // gpw 8-position groups per wave (gpb <= waves * gpw)
    int gpb;                  // > 0: static partition, 8-position groups per block (rows < head_stride / D)
    float eps, scale;
    // multi-stream decode: blockIdx.y = stream; per-stream strides of the cache
    // (elements), the qkv rows, the partials and the state / rope_cur rows
    int batch;                // streams (0 or 1: one)
    int64_t batch_kv_stride, batch_qkv_stride, batch_part_stride;
    const int *gpb_dev;       // nullable: per-stream groups per block [batch] (overrides gpb)
    const int *stream_order;  // nullable: grid row -> stream of a multi-stream step (largest units first)
    int depth;                // multi-stream mode: groups in flight per wave (1 or 2; 0: 2)
    // multi-stream mode: the streams a launch serves.  A stream whose partition
    // (gpb_dev) has at most QASR_STEP_MAX_GPB groups per block takes the
    // single-stream step form (k_attn_step_batch), a longer one k_attn_decode's,
    // as the single-stream decoder chooses per context bucket.  0: every stream
    // (the step's streams all take this launch's form); 1: only the short
    // partitions; 2: only the long ones (k_qk_prep_rows, k_attn_decode)
    int select;
    // qkv + attention in one launch (launch_qkv_attn): the (tag, value) pairs
    // of the qkv rows, the layer (tag = state[4] * 32 + layer) and the flag a
    // poll that never matched sets
    unsigned long long *qkv_tag;
    int layer;
    int *fault;
    // profiling build only: [layer][block][QASR_STAMP_SLOTS] phase times of the
    // fused launch (null: none)
    unsigned long long *stamps;
};

// one launch for a layer's RMSNorm + qkv matvec (m: the MvArgs of the plain
// qkv launch, R = 4 rows per wave) and its decode attention (a: k_attn_step's
// arguments plus qkv_tag, layer, fault)
hipError_t launch_qkv_attn(const MvArgs &m, const AttnDecodeArgs &a, int n_heads, int n_kv_heads, int head_dim,
                           int kv_bf16, bool embed, int rows_per_wave, hipStream_t st);
// epoch[0] += 1 (one thread)
hipError_t launch_epoch_advance(int *epoch, hipStream_t st);

// multi-stream step prologue (k_qk_prep_rows): q/k per-head norm + RoPE, the new
// K/V row of every stream; run before launch_attn_decode with gpb_dev set
hipError_t launch_qk_prep_rows(const AttnDecodeArgs &a, int n_heads, int n_kv_heads, int head_dim, int kv_bf16,
                               hipStream_t st);
// merge: the last block of each KV head merges the split partials into out;
// otherwise the partials are left for k_oproj_merge (n_split 1, 2, 4 or 8)
hipError_t launch_attn_decode(const AttnDecodeArgs &a, int n_heads, int n_kv_heads, int head_dim,
                              int kv_bf16, hipStream_t st, bool merge = true);

// o_proj += Wo attn with the split-attention merge as its prologue (decode step)
struct OprojMergeArgs {
    const float *part;        // attention partials, split index fastest: (m, l) [2 Hq][S], o [Hq][128][S]
    int n_split, Hkv;
    const int8_t *w;          // [N, K = 2 * Hkv * 128] int8
    const float *ws;          // [N]
    float *y;                 // [N], y += W attn
    int N;
    unsigned long long *stamps;   // profiling build only: [layer][block][QASR_STAMP_SLOTS] (null: none)
    int layer;
};
hipError_t launch_oproj_merge(const OprojMergeArgs &a, int rows_per_wave, hipStream_t st);

hipError_t launch_rms_norm_rows(float *out, const float *x, const float *w, int64_t seq, int hidden,
                                float eps, hipStream_t st);
hipError_t launch_head_norm_rope(float *x, const float *w, const float *cos_t, const float *sin_t,
                                 int64_t seq, int heads, int hd, float eps, int do_norm,
                                 int do_rope, hipStream_t st);

}  // namespace qasr

namespace qasr {
// ---- GEMM ----------------------------------------------------------------
enum { A_F32_SPLIT = 0, A_BF16 = 1, A_CONV = 2 };
enum { B_BF16 = 0, B_I8 = 1 };
// EPI_SWIGLU: B rows interleave (gate, up); C[m][n / 2] = silu(gate) up (ldc
// in outputs, N / 2 of them), the decoder's SwiGLU with its AVX / tail paths
enum { EPI_NONE = 0, EPI_ACCUM = 1, EPI_SCALE = 2, EPI_GELU = 4, EPI_TRANS = 8, EPI_CHW = 16, EPI_SWIGLU = 32 };

struct GemmArgs {
    int M, N, K;
    const void *A;            // [M, lda]  f32 or bf16
    int64_t lda;
    const void *B;            // [N, ldb]  bf16 or int8
    int64_t ldb;
    float *C;                 // [M, ldc]  (EPI_TRANS: [M / gelu_rows][N][gelu_rows])
    int64_t ldc;
    const float *bias;        // [N] or null: C = acc + bias (EPI_ACCUM: C = (C + bias) + acc)
    const float *scale;       // [N] (EPI_SCALE)
    int64_t gelu_n;           // elements of the buffer gelu() sees (EPI_GELU / EPI_TRANS: per chunk)
    int gelu_rows;            // EPI_TRANS: spatial positions per chunk
    int a_vec4, b_vec;        // set by the launcher
    float *ws;                // optional workspace for split-K partials (null: no split)
    int64_t ws_bytes;
    // f32-class path: split K by the shape alone (N <= 1024 and K / 32 >= 16),
    // whatever M, so that a row's result does not depend on how many rows
    // share the call; the launch fails if the workspace is too small
    int split_by_shape;
    // A_CONV (f32-class, implicit im2col): A is a channels-last activation
    // [chunks][conv_hin][conv_win][conv_c]; GEMM row m is output position
    // (chunk, oy, ox) of a conv_hout x conv_wout grid and K index (ky, kx, c)
    // of a conv_kh x conv_kw kernel: input (oy sy - py + ky, ox sx - px + kx),
    // zero outside the input.  conv_c % 32 == 0.
    int conv_hin, conv_win, conv_c, conv_hout, conv_wout, conv_kh, conv_kw, conv_sy, conv_sx, conv_py, conv_px;
    float conv_rc, conv_rkw;  // 1 / conv_c, 1 / conv_kw (set by the launcher)
};

hipError_t launch_gemm(const GemmArgs &g, int asrc, int bsrc, int epi, hipStream_t st);
hipError_t launch_gemm_f32(const GemmArgs &g, hipStream_t st);
}  // namespace qasr

namespace qasr {
// ---- prefill / encoder / mel ------------------------------------------------
#define QASR_ATTN_MAX_SEG 64
struct AttnRowsArgs {
    const float *q;           // row i, head h at q + i * q_rs + h * hd
    int64_t q_rs;
    const float *k, *v;       // kv head g, position j at k + g * k_hs + j * k_rs
    int64_t k_hs, k_rs;
    float *out;               // row i, head h at out + i * o_rs + h * hd
    int64_t o_rs;
    int n_q, n_k;             // query rows; key positions available
    int G;                    // query heads per KV head (32 % G == 0)
    int q_offset;             // causal: query i sees keys [0, q_offset + i]
    int window;               // > 0: query i sees its window [w*window, min((w+1)*window, n_k))
    float scale;
    int kv_div;               // set by launch_attn_rows: block x reads KV head x / kv_div (0 = 1)
    // windowed calls over several sequences (n_seg > 0): sequence j holds rows
    // [seg_lo[j], seg_hi[j]) and its windows start at seg_lo[j]; every seg_lo
    // is a multiple of 32, so no block of rows straddles two sequences and a
    // row meets the same blocks, key chunks and order as in a call of its own
    // sequence alone; rows outside every range are not computed
    int n_seg;
    int seg_lo[QASR_ATTN_MAX_SEG], seg_hi[QASR_ATTN_MAX_SEG];
};
hipError_t launch_attn_rows(const AttnRowsArgs &a, int n_kv_heads, int head_dim, hipStream_t st);
// Causal attention of n sequences (<= QASR_ATTN_MAX_SEQ) in one launch: base
// holds the shared fields (strides, G, scale; q and out at row 0), sequence j
// its first query / output row, KV cache bases, query rows, keys and query
// offset.  Each sequence's rows get the bits of a launch_attn_rows call of its
// own.  128-dim heads with G = 2 (the decoder) only.
#define QASR_ATTN_MAX_SEQ 32
struct AttnSeqArgs {
    AttnRowsArgs base;
    int n;
    int blk[QASR_ATTN_MAX_SEQ + 1];        // set by the launcher
    int64_t row[QASR_ATTN_MAX_SEQ];
    const float *k[QASR_ATTN_MAX_SEQ], *v[QASR_ATTN_MAX_SEQ];
    int n_q[QASR_ATTN_MAX_SEQ], n_k[QASR_ATTN_MAX_SEQ], q_offset[QASR_ATTN_MAX_SEQ];
};
hipError_t launch_attn_rows_seqs(const AttnSeqArgs &s, int n_kv_heads, int head_dim, hipStream_t st);
hipError_t launch_layer_norm_rows(float *out, const float *x, const float *w, const float *b, int64_t seq,
                                  int hidden, float eps, hipStream_t st);
hipError_t launch_swiglu_rows(float *out, const float *gu, int64_t seq, int inter, hipStream_t st);
hipError_t launch_gelu(float *x, int64_t n, hipStream_t st);
hipError_t launch_add_periodic(float *y, const float *table, int64_t rows, int cols, int period, hipStream_t st);
hipError_t launch_im2col3x3s2(float *cols, const float *in, int n_chunks, int C, int H, int W, int64_t cs,
                              int64_t chs, int64_t rs, int Ho, int Wo, hipStream_t st);
hipError_t launch_conv_reshape(float *out, const float *in, int n_chunks, int C, int F, int T, hipStream_t st);
// stem conv1 + bias + GELU, direct (input element (c, ih, iw) at in + c * cs + ih * rs + iw;
// (H + 2) * (W + 2) <= 13312, Ho / Wo the stride-2 output sizes, C >= 16)
hipError_t launch_conv1_direct(float *out, const float *in, int n_chunks, int64_t cs, int64_t rs, int H, int W,
                               const uint16_t *w, const float *bias, int C, int Ho, int Wo, bool nhwc,
                               hipStream_t st);
hipError_t launch_taps_last(uint16_t *out, const uint16_t *in, int O, int Cin, int T, hipStream_t st);
// idle one wave for `us` microseconds (timing helper)
hipError_t launch_delay(int us, hipStream_t st);
// the prefill's q/k per-head norm + RoPE and K/V cache write (one launch)
struct PrefillPostArgs {
    float *qkv;                          // [S][row_stride]: q (Hq heads) | k (Hkv) | v (Hkv), 128 dims each
    int64_t row_stride, S;
    int Hq, Hkv;
    const float *q_norm, *k_norm;        // [128]
    const float *cos_t, *sin_t;          // RoPE rows of positions start .. start + S - 1
    float *kc, *vc;                      // [Hkv][head_stride]
    int64_t head_stride;
    int64_t start;
    float eps;
};
hipError_t launch_prefill_qkv_post(const PrefillPostArgs &a, hipStream_t st);
// The same over n sequences of consecutive rows (<= QASR_ATTN_MAX_SEQ): base
// holds qkv (row 0), row_stride, heads, norms, eps and cos_t / sin_t at
// position 0; sequence j its first row, position, KV bases (this layer) and
// head stride.
struct PrefillPostSeqArgs {
    PrefillPostArgs base;
    int n;
    int64_t row[QASR_ATTN_MAX_SEQ + 1];    // row[n] = all rows
    int64_t start[QASR_ATTN_MAX_SEQ], head_stride[QASR_ATTN_MAX_SEQ];
    float *kc[QASR_ATTN_MAX_SEQ], *vc[QASR_ATTN_MAX_SEQ];
};
hipError_t launch_prefill_qkv_post_seqs(const PrefillPostSeqArgs &a, hipStream_t st);
hipError_t launch_row_diff(const float *a, const float *b, int64_t rows, int64_t H, int *flags, hipStream_t st);
// idx[r] = lowest column of the maximum of row r's non-NaN values (0 when column 0 is NaN)
hipError_t launch_argmax_f32_rows(const float *x, int64_t ld, int64_t rows, int64_t cols, int32_t *idx,
                                  hipStream_t st);
hipError_t launch_gather_rows(float *dst, const float *src, const int32_t *rows, int64_t n, int64_t H,
                              hipStream_t st);
hipError_t launch_build_prompt(float *out, const uint16_t *embed, const int *toks, int n_head, const float *mid,
                               int n_mid, int n_tail, int H, hipStream_t st);
hipError_t launch_mel_frames(float *fr, const float *x, int64_t ns, const float *window, int nf, hipStream_t st);
hipError_t launch_mel_power(float *pT, const float *re, const float *im, int nf, hipStream_t st);
hipError_t launch_mel_log_norm(float *mel, int64_t n, float *bmax, hipStream_t st);
hipError_t launch_head_norm_rope_strided(float *x, int64_t row_stride, const float *w, const float *cos_t,
                                         const float *sin_t, int64_t seq, int heads, float eps, int do_norm,
                                         int do_rope, hipStream_t st);
}  // namespace qasr
