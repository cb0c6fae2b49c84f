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
};

struct ArgmaxArgs {
    const float *x;
    const float *norm_w;
    float eps;
    int K, N;
    const int8_t *w;
    const float *ws;
    float *part_val;          // [gridDim.x]
    int *part_idx;            // [gridDim.x]
    unsigned *counter;        // zero before the first launch; the last block resets it
    int *out_idx;             // [1]
    int *state;               // nullable decode-loop state
    int *token_log;           // nullable
};

hipError_t launch_pack_int8(const uint16_t *w, int64_t n, int K, int mode, int8_t *q, float *s,
                            hipStream_t st);
hipError_t launch_quant_act(const float *x, int K, int8_t *q, float *xs, hipStream_t st);
hipError_t launch_w8a8(const MvArgs &a, int mode, bool norm, bool embed, int rows_per_wave,
                       hipStream_t st);
hipError_t launch_argmax(const ArgmaxArgs &a, bool norm, int blocks, hipStream_t st);

// ---- attention / norms / rope ---------------------------------------------
struct AttnDecodeArgs {
    const float *qkv;         // raw projections: q [Hq*D] | k [Hkv*D] | v [Hkv*D]
    const float *q_norm, *k_norm;   // per-head RMSNorm gains [D] (nullable: skip norm+rope)
    const float *rope_cos, *rope_sin;   // [max_pos][D]
    const int *state;         // decode state (pos = state[1]); nullable -> use pos
    int pos;
    void *kcache, *vcache;    // layer base, layout [Hkv][max_seq][D]
    int64_t head_stride;      // max_seq * D (elements)
    float *part;              // [Hkv][n_split][G][D + 2]
    unsigned *counters;       // [Hkv], zero-initialised; the merging block resets its counter
    float *out;               // [Hq * D]
    int n_split;
    float eps, scale;
};

hipError_t launch_attn_decode(const AttnDecodeArgs &a, int n_heads, int n_kv_heads, int head_dim,
                              int kv_bf16, hipStream_t st);

hipError_t launch_rms_norm_rows(float *out, const float *x, const float *w, int64_t seq, int hidden,
                                float eps, hipStream_t st);
hipError_t launch_head_norm_rope(float *x, const float *w, const float *cos_t, const float *sin_t,
                                 int64_t seq, int heads, int hd, float eps, int do_norm,
                                 int do_rope, hipStream_t st);

}  // namespace qasr
