// int8 kernels of the decode hot path: weight packer, activation quantizer,
// W8A8 matvec family (plain / residual-add / SwiGLU / bias) and the LM-head
// argmax.  Integer accumulation is exact, so every output here is bit-identical
// to the reference's NEON SDOT path for the same f32 input vector.
#include "kernels.h"
#include "mv_wave.h"

namespace qasr {

// ---------------------------------------------------------------------------
// Weight packer: quantize_bf16_weights_to_int8 (kernels/mod.rs:1805-1829,
// generic/x86 rounding) or neon::quantize_bf16_to_int8 (kernels/neon.rs:637-694,
// truncation on the 8-wide body, rounding on the tail).  One wave per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_pack_int8_rows(const uint16_t *__restrict__ w, int64_t n,
                                                        int K, int mode, int8_t *__restrict__ q,
                                                        float *__restrict__ scales) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    const uint16_t *src = w + row * K;
    float m = 0.0f;
    for (int k = lane; k < K; k += 64) m = fmaxf(m, fabsf(bf16_to_f32(src[k])));
    m = wave_max_f32(m);
    const float scale = m > 0.0f ? __fdiv_rn(m, 127.0f) : 1.0f;
    const float inv = __fdiv_rn(127.0f, fmaxf(m, 1e-10f));
    if (lane == 0) scales[row] = scale;
    const int vec_end = mode == QASR_TRUNC ? K - (K % 8) : 0;
    int8_t *dst = q + row * K;
    for (int k = lane; k < K; k += 64) {
        const float v = __fmul_rn(bf16_to_f32(src[k]), inv);
        int r;
        if (k < vec_end) {
            // vcvtq_s32_f32 (truncate, saturating) then saturating narrows to int8
            r = (int)truncf(v);
            r = r > 127 ? 127 : (r < -128 ? -128 : r);
        } else {
            r = round_clamp_i8(v);
        }
        dst[k] = (int8_t)r;
    }
}

template <int NS, int R, int MODE, bool NORM, bool EMBED>
__global__ __launch_bounds__(256) void k_w8a8(MvArgs a) {
    __shared__ float lds[NORM ? 4 * QASR_NORM_LDS(NS) : 1];
    __shared__ __attribute__((aligned(16))) int qlds[NS * 256];
    unsigned long long *stamp = nullptr;
#ifdef QASR_STAMPS
    if (a.stamps) stamp = a.stamps + ((int64_t)a.layer * QASR_STAMP_BLOCKS + blockIdx.x) * QASR_STAMP_SLOTS;
    if ((threadIdx.x >> 6) == 0) QASR_STAMP(stamp, 0);
#endif
    w8a8_wave<NS, R, MODE, NORM, EMBED>(a, blockIdx.x, lds, qlds, nullptr, 0, stamp);
}

// ---------------------------------------------------------------------------
// o_proj of the decode step with the split-attention merge in front
// (causal_attention's result, mod.rs:1527-1535, then linear_nobias_int8_addto,
// decoder.rs:616-617).  The attention kernel leaves S partials per query head
// h = 2 kvh + g: max m and sum l at part[(2h + {0,1}) S + s], and o[128] at
// part[32 S + (128 h + d) S + s] (split index fastest).  Every block merges
// all 16 heads: thread (g, d) loads its 8 heads' S partials as vectors,
// threads t < 16 S turn (m, l) into log-sum-exp weights with 8-lane DPP
// reductions; each thread merges its 8 values in registers, the block takes
// their absmax, and each thread writes its 8 int8 values of the quantized row
// (the activation of the W8A8 += matvec) into LDS, which every wave reads back
// as its 16-byte slots.  All loads (partials, weights, epilogue operands) are
// issued before the first wait.
// ---------------------------------------------------------------------------
template <int S>
__device__ __forceinline__ void ld_split(const float *p, float (&v)[S]) {
    if constexpr (S >= 8) {
#pragma unroll
        for (int i = 0; i < S / 4; i++) {
            const float4 a = reinterpret_cast<const float4 *>(p)[i];
            v[4 * i] = a.x; v[4 * i + 1] = a.y; v[4 * i + 2] = a.z; v[4 * i + 3] = a.w;
        }
    } else if constexpr (S == 8) {
        const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else if constexpr (S == 4) {
        const float4 a = reinterpret_cast<const float4 *>(p)[0];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    } else if constexpr (S == 2) {
        const float2 a = reinterpret_cast<const float2 *>(p)[0];
        v[0] = a.x; v[1] = a.y;
    } else {
        v[0] = p[0];
    }
}
// max / sum over aligned groups of S lanes (S = 1, 2, 4, 8, 16; row_mirror
// pairs the two 8-lane halves of a 16-lane row)
template <int S>
__device__ __forceinline__ float split_max(float v) {
    if (S >= 2) v = fmaxf(v, dpp_f32<QASR_DPP_QP_1032>(v));
    if (S >= 4) v = fmaxf(v, dpp_f32<QASR_DPP_QP_2301>(v));
    if (S >= 8) v = fmaxf(v, dpp_f32<QASR_DPP_ROW_HALF_MIRROR>(v));
    if (S >= 16) v = fmaxf(v, dpp_f32<QASR_DPP_ROW_MIRROR>(v));
    return v;
}
template <int S>
__device__ __forceinline__ float split_sum(float v) {
    if (S >= 2) v = __fadd_rn(v, dpp_f32<QASR_DPP_QP_1032>(v));
    if (S >= 4) v = __fadd_rn(v, dpp_f32<QASR_DPP_QP_2301>(v));
    if (S >= 8) v = __fadd_rn(v, dpp_f32<QASR_DPP_ROW_HALF_MIRROR>(v));
    if (S >= 16) v = __fadd_rn(v, dpp_f32<QASR_DPP_ROW_MIRROR>(v));
    return v;
}

template <int S, int R>
__global__ __launch_bounds__(256) void k_oproj_merge(OprojMergeArgs a) {
    constexpr int D = 128, NS = 2, HQ = 16, K = HQ * D;
    __shared__ __attribute__((aligned(16))) int8_t qb[K];
    __shared__ float fw[HQ][S], lsum[HQ], wmax[4];
    const int t = threadIdx.x, lane = t & 63;
    const int wid = __builtin_amdgcn_readfirstlane(t >> 6);
    const int g = t >> 7, d = t & 127;
    unsigned long long *stamp = nullptr;
#ifdef QASR_STAMPS
    if (a.stamps) stamp = a.stamps + ((int64_t)a.layer * QASR_STAMP_BLOCKS + blockIdx.x) * QASR_STAMP_SLOTS;
#endif
    if (wid == 0) QASR_STAMP(stamp, 0);
    // (1) (m, l) of entry e = (head, split) = (e / S, e % S), first, so that
    // the merge weights form while the o partials are still arriving (loads
    // complete in issue order); threads past 16 S reload entry t % (16 S).
    // Then this thread's o partials: heads h = 2 j + g, dim d, all splits
    const int e = t % (HQ * S), eh = e / S, es = e % S;
    const float pm = a.part[(2 * eh) * S + es], pl = a.part[(2 * eh + 1) * S + es];
    const float *po = a.part + 2 * HQ * S;
    float ov[HQ / 2][S];
#pragma unroll
    for (int j = 0; j < HQ / 2; j++) ld_split<S>(po + ((2 * j + g) * D + d) * S, ov[j]);
    // (2) weights and epilogue operands of this wave's rows (rows past N read row 0 and are not stored)
    const int row0 = (blockIdx.x * 4 + wid) * R;
    const bool live = row0 < a.N;
    const int r0 = live ? row0 : 0;
    i32x4 wv[R][NS];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int c = 0; c < NS; c++)
            wv[r][c] = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(a.w + (int64_t)(r0 + r) * K) +
                                                  lane + 64 * c);
    // each lane's epilogue serves the row the reduce-scatter leaves in it
    const int item = scatter_item<R>();
    const float ws0 = __builtin_nontemporal_load(a.ws + r0 + item);
    const float yb = __builtin_nontemporal_load(a.y + r0 + item);
    __builtin_amdgcn_sched_barrier(0);
    if (wid == 0) QASR_STAMP(stamp, 1);
    // (3) log-sum-exp weights per (head, split)
    {
        const float M = split_max<S>(pm);
        const float f = pm == -INFINITY ? 0.0f : expf(__fsub_rn(pm, M));
        const float lt = split_sum<S>(__fmul_rn(pl, f));
        if (t < HQ * S) {
            fw[eh][es] = f;
            if (es == 0) lsum[eh] = lt;
        }
    }
    __syncthreads();
    if (wid == 0) QASR_STAMP(stamp, 2);
    // (4) merged attention output of heads 2 j + g, dim d, kept in registers;
    // the block's absmax over all of them
    float mv[HQ / 2], mx = 0.0f;
#pragma unroll
    for (int j = 0; j < HQ / 2; j++) {
        const int h = 2 * j + g;
        float ot = 0.0f;
#pragma unroll
        for (int s = 0; s < S; s++) ot = fmaf(ov[j][s], fw[h][s], ot);
        const float lt = lsum[h];
        mv[j] = lt > 0.0f ? __fdiv_rn(ot, lt) : 0.0f;
        mx = fmaxf(mx, fabsf(mv[j]));
    }
    mx = wave_max_f32(mx);
    if (lane == 0) wmax[wid] = mx;
    __syncthreads();
    if (wid == 0) QASR_STAMP(stamp, 3);
    // (5) quantize_f32_to_int8 of the merged row: each thread converts its own
    // 8 values with the block's scale into the int8 row in LDS (element e at
    // byte e), then every lane reads its 16-byte slots back
    float xs, inv;
    act_scales(fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3])), &xs, &inv);
#pragma unroll
    for (int j = 0; j < HQ / 2; j++) qb[(2 * j + g) * D + d] = (int8_t)round_clamp_i8(__fmul_rn(mv[j], inv));
    __syncthreads();
    int xd[NS][4];
#pragma unroll
    for (int c = 0; c < NS; c++) {
        const int4 q4 = reinterpret_cast<const int4 *>(qb)[lane + 64 * c];
        xd[c][0] = q4.x; xd[c][1] = q4.y; xd[c][2] = q4.z; xd[c][3] = q4.w;
    }
    if (wid == 0) QASR_STAMP(stamp, 4);
    // (6) dots, one reduce-scatter of the R row sums and the residual-add
    // epilogue (branch-free: lanes holding the same row store the same value)
    int part[R][1];
#pragma unroll
    for (int r = 0; r < R; r++) {
        int q = 0;
#pragma unroll
        for (int c = 0; c < NS; c++) q = dot16(wv[r][c], xd[c], q);
        part[r][0] = q;
    }
    int av[1];
    scatter_items<R, 1>(part, av);
    if (wid == 0) QASR_STAMP(stamp, 5);
    const float v = __fadd_rn(__fmul_rn(__fmul_rn((float)av[0], xs), ws0), yb);
    if (live) a.y[r0 + item] = v;
    if (wid == 0) QASR_STAMP(stamp, 6);
}

template <int R>
static hipError_t go_oproj_merge(const OprojMergeArgs &a, hipStream_t st) {
    const unsigned blocks = (unsigned)((a.N / R + 3) / 4);
    switch (a.n_split) {
        case 1: hipLaunchKernelGGL((k_oproj_merge<1, R>), dim3(blocks), dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL((k_oproj_merge<2, R>), dim3(blocks), dim3(256), 0, st, a); break;
        case 4: hipLaunchKernelGGL((k_oproj_merge<4, R>), dim3(blocks), dim3(256), 0, st, a); break;
        case 8: hipLaunchKernelGGL((k_oproj_merge<8, R>), dim3(blocks), dim3(256), 0, st, a); break;
        case 16: hipLaunchKernelGGL((k_oproj_merge<16, R>), dim3(blocks), dim3(256), 0, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_oproj_merge(const OprojMergeArgs &a, int rows_per_wave, hipStream_t st) {
    if (a.Hkv != 8 || a.N % rows_per_wave != 0) return hipErrorInvalidValue;
    switch (rows_per_wave) {
        case 1: return go_oproj_merge<1>(a, st);
        case 2: return go_oproj_merge<2>(a, st);
        case 4: return go_oproj_merge<4>(a, st);
        default: return hipErrorInvalidValue;
    }
}

// ---------------------------------------------------------------------------
// LM-head argmax: argmax_matvec_int8 (kernels/mod.rs:1832-1893).  Optional
// final RMSNorm prologue; grid-stride over row groups; strict > per wave
// (rows visited in increasing order), then block and grid merges with the
// rule "larger value wins, lower index on ties" — the reference's result for
// any thread split.  The last block to finish merges the per-block partials
// and, in decode-loop mode, advances the device-side step state.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i >= 0 && (bi < 0 || i < bi));
}

template <int NS, int R, bool NORM>
__global__ __launch_bounds__(256) void k_argmax_w8a8(ArgmaxArgs a) {
    __shared__ float lds[NORM ? 4 * QASR_NORM_LDS(NS) : 1];
    __shared__ __attribute__((aligned(16))) int qlds[NS * 256];
    __shared__ float bvals[4];
    __shared__ int bidx[4];
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = a.K, nslot = K >> 4;
    const int n_groups = (a.N + R - 1) / R;
    const int gw = blockIdx.x * 4 + wid, n_waves = gridDim.x * 4;
    int xd[NS][4];
    float xs;
    float best_v = -1e30f;
    int best_i = -1;
    // Two groups in flight per wave: buffer A holds groups gw, gw + 2n, ...,
    // buffer B groups gw + n, gw + 3n, ... (n = waves in the grid).  Rows past
    // N load row 0 (discarded by the row < N test); slots past K load slot 0
    // (their activation bytes are zero).
    i32x4 wa[R][NS], wb[R][NS];
    float sa[R], sb[R];
    auto load_group = [&](i32x4 (&wv)[R][NS], float (&sc)[R], int grp) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = grp * R + r < a.N ? grp * R + r : 0;
#pragma unroll
            for (int c = 0; c < NS; c++) {
                const int s = lane + 64 * c;
                wv[r][c] = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(a.w + (int64_t)row * K) +
                                                      (s < nslot ? s : 0));
            }
            sc[r] = a.ws[row];
        }
    };
    // rows visited in increasing order per wave, strict > (first index wins)
    auto consume = [&](const i32x4 (&wv)[R][NS], const float (&sc)[R], int grp) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            int t = 0;
#pragma unroll
            for (int c = 0; c < NS; c++) t = dot16(wv[r][c], xd[c], t);
            const int sum = wave_sum_i32(t);
            const int row = grp * R + r;
            if (row < a.N) {
                const float v = __fadd_rn(__fmul_rn(__fmul_rn((float)sum, xs), sc[r]), 0.0f);
                if (v > best_v) { best_v = v; best_i = row; }
            }
        }
    };
    ActIn<NS, NORM, false> in;
    act_load<NS, NORM, false>(a.x, nullptr, a.norm_w, K, in);
    if (gw < n_groups) load_group(wa, sa, gw);
    if (gw + n_waves < n_groups) load_group(wb, sb, gw + n_waves);
    __builtin_amdgcn_sched_barrier(0);
    act_convert<NS, NORM, false>(in, K, nullptr);
    act_finish_block<NS, NORM, false>(in, a.eps, K, lds + wid * QASR_NORM_LDS(NS), qlds, xd, &xs);
    for (int g = gw; g < n_groups; g += 2 * n_waves) {
        consume(wa, sa, g);
        if (g + 2 * n_waves < n_groups) load_group(wa, sa, g + 2 * n_waves);
        if (g + n_waves < n_groups) {
            consume(wb, sb, g + n_waves);
            if (g + 3 * n_waves < n_groups) load_group(wb, sb, g + 3 * n_waves);
        }
    }
    if (lane == 0) { bvals[wid] = best_v; bidx[wid] = best_i; }
    __syncthreads();
    if (threadIdx.x == 0) {
        float bv = bvals[0];
        int bi = bidx[0];
        for (int w = 1; w < 4; w++)
            if (better(bvals[w], bidx[w], bv, bi)) { bv = bvals[w]; bi = bidx[w]; }
        a.part_val[blockIdx.x] = bv;   // published by the kernel boundary
        a.part_idx[blockIdx.x] = bi;
    }
}

// ---------------------------------------------------------------------------
// Second pass of the LM-head argmax: one block merges the per-block
// (value, index) partials with the same rule (larger value, lower index on
// ties) and, in decode-loop mode, advances the device-side step state: the
// token, the position, the token log and the next position's RoPE rows for the
// next step's attention kernels.  A separate launch costs less than merging in
// the streaming kernel: its last-block hand-off (an agent-scope counter bumped
// by every block) measured 6-12 us at 512-1024 blocks.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_argmax_finish(ArgmaxArgs a, int n_parts) {
    __shared__ float bvals[4];
    __shared__ int bidx[4];
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    // the next position's RoPE rows do not depend on the token: thread t < 128
    // copies cos[t], t >= 128 sin[t - 128], issued alongside the partial loads
    // (every thread reads the position before the barrier below; lane 0 of
    // wave 0 advances it after)
    const int next_pos = a.state ? a.state[1] + 1 : 0;
    if (a.state && a.rope_cur && next_pos < a.max_pos) {
        const int i = threadIdx.x & 127;
        const float *tab = threadIdx.x < 128 ? a.rope_cos : a.rope_sin;
        a.rope_cur[threadIdx.x] = tab[(int64_t)next_pos * 128 + i];
    }
    float bv = -1e30f;
    int bi = -1;
    for (int b = threadIdx.x; b < n_parts; b += 256) {
        const float v = a.part_val[b];
        const int i = a.part_idx[b];
        if (better(v, i, bv, bi)) { bv = v; bi = i; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) { bvals[wid] = bv; bidx[wid] = bi; }
    __syncthreads();
    if (wid != 0) return;
    bv = bvals[0];
    bi = bidx[0];
    for (int w = 1; w < 4; w++)
        if (better(bvals[w], bidx[w], bv, bi)) { bv = bvals[w]; bi = bidx[w]; }
    if (lane == 0) {
        const int tok = bi < 0 ? 0 : bi;
        a.out_idx[0] = tok;
        if (a.out_val) a.out_val[0] = bv;
        if (a.state) {
            a.state[0] = tok;
            a.state[1] = next_pos;
            if (a.token_log) a.token_log[a.state[2]] = tok;
            a.state[2] += 1;
        }
        if (a.epoch) a.epoch[0] += 1;
    }
}

// ---------------------------------------------------------------------------
// standalone activation quantizer (quantize_f32_to_int8), one block
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_quant_act(const float *__restrict__ x, int K,
                                                   int8_t *__restrict__ q, float *__restrict__ xs) {
    __shared__ float red[4];
    float m = 0.0f;
    for (int k = threadIdx.x; k < K; k += 256) m = fmaxf(m, fabsf(x[k]));
    m = wave_max_f32(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float scale, inv;
    act_scales(m, &scale, &inv);
    if (threadIdx.x == 0) *xs = scale;
    for (int k = threadIdx.x; k < K; k += 256) q[k] = (int8_t)round_clamp_i8(__fmul_rn(x[k], inv));
}

// ---------------------------------------------------------------------------
// device-to-device copy (16-byte vectors when both pointers and the size allow)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_copy16(int4 *__restrict__ dst, const int4 *__restrict__ src, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) dst[i] = src[i];
}
__global__ __launch_bounds__(256) void k_copy1(uint8_t *__restrict__ dst, const uint8_t *__restrict__ src, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) dst[i] = src[i];
}
hipError_t launch_copy(void *dst, const void *src, int64_t bytes, hipStream_t st) {
    if (bytes <= 0) return hipSuccess;
    const bool v16 = ((uintptr_t)dst % 16 == 0) && ((uintptr_t)src % 16 == 0) && (bytes % 16 == 0);
    const int64_t n = v16 ? bytes / 16 : bytes;
    const unsigned blocks = (unsigned)std::min<int64_t>((n + 255) / 256, 4096);
    if (v16) hipLaunchKernelGGL(k_copy16, dim3(blocks), dim3(256), 0, st, (int4 *)dst, (const int4 *)src, n);
    else hipLaunchKernelGGL(k_copy1, dim3(blocks), dim3(256), 0, st, (uint8_t *)dst, (const uint8_t *)src, n);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
hipError_t launch_pack_int8(const uint16_t *w, int64_t n, int K, int mode, int8_t *q, float *s,
                            hipStream_t st) {
    const unsigned blocks = (unsigned)((n + 3) / 4);
    hipLaunchKernelGGL(k_pack_int8_rows, dim3(blocks), dim3(256), 0, st, w, n, K, mode, q, s);
    return hipGetLastError();
}

hipError_t launch_quant_act(const float *x, int K, int8_t *q, float *xs, hipStream_t st) {
    hipLaunchKernelGGL(k_quant_act, dim3(1), dim3(256), 0, st, x, K, q, xs);
    return hipGetLastError();
}

template <int NS, int R, int MODE, bool NORM, bool EMBED>
static hipError_t go_mv(const MvArgs &a, hipStream_t st) {
    const int waves = (a.n_total + R - 1) / R;
    const unsigned blocks = (unsigned)((waves + 3) / 4);
    hipLaunchKernelGGL((k_w8a8<NS, R, MODE, NORM, EMBED>), dim3(blocks), dim3(256), 0, st, a);
    return hipGetLastError();
}

// dispatch on slots-per-lane (ceil(K / 1024))
template <int R, int MODE, bool NORM, bool EMBED>
static hipError_t go_mv_ns(const MvArgs &a, hipStream_t st) {
    const int ns = (a.K + 1023) / 1024;
    switch (ns) {
        case 1: return go_mv<1, R, MODE, NORM, EMBED>(a, st);
        case 2: return go_mv<2, R, MODE, NORM, EMBED>(a, st);
        case 3: return go_mv<3, R, MODE, NORM, EMBED>(a, st);
        case 4: return go_mv<4, R, MODE, NORM, EMBED>(a, st);
        case 6: if (!NORM) return go_mv<6, R, MODE, false, EMBED>(a, st); break;
        default: break;
    }
    return hipErrorInvalidValue;
}

hipError_t launch_w8a8(const MvArgs &a, int mode, bool norm, bool embed, int rows_per_wave,
                       hipStream_t st) {
    if (a.K % 64 != 0 || a.K > 6144) return hipErrorInvalidValue;
    if (norm && a.K > 4096) return hipErrorInvalidValue;
#define QASR_MV(R)                                                                     \
    switch (mode) {                                                                     \
        case MV_PLAIN:                                                                  \
            if (embed) return go_mv_ns<R, MV_PLAIN, true, true>(a, st);                 \
            return norm ? go_mv_ns<R, MV_PLAIN, true, false>(a, st)                     \
                        : go_mv_ns<R, MV_PLAIN, false, false>(a, st);                   \
        case MV_ADDTO: return norm ? hipErrorInvalidValue : go_mv_ns<R, MV_ADDTO, false, false>(a, st); \
        case MV_SWIGLU:                                                                 \
            return norm ? go_mv_ns<R, MV_SWIGLU, true, false>(a, st)                    \
                        : go_mv_ns<R, MV_SWIGLU, false, false>(a, st);                  \
        case MV_BIAS: return norm ? hipErrorInvalidValue : go_mv_ns<R, MV_BIAS, false, false>(a, st); \
        default: return hipErrorInvalidValue;                                           \
    }
    if (rows_per_wave == 1 && mode != MV_SWIGLU) { QASR_MV(1) }
    if (rows_per_wave == 2) { QASR_MV(2) }
    if (rows_per_wave == 4) { QASR_MV(4) }
    if (rows_per_wave == 8) { QASR_MV(8) }
#undef QASR_MV
    return hipErrorInvalidValue;
}

hipError_t launch_argmax(const ArgmaxArgs &a, bool norm, int blocks, hipStream_t st, bool stream, bool finish) {
    if (a.K % 64 != 0 || a.K > 4096) return hipErrorInvalidValue;
    const int ns = (a.K + 1023) / 1024;
    if (ns < 1 || ns > 4) return hipErrorInvalidValue;
#define QASR_AM(NS)                                                                           \
    if (ns == NS) {                                                                           \
        if (norm) hipLaunchKernelGGL((k_argmax_w8a8<NS, 4, true>), dim3(blocks), dim3(256), 0, st, a); \
        else hipLaunchKernelGGL((k_argmax_w8a8<NS, 4, false>), dim3(blocks), dim3(256), 0, st, a);     \
    }
    if (stream) { QASR_AM(1) QASR_AM(2) QASR_AM(3) QASR_AM(4) }
    if (finish) hipLaunchKernelGGL(k_argmax_finish, dim3(1), dim3(256), 0, st, a, blocks);
    return hipGetLastError();
#undef QASR_AM
}


// ===========================================================================
// Multi-stream decode: B <= 32 independent streams step
// together.  Every per-row operation is the single-stream one (the same
// prologue helpers, the same epilogue operation order), and the W8A8 dots run
// on int8 MFMA (v_mfma_i32_16x16x64_i8) with exact int32 accumulation, so each
// stream's output is bit-identical to its own M = 1 step.
// ===========================================================================

// layer-0 input: x[b] = f32(embedding row of stream b's token)
__global__ __launch_bounds__(256) void k_embed_rows(float *__restrict__ x, const uint16_t *__restrict__ embed,
                                                    const int *__restrict__ state, int H) {
    const int b = blockIdx.x;
    const int tok = state[4 * b];
    for (int i = threadIdx.x; i < H; i += 256) x[(int64_t)b * H + i] = bf16_to_f32(embed[(int64_t)tok * H + i]);
}

hipError_t launch_embed_rows(float *x, const uint16_t *embed, const int *state, int B, int H, hipStream_t st) {
    hipLaunchKernelGGL(k_embed_rows, dim3(B), dim3(256), 0, st, x, embed, state, H);
    return hipGetLastError();
}

// per-row activation prologue: optional RMSNorm (AVX order) + absmax int8
// quantization of x[b][K] -> xq[b][K], xs[b]; one wave per row
template <int NS, bool NORM>
__global__ __launch_bounds__(256) void k_quant_rows(const float *__restrict__ x, const float *__restrict__ norm_w,
                                                    float eps, int K, int B, int8_t *__restrict__ xq,
                                                    float *__restrict__ xs) {
    __shared__ float lds[NORM ? 4 * QASR_NORM_LDS(NS) : 1];
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int b = blockIdx.x * 4 + wid;
    if (b >= B) return;
    ActIn<NS, NORM, false> in;
    act_load<NS, NORM, false>(x + (int64_t)b * K, nullptr, norm_w, K, in);
    act_convert<NS, NORM, false>(in, K, nullptr);
    int xd[NS][4];
    float s;
    act_finish<NS, NORM, false>(in, eps, K, lds + wid * QASR_NORM_LDS(NS), xd, &s);
    const int nslot = K >> 4;
#pragma unroll
    for (int c = 0; c < NS; c++) {
        const int sl = lane + 64 * c;
        if (sl < nslot)
            reinterpret_cast<int4 *>(xq + (int64_t)b * K)[sl] = make_int4(xd[c][0], xd[c][1], xd[c][2], xd[c][3]);
    }
    if (lane == 0) xs[b] = s;
}

hipError_t launch_quant_rows(const float *x, const float *norm_w, float eps, int K, int B, int8_t *xq, float *xs,
                             hipStream_t st) {
    if (K % 64 != 0 || K > 6144 || B <= 0) return hipErrorInvalidValue;
    if (norm_w && K > 4096) return hipErrorInvalidValue;
    const unsigned blocks = (unsigned)((B + 3) / 4);
    const int ns = (K + 1023) / 1024;
#define QR(NS)                                                                                                  \
    if (ns == NS) {                                                                                             \
        if (norm_w) hipLaunchKernelGGL((k_quant_rows<NS, true>), dim3(blocks), dim3(256), 0, st, x, norm_w, eps, K, B, xq, xs); \
        else hipLaunchKernelGGL((k_quant_rows<NS, false>), dim3(blocks), dim3(256), 0, st, x, norm_w, eps, K, B, xq, xs);      \
        return hipGetLastError();                                                                               \
    }
    QR(1) QR(2) QR(3) QR(4)
    if (ns == 6 && !norm_w) {
        hipLaunchKernelGGL((k_quant_rows<6, false>), dim3(blocks), dim3(256), 0, st, x, norm_w, eps, K, B, xq, xs);
        return hipGetLastError();
    }
#undef QR
    return hipErrorInvalidValue;
}

// C[b][n] for 16 weight rows n x 32 stream columns b per wave: two
// v_mfma_i32_16x16x64_i8 tiles per 64-wide K step.  Lane l supplies 16
// consecutive K bytes of weight row n0 + l % 16 and of activation rows
// l % 16 and 16 + l % 16 at K offset 16 (l / 16) (the same lane -> k map on
// both operands, so the exact int32 sums do not depend on the hardware's k
// order); it receives C[n0 + 4 (l / 16) + j][l % 16 (+16)], j < 4.
__device__ __forceinline__ void mfma_rows16(const int8_t *__restrict__ wrow, const int8_t *__restrict__ xa,
                                            const int8_t *__restrict__ xb, int K, i32x4 &c0, i32x4 &c1) {
    constexpr int CH = 16;                       // K steps per chunk (1024 bytes of a row)
    for (int k0 = 0; k0 < K; k0 += 64 * CH) {
        const int steps = min(CH, (K - k0) / 64);
        i32x4 wa[CH], xa_[CH], xb_[CH];
#pragma unroll
        for (int s = 0; s < CH; s++) {
            if (s < steps) {
                wa[s] = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(wrow + k0 + 64 * s));
                xa_[s] = *reinterpret_cast<const i32x4 *>(xa + k0 + 64 * s);
                xb_[s] = *reinterpret_cast<const i32x4 *>(xb + k0 + 64 * s);
            }
        }
#pragma unroll
        for (int s = 0; s < CH; s++) {
            if (s < steps) {
                c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa[s], xa_[s], c0, 0, 0, 0);
                c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa[s], xb_[s], c1, 0, 0, 0);
            }
        }
    }
}

// Batched W8A8 projection: out = epilogue((sum_k xq[b][k] w[n][k]) * xs[b] * ws[n])
// with the single-stream epilogues (MV_PLAIN / MV_ADDTO / MV_SWIGLU).  xq has
// 32 rows; rows >= B hold stale bytes, and since each output column depends
// only on its own activation row, their columns are computed and dropped.
//
// One block per 16-row tile, 16 waves splitting K (ST steps of 64 each, every
// load issued up front: the weight tile streams in one round trip); the 16
// int32 partial tiles are summed through LDS (exact, so the order is free) and
// the block applies the epilogue, threads over (stream, row) so that stores
// are row-contiguous.  (Measured and rejected for the 64-tile shapes, o_proj
// and down at 0.6B: K split over 2-3 blocks per tile, each publishing its
// int32 tile and the last to arrive (arrive_last) adding them, 5.3 -> 14.9
// and 7.0 -> 16.6 us per launch: the agent-scope release before the counter
// bump costs more than the CUs the 64 blocks leave idle.)
template <int MODE, int ST>
__global__ __launch_bounds__(1024) void k_w8a8_batch(BatchMvArgs a) {
    constexpr int W = 16;
    __shared__ int red[W][512];
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * 16;
    const int K = a.K, r = lane & 15, kg = lane >> 4;
    const int kb = wid * ST * 64 + 16 * kg;
    const int8_t *wr = a.w + (int64_t)(n0 + r) * K + kb;
    const int8_t *xa = a.xq + (int64_t)r * K + kb, *xb = a.xq + (int64_t)(16 + r) * K + kb;
    i32x4 wv[ST], av[ST], bv[ST];
#pragma unroll
    for (int s = 0; s < ST; s++) {
        wv[s] = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(wr + 64 * s));
        av[s] = *reinterpret_cast<const i32x4 *>(xa + 64 * s);
        bv[s] = *reinterpret_cast<const i32x4 *>(xb + 64 * s);
    }
    // epilogue operands of this thread's output(s), requested with the tile
    // (threads past B read stream 0's and do not store)
    const int t = threadIdx.x;
    const int eb = MODE == MV_SWIGLU ? (t >> 3) & 31 : (t >> 4) & 31;
    const int er = MODE == MV_SWIGLU ? 2 * (t & 7) : t & 15;
    const int ebs = eb < a.B ? eb : 0;
    const float e_xs = __builtin_nontemporal_load(a.xs + ebs);
    const float e_w0 = __builtin_nontemporal_load(a.ws + n0 + er);
    const float e_w1 = MODE == MV_SWIGLU ? __builtin_nontemporal_load(a.ws + n0 + er + 1) : 0.0f;
    const float e_y = MODE == MV_ADDTO ? __builtin_nontemporal_load(a.y + (int64_t)ebs * a.ldy + n0 + er) : 0.0f;
    __builtin_amdgcn_sched_barrier(0);
    i32x4 c0 = {0, 0, 0, 0}, c1 = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < ST; s++) {
        c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(wv[s], av[s], c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(wv[s], bv[s], c1, 0, 0, 0);
    }
    // lane holds C[row 4 kg + j][stream r] (c0) and [stream 16 + r] (c1); LDS index stream * 16 + row
#pragma unroll
    for (int j = 0; j < 4; j++) {
        red[wid][r * 16 + 4 * kg + j] = c0[j];
        red[wid][(16 + r) * 16 + 4 * kg + j] = c1[j];
    }
    __syncthreads();
    if (MODE == MV_SWIGLU) {
        // 8 outputs per stream: rows (2 p, 2 p + 1) = (gate, up) of output n0 / 2 + p
        if (t < 256) {
            const int b = t >> 3, p = t & 7;
            int g = 0, u = 0;
#pragma unroll
            for (int w = 0; w < W; w++) {
                g += red[w][b * 16 + 2 * p];
                u += red[w][b * 16 + 2 * p + 1];
            }
            if (b < a.B) {
                const float gf = __fmul_rn(__fmul_rn((float)g, e_xs), e_w0);
                const float uf = __fmul_rn(__fmul_rn((float)u, e_xs), e_w1);
                a.y[(int64_t)b * a.ldy + n0 / 2 + p] = __fmul_rn(__fdiv_rn(gf, __fadd_rn(1.0f, expf(-gf))), uf);
            }
        }
    } else if (t < 512) {
        const int b = t >> 4, rr = t & 15;
        int acc = 0;
#pragma unroll
        for (int w = 0; w < W; w++) acc += red[w][t];
        if (b < a.B) {
            float v = __fmul_rn(__fmul_rn((float)acc, e_xs), e_w0);
            if (MODE == MV_ADDTO) v = __fadd_rn(v, e_y);
            a.y[(int64_t)b * a.ldy + n0 + rr] = v;
        }
    }
}

hipError_t launch_w8a8_batch(const BatchMvArgs &a, int mode, hipStream_t st) {
    // K = 16 waves x ST steps x 64
    if (a.K % 1024 != 0 || a.N % 16 != 0 || a.B <= 0 || a.B > 32) return hipErrorInvalidValue;
    const int st_ = a.K / 1024;
    const unsigned blocks = (unsigned)(a.N / 16);
#define QB(S)                                                                                              \
    if (st_ == S) {                                                                                        \
        switch (mode) {                                                                                    \
            case MV_PLAIN: hipLaunchKernelGGL((k_w8a8_batch<MV_PLAIN, S>), dim3(blocks), dim3(1024), 0, st, a); break;   \
            case MV_ADDTO: hipLaunchKernelGGL((k_w8a8_batch<MV_ADDTO, S>), dim3(blocks), dim3(1024), 0, st, a); break;   \
            case MV_SWIGLU: hipLaunchKernelGGL((k_w8a8_batch<MV_SWIGLU, S>), dim3(blocks), dim3(1024), 0, st, a); break; \
            default: return hipErrorInvalidValue;                                                          \
        }                                                                                                  \
        return hipGetLastError();                                                                          \
    }
    QB(1) QB(2) QB(3) QB(4) QB(6)
#undef QB
    return hipErrorInvalidValue;
}

// Batched LM-head argmax: per stream the larger value wins, lower index on
// ties (argmax_matvec_int8, kernels/mod.rs:1832-1893).  A block of 16 waves
// stages the 32 activation rows in LDS once (32 K bytes) and each wave takes
// one 16-row tile per pass (grid-stride), all weight loads of a tile issued up
// front; the MFMA's activation operands come from LDS.  Each lane keeps the
// best of its rows for its two stream columns, then the 4 lanes of a column
// and the block's waves merge; block partials go to part_val / part_idx
// [blocks][32].
template <int KC>
__global__ __launch_bounds__(1024) void k_argmax_batch(BatchMvArgs a) {
    extern __shared__ int4 xs_lds[];                 // [32][K / 16]
    __shared__ float sv[16][32];
    __shared__ int si[16][32];
    const int t = threadIdx.x, lane = t & 63;
    const int wid = __builtin_amdgcn_readfirstlane(t >> 6);
    const int K = a.K, r = lane & 15, kg = lane >> 4, kv = K >> 4;
    for (int i = t; i < 32 * kv; i += 1024) xs_lds[i] = reinterpret_cast<const int4 *>(a.xq)[i];
    __syncthreads();
    const int n_tiles = a.N / 16;
    float bv[2] = {-1e30f, -1e30f};
    int bi[2] = {-1, -1};
    float xsv[2];
    xsv[0] = a.xs[r < a.B ? r : 0];
    xsv[1] = a.xs[16 + r < a.B ? 16 + r : 0];
    for (int tile = blockIdx.x * 16 + wid; tile < n_tiles; tile += gridDim.x * 16) {
        const int n0 = tile * 16;
        const int8_t *wr = a.w + (int64_t)(n0 + r) * K + 16 * kg;
        i32x4 c0 = {0, 0, 0, 0}, c1 = {0, 0, 0, 0};
        for (int k0 = 0; k0 < K; k0 += 64 * KC) {
            i32x4 wv[KC];
#pragma unroll
            for (int s = 0; s < KC; s++) wv[s] = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(wr + k0 + 64 * s));
            __builtin_amdgcn_sched_barrier(0);       // every weight load of the tile before the first MFMA
#pragma unroll
            for (int s = 0; s < KC; s++) {
                const int kq = (k0 + 64 * s) / 16 + kg;
                const int4 xa = xs_lds[r * kv + kq], xb = xs_lds[(16 + r) * kv + kq];
                const i32x4 av = {xa.x, xa.y, xa.z, xa.w}, bvv = {xb.x, xb.y, xb.z, xb.w};
                c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(wv[s], av, c0, 0, 0, 0);
                c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(wv[s], bvv, c1, 0, 0, 0);
            }
        }
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
            const i32x4 c = tt ? c1 : c0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int n = n0 + 4 * kg + j;
                const float v = __fadd_rn(__fmul_rn(__fmul_rn((float)c[j], xsv[tt]), a.ws[n]), 0.0f);
                if (better(v, n, bv[tt], bi[tt])) { bv[tt] = v; bi[tt] = n; }
            }
        }
    }
    // the 4 lanes (kg) of a column hold disjoint rows: merge with xor 16, 32
#pragma unroll
    for (int tt = 0; tt < 2; tt++) {
#pragma unroll
        for (int o = 16; o <= 32; o <<= 1) {
            const float ov = __shfl_xor(bv[tt], o, 64);
            const int oi = __shfl_xor(bi[tt], o, 64);
            if (better(ov, oi, bv[tt], bi[tt])) { bv[tt] = ov; bi[tt] = oi; }
        }
        if (kg == 0) { sv[wid][16 * tt + r] = bv[tt]; si[wid][16 * tt + r] = bi[tt]; }
    }
    __syncthreads();
    if (t < 32) {
        float v = sv[0][t];
        int i = si[0][t];
        for (int w = 1; w < 16; w++)
            if (better(sv[w][t], si[w][t], v, i)) { v = sv[w][t]; i = si[w][t]; }
        a.part_val[blockIdx.x * 32 + t] = v;
        a.part_idx[blockIdx.x * 32 + t] = i;
    }
}

// merge of the block partials per stream (one wave per stream) and the
// per-stream step-state update (token, position, token log, the next
// position's RoPE rows and attention partition)
__global__ __launch_bounds__(64) void k_argmax_batch_finish(BatchMvArgs a, int n_parts, int *state, int *token_log,
                                                            int64_t log_stride, const float *rope_cos,
                                                            const float *rope_sin, float *rope_cur, int max_pos,
                                                            const int *gpb_table, int *gpb_dev) {
    const int lane = threadIdx.x, b = blockIdx.x;
    float bv = -1e30f;
    int bi = -1;
    for (int p = lane; p < n_parts; p += 64) {
        const float v = a.part_val[p * 32 + b];
        const int i = a.part_idx[p * 32 + b];
        if (better(v, i, bv, bi)) { bv = v; bi = i; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    int *s = state + 4 * b;
    const int next_pos = s[1] + 1;
    if (next_pos < max_pos)
        for (int i = lane; i < 128; i += 64) {
            rope_cur[b * 256 + i] = rope_cos[(int64_t)next_pos * 128 + i];
            rope_cur[b * 256 + 128 + i] = rope_sin[(int64_t)next_pos * 128 + i];
        }
    if (lane == 0) {
        const int tok = bi < 0 ? 0 : bi;
        s[0] = tok;
        s[1] = next_pos;
        token_log[b * log_stride + s[2]] = tok;
        s[2] += 1;
        if (gpb_table && next_pos < max_pos) gpb_dev[b] = gpb_table[next_pos];
    }
}

hipError_t launch_argmax_batch(const BatchMvArgs &a, int blocks, int *state, int *token_log, int64_t log_stride,
                               const float *rope_cos, const float *rope_sin, float *rope_cur, int max_pos,
                               const int *gpb_table, int *gpb_dev, hipStream_t st, bool stream, bool finish) {
    if (a.K % 1024 != 0 || a.K > 4096 || a.N % 16 != 0 || a.B <= 0 || a.B > 32 || blocks <= 0)
        return hipErrorInvalidValue;
    if (gpb_table && !gpb_dev) return hipErrorInvalidValue;
    if (stream) {
        const size_t lds = (size_t)32 * a.K;
        hipLaunchKernelGGL(k_argmax_batch<16>, dim3(blocks), dim3(1024), lds, st, a);
    }
    if (finish)
        hipLaunchKernelGGL(k_argmax_batch_finish, dim3(a.B), dim3(64), 0, st, a, blocks, state, token_log, log_stride,
                           rope_cos, rope_sin, rope_cur, max_pos, gpb_table, gpb_dev);
    return hipGetLastError();
}

// attention partial merge per stream (the o_proj prologue's merge as its own
// pass), split index slowest, then the o_proj activation quantization of the
// merged row (absmax over the 16 heads x 128 dims, act_finish's scale and
// rounding): xq[b][128 h + d], xs[b]; att (nullable) receives the f32 row
template <int S>
__global__ __launch_bounds__(256) void k_attn_merge_rows(const float *__restrict__ part, int64_t part_stride,
                                                         float *__restrict__ att, int64_t att_stride,
                                                         int8_t *__restrict__ xq, float *__restrict__ xs) {
    constexpr int D = 128, HQ = 16, K = HQ * D;
    __shared__ float fw[HQ][S], lsum[HQ], wmax[4];
    const int b = blockIdx.x, t = threadIdx.x, lane = t & 63;
    const float *pb = part + (int64_t)b * part_stride;
    // o partials split index slowest (part_o_index_slow): items u = t, t + 256
    // are (head u / 32, dims 4 (u % 32) .. + 3), one float4 per split
    float4 ov[2][S];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int it = t + 256 * u, h = it >> 5, c4 = it & 31;
#pragma unroll
        for (int s = 0; s < S; s++)
            ov[u][s] = *reinterpret_cast<const float4 *>(pb + part_o_index_slow(S, s, HQ, h * D + 4 * c4));
    }
    const int e = t % (HQ * S), eh = e / S, es = e % S;
    const float pm = pb[(2 * eh) * S + es], pl = pb[(2 * eh + 1) * S + es];
    {
        const float M = split_max<S>(pm);
        const float f = pm == -INFINITY ? 0.0f : expf(__fsub_rn(pm, M));
        const float lt = split_sum<S>(__fmul_rn(pl, f));
        if (t < HQ * S) {
            fw[eh][es] = f;
            if (es == 0) lsum[eh] = lt;
        }
    }
    __syncthreads();
    float o[2][4], m = 0.0f;
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int it = t + 256 * u, h = it >> 5, c4 = it & 31;
        const float lt = lsum[h];
        float ot[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < S; s++) {
            const float w = fw[h][s];
            ot[0] = fmaf(ov[u][s].x, w, ot[0]);
            ot[1] = fmaf(ov[u][s].y, w, ot[1]);
            ot[2] = fmaf(ov[u][s].z, w, ot[2]);
            ot[3] = fmaf(ov[u][s].w, w, ot[3]);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o[u][i] = lt > 0.0f ? __fdiv_rn(ot[i], lt) : 0.0f;
            m = fmaxf(m, fabsf(o[u][i]));
            if (att) att[(int64_t)b * att_stride + h * D + 4 * c4 + i] = o[u][i];
        }
    }
    m = wave_max_f32(m);
    if (lane == 0) wmax[t >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    float scale, inv;
    act_scales(m, &scale, &inv);
    if (t == 0) xs[b] = scale;
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int it = t + 256 * u, h = it >> 5, c4 = it & 31;
#pragma unroll
        for (int i = 0; i < 4; i++)
            xq[(int64_t)b * K + h * D + 4 * c4 + i] = (int8_t)round_clamp_i8(__fmul_rn(o[u][i], inv));
    }
}

// The merge for the split counts the o_proj prologue does not take (any
// other count <= 64; partials split index slowest).  Per head, one wave with
// one split per lane: the max and sum_s l_s f_s by fixed-order wave
// reductions, f_s = exp(m_s - max) to LDS; then per (head, dim) the o
// partials weighted in split order.  Two kernels share these steps:
// k_attn_merge_seq (one block per stream, all heads, with the o_proj
// activation quantization fused) and k_attn_merge_heads (one block per
// (head, stream), the f32 row only).
__device__ __forceinline__ void merge_head_weights(const float *pb, int S, int h, float *fw, float *lsum) {
    const int sp = threadIdx.x & 63;
    const float m = sp < S ? pb[(2 * h) * S + sp] : -INFINITY;
    const float l = sp < S ? pb[(2 * h + 1) * S + sp] : 0.0f;
    const float M = wave_max_f32(m);
    const float f = m == -INFINITY ? 0.0f : expf(__fsub_rn(m, M));
    fw[sp] = f;
    const float lt = wave_sum_f32(__fmul_rn(l, f));
    if (sp == 0) *lsum = lt;
}
__device__ __forceinline__ float merge_head_dim(const float *pb, int S, int h, int d, const float *fw, float lt) {
    constexpr int D = 128, HQ = 16;
    const float *po = pb + 2 * HQ * S + h * D + d;
    float ot = 0.0f;
    for (int s = 0; s < S; s++) ot = fmaf(po[(int64_t)s * HQ * D], fw[s], ot);
    return lt > 0.0f ? __fdiv_rn(ot, lt) : 0.0f;
}

__global__ __launch_bounds__(1024) void k_attn_merge_seq(const float *__restrict__ part, int64_t part_stride, int S,
                                                        float *__restrict__ att, int64_t att_stride,
                                                        int8_t *__restrict__ xq, float *__restrict__ xs) {
    constexpr int D = 128, HQ = 16, K = HQ * D;
    __shared__ float fw[HQ][64], lsum[HQ], wmax[16];
    const int b = blockIdx.x, t = threadIdx.x, lane = t & 63, wid = t >> 6;
    const float *pb = part + (int64_t)b * part_stride;
    merge_head_weights(pb, S, wid, fw[wid], &lsum[wid]);
    __syncthreads();
    const int hp = t >> 7, d = t & 127;
    float o[2], am = 0.0f;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int h = 2 * hp + j;
        o[j] = merge_head_dim(pb, S, h, d, fw[h], lsum[h]);
        am = fmaxf(am, fabsf(o[j]));
        if (att) att[(int64_t)b * att_stride + h * D + d] = o[j];
    }
    if (!xq) return;
    am = wave_max_f32(am);
    if (lane == 0) wmax[wid] = am;
    __syncthreads();
    am = 0.0f;
#pragma unroll
    for (int w = 0; w < 16; w++) am = fmaxf(am, wmax[w]);
    float scale, inv;
    act_scales(am, &scale, &inv);
    if (t == 0) xs[b] = scale;
#pragma unroll
    for (int j = 0; j < 2; j++)
        xq[(int64_t)b * K + (2 * hp + j) * D + d] = (int8_t)round_clamp_i8(__fmul_rn(o[j], inv));
}

__global__ __launch_bounds__(128) void k_attn_merge_heads(const float *__restrict__ part, int64_t part_stride, int S,
                                                         float *__restrict__ att, int64_t att_stride) {
    constexpr int D = 128;
    __shared__ float fw[64], lsum;
    const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    const float *pb = part + (int64_t)b * part_stride;
    if (t < 64) merge_head_weights(pb, S, h, fw, &lsum);
    __syncthreads();
    att[(int64_t)b * att_stride + h * D + t] = merge_head_dim(pb, S, h, t, fw, lsum);
}

hipError_t launch_attn_merge_rows(const float *part, int64_t part_stride, int n_split, float *att,
                                  int64_t att_stride, int8_t *xq, float *xs, int B, hipStream_t st) {
    if ((!xq) != (!xs) || (!xq && !att) || B <= 0 || n_split <= 0 || n_split > 64) return hipErrorInvalidValue;
    switch (n_split) {
#define AM(S) case S: if (!xq) return hipErrorInvalidValue; \
        hipLaunchKernelGGL(k_attn_merge_rows<S>, dim3(B), dim3(256), 0, st, part, part_stride, att, att_stride, xq, xs); break;
        AM(1) AM(2) AM(4) AM(8) AM(16)
#undef AM
        default:
            if (xq)
                hipLaunchKernelGGL(k_attn_merge_seq, dim3(B), dim3(1024), 0, st, part, part_stride, n_split, att,
                                   att_stride, xq, xs);
            else
                hipLaunchKernelGGL(k_attn_merge_heads, dim3(16, B), dim3(128), 0, st, part, part_stride, n_split, att,
                                   att_stride);
    }
    return hipGetLastError();
}

}  // namespace qasr
