// int8 kernels of the decode hot path: weight packer, activation quantizer,
// W8A8 matvec family (plain / residual-add / SwiGLU / bias) and the LM-head
// argmax.  Integer accumulation is exact, so every output here is bit-identical
// to the reference's NEON SDOT path for the same f32 input vector.
#include "kernels.h"

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

// ---------------------------------------------------------------------------
// Activation prologue shared by the matvec kernels.
//
// Lane l owns the 16-element slots s = l + 64 c (c < NS); element e = 16 s + r.
// The wave (a) loads its slice of x (from f32 or from a bf16 embedding row),
// (b) optionally applies RMSNorm with the reference's exact AVX2 summation
// order (kernels/avx.rs:377-415: 16 lanes of sequential FMAs over 16-element
// blocks, then the hsum tree), and (c) quantizes with the absmax rule of
// quantize_f32_to_int8 (kernels/mod.rs:1795-1802).  The result is the lane's
// int8 dwords plus the activation scale.  No LDS barrier: each wave computes
// the prologue redundantly (x is a few KiB and sits in L2).
// ---------------------------------------------------------------------------
template <int NS, bool NORM, bool EMBED>
struct ActIn {
    float xv[NS][16];
    float wn[NORM ? NS : 1][16];
};

// Phase 1: issue the loads of the lane's activation slice (and RMSNorm gains).
// Called before the weight loads: vmcnt retires loads in issue order, so these
// small L2-resident reads complete while the weight stream is still in flight.
template <int NS, bool NORM, bool EMBED>
__device__ __forceinline__ void act_load(const float *__restrict__ x, const uint16_t *__restrict__ xe,
                                         const float *__restrict__ norm_w, int K, ActIn<NS, NORM, EMBED> &in,
                                         float *__restrict__ resid_out) {
    const int lane = threadIdx.x & 63;
    const int nslot = K >> 4;
    // branch-free: out-of-range slots load slot 0 and are zeroed by a select
#pragma unroll
    for (int c = 0; c < NS; c++) {
        const int s = lane + 64 * c;
        const bool ok = s < nslot;
        const int se = ok ? s : 0;
        if (EMBED) {
            const uint4 *p = reinterpret_cast<const uint4 *>(xe + 16 * se);
            const uint4 a = p[0], b = p[1];
            const uint32_t wds[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                in.xv[c][2 * i] = ok ? __uint_as_float(wds[i] << 16) : 0.0f;
                in.xv[c][2 * i + 1] = ok ? __uint_as_float(wds[i] & 0xFFFF0000u) : 0.0f;
            }
        } else {
            const float4 *p = reinterpret_cast<const float4 *>(x + 16 * se);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 v = p[i];
                in.xv[c][4 * i] = ok ? v.x : 0.0f;
                in.xv[c][4 * i + 1] = ok ? v.y : 0.0f;
                in.xv[c][4 * i + 2] = ok ? v.z : 0.0f;
                in.xv[c][4 * i + 3] = ok ? v.w : 0.0f;
            }
        }
        if (NORM) {
            const float4 *wp = reinterpret_cast<const float4 *>(norm_w + 16 * se);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 v = wp[i];
                in.wn[c][4 * i] = v.x; in.wn[c][4 * i + 1] = v.y;
                in.wn[c][4 * i + 2] = v.z; in.wn[c][4 * i + 3] = v.w;
            }
        }
        if (resid_out && ok) {
            float4 *o = reinterpret_cast<float4 *>(resid_out + 16 * s);
#pragma unroll
            for (int i = 0; i < 4; i++)
                o[i] = make_float4(in.xv[c][4 * i], in.xv[c][4 * i + 1], in.xv[c][4 * i + 2], in.xv[c][4 * i + 3]);
        }
    }
}

// Phase 2: optional RMSNorm with the reference's exact AVX2 summation order
// (kernels/avx.rs:377-415: 16 lanes of sequential FMAs over 16-element blocks,
// then the hsum tree), then the absmax int8 quantization of
// quantize_f32_to_int8 (kernels/mod.rs:1795-1802).  Lane l owns the 16-element
// slots s = l + 64 c; the result is its int8 dwords plus the activation scale.
// Each wave computes this redundantly — x is a few KiB and sits in L2 — so no
// block barrier is needed.
template <int NS, bool NORM, bool EMBED>
__device__ __forceinline__ void act_finish(ActIn<NS, NORM, EMBED> &in, float eps, int K, float *lds_t,
                                           int xd[NS][4], float *xs) {
    const int lane = threadIdx.x & 63;
    const int nslot = K >> 4;
    if (NORM) {
        // transpose through LDS: T[r][s] = x[16 s + r]
#pragma unroll
        for (int c = 0; c < NS; c++) {
            const int s = lane + 64 * c;
            if (s < nslot) {
#pragma unroll
                for (int r = 0; r < 16; r++) lds_t[r * nslot + s] = in.xv[c][r];
            }
        }
        __builtin_amdgcn_wave_barrier();
        float acc = 0.0f;
        if (lane < 16) {
            const float4 *t = reinterpret_cast<const float4 *>(lds_t + lane * nslot);
            for (int i = 0; i < (nslot >> 2); i++) {
                float4 v = t[i];
                acc = fmaf(v.x, v.x, acc);
                acc = fmaf(v.y, v.y, acc);
                acc = fmaf(v.z, v.z, acc);
                acc = fmaf(v.w, v.w, acc);
            }
        }
        __builtin_amdgcn_wave_barrier();
        const float ss = avx16_tree(acc);
        const float rinv = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)K), eps)));
#pragma unroll
        for (int c = 0; c < NS; c++)
#pragma unroll
            for (int r = 0; r < 16; r++) in.xv[c][r] = __fmul_rn(__fmul_rn(in.xv[c][r], rinv), in.wn[c][r]);
    }
    float m = 0.0f;
#pragma unroll
    for (int c = 0; c < NS; c++)
#pragma unroll
        for (int r = 0; r < 16; r++) m = fmaxf(m, fabsf(in.xv[c][r]));
    m = wave_max_f32(m);
    float scale, inv;
    act_scales(m, &scale, &inv);
    *xs = scale;
#pragma unroll
    for (int c = 0; c < NS; c++)
#pragma unroll
        for (int d = 0; d < 4; d++)
            xd[c][d] = pack4_i8(round_clamp_i8(__fmul_rn(in.xv[c][4 * d], inv)),
                                round_clamp_i8(__fmul_rn(in.xv[c][4 * d + 1], inv)),
                                round_clamp_i8(__fmul_rn(in.xv[c][4 * d + 2], inv)),
                                round_clamp_i8(__fmul_rn(in.xv[c][4 * d + 3], inv)));
}

__device__ __forceinline__ int dot16(const i32x4 w, const int xd[4], int acc) {
    acc = __builtin_amdgcn_sdot4(w.x, xd[0], acc, false);
    acc = __builtin_amdgcn_sdot4(w.y, xd[1], acc, false);
    acc = __builtin_amdgcn_sdot4(w.z, xd[2], acc, false);
    acc = __builtin_amdgcn_sdot4(w.w, xd[3], acc, false);
    return acc;
}

// ---------------------------------------------------------------------------
// W8A8 matvec family.  Wave gw owns rows [gw R, gw R + R) of the concatenated
// segments (q | k | v for the fused QKV projection); its weight loads are
// issued before the activation prologue so the prologue hides under HBM
// latency.  Epilogue ((float)acc * xs) * ws[row] as neon.rs:751-765, then:
//   MV_PLAIN  y = v                       (linear_nobias_int8_qkv, mod.rs:884)
//   MV_ADDTO  y = v + y                   (linear_nobias_int8_addto, mod.rs:1030)
//   MV_SWIGLU out[j] = g/(1+expf(-g))*u   (linear_nobias_int8_swiglu, mod.rs:970)
//   MV_BIAS   y = v + bias[row]           (matvec_int8 with bias, neon.rs:762)
// ---------------------------------------------------------------------------
template <int NS, int R, int MODE, bool NORM, bool EMBED>
__global__ __launch_bounds__(256) void k_w8a8(MvArgs a) {
    __shared__ float lds[NORM ? 4 * NS * 1024 : 1];
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = (blockIdx.x * 4 + wid) * R;
    if (row0 >= a.n_total) return;
    const int K = a.K, nslot = K >> 4;
    // segment of this wave (segments are multiples of R rows); scalar selects
    // keep the segment fields in SGPRs
    const int n0 = a.seg[0].n, n1 = a.seg[1].n;
    const bool in0 = row0 < n0, in1 = !in0 && row0 < n0 + n1;
    MvSeg S;
    S.w = in0 ? a.seg[0].w : (in1 ? a.seg[1].w : a.seg[2].w);
    S.ws = in0 ? a.seg[0].ws : (in1 ? a.seg[1].ws : a.seg[2].ws);
    S.y = in0 ? a.seg[0].y : (in1 ? a.seg[1].y : a.seg[2].y);
    const int lrow0 = row0 - (in0 ? 0 : (in1 ? n0 : n0 + n1));
    const uint16_t *xe = nullptr;
    if (EMBED) xe = a.embed + (int64_t)a.state[0] * K;
    float *resid = (EMBED && blockIdx.x == 0 && wid == 0) ? a.resid_out : nullptr;
    ActIn<NS, NORM, EMBED> in;
    act_load<NS, NORM, EMBED>(a.x, xe, a.norm_w, K, in, resid);
    i32x4 wv[R][NS];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int c = 0; c < NS; c++) {
            const int s = lane + 64 * c;
            const i32x4 v = __builtin_nontemporal_load(
                reinterpret_cast<const i32x4 *>(S.w + (int64_t)(lrow0 + r) * K) + (s < nslot ? s : 0));
            wv[r][c] = s < nslot ? v : i32x4{0, 0, 0, 0};
        }
    int xd[NS][4];
    float xs;
    act_finish<NS, NORM, EMBED>(in, a.eps, K, lds + wid * NS * 1024, xd, &xs);
    int acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        int t = 0;
#pragma unroll
        for (int c = 0; c < NS; c++) t = dot16(wv[r][c], xd[c], t);
        acc[r] = wave_sum_i32(t);
    }
    if (MODE == MV_SWIGLU) {
        if (lane < R / 2) {
            float g = 0.0f, u = 0.0f;
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float v = __fmul_rn(__fmul_rn((float)acc[r], xs), S.ws[lrow0 + r]);
                if (r == 2 * lane) g = v;
                if (r == 2 * lane + 1) u = v;
            }
            S.y[(lrow0 >> 1) + lane] = __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), u);
        }
    } else {
        if (lane < R) {
            int av = 0;
#pragma unroll
            for (int r = 0; r < R; r++) if (r == lane) av = acc[r];
            const int row = lrow0 + lane;
            float v = __fmul_rn(__fmul_rn((float)av, xs), S.ws[row]);
            if (MODE == MV_ADDTO) v = __fadd_rn(v, S.y[row]);
            if (MODE == MV_BIAS) v = __fadd_rn(v, a.bias[row]);
            S.y[row] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// o_proj of the decode step with the split-attention merge in front
// (causal_attention's result, mod.rs:1527-1535, then linear_nobias_int8_addto,
// decoder.rs:616-617).  The attention kernel leaves n_split partials
// (max, sum, o[128]) per query head; every block loads them (L2/MALL), merges
// with log-sum-exp weights into LDS, and its waves quantize the merged vector
// as the activation of a 4-rows-per-wave W8A8 addto matvec.  The partial loads
// are issued before the weight loads so the merge overlaps the weight stream.
// ---------------------------------------------------------------------------
#define OM_MAXS 8
__global__ __launch_bounds__(256) void k_oproj_merge(OprojMergeArgs a) {
    constexpr int D = 128, G = 2, NS = 2, R = 4, HQ = 16, K = HQ * D;
    __shared__ float att[K];
    __shared__ float ms[HQ][OM_MAXS], ls[HQ][OM_MAXS], wf[HQ][OM_MAXS], lsum[HQ];
    const int t = threadIdx.x, lane = t & 63;
    const int wid = __builtin_amdgcn_readfirstlane(t >> 6);
    const int S = a.n_split;
    const int row0 = (blockIdx.x * 4 + wid) * R;
    // (1) partial statistics and outputs of this thread
    float pm = -INFINITY, pl = 0.0f;
    if (t < HQ * S) {
        const int h = t / S, sp = t % S, kvh = h / G, g = h % G;
        const float *b = a.part + ((int64_t)(kvh * S + sp) * G + g) * (D + 2);
        pm = b[0];
        pl = b[1];
    }
    float ov[K / 256][OM_MAXS];
#pragma unroll
    for (int j = 0; j < K / 256; j++) {
        const int i = t + 256 * j, h = i / D, d = i % D, kvh = h / G, g = h % G;
#pragma unroll
        for (int sp = 0; sp < OM_MAXS; sp++) {
            const int se = sp < S ? sp : 0;
            const float v = a.part[((int64_t)(kvh * S + se) * G + g) * (D + 2) + 2 + d];
            ov[j][sp] = sp < S ? v : 0.0f;
        }
    }
    // (2) weights of this wave's rows
    const int nslot = K >> 4;
    const bool live = row0 < a.N;
    const int r0 = live ? row0 : 0;
    i32x4 wv[R][NS];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int c = 0; c < NS; c++)
            wv[r][c] = __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(a.w + (int64_t)(r0 + r) * K) +
                                                  lane + 64 * c);
    // (3) log-sum-exp weights per head
    if (t < HQ * S) {
        ms[t / S][t % S] = pm;
        ls[t / S][t % S] = pl;
    }
    __syncthreads();
    if (t < HQ) {
        float M = -INFINITY;
        for (int sp = 0; sp < S; sp++) M = fmaxf(M, ms[t][sp]);
        float lt = 0.0f;
        for (int sp = 0; sp < S; sp++) {
            const float f = ms[t][sp] == -INFINITY ? 0.0f : expf(__fsub_rn(ms[t][sp], M));
            wf[t][sp] = f;
            lt = fmaf(ls[t][sp], f, lt);
        }
        lsum[t] = lt;
    }
    __syncthreads();
    // (4) merged attention output
#pragma unroll
    for (int j = 0; j < K / 256; j++) {
        const int i = t + 256 * j, h = i / D;
        float ot = 0.0f;
#pragma unroll
        for (int sp = 0; sp < OM_MAXS; sp++)
            if (sp < S) ot = fmaf(ov[j][sp], wf[h][sp], ot);
        att[i] = lsum[h] > 0.0f ? __fdiv_rn(ot, lsum[h]) : 0.0f;
    }
    __syncthreads();
    if (!live) return;
    // (5) quantize (each wave covers the whole vector with its lanes' slots)
    ActIn<NS, false, false> in;
#pragma unroll
    for (int c = 0; c < NS; c++) {
        const float4 *p = reinterpret_cast<const float4 *>(att + 16 * (lane + 64 * c));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 v = p[i];
            in.xv[c][4 * i] = v.x; in.xv[c][4 * i + 1] = v.y; in.xv[c][4 * i + 2] = v.z; in.xv[c][4 * i + 3] = v.w;
        }
    }
    int xd[NS][4];
    float xs;
    act_finish<NS, false, false>(in, 0.0f, K, nullptr, xd, &xs);
    (void)nslot;
    // (6) dots and the residual-add epilogue
    int acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        int q = 0;
#pragma unroll
        for (int c = 0; c < NS; c++) q = dot16(wv[r][c], xd[c], q);
        acc[r] = wave_sum_i32(q);
    }
    if (lane < R) {
        int av = 0;
#pragma unroll
        for (int r = 0; r < R; r++) if (r == lane) av = acc[r];
        const int row = row0 + lane;
        const float v = __fmul_rn(__fmul_rn((float)av, xs), a.ws[row]);
        a.y[row] = __fadd_rn(v, a.y[row]);
    }
}

hipError_t launch_oproj_merge(const OprojMergeArgs &a, hipStream_t st) {
    if (a.Hkv != 8 || a.n_split <= 0 || a.n_split > OM_MAXS || a.N % 4 != 0) return hipErrorInvalidValue;
    const unsigned blocks = (unsigned)((a.N / 4 + 3) / 4);
    hipLaunchKernelGGL(k_oproj_merge, dim3(blocks), dim3(256), 0, st, a);
    return hipGetLastError();
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
    __shared__ float lds[NORM ? 4 * NS * 1024 : 1];
    __shared__ float bvals[4];
    __shared__ int bidx[4];
    __shared__ int last;
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = a.K, nslot = K >> 4;
    const int n_groups = (a.N + R - 1) / R;
    const int gw = blockIdx.x * 4 + wid, n_waves = gridDim.x * 4;
    int xd[NS][4];
    float xs;
    float best_v = -1e30f;
    int best_i = -1;
    int g = gw;
    i32x4 wv[R][NS];
    auto load_group = [&](int grp) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = grp * R + r;
#pragma unroll
            for (int c = 0; c < NS; c++) {
                const int s = lane + 64 * c;
                const bool ok = row < a.N && s < nslot;
                const i32x4 v = __builtin_nontemporal_load(
                    reinterpret_cast<const i32x4 *>(a.w + (int64_t)(row < a.N ? row : 0) * K) + (s < nslot ? s : 0));
                wv[r][c] = ok ? v : i32x4{0, 0, 0, 0};
            }
        }
    };
    ActIn<NS, NORM, false> in;
    act_load<NS, NORM, false>(a.x, nullptr, a.norm_w, K, in, nullptr);
    if (g < n_groups) load_group(g);
    act_finish<NS, NORM, false>(in, a.eps, K, lds + wid * NS * 1024, xd, &xs);
    for (; g < n_groups; g += n_waves) {
        int acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            int t = 0;
#pragma unroll
            for (int c = 0; c < NS; c++) t = dot16(wv[r][c], xd[c], t);
            acc[r] = t;
        }
        const int gn = g + n_waves;
        if (gn < n_groups) load_group(gn);   // prefetch the next group before reducing
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = g * R + r;
            const int s = wave_sum_i32(acc[r]);
            if (row < a.N) {
                const float v = __fadd_rn(__fmul_rn(__fmul_rn((float)s, xs), a.ws[row]), 0.0f);
                if (v > best_v) { best_v = v; best_i = row; }
            }
        }
    }
    if (lane == 0) { bvals[wid] = best_v; bidx[wid] = best_i; }
    __syncthreads();
    if (threadIdx.x == 0) {
        float bv = bvals[0];
        int bi = bidx[0];
        for (int w = 1; w < 4; w++)
            if (better(bvals[w], bidx[w], bv, bi)) { bv = bvals[w]; bi = bidx[w]; }
        st_agent(a.part_val + blockIdx.x, bv);
        st_agent(a.part_idx + blockIdx.x, bi);
    }
    if (!arrive_last(a.counter, gridDim.x, &last)) return;
    // final merge by one wave
    if (wid == 0) {
        float bv = -1e30f;
        int bi = -1;
        for (int b = lane; b < (int)gridDim.x; b += 64) {
            const float v = ld_agent(a.part_val + b);
            const int i = ld_agent(a.part_idx + b);
            if (better(v, i, bv, bi)) { bv = v; bi = i; }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        }
        if (lane == 0) {
            const int tok = bi < 0 ? 0 : bi;
            a.out_idx[0] = tok;
            if (a.state) {
                a.state[0] = tok;
                a.state[1] += 1;
                if (a.token_log) a.token_log[a.state[2]] = tok;
                a.state[2] += 1;
            }
            reset_counter(a.counter);
        }
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
#undef QASR_MV
    return hipErrorInvalidValue;
}

hipError_t launch_argmax(const ArgmaxArgs &a, bool norm, int blocks, hipStream_t st) {
    if (a.K % 64 != 0 || a.K > 4096) return hipErrorInvalidValue;
    const int ns = (a.K + 1023) / 1024;
#define QASR_AM(NS)                                                                           \
    if (ns == NS) {                                                                           \
        if (norm) hipLaunchKernelGGL((k_argmax_w8a8<NS, 4, true>), dim3(blocks), dim3(256), 0, st, a); \
        else hipLaunchKernelGGL((k_argmax_w8a8<NS, 4, false>), dim3(blocks), dim3(256), 0, st, a);     \
        return hipGetLastError();                                                             \
    }
    QASR_AM(1) QASR_AM(2) QASR_AM(3) QASR_AM(4)
#undef QASR_AM
    return hipErrorInvalidValue;
}

}  // namespace qasr
