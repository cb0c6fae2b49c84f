// Device code of the W8A8 decode matvecs shared by the kernels that run them:
// the activation prologue (load, RMSNorm in the reference's order, absmax
// quantization) and one wave's rows of the matvec.  Included by k_int8.hip
// (the matvec kernels) and k_attn.hip (the qkv + attention launch).
#pragma once
#include "kernels.h"

namespace qasr {

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
    float4 xf[EMBED ? 1 : NS][4];     // raw f32 activation loads
    uint4 xb[EMBED ? NS : 1][2];      // raw bf16 embedding-row loads
    float4 wf[NORM ? NS : 1][4];      // raw RMSNorm gain loads
    float xv[NS][16];
    float wn[NORM ? NS : 1][16];
};

// Phase 1: issue the loads of the lane's activation slice (and RMSNorm gains)
// into raw registers, nothing else.  Callers issue their weight loads right
// after and then place a scheduling barrier, so no instruction that consumes
// these values (and would make the wave wait for them) can be hoisted above
// the weight loads: the weight stream is in flight before the wave first
// waits on memory.  vmcnt retires loads in issue order, so these small
// L2-resident reads are the first to complete.
template <int NS, bool NORM, bool EMBED>
__device__ __forceinline__ void act_load(const float *__restrict__ x, const uint16_t *__restrict__ xe,
                                         const float *__restrict__ norm_w, int K, ActIn<NS, NORM, EMBED> &in) {
    const int lane = threadIdx.x & 63;
    const int nslot = K >> 4;
    // out-of-range slots load slot 0; act_convert zeroes them
#pragma unroll
    for (int c = 0; c < NS; c++) {
        const int s = lane + 64 * c;
        const int se = s < nslot ? s : 0;
        if (EMBED) {
            const uint4 *p = reinterpret_cast<const uint4 *>(xe + 16 * se);
            in.xb[c][0] = p[0];
            in.xb[c][1] = p[1];
        } else {
            const float4 *p = reinterpret_cast<const float4 *>(x + 16 * se);
#pragma unroll
            for (int i = 0; i < 4; i++) in.xf[c][i] = p[i];
        }
        if (NORM) {
            const float4 *wp = reinterpret_cast<const float4 *>(norm_w + 16 * se);
#pragma unroll
            for (int i = 0; i < 4; i++) in.wf[c][i] = wp[i];
        }
    }
}

// Phase 1b: raw loads -> f32 slots (zero beyond K); optionally stores the f32
// slice to resid_out (the embedding row becomes the residual stream).
template <int NS, bool NORM, bool EMBED>
__device__ __forceinline__ void act_convert(ActIn<NS, NORM, EMBED> &in, int K, float *__restrict__ resid_out) {
    const int lane = threadIdx.x & 63;
    const int nslot = K >> 4;
#pragma unroll
    for (int c = 0; c < NS; c++) {
        const int s = lane + 64 * c;
        const bool ok = s < nslot;
        if (EMBED) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t wds[4] = {in.xb[c][h].x, in.xb[c][h].y, in.xb[c][h].z, in.xb[c][h].w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    in.xv[c][8 * h + 2 * i] = ok ? __uint_as_float(wds[i] << 16) : 0.0f;
                    in.xv[c][8 * h + 2 * i + 1] = ok ? __uint_as_float(wds[i] & 0xFFFF0000u) : 0.0f;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 v = in.xf[c][i];
                in.xv[c][4 * i] = ok ? v.x : 0.0f;
                in.xv[c][4 * i + 1] = ok ? v.y : 0.0f;
                in.xv[c][4 * i + 2] = ok ? v.z : 0.0f;
                in.xv[c][4 * i + 3] = ok ? v.w : 0.0f;
            }
        }
        if (NORM) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 v = in.wf[c][i];
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
template <int NS, bool NORM, bool EMBED, bool UNROLL = false>
__device__ __forceinline__ void act_norm_scale(ActIn<NS, NORM, EMBED> &in, float eps, int K, float *lds_t,
                                               float *xs, float *xinv) {
    const int lane = threadIdx.x & 63;
    const int nslot = K >> 4;
    if (NORM) {
        // transpose through LDS: T[r][s] = x[16 s + r], rows QASR_NORM_PAD
        // floats apart beyond their nslot so that the 16 row-reading lanes
        // start on different banks
        const int ts = nslot + QASR_NORM_PAD;
#pragma unroll
        for (int c = 0; c < NS; c++) {
            const int s = lane + 64 * c;
            if (s < nslot) {
#pragma unroll
                for (int r = 0; r < 16; r++) lds_t[r * ts + s] = in.xv[c][r];
            }
        }
        __builtin_amdgcn_wave_barrier();
        float acc = 0.0f;
        if (lane < 16) {
            const float4 *t = reinterpret_cast<const float4 *>(lds_t + lane * ts);
            auto chain = [&acc](const float4 v) {
                acc = fmaf(v.x, v.x, acc);
                acc = fmaf(v.y, v.y, acc);
                acc = fmaf(v.z, v.z, acc);
                acc = fmaf(v.w, v.w, acc);
            };
            if (UNROLL && nslot == 64 * NS) {
                // whole slots: each chunk's 16 LDS reads issued before its FMA
                // chain (more VGPRs: for kernels whose occupancy does not bind)
#pragma unroll
                for (int h = 0; h < NS; h++) {
                    float4 v[16];
#pragma unroll
                    for (int i = 0; i < 16; i++) v[i] = t[16 * h + i];
#pragma unroll
                    for (int i = 0; i < 16; i++) chain(v[i]);
                }
            } else {
                for (int i = 0; i < (nslot >> 2); i++) chain(t[i]);
            }
        }
        __builtin_amdgcn_wave_barrier();
        const float ss = avx16_tree(acc);
        const float rinv = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(div_by_count(ss, K), eps)));
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
    act_scales(m, xs, xinv);
}

// int8 dword d (elements 4d .. 4d + 3) of slot c
template <int NS, bool NORM, bool EMBED>
__device__ __forceinline__ int act_quant_dword(const ActIn<NS, NORM, EMBED> &in, int c, int d, float inv) {
    return pack4_i8(round_clamp_i8(__fmul_rn(in.xv[c][4 * d], inv)),
                    round_clamp_i8(__fmul_rn(in.xv[c][4 * d + 1], inv)),
                    round_clamp_i8(__fmul_rn(in.xv[c][4 * d + 2], inv)),
                    round_clamp_i8(__fmul_rn(in.xv[c][4 * d + 3], inv)));
}

template <int NS, bool NORM, bool EMBED>
__device__ __forceinline__ void act_finish(ActIn<NS, NORM, EMBED> &in, float eps, int K, float *lds_t,
                                           int xd[NS][4], float *xs) {
    float inv;
    act_norm_scale<NS, NORM, EMBED>(in, eps, K, lds_t, xs, &inv);
#pragma unroll
    for (int c = 0; c < NS; c++)
#pragma unroll
        for (int d = 0; d < 4; d++) xd[c][d] = act_quant_dword<NS, NORM, EMBED>(in, c, d, inv);
}

// act_finish for the 4 waves of a block that all need the same quantized
// vector: each wave forms the scale itself (the absmax is over the whole
// vector), quantizes dword wid of every slot its lanes hold (a quarter of the
// per-lane work) into qlds, and after one block barrier every lane reads its
// slots' 16 bytes back.  The values are act_finish's, bit for bit.  Every
// wave of the block must call it.  qlds: NS * 64 * 4 ints.
template <int NS, bool NORM, bool EMBED, bool UNROLL = false>
__device__ __forceinline__ void act_finish_block(ActIn<NS, NORM, EMBED> &in, float eps, int K, float *lds_t,
                                                 int *qlds, int xd[NS][4], float *xs) {
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    float inv;
    act_norm_scale<NS, NORM, EMBED, UNROLL>(in, eps, K, lds_t, xs, &inv);
#pragma unroll
    for (int c = 0; c < NS; c++) {
        int q;
        // wid is wave-uniform: one of four static register selections
        if (wid == 0) q = act_quant_dword<NS, NORM, EMBED>(in, c, 0, inv);
        else if (wid == 1) q = act_quant_dword<NS, NORM, EMBED>(in, c, 1, inv);
        else if (wid == 2) q = act_quant_dword<NS, NORM, EMBED>(in, c, 2, inv);
        else q = act_quant_dword<NS, NORM, EMBED>(in, c, 3, inv);
        qlds[(c * 64 + lane) * 4 + wid] = q;
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < NS; c++) {
        const int4 t = reinterpret_cast<const int4 *>(qlds)[c * 64 + lane];
        xd[c][0] = t.x; xd[c][1] = t.y; xd[c][2] = t.z; xd[c][3] = t.w;
    }
}

__device__ __forceinline__ int dot16(const i32x4 w, const int xd[4], int acc) {
    acc = __builtin_amdgcn_sdot4(w.x, xd[0], acc, false);
    acc = __builtin_amdgcn_sdot4(w.y, xd[1], acc, false);
    acc = __builtin_amdgcn_sdot4(w.z, xd[2], acc, false);
    acc = __builtin_amdgcn_sdot4(w.w, xd[3], acc, false);
    return acc;
}


// ---------------------------------------------------------------------------
// Reduce-scatter of a wave's integer partial dots.  Each lane holds W partial
// sums for each of N items (rows, or gate/up row pairs); after
// scatter_items<N, W> every lane holds the complete wave sums (all 64 lanes)
// of item scatter_item<N>(), replicated over 64 / N lanes: a permlane32 swap
// halves the items, a permlane16 swap halves them again, a row_ror:8 DPP step
// once more, and DPP steps (row_half_mirror, quad perms) finish the sums over
// the lanes left.  N = 8 takes 10 cross-lane steps per value where N
// separate wave sums take 48.  Integer sums are exact in any order, so the
// results equal the per-item wave sums bit for bit.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int swap32_sum_i(int keep_lo, int keep_hi) {
    const auto p = __builtin_amdgcn_permlane32_swap(keep_lo, keep_hi, false, false);
    return (int)p[0] + (int)p[1];
}
__device__ __forceinline__ int swap16_sum_i(int keep_even, int keep_odd) {
    const auto p = __builtin_amdgcn_permlane16_swap(keep_even, keep_odd, false, false);
    return (int)p[0] + (int)p[1];
}
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
    return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xF, 0xF, false);
}
// the item this lane holds after scatter_items<N, W> (the swap halves are
// told apart by running the same swaps on indicators)
template <int N>
__device__ __forceinline__ int scatter_item() {
    int it = 0;
    if (N >= 2) it += swap32_sum_i(0, 1) > 1 ? N / 2 : 0;
    if (N >= 4) it += swap16_sum_i(0, 1) > 1 ? N / 4 : 0;
    if (N >= 8) it += (threadIdx.x >> 3) & 1;
    return it;
}
template <int N, int W>
__device__ __forceinline__ void scatter_items(int (&v)[N][W], int (&out)[W]) {
    static_assert(N == 1 || N == 2 || N == 4 || N == 8, "1, 2, 4 or 8 items");
    if constexpr (N >= 2) {
#pragma unroll
        for (int i = 0; i < N / 2; i++)
#pragma unroll
            for (int w = 0; w < W; w++) v[i][w] = swap32_sum_i(v[i][w], v[i + N / 2][w]);
    }
    if constexpr (N >= 4) {
#pragma unroll
        for (int i = 0; i < N / 4; i++)
#pragma unroll
            for (int w = 0; w < W; w++) v[i][w] = swap16_sum_i(v[i][w], v[i + N / 4][w]);
    }
    if constexpr (N >= 8) {
        const int bit3 = (threadIdx.x >> 3) & 1;
#pragma unroll
        for (int w = 0; w < W; w++) {
            const int keep = bit3 ? v[1][w] : v[0][w], send = bit3 ? v[0][w] : v[1][w];
            v[0][w] = keep + dpp_i32<QASR_DPP_ROW_ROR8>(send);
        }
    }
#pragma unroll
    for (int w = 0; w < W; w++) {
        int x = v[0][w];
        if constexpr (N < 2) x = swap32_sum_i(x, x);
        if constexpr (N < 4) x = swap16_sum_i(x, x);
        if constexpr (N < 8) x += dpp_i32<QASR_DPP_ROW_ROR8>(x);
        x += dpp_i32<QASR_DPP_ROW_HALF_MIRROR>(x);
        x += dpp_i32<QASR_DPP_QP_1032>(x);
        x += dpp_i32<QASR_DPP_QP_2301>(x);
        out[w] = x;
    }
}

// ---------------------------------------------------------------------------
// W8A8 matvec family, one wave of block blk (4 waves per block).  Wave gw
// owns rows [gw R, gw R + R) of the concatenated segments (q | k | v for the
// fused QKV projection); its weight loads are issued before the activation
// prologue so the prologue hides under HBM latency.  Epilogue
// ((float)acc * xs) * ws[row] as neon.rs:751-765, then:
//   MV_PLAIN  y = v                       (linear_nobias_int8_qkv, mod.rs:884)
//   MV_ADDTO  y = v + y                   (linear_nobias_int8_addto, mod.rs:1030)
//   MV_SWIGLU out[j] = g/(1+expf(-g))*u   (linear_nobias_int8_swiglu, mod.rs:970)
//   MV_BIAS   y = v + bias[row]           (matvec_int8 with bias, neon.rs:762)
// TAG (plain rows only): row r's value goes to tag_out[r] as one 64-bit
// (tag << 32 | f32 bits) agent-scope store instead of to the segment's y, for
// a consumer in the same launch that polls until the tag matches.
// lds: 4 QASR_NORM_LDS(NS) floats per block when NORM; qlds: NS 256 ints per block (the
// block's 4 waves share the quantized activation).  All 4 waves of the block
// must call it (one block barrier).
// ---------------------------------------------------------------------------
template <int NS, int R, int MODE, bool NORM, bool EMBED, bool TAG = false>
__device__ __forceinline__ void w8a8_wave(const MvArgs &a, int blk, float *lds, int *qlds,
                                          unsigned long long *tag_out = nullptr, unsigned tag = 0,
                                          unsigned long long *stamp = nullptr) {
    static_assert(!TAG || MODE == MV_PLAIN, "tagged outputs: plain rows only");
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // waves past the last row compute row 0 and store nothing
    const bool live = (blk * 4 + wid) * R < a.n_total;
    const int row0 = live ? (blk * 4 + wid) * R : 0;
    const int K = a.K, nslot = K >> 4;
    // segment of this wave (segments are multiples of R rows); scalar selects
    // keep the segment fields in SGPRs.  (The compiler loads the selected
    // fields from a selected argument address, a second scalar round trip
    // after the first batch of argument loads.  Reading all nine fields in
    // the first batch and selecting the values moved the first weight loads
    // 0.16 us earlier inside the launch but measured slower per launch:
    // gate_up 3.99 -> 4.33, down 3.45 -> 4.24 us.)
    const int n0 = a.seg[0].n, n1 = a.seg[1].n;
    const bool in0 = row0 < n0, in1 = !in0 && row0 < n0 + n1;
    MvSeg S;
    S.w = in0 ? a.seg[0].w : (in1 ? a.seg[1].w : a.seg[2].w);
    S.ws = in0 ? a.seg[0].ws : (in1 ? a.seg[1].ws : a.seg[2].ws);
    S.y = in0 ? a.seg[0].y : (in1 ? a.seg[1].y : a.seg[2].y);
    const int lrow0 = row0 - (in0 ? 0 : (in1 ? n0 : n0 + n1));
    const uint16_t *xe = nullptr;
    if (EMBED) xe = a.embed + (int64_t)a.state[0] * K;
    float *resid = (EMBED && blk == 0 && wid == 0) ? a.resid_out : nullptr;
    ActIn<NS, NORM, EMBED> in;
    act_load<NS, NORM, EMBED>(a.x, xe, a.norm_w, K, in);
    // weight slots beyond K load slot 0; their activation bytes are zero
    i32x4 wv[R][NS];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int c = 0; c < NS; c++) {
            const int s = lane + 64 * c;
            wv[r][c] = __builtin_nontemporal_load(
                reinterpret_cast<const i32x4 *>(S.w + (int64_t)(lrow0 + r) * K) + (s < nslot ? s : 0));
        }
    // epilogue operands (row scales, the old y of +=, the bias), loaded with the
    // weights so that no load is left on the path after the dot products.
    // SwiGLU: lane j < R/2 owns the gate/up row pair (2j, 2j+1); otherwise lane r < R owns row r.
    // (Vector loads on purpose: as scalar loads of uniform addresses they get
    // scheduled after the dot products.)
    // Each lane's epilogue serves the item the reduce-scatter leaves in it:
    // SwiGLU, the gate/up row pair (2j, 2j + 1) of item j; otherwise row r.
    constexpr int NI = MODE == MV_SWIGLU ? (R >= 2 ? R / 2 : 1) : R;   // (SwiGLU needs R >= 2)
    const int item = scatter_item<NI>();
    float ws0 = 0.0f, ws1 = 0.0f, yb = 0.0f;
    if (MODE == MV_SWIGLU) {
        ws0 = __builtin_nontemporal_load(S.ws + lrow0 + 2 * item);
        ws1 = __builtin_nontemporal_load(S.ws + lrow0 + 2 * item + 1);
    } else {
        ws0 = __builtin_nontemporal_load(S.ws + lrow0 + item);
        if (MODE == MV_ADDTO) yb = __builtin_nontemporal_load(S.y + lrow0 + item);
        if (MODE == MV_BIAS) yb = __builtin_nontemporal_load(a.bias + lrow0 + item);
    }
    // keep every load above here: the scheduling barrier stops the machine
    // scheduler, the empty memory-clobbering asm stops the earlier sinking
    // passes, which otherwise move the weight loads of the kernels without the
    // RMSNorm prologue below the activation wait (two HBM round trips in a
    // row instead of one)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    if (wid == 0) QASR_STAMP(stamp, 1);
    act_convert<NS, NORM, EMBED>(in, K, resid);
    if (wid == 0) QASR_STAMP(stamp, 2);
    int xd[NS][4];
    float xs;
    // (the fused qkv + attention launch, TAG, takes the unrolled RMSNorm reads
    // at K = 1024; at K = 2048 they raised its VGPRs 120 -> 169, leaving 2
    // waves per SIMD, one block per CU, and the 1.7B launch at L = 4096 grew
    // 16.8 -> 22.1 us)
    act_finish_block<NS, NORM, EMBED, TAG && NS == 1>(in, a.eps, K, lds + wid * QASR_NORM_LDS(NS), qlds, xd, &xs);
    if (wid == 0) QASR_STAMP(stamp, 3);
    // per-lane partial dots, then one reduce-scatter: every lane ends with its
    // item's complete sums.  The epilogue runs in every lane with no branch
    // (lanes holding the same item store the same value to the same address):
    // a predicated store would let the compiler sink the operand loads above
    // into the branch, after the dot products.
    if constexpr (MODE == MV_SWIGLU) {
        int part[NI][2];
#pragma unroll
        for (int j = 0; j < NI; j++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                int t = 0;
#pragma unroll
                // (% R: the R = 1 SwiGLU form is never launched; this keeps it in bounds)
                for (int c = 0; c < NS; c++) t = dot16(wv[(2 * j + h) % R][c], xd[c], t);
                part[j][h] = t;
            }
        int gu[2];
        scatter_items<NI, 2>(part, gu);
        const float g = __fmul_rn(__fmul_rn((float)gu[0], xs), ws0);
        const float u = __fmul_rn(__fmul_rn((float)gu[1], xs), ws1);
        if (wid == 0) QASR_STAMP(stamp, 4);
        const float o = __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), u);
        if (live) S.y[(lrow0 >> 1) + item] = o;
        if (wid == 0) QASR_STAMP(stamp, 5);
    } else {
        int part[NI][1];
#pragma unroll
        for (int r = 0; r < R; r++) {
            int t = 0;
#pragma unroll
            for (int c = 0; c < NS; c++) t = dot16(wv[r][c], xd[c], t);
            part[r][0] = t;
        }
        int av[1];
        scatter_items<NI, 1>(part, av);
        if (wid == 0) QASR_STAMP(stamp, 4);
        float v = __fmul_rn(__fmul_rn((float)av[0], xs), ws0);
        if (MODE == MV_ADDTO || MODE == MV_BIAS) v = __fadd_rn(v, yb);
        if (TAG) {
            // (value, tag) in one 64-bit agent-scope store: a consumer in the
            // same launch polls it (row0 is the row in the concatenation)
            if (live)
                __hip_atomic_store(tag_out + row0 + item, ((unsigned long long)tag << 32) | __float_as_uint(v),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (wid == 0) QASR_STAMP(stamp, 5);
        } else {
            if (live) S.y[lrow0 + item] = v;
            if (wid == 0) QASR_STAMP(stamp, 5);
        }
    }
}


}  // namespace qasr
