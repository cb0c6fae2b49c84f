// Dense GEMMs of the prefill, the audio encoder and the mel front end.
//
//   C[m, n] (op)= sum_k A[m, k] * B[n, k]          ("NT": both operands K-contiguous)
//
// k_gemm_mfma: CDNA4 MFMA (v_mfma_f32_16x16x32_bf16), 64x64 block tile, four
// waves of 32x32, K-step 32, LDS double buffer.  Operand sources:
//   A f32, split: A = hi + mid + lo with three bf16 terms (each the RNE rounding
//                 of the remaining residual), so A*B is formed from exact bf16
//                 products accumulated in f32 — f32-class accuracy against the
//                 reference's cblas_sgemm on bf16-valued weights (mod.rs:550-628)
//   A bf16        activations already in bf16 (the int8 x bf16 GEMM)
//   B bf16        the reference's weights (exact)
//   B int8        per-row int8 weights, dequantised exactly to bf16 in LDS; the
//                 per-row scale is applied in the epilogue
//   A conv       (k_gemm_lds only) f32 channels-last activations read as the
//                 im2col matrix of a strided convolution without forming it:
//                 each K-step is one kernel tap's run of 32 channels, loaded
//                 straight from the activation row (zero past the borders),
//                 then split like A f32
// k_gemm_f32: plain f32 FMA tiles for the small GEMMs whose operands are both
// f32 tables (mel DFT and filterbank, audio.rs:339-351).
#include <cstdlib>

#include "kernels.h"

namespace qasr {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float bf16_round(float v) {
    return __uint_as_float((uint32_t)f32_to_bf16_rne(v) << 16);
}

template <int ASRC, int BSRC, int EPI>
__global__ __launch_bounds__(256) void k_gemm_mfma(GemmArgs g) {
    constexpr int BM = 64, BN = 64, BK = 32, LDK = BK + 8;
    constexpr int NA = ASRC == A_F32_SPLIT ? 3 : 1;
    __shared__ __attribute__((aligned(16))) uint16_t As[2][NA][BM][LDK];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN][LDK];
    const int t = threadIdx.x, lane = t & 63;
    const int wid = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wid >> 1, wn = wid & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int M = g.M, N = g.N, K = g.K;
    // global -> register staging: thread t covers row t/4, k-offset (t%4)*8 of the tile
    const int lr = t >> 2, lk = (t & 3) * 8;
    const int am = m0 + lr, bn = n0 + lr;
    float ar[8];
    u16x8 ab;
    u16x8 br;

    auto load_tile = [&](int k0) {
        const int kk = k0 + lk;
        if (ASRC == A_F32_SPLIT) {
            const float *ap = reinterpret_cast<const float *>(g.A) + (int64_t)am * g.lda + kk;
            if (am < M && kk + 8 <= K && g.a_vec4) {
                const float4 x0 = reinterpret_cast<const float4 *>(ap)[0];
                const float4 x1 = reinterpret_cast<const float4 *>(ap)[1];
                ar[0] = x0.x; ar[1] = x0.y; ar[2] = x0.z; ar[3] = x0.w;
                ar[4] = x1.x; ar[5] = x1.y; ar[6] = x1.z; ar[7] = x1.w;
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float *q = reinterpret_cast<const float *>(g.A) + (int64_t)min(am, M - 1) * g.lda + min(kk + i, K - 1);
                    ar[i] = (am < M && kk + i < K) ? *q : 0.0f;
                }
            }
        } else {
            const uint16_t *ap = reinterpret_cast<const uint16_t *>(g.A) + (int64_t)am * g.lda + kk;
            if (am < M && kk + 8 <= K && g.a_vec4) {
                ab = *reinterpret_cast<const u16x8 *>(ap);
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const uint16_t *q = reinterpret_cast<const uint16_t *>(g.A) + (int64_t)min(am, M - 1) * g.lda + min(kk + i, K - 1);
                    ab[i] = (am < M && kk + i < K) ? *q : (uint16_t)0;
                }
            }
        }
        if (BSRC == B_BF16) {
            const uint16_t *bp = reinterpret_cast<const uint16_t *>(g.B) + (int64_t)bn * g.ldb + kk;
            if (bn < N && kk + 8 <= K && g.b_vec) {
                br = *reinterpret_cast<const u16x8 *>(bp);
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const uint16_t *q = reinterpret_cast<const uint16_t *>(g.B) + (int64_t)min(bn, N - 1) * g.ldb + min(kk + i, K - 1);
                    br[i] = (bn < N && kk + i < K) ? *q : (uint16_t)0;
                }
            }
        } else {
            const int8_t *bp = reinterpret_cast<const int8_t *>(g.B) + (int64_t)bn * g.ldb + kk;
            int8_t q[8];
            if (bn < N && kk + 8 <= K && g.b_vec) {
                const uint2 v = *reinterpret_cast<const uint2 *>(bp);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    q[i] = (int8_t)(v.x >> (8 * i));
                    q[4 + i] = (int8_t)(v.y >> (8 * i));
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const int8_t *qp = reinterpret_cast<const int8_t *>(g.B) + (int64_t)min(bn, N - 1) * g.ldb + min(kk + i, K - 1);
                    q[i] = (bn < N && kk + i < K) ? *qp : (int8_t)0;
                }
            }
#pragma unroll
            for (int i = 0; i < 8; i++) br[i] = f32_to_bf16_rne((float)q[i]);   // exact, |q| <= 128
        }
    };
    auto store_tile = [&](int buf) {
        if (ASRC == A_F32_SPLIT) {
            u16x8 hi, mi, lo;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float x = ar[i];
                const uint16_t h = f32_to_bf16_rne(x);
                const float r1 = __fsub_rn(x, __uint_as_float((uint32_t)h << 16));
                const uint16_t m = f32_to_bf16_rne(r1);
                const float r2 = __fsub_rn(r1, __uint_as_float((uint32_t)m << 16));
                hi[i] = h; mi[i] = m; lo[i] = f32_to_bf16_rne(r2);
            }
            *reinterpret_cast<u16x8 *>(&As[buf][0][lr][lk]) = hi;
            *reinterpret_cast<u16x8 *>(&As[buf][1][lr][lk]) = mi;
            *reinterpret_cast<u16x8 *>(&As[buf][2 % NA][lr][lk]) = lo;
        } else {
            *reinterpret_cast<u16x8 *>(&As[buf][0][lr][lk]) = ab;
        }
        *reinterpret_cast<u16x8 *>(&Bs[buf][lr][lk]) = br;
    };

    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int nk = (K + BK - 1) / BK;
    load_tile(0);
    store_tile(0);
    __syncthreads();
    const int fr = lane & 15, fk = (lane >> 4) * 8;
    for (int kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load_tile((kt + 1) * BK);
        bf16x8 bfrag[2];
#pragma unroll
        for (int j = 0; j < 2; j++)
            bfrag[j] = *reinterpret_cast<const bf16x8 *>(&Bs[buf][wn * 32 + j * 16 + fr][fk]);
#pragma unroll
        for (int s = NA - 1; s >= 0; s--) {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const bf16x8 afrag = *reinterpret_cast<const bf16x8 *>(&As[buf][s][wm * 32 + i * 16 + fr][fk]);
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afrag, bfrag[j], acc[i][j], 0, 0, 0);
            }
        }
        if (kt + 1 < nk) store_tile(buf ^ 1);
        __syncthreads();
    }

    // epilogue: lane holds rows 4*(lane/16)+r, column lane%16 of each 16x16 tile
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * 32 + i * 16 + (lane >> 4) * 4 + r;
                const int n = n0 + wn * 32 + j * 16 + (lane & 15);
                if (m >= M || n >= N) continue;
                float v = acc[i][j][r];
                // EPI_TRANS: rows are (chunk, spatial) of a batched conv and the
                // output keeps the reference layout [chunk][channel][spatial];
                // EPI_CHW: the same GELU index, row-major (channels-last) output
                int64_t off, gidx;
                if (EPI & EPI_TRANS) {
                    const int c = m / g.gelu_rows, sp = m % g.gelu_rows;
                    gidx = (int64_t)n * g.gelu_rows + sp;
                    off = (int64_t)c * g.gelu_n + gidx;
                } else if (EPI & EPI_CHW) {
                    gidx = (int64_t)n * g.gelu_rows + m % g.gelu_rows;
                    off = (int64_t)m * g.ldc + n;
                } else {
                    gidx = (int64_t)m * g.ldc + n;
                    off = gidx;
                }
                float *cp = g.C + off;
                if (EPI & EPI_SCALE) v = __fmul_rn(v, g.scale[n]);
                if (EPI & EPI_ACCUM) {
                    float c = *cp;
                    if (g.bias) c = __fadd_rn(c, g.bias[n]);
                    v = __fadd_rn(c, v);
                } else if (g.bias) {
                    v = __fadd_rn(v, g.bias[n]);
                }
                if (EPI & EPI_GELU) v = gelu_ref(v, gidx, g.gelu_n);
                *cp = v;
            }
}

// ---------------------------------------------------------------------------
// k_gemm_lds: the same tile shape, MFMA and epilogues as k_gemm_mfma, fed by
// direct global -> LDS loads (global_load_lds_dwordx4) through a ring of NS
// stages, so NS - 1 K-steps are in flight while one is computed (the
// register-staged kernel above keeps one, and its K loop is a chain of HBM
// round trips at these M ~ 400 shapes).  A stage holds the block's A tile
// (64 rows x BK, f32 or bf16, 8 KiB) and B tile (64 rows x BK, bf16 or int8,
// 4 KiB); each wave issues 3 of the stage's 12 one-KiB loads.  A load writes
// lane l's 16 bytes at LDS offset 16 l, so the lane -> (row, 16-byte slot)
// map is chosen with an XOR swizzle of the slot by the row, which spreads a
// fragment read's 16 rows over the banks.  f32 A is split into its three
// bf16 terms when the fragment is read; int8 B is widened to bf16 (exact).
// K-steps past the end load a zero page, so the wait count is the same in
// every iteration.  Requires K % BK == 0 and 16-byte aligned rows.
//
// KP > 1 splits the K loop inside the block: 4 KP waves in KP groups of 4,
// group p taking the K-steps p, p + KP, ... through a ring of its own; at the
// end groups 1 .. KP - 1 leave their partial tiles in LDS and group 0 adds
// them in group order and runs the epilogue.  At the M ~ 400 shapes of the
// prefill and config 1 a 64 x 64 tile's K loop is a chain of K-steps that one
// wave per SIMD walks alone (the grid holds 96-384 tiles for 256 CUs); KP
// groups shorten the chain KP times and give each SIMD KP waves to overlap.
// ---------------------------------------------------------------------------
__device__ __attribute__((aligned(256))) int4 g_gemm_zero16[16];

// One global_load_lds_dwordx4: lane l's 16 bytes from g land at LDS byte
// lds + 16 l.  Written as inline assembly, with the waits below, because the
// compiler otherwise treats every LDS read as possibly aliasing any load in
// flight and waits for all of them (vmcnt(0)) before it, which would drain
// the ring every K-step.  The compiler does not see these loads: the kernel
// issues no other vector-memory load until its final vmcnt(0), and it makes
// no other use of M0 (the generated code was checked for both).
// LDS placement of the ring's 16-byte slots: slot q of tile row r sits at
// slot q ^ a_swz(r) (A rows: 128 B, 8 slots) or q ^ b_swz(r) (B rows: 64 B, 4
// slots).  The f32-split kernels keep r & 7 and r & 3 (A by (r >> 1) & 7,
// conflict-free for 16-lane bank passes, measured 2.9 -> 3.15 ms on the
// encoder's GEMMs).  The bf16 x int8 kernels take the conflict-free forms
// (r >> 1) & 7 and (r & 3) ^ ((r >> 2) & 3): config-1 LM head at M = 375
// 184 -> 178 us, the seven 64 x 64 shapes within 2%.
template <bool AF>
__device__ __forceinline__ int a_swz(int r) { return AF ? (r & 7) : ((r >> 1) & 7); }
template <bool AF>
__device__ __forceinline__ int b_swz(int r) { return AF ? (r & 3) : ((r & 3) ^ ((r >> 2) & 3)); }

__device__ __forceinline__ void lds_dma16(const void *g, const void *lds) {
    const uint32_t la = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)lds;
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(la) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// float pair -> bf16 pair, round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// the GEMM epilogue of one output element (C row-major, or EPI_TRANS:
// [M / gelu_rows][N][gelu_rows]; EPI_CHW: row-major with EPI_TRANS's GELU
// index): scale, then C = (C + bias) + v for EPI_ACCUM or v + bias, then GELU
template <int EPI>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs &g, int m, int n, float v) {
    int64_t off, gidx;
    if (EPI & EPI_TRANS) {
        const int c = m / g.gelu_rows, sp = m % g.gelu_rows;
        gidx = (int64_t)n * g.gelu_rows + sp;
        off = (int64_t)c * g.gelu_n + gidx;
    } else if (EPI & EPI_CHW) {
        gidx = (int64_t)n * g.gelu_rows + m % g.gelu_rows;
        off = (int64_t)m * g.ldc + n;
    } else {
        gidx = (int64_t)m * g.ldc + n;
        off = gidx;
    }
    float *cp = g.C + off;
    if (EPI & EPI_SCALE) v = __fmul_rn(v, g.scale[n]);
    if (EPI & EPI_ACCUM) {
        float c = *cp;
        if (g.bias) c = __fadd_rn(c, g.bias[n]);
        v = __fadd_rn(c, v);
    } else if (g.bias) {
        v = __fadd_rn(v, g.bias[n]);
    }
    if (EPI & EPI_GELU) v = gelu_ref(v, gidx, g.gelu_n);
    *cp = v;
}

template <int ASRC, int BSRC, int EPI, int NS, int BM, int BN, int KS, int KP>
__global__ __launch_bounds__(256 * KP) void k_gemm_lds(GemmArgs g) {
    constexpr bool CONV = ASRC == A_CONV;
    constexpr bool AF = ASRC == A_F32_SPLIT || CONV;
    constexpr int AE = AF ? 4 : 2, BE = BSRC == B_BF16 ? 2 : 1;     // element bytes
    constexpr int BK = AF ? 32 : 64;                                 // A rows are 128 B, B rows 64 B per stage
    constexpr int ASZ = BM * 128, BSZ = BN * 64, STG = ASZ + BSZ;
    constexpr int LA = BM / 32, LB = BN / 64;                        // one-KiB loads per wave per stage
    constexpr int NA = AF ? 3 : 1;
    // wave tiling: the operand that needs converting is owned by one wave per
    // fragment (f32 A: waves take BM/4-row strips; int8 B: BN/4-column strips),
    // so no fragment is converted twice.  (Measured and rejected for the
    // int8 LM head at M = 375: 2 x 2 waves of (BM/2) x (BN/2), which halve the
    // A reads from LDS but widen every B fragment in two waves: 189 -> 209 us
    // with 128 x 128 tiles, 248 us with 128 x 256 tiles of one block per CU.)
    constexpr int WR = (AF ? BM / 4 : BM) / 16, WC = (AF ? BN : BN / 4) / 16;
    static_assert(BSRC == (AF ? B_BF16 : B_I8), "operand pair");
    static_assert(BM % 32 == 0 && BN % 64 == 0, "tile");
    static_assert(KP == 1 || KS == 1, "split K across blocks or inside them, not both");
    static_assert((KP - 1) * 4 * WR * WC * 4 * 64 * 4 <= KP * NS * STG, "partials fit the rings");
    __shared__ __attribute__((aligned(16))) char smem_all[KP][NS][STG];
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int grp = wave >> 2, wid = wave & 3;          // K group, wave within the group
    auto &smem = smem_all[grp];
    const int mw = AF ? (BM / 4) * wid : 0, nw = AF ? 0 : (BN / 4) * wid;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int M = g.M, N = g.N, K = g.K;
    // split K (KS > 1, grid z = KS): this block's K-steps [k0s, k0s + nk); its
    // raw partial sums go to the workspace and a reduction pass runs the
    // epilogue.  A compile-time count, so that the unsplit kernels keep their
    // main loop unchanged.
    const int nk_all = K / BK, kz = KS > 1 ? (int)blockIdx.z : 0;
    const int k0s = KS > 1 ? nk_all * kz / KS : 0, nk = KS > 1 ? nk_all * (kz + 1) / KS - k0s : nk_all;
    // KP groups: this group's i-th K-step is k0s + grp + KP i; nit iterations each
    const int nit = (nk + KP - 1) / KP;
    // this lane's rows and swizzled 16-byte slots in the wave's loads: A load j
    // covers tile rows 8 j .. 8 j + 7 (8 slots each), B load j rows 16 j .. 16 j + 15 (4 slots)
    const char *A = reinterpret_cast<const char *>(g.A), *B = reinterpret_cast<const char *>(g.B);
    const char *a_src[LA], *b_src[LB];
    int a_iy[CONV ? LA : 1], a_ix[CONV ? LA : 1];   // A_CONV: the row's input origin (may be outside)
#pragma unroll
    for (int u = 0; u < LA; u++) {
        const int r = 8 * (wid * LA + u) + (lane >> 3), p = (lane & 7) ^ a_swz<AF>(r);
        const int m = min(m0 + r, M - 1);
        if constexpr (CONV) {
            const int plane = g.conv_hout * g.conv_wout, ch = m / plane, rem = m - ch * plane;
            const int oy = rem / g.conv_wout, ox = rem - oy * g.conv_wout;
            a_iy[u] = oy * g.conv_sy - g.conv_py;
            a_ix[u] = ox * g.conv_sx - g.conv_px;
            a_src[u] = A + (int64_t)ch * g.conv_hin * g.conv_win * g.conv_c * AE + 16 * p;
        } else {
            a_src[u] = A + ((int64_t)m * g.lda) * AE + 16 * p;
        }
    }
#pragma unroll
    for (int u = 0; u < LB; u++) {
        const int r = 16 * (wid * LB + u) + (lane >> 2), p = (lane & 3) ^ b_swz<AF>(r);
        b_src[u] = B + ((int64_t)min(n0 + r, N - 1) * g.ldb) * BE + 16 * p;
    }
    const char *zero = reinterpret_cast<const char *>(g_gemm_zero16);
    auto issue = [&](int buf, int kt) {
        char *st = smem[buf];
        const int kg = grp + KP * kt;       // the group's kt-th K-step
        const bool live = kt < nit && kg < nk;
        const int64_t ka = live ? (int64_t)(k0s + kg) * BK * AE : 0, kb = live ? (int64_t)(k0s + kg) * BK * BE : 0;
        if constexpr (CONV) {
            // K-step (ky, kx, c0 .. c0 + 31): one 128-byte run of channels per
            // row.  The quotients by reciprocal: k0 is a multiple of 32 below
            // conv_c kh kw, so (k0 + 16) / conv_c sits at least 16 / conv_c
            // from an integer, far beyond the float error of the product
            // (and likewise t + 0.5 over conv_kw)
            const int k0 = live ? (k0s + kg) * BK : 0;
            const int t = (int)(((float)k0 + 16.0f) * g.conv_rc), c0 = k0 - t * g.conv_c;
            const int ky = (int)(((float)t + 0.5f) * g.conv_rkw), kx = t - ky * g.conv_kw;
#pragma unroll
            for (int u = 0; u < LA; u++) {
                const int iy = a_iy[u] + ky, ix = a_ix[u] + kx;
                const bool in = live && iy >= 0 && iy < g.conv_hin && ix >= 0 && ix < g.conv_win;
                const int64_t off = ((int64_t)(in ? iy : 0) * g.conv_win + (in ? ix : 0)) * g.conv_c + c0;
                lds_dma16(in ? a_src[u] + off * AE : zero, st + 1024 * (wid * LA + u));
            }
        } else {
#pragma unroll
            for (int u = 0; u < LA; u++) lds_dma16(live ? a_src[u] + ka : zero, st + 1024 * (wid * LA + u));
        }
#pragma unroll
        for (int u = 0; u < LB; u++) lds_dma16(live ? b_src[u] + kb : zero, st + ASZ + 1024 * (wid * LB + u));
    };

    f32x4 acc[WR][WC];
#pragma unroll
    for (int i = 0; i < WR; i++)
#pragma unroll
        for (int j = 0; j < WC; j++) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // The epilogue's operands do not depend on the products: the unsplit
    // kernels load them (column scale and bias, the old C of +=) before the
    // ring's first stage, so that no load is left after the K loop.  Being
    // older than every ring load, they are complete by the first wait.
    constexpr bool PRE = KS == 1;
    float pre_s[WC], pre_b[WC], pre_c[PRE && (EPI & EPI_ACCUM) ? WR : 1][WC][4];
    if (PRE && grp == 0) {
#pragma unroll
        for (int j = 0; j < WC; j++) {
            const int n = min(n0 + nw + j * 16 + (lane & 15), N - 1);
            pre_s[j] = (EPI & EPI_SCALE) ? g.scale[n] : 1.0f;
            pre_b[j] = g.bias ? g.bias[n] : 0.0f;
        }
        if constexpr ((EPI & EPI_ACCUM) != 0) {
#pragma unroll
            for (int i = 0; i < WR; i++)
#pragma unroll
                for (int j = 0; j < WC; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int m = min(m0 + mw + i * 16 + (lane >> 4) * 4 + r, M - 1);
                        const int n = min(n0 + nw + j * 16 + (lane & 15), N - 1);
                        pre_c[i][j][r] = g.C[(int64_t)m * g.ldc + n];
                    }
        }
    }

#pragma unroll
    for (int s = 0; s < NS - 1; s++) issue(s, s);
    const int fr = lane & 15, fg = lane >> 4;
    for (int kt = 0; kt < nit; kt++) {
        wait_vmcnt<(LA + LB) * (NS - 2)>();   // this wave's loads of stage kt have landed
        __syncthreads();                      // ... and every wave's; stage kt - 1 is free
        issue((kt + NS - 1) % NS, kt + NS - 1);
        const char *st = smem[kt % NS];
#pragma unroll
        for (int s = 0; s < BK / 32; s++) {
            bf16x8 bfrag[WC];
#pragma unroll
            for (int j = 0; j < WC; j++) {
                const int n = nw + j * 16 + fr;
                if (BSRC == B_BF16) {
                    const int p = fg ^ b_swz<AF>(n);
                    bfrag[j] = *reinterpret_cast<const bf16x8 *>(st + ASZ + n * 64 + p * 16);
                } else {
                    // 8 int8 weights -> bf16 (exact: |q| <= 128 has 8 significant bits)
                    const int p = (2 * s + (fg >> 1)) ^ b_swz<AF>(n);
                    const uint2 v = *reinterpret_cast<const uint2 *>(st + ASZ + n * 64 + p * 16 + (fg & 1) * 8);
                    uint32_t w[4];
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const uint32_t x = e ? v.y : v.x;
                        w[2 * e] = cvt_pk_bf16((float)(int8_t)(x & 0xFF), (float)(int8_t)((x >> 8) & 0xFF));
                        w[2 * e + 1] = cvt_pk_bf16((float)(int8_t)((x >> 16) & 0xFF), (float)(int8_t)(x >> 24));
                    }
                    bfrag[j] = __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3]));
                }
            }
#pragma unroll
            for (int i = 0; i < WR; i++) {
                const int r = mw + i * 16 + fr;
                bf16x8 af[NA];
                if (AF) {
                    // f32 A = hi + mid + lo, each term the RNE bf16 of the remaining residual
                    const int k4 = 2 * fg;
                    const float4 x0 = *reinterpret_cast<const float4 *>(st + r * 128 + ((k4 ^ a_swz<AF>(r)) * 16));
                    const float4 x1 = *reinterpret_cast<const float4 *>(st + r * 128 + (((k4 + 1) ^ a_swz<AF>(r)) * 16));
                    const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                    uint32_t hi[4], mi[4], lo[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float a0 = xv[2 * e], a1 = xv[2 * e + 1];
                        const uint32_t h = cvt_pk_bf16(a0, a1);
                        const float r0 = __fsub_rn(a0, __uint_as_float(h << 16));
                        const float r1 = __fsub_rn(a1, __uint_as_float(h & 0xFFFF0000u));
                        const uint32_t m = cvt_pk_bf16(r0, r1);
                        const float s0 = __fsub_rn(r0, __uint_as_float(m << 16));
                        const float s1 = __fsub_rn(r1, __uint_as_float(m & 0xFFFF0000u));
                        hi[e] = h;
                        mi[e] = m;
                        lo[e] = cvt_pk_bf16(s0, s1);
                    }
                    af[0] = __builtin_bit_cast(bf16x8, make_uint4(hi[0], hi[1], hi[2], hi[3]));
                    af[NA > 1 ? 1 : 0] = __builtin_bit_cast(bf16x8, make_uint4(mi[0], mi[1], mi[2], mi[3]));
                    af[NA - 1] = __builtin_bit_cast(bf16x8, make_uint4(lo[0], lo[1], lo[2], lo[3]));
                } else {
                    const int p = (4 * s + fg) ^ a_swz<AF>(r);
                    af[0] = *reinterpret_cast<const bf16x8 *>(st + r * 128 + p * 16);
                }
#pragma unroll
                for (int a = NA - 1; a >= 0; a--)
#pragma unroll
                    for (int j = 0; j < WC; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[a], bfrag[j], acc[i][j], 0, 0, 0);
            }
        }
    }
    wait_vmcnt<0>();                          // no load may land in LDS after the block ends
    if constexpr (KP > 1) {
        // groups 1 .. KP - 1 hand their partial tiles to group 0 through the
        // rings' LDS (every wave is past its last ring read at the barrier)
        constexpr int EW = WR * WC * 4;      // accumulator values per lane
        float *red = reinterpret_cast<float *>(&smem_all[0][0][0]);
        __syncthreads();
        if (grp > 0) {
            float *dst = red + ((grp - 1) * 4 + wid) * EW * 64 + lane;
#pragma unroll
            for (int i = 0; i < WR; i++)
#pragma unroll
                for (int j = 0; j < WC; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++) dst[((i * WC + j) * 4 + r) * 64] = acc[i][j][r];
        }
        __syncthreads();
        if (grp > 0) return;
#pragma unroll
        for (int p = 1; p < KP; p++) {
            const float *src = red + ((p - 1) * 4 + wid) * EW * 64 + lane;
#pragma unroll
            for (int i = 0; i < WR; i++)
#pragma unroll
                for (int j = 0; j < WC; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        acc[i][j][r] = __fadd_rn(acc[i][j][r], src[((i * WC + j) * 4 + r) * 64]);
        }
    }

    // epilogue: lane holds rows 4*(lane/16)+r, column lane%16 of each 16x16 tile
    if constexpr (PRE) {
        // every value first, then only stores under the bounds tests: an
        // operand use inside a store's branch would make the compiler wait
        // for all vector memory there, the previous stores included
        float outv[WR][WC][4];
#pragma unroll
        for (int i = 0; i < WR; i++)
#pragma unroll
            for (int j = 0; j < WC; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = m0 + mw + i * 16 + (lane >> 4) * 4 + r;
                    const int n = n0 + nw + j * 16 + (lane & 15);
                    // gemm_epilogue's arithmetic on the preloaded operands
                    int64_t gidx;              // gelu()'s element index
                    if (EPI & (EPI_TRANS | EPI_CHW)) gidx = (int64_t)n * g.gelu_rows + m % g.gelu_rows;
                    else gidx = (int64_t)m * g.ldc + n;
                    float v = acc[i][j][r];
                    if (EPI & EPI_SCALE) v = __fmul_rn(v, pre_s[j]);
                    if constexpr ((EPI & EPI_ACCUM) != 0) {
                        float c = pre_c[i][j][r];
                        if (g.bias) c = __fadd_rn(c, pre_b[j]);
                        v = __fadd_rn(c, v);
                    } else {
                        if (g.bias) v = __fadd_rn(v, pre_b[j]);
                    }
                    if (EPI & EPI_GELU) v = gelu_ref(v, gidx, g.gelu_n);
                    if constexpr ((EPI & EPI_SWIGLU) != 0) {
                        // (gate, up) are columns (n, n + 1), held by lanes (l, l ^ 1)
                        // with the same rows: the even lane forms output n / 2 with
                        // the expression and AVX / tail choice of k_swiglu_rows
                        const float up = __shfl_xor(v, 1, 64);
                        const int jj = n >> 1, half = N >> 1, nv = half - half % 8;
                        const float e = jj < nv ? fast_exp_ref(__fsub_rn(0.0f, v)) : expf(-v);
                        v = __fmul_rn(__fdiv_rn(v, __fadd_rn(1.0f, e)), up);
                    }
                    // materialised here: otherwise the compiler sinks the
                    // arithmetic into the store branches below
                    asm volatile("" : "+v"(v));
                    outv[i][j][r] = v;
                }
#pragma unroll
        for (int i = 0; i < WR; i++)
#pragma unroll
            for (int j = 0; j < WC; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = m0 + mw + i * 16 + (lane >> 4) * 4 + r;
                    const int n = n0 + nw + j * 16 + (lane & 15);
                    if (m >= M || n >= N) continue;
                    if ((EPI & EPI_SWIGLU) && (n & 1)) continue;
                    int64_t off;
                    if (EPI & EPI_TRANS) {
                        const int c = m / g.gelu_rows, sp = m % g.gelu_rows;
                        off = (int64_t)c * g.gelu_n + (int64_t)n * g.gelu_rows + sp;
                    } else if (EPI & EPI_SWIGLU) {
                        off = (int64_t)m * g.ldc + (n >> 1);
                    } else {
                        off = (int64_t)m * g.ldc + n;
                    }
                    g.C[off] = outv[i][j][r];
                }
    } else {
#pragma unroll
        for (int i = 0; i < WR; i++)
#pragma unroll
            for (int j = 0; j < WC; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = m0 + mw + i * 16 + (lane >> 4) * 4 + r;
                    const int n = n0 + nw + j * 16 + (lane & 15);
                    if (m < M && n < N) g.ws[((int64_t)kz * M + m) * N + n] = acc[i][j][r];
                }
    }
}

// split-K reduction: the partials summed in split order, then the epilogue
template <int EPI>
__global__ __launch_bounds__(256) void k_gemm_splitk_reduce(GemmArgs g, int ks) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x, mn = (int64_t)g.M * g.N;
    if (i >= mn) return;
    float v = g.ws[i];
    for (int z = 1; z < ks; z++) v = __fadd_rn(v, g.ws[z * mn + i]);
    gemm_epilogue<EPI>(g, (int)(i / g.N), (int)(i % g.N), v);
}

// ---------------------------------------------------------------------------
// f32 SIMT GEMM (NT), 64x64 tile, 4x4 outputs per thread, K-step 16
// ---------------------------------------------------------------------------
// T x T output tile per block of 16 x 16 threads, (T / 16)^2 outputs per
// thread; each output's sum runs over k in order in one thread (fmaf), so the
// tile size does not change a bit
template <int T>
__global__ __launch_bounds__(256) void k_gemm_f32(GemmArgs g) {
    constexpr int R = T / 16;
    __shared__ float As[16][T + 1], Bs[16][T + 1];
    const int t = threadIdx.x, tx = t & 15, ty = t >> 4;
    const int m0 = blockIdx.y * T, n0 = blockIdx.x * T;
    const float *A = reinterpret_cast<const float *>(g.A), *B = reinterpret_cast<const float *>(g.B);
    float acc[R][R] = {};
    for (int k0 = 0; k0 < g.K; k0 += 16) {
        for (int i = t; i < T * 16; i += 256) {
            const int r = i >> 4, k = i & 15;
            const int m = m0 + r, n = n0 + r, kk = k0 + k;
            const float av = A[(int64_t)min(m, g.M - 1) * g.lda + min(kk, g.K - 1)];
            const float bv = B[(int64_t)min(n, g.N - 1) * g.ldb + min(kk, g.K - 1)];
            As[k][r] = (m < g.M && kk < g.K) ? av : 0.0f;
            Bs[k][r] = (n < g.N && kk < g.K) ? bv : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 16; k++) {
            float a[R], b[R];
#pragma unroll
            for (int i = 0; i < R; i++) { a[i] = As[k][ty * R + i]; b[i] = Bs[k][tx * R + i]; }
#pragma unroll
            for (int i = 0; i < R; i++)
#pragma unroll
                for (int j = 0; j < R; j++) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int j = 0; j < R; j++) {
            const int m = m0 + ty * R + i, n = n0 + tx * R + j;
            if (m < g.M && n < g.N) g.C[(int64_t)m * g.ldc + n] = acc[i][j];
        }
}

template <int ASRC, int BSRC>
static hipError_t go_gemm(const GemmArgs &g, int epi, hipStream_t st) {
    const dim3 grid((g.N + 63) / 64, (g.M + 63) / 64);
    switch (epi) {
#define QE(E) case E: hipLaunchKernelGGL((k_gemm_mfma<ASRC, BSRC, E>), grid, dim3(256), 0, st, g); break;
        QE(EPI_NONE) QE(EPI_ACCUM) QE(EPI_SCALE) QE(EPI_GELU) QE(EPI_TRANS) QE(EPI_TRANS | EPI_GELU)
        QE(EPI_GELU | EPI_CHW)
#undef QE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// the epilogues each operand source is launched with (the implicit-im2col
// conv source: its plain and GELU forms, channels-last output)
constexpr bool epi_used(int asrc, int e) {
    if (asrc == A_CONV) return e == EPI_NONE || e == (EPI_GELU | EPI_CHW);
    if (e == EPI_SWIGLU) return asrc == A_F32_SPLIT;
    return (e & (EPI_CHW | EPI_SWIGLU)) == 0;
}

// the unsplit kernel with KP K groups per block
template <int ASRC, int BSRC, int NS, int BM, int BN, int KP>
static hipError_t go_gemm_lds_kp(const GemmArgs &g, int epi, dim3 grid, hipStream_t st) {
    switch (epi) {
#define QE(E)                                                                                                     \
    case E:                                                                                                       \
        if constexpr (epi_used(ASRC, E)) {                                                                        \
            hipLaunchKernelGGL((k_gemm_lds<ASRC, BSRC, E, NS, BM, BN, 1, KP>), grid, dim3(256 * KP), 0, st, g); \
            break;                                                                                                \
        } else {                                                                                                  \
            return hipErrorInvalidValue;                                                                          \
        }
        QE(EPI_NONE) QE(EPI_ACCUM) QE(EPI_SCALE) QE(EPI_GELU) QE(EPI_TRANS) QE(EPI_TRANS | EPI_GELU)
        QE(EPI_GELU | EPI_CHW) QE(EPI_SWIGLU)
#undef QE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// K groups per block of the 64 x 64 kernel: 4 while a block has at least 16
// K-steps and the tile columns number at most 32.  Measured at M = 375 (config 1, us per launch, KP 1 -> 4): k / v
// 7.7 -> 6.6, q 8.5 -> 7.5, o 12.4 -> 9.2, down 17.1 -> 11.9; gate / up (48
// tile columns, 288 blocks of 16 waves for 256 CUs) 10.2 -> 12.2, so they
// keep one group.  The rule reads N and K only, so a row's bits do not
// depend on how many rows share the call.
static int gemm_kp(const GemmArgs &g, int bk) {
    return (g.K / bk >= 16 && (g.N + 63) / 64 <= 32) ? 4 : 1;
}

template <int ASRC, int BSRC, int NS, int BM, int BN>
static hipError_t go_gemm_lds_ns(const GemmArgs &g, int epi, hipStream_t st) {
    const int gx = (g.N + BN - 1) / BN, gy = (g.M + BM - 1) / BM;
    if constexpr (BM == 64 && BN == 64) {
        const int kp = gemm_kp(g, ASRC == A_BF16 ? 64 : 32);
        if (kp == 4) return go_gemm_lds_kp<ASRC, BSRC, 3, 64, 64, 4>(g, epi, dim3(gx, gy), st);
        if (kp == 2) return go_gemm_lds_kp<ASRC, BSRC, 4, 64, 64, 2>(g, epi, dim3(gx, gy), st);
    }
    // split K in two (epilogues without a transposed store)
    // when the tile grid leaves most CUs idle and the caller gave a workspace
    // for the partials
    // (K-steps: at least 16 of the f32-class path, whose steps cost three MFMA
    // passes; the bf16 path does not split: with its loads of the epilogue
    // operands ahead of the K loop, the unsplit kernel measured faster at
    // M = 375, K = 2048 (11.7 against 13.2 us) and equal at K = 3072)
    if constexpr (ASRC == A_F32_SPLIT) {
    const int bk = 32, min_steps = 16;
    const bool epi_ok = epi == EPI_NONE || epi == EPI_ACCUM || epi == EPI_GELU || epi == EPI_SCALE;
    const bool ws_ok = g.ws && g.ws_bytes >= (int64_t)2 * g.M * g.N * (int64_t)sizeof(float);
    bool split;
    if (g.split_by_shape && ASRC == A_F32_SPLIT) {
        // (the tile-count rule's choice too for N <= 1024 up to 640 rows; that
        // rule also splits N > 1024 when the rows are few enough)
        split = gx <= 16 && g.K / bk >= min_steps && epi_ok;
        if (split && !ws_ok) return hipErrorInvalidValue;
    } else {
        split = ASRC == A_F32_SPLIT && gx * gy <= 160 && g.K / bk >= min_steps && epi_ok && ws_ok;
    }
    if (split) {
        const dim3 grid(gx, gy, 2), rg((unsigned)(((int64_t)g.M * g.N + 255) / 256));
        switch (epi) {
#define QE(E)                                                                                          \
    case E:                                                                                            \
        hipLaunchKernelGGL((k_gemm_lds<ASRC, BSRC, E, NS, BM, BN, 2, 1>), grid, dim3(256), 0, st, g);  \
        hipLaunchKernelGGL((k_gemm_splitk_reduce<E>), rg, dim3(256), 0, st, g, 2);                     \
        break;
            QE(EPI_NONE) QE(EPI_ACCUM) QE(EPI_GELU) QE(EPI_SCALE)
#undef QE
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    }
    // (measured and rejected: each block walking every M tile of its column
    // strip, so that the strip's weights are read from HBM once: for the
    // config-1 LM head, 1187 strips at M = 375, 205 us against 160-184 with a
    // block per tile)
    const dim3 grid(gx, gy);
    switch (epi) {
#define QE(E)                                                                                           \
    case E:                                                                                             \
        if constexpr (epi_used(ASRC, E)) {                                                              \
            hipLaunchKernelGGL((k_gemm_lds<ASRC, BSRC, E, NS, BM, BN, 1, 1>), grid, dim3(256), 0, st, g); \
            break;                                                                                      \
        } else {                                                                                        \
            return hipErrorInvalidValue;                                                                \
        }
        QE(EPI_NONE) QE(EPI_ACCUM) QE(EPI_SCALE) QE(EPI_GELU) QE(EPI_TRANS) QE(EPI_TRANS | EPI_GELU)
        QE(EPI_GELU | EPI_CHW) QE(EPI_SWIGLU)
#undef QE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int ASRC, int BSRC>
static hipError_t go_gemm_lds(const GemmArgs &g, int epi, hipStream_t st) {
    // 64 x 64 tiles (4 stages of 12 KiB, 3 blocks per CU) while they leave
    // fewer than ~2 blocks per CU; beyond, 128 x 128 tiles: four times the
    // MFMA work per K-step and barrier.  Their bf16 x int8 form keeps 2
    // stages of 24 KiB, so that 3 blocks share a CU (LM head at M = 375, 3
    // stages -> 2: 174 -> 155 us, the same bits).  Measured and rejected
    // there: 128 x 256 tiles (218-226 us); 2 waves of 64-column strips, which
    // halve the A reads from LDS but need 287 registers (206 us); the M tiles
    // of one column strip grouped on one XCD (162 us, against 155); and the
    // activations split into three int8 planes on the int8 MFMA (273-282 us:
    // three bytes per activation through the ring and the LDS reads).
    // The implicit-im2col conv GEMM keeps 2 stages as well (the encoder's
    // conv2, M = 24000, N = 480, K = 4320: encoder 2.62-2.64 -> 2.59 ms; its
    // 64 x 64 and 128 x 64 tiles measured 2.79 and 2.77 ms).
    const int64_t small_blocks = (int64_t)((g.N + 63) / 64) * ((g.M + 63) / 64);
    const bool big = small_blocks >= 2048;
    constexpr int big_ns = ASRC == A_F32_SPLIT ? 3 : 2;
    return big ? go_gemm_lds_ns<ASRC, BSRC, big_ns, 128, 128>(g, epi, st)
               : go_gemm_lds_ns<ASRC, BSRC, 4, 64, 64>(g, epi, st);
}

// the LDS-ring kernel applies when every stage is whole and rows are 16-byte aligned
static bool gemm_lds_ok(const GemmArgs &g, int asrc, int bsrc) {
    const int bk = asrc == A_F32_SPLIT ? 32 : 64;
    const int ae = asrc == A_F32_SPLIT ? 4 : 2, be = bsrc == B_BF16 ? 2 : 1;
    return g.K % bk == 0 && (g.lda * ae) % 16 == 0 && (g.ldb * be) % 16 == 0 && (uintptr_t)g.A % 16 == 0 &&
           (uintptr_t)g.B % 16 == 0;
}

hipError_t launch_gemm(const GemmArgs &g0, int asrc, int bsrc, int epi, hipStream_t st) {
    GemmArgs g = g0;
    if (g.M <= 0 || g.N <= 0 || g.K <= 0) return hipErrorInvalidValue;
    g.a_vec4 = (g.lda % 8 == 0) && ((uintptr_t)g.A % 16 == 0);
    g.b_vec = (g.ldb % 8 == 0) && ((uintptr_t)g.B % 16 == 0);
    if ((epi & (EPI_TRANS | EPI_CHW)) && g.gelu_rows <= 0) return hipErrorInvalidValue;
    if ((epi & EPI_SWIGLU) && (g.N % 2 != 0 || !gemm_lds_ok(g, asrc, bsrc))) return hipErrorInvalidValue;
    if (asrc == A_CONV) {
        // implicit im2col: whole 32-channel runs, every K-step inside one tap
        const bool ok = bsrc == B_BF16 && g.conv_c > 0 && g.conv_c % 32 == 0 && g.conv_kh > 0 && g.conv_kw > 0 &&
                        g.K == g.conv_c * g.conv_kh * g.conv_kw && g.conv_hout > 0 && g.conv_wout > 0 &&
                        g.conv_hin > 0 && g.conv_win > 0 && g.M % (g.conv_hout * g.conv_wout) == 0 &&
                        (g.ldb * 2) % 16 == 0 && (uintptr_t)g.A % 16 == 0 && (uintptr_t)g.B % 16 == 0;
        if (!ok || g.K >= (1 << 22)) return hipErrorInvalidValue;
        g.conv_rc = 1.0f / (float)g.conv_c;
        g.conv_rkw = 1.0f / (float)g.conv_kw;
        return go_gemm_lds<A_CONV, B_BF16>(g, epi, st);
    }
    if (asrc == A_F32_SPLIT && bsrc == B_BF16)
        return gemm_lds_ok(g, asrc, bsrc) ? go_gemm_lds<A_F32_SPLIT, B_BF16>(g, epi, st)
                                          : go_gemm<A_F32_SPLIT, B_BF16>(g, epi, st);
    if (asrc == A_BF16 && bsrc == B_I8)
        return gemm_lds_ok(g, asrc, bsrc) ? go_gemm_lds<A_BF16, B_I8>(g, epi, st) : go_gemm<A_BF16, B_I8>(g, epi, st);
    if (asrc == A_BF16 && bsrc == B_BF16) return go_gemm<A_BF16, B_BF16>(g, epi, st);
    return hipErrorInvalidValue;
}

hipError_t launch_gemm_f32(const GemmArgs &g, hipStream_t st) {
    if (g.M <= 0 || g.N <= 0 || g.K <= 0) return hipErrorInvalidValue;
    // 32 x 32 tiles while 64 x 64 ones would leave CUs idle (the mel DFT and
    // filterbank: 94-188 blocks of 64 x 64)
    const int64_t tiles64 = (int64_t)((g.N + 63) / 64) * ((g.M + 63) / 64);
    if (tiles64 < 512) {
        hipLaunchKernelGGL(k_gemm_f32<32>, dim3((g.N + 31) / 32, (g.M + 31) / 32), dim3(256), 0, st, g);
    } else {
        hipLaunchKernelGGL(k_gemm_f32<64>, dim3((g.N + 63) / 64, (g.M + 63) / 64), dim3(256), 0, st, g);
    }
    return hipGetLastError();
}

}  // namespace qasr
