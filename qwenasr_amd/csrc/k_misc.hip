// Row-wise and element-wise kernels of the prefill, the audio encoder and the
// mel front end, plus the multi-row (prefill / encoder-window) attention.
#include <climits>
#include <cstdlib>

#include "kernels.h"

namespace qasr {

// ---------------------------------------------------------------------------
// LayerNorm rows: avx::layer_norm_row (avx.rs:420-481) in its exact order —
// mean over 2x8 lane accumulators, variance with FMA accumulators, both
// through the hsum tree, then fma((x - mean) * inv, w, b) (hidden % 16 == 0,
// so every element takes the 8-wide path).  One single-wave block per row:
// lane l holds the 16-element slots s = l + 64 c in registers, the row goes
// through LDS transposed so that lanes r < 16 run the reference's sequential
// accumulator chains.
// ---------------------------------------------------------------------------
template <int NS>
__global__ __launch_bounds__(64) void k_layer_norm_rows(float *__restrict__ out, const float *__restrict__ x,
                                                        const float *__restrict__ w, const float *__restrict__ b,
                                                        int H, float eps) {
    __shared__ float T[16 * (64 * NS + 1)];   // rows one float apart beyond nslot: conflict-free reads
    const int lane = threadIdx.x;
    const int64_t row = blockIdx.x;
    const float *xr = x + row * H;
    float *o = out + row * H;
    const int nslot = H >> 4, ts = nslot + 1;
    float4 xv[NS][4];
#pragma unroll
    for (int c = 0; c < NS; c++) {
        const int sl = lane + 64 * c, se = sl < nslot ? sl : 0;
#pragma unroll
        for (int i = 0; i < 4; i++) xv[c][i] = reinterpret_cast<const float4 *>(xr + 16 * se)[i];
    }
#pragma unroll
    for (int c = 0; c < NS; c++) {
        const int sl = lane + 64 * c;
        if (sl < nslot) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                T[(4 * i) * ts + sl] = xv[c][i].x;
                T[(4 * i + 1) * ts + sl] = xv[c][i].y;
                T[(4 * i + 2) * ts + sl] = xv[c][i].z;
                T[(4 * i + 3) * ts + sl] = xv[c][i].w;
            }
        }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    const float *t = T + (lane < 16 ? lane : 0) * ts;
    float acc = 0.0f;
    if (lane < 16)
        for (int i = 0; i < nslot; i++) acc = __fadd_rn(acc, t[i]);
    const float mean = div_by_count(avx16_tree(acc), H);
    acc = 0.0f;
    if (lane < 16)
        for (int i = 0; i < nslot; i++) {
            const float d = __fsub_rn(t[i], mean);
            acc = fmaf(d, d, acc);
        }
    const float var = avx16_tree(acc);
    const float inv = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(div_by_count(var, H), eps)));
#pragma unroll
    for (int c = 0; c < NS; c++) {
        const int sl = lane + 64 * c;
        if (sl < nslot) {
            float4 *op = reinterpret_cast<float4 *>(o + 16 * sl);
            const float4 *wp = reinterpret_cast<const float4 *>(w + 16 * sl);
            const float4 *bp = reinterpret_cast<const float4 *>(b + 16 * sl);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 a = xv[c][i], ww = wp[i], bb = bp[i];
                op[i] = make_float4(fmaf(__fmul_rn(__fsub_rn(a.x, mean), inv), ww.x, bb.x),
                                    fmaf(__fmul_rn(__fsub_rn(a.y, mean), inv), ww.y, bb.y),
                                    fmaf(__fmul_rn(__fsub_rn(a.z, mean), inv), ww.z, bb.z),
                                    fmaf(__fmul_rn(__fsub_rn(a.w, mean), inv), ww.w, bb.w));
            }
        }
    }
}

hipError_t launch_layer_norm_rows(float *out, const float *x, const float *w, const float *b, int64_t seq,
                                  int hidden, float eps, hipStream_t st) {
    if (hidden % 16 != 0 || hidden > 4096 || seq <= 0) return hipErrorInvalidValue;
    const dim3 grid((unsigned)seq);
    switch ((hidden + 1023) / 1024) {
        case 1: hipLaunchKernelGGL(k_layer_norm_rows<1>, grid, dim3(64), 0, st, out, x, w, b, hidden, eps); break;
        case 2: hipLaunchKernelGGL(k_layer_norm_rows<2>, grid, dim3(64), 0, st, out, x, w, b, hidden, eps); break;
        case 3: hipLaunchKernelGGL(k_layer_norm_rows<3>, grid, dim3(64), 0, st, out, x, w, b, hidden, eps); break;
        default: hipLaunchKernelGGL(k_layer_norm_rows<4>, grid, dim3(64), 0, st, out, x, w, b, hidden, eps); break;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// SwiGLU over rows of interleaved gate/up (swiglu_multiply, mod.rs:1291-1341 ->
// avx::swiglu_interleaved, avx.rs:568-599): fast_exp on 8-wide blocks, libm
// expf on the tail.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_swiglu_rows(float *__restrict__ out, const float *__restrict__ gu,
                                                     int64_t seq, int inter) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= seq * inter) return;
    const int64_t s = i / inter;
    const int j = (int)(i % inter);
    const float g = gu[s * 2 * inter + 2 * j], u = gu[s * 2 * inter + 2 * j + 1];
    const int nv = inter - inter % 8;
    const float e = j < nv ? fast_exp_ref(__fsub_rn(0.0f, g)) : expf(-g);
    out[i] = __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, e)), u);
}

hipError_t launch_swiglu_rows(float *out, const float *gu, int64_t seq, int inter, hipStream_t st) {
    const int64_t n = seq * inter;
    hipLaunchKernelGGL(k_swiglu_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, out, gu, seq, inter);
    return hipGetLastError();
}

// gelu in place over a buffer of n elements (gelu, mod.rs:1250-1289)
__global__ __launch_bounds__(256) void k_gelu(float *__restrict__ x, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = gelu_ref(x[i], i, n);
}

hipError_t launch_gelu(float *x, int64_t n, hipStream_t st) {
    hipLaunchKernelGGL(k_gelu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n);
    return hipGetLastError();
}

// y[r][c] += table[r % period][c]  (add_inplace of the per-chunk sinusoidal PE)
__global__ __launch_bounds__(256) void k_add_periodic(float *__restrict__ y, const float *__restrict__ table,
                                                      int64_t rows, int cols, int period) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * cols) return;
    const int64_t r = i / cols;
    const int c = (int)(i % cols);
    y[i] = __fadd_rn(y[i], table[(r % period) * cols + c]);
}

hipError_t launch_add_periodic(float *y, const float *table, int64_t rows, int cols, int period, hipStream_t st) {
    const int64_t n = rows * cols;
    hipLaunchKernelGGL(k_add_periodic, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, y, table, rows, cols, period);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// im2col for a batch of independent 3x3 / stride-2 / pad-1 convolutions
// (conv2d, mod.rs:1077-1154), transposed: cols[(c * Ho + oh) * Wo + ow][p] with
// p = (ic * 3 + ki) * 3 + kj.  Input element (c, ic, ih, iw) lives at
//   in + c * cs + ic * chs + ih * rs + iw.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_im2col3x3s2(float *__restrict__ cols, const float *__restrict__ in,
                                                     int n_chunks, int C, int H, int W, int64_t cs, int64_t chs,
                                                     int64_t rs, int Ho, int Wo) {
    const int P = C * 9;
    const int64_t total = (int64_t)n_chunks * Ho * Wo * P;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int p = (int)(i % P);
        const int64_t row = i / P;
        const int ow = (int)(row % Wo);
        const int oh = (int)((row / Wo) % Ho);
        const int c = (int)(row / ((int64_t)Wo * Ho));
        const int ic = p / 9, ki = (p % 9) / 3, kj = p % 3;
        const int ih = oh * 2 + ki - 1, iw = ow * 2 + kj - 1;
        float v = 0.0f;
        if (ih >= 0 && ih < H && iw >= 0 && iw < W) v = in[c * cs + ic * chs + (int64_t)ih * rs + iw];
        cols[i] = v;
    }
}

// the same patches with one block per output position (row) and the threads
// over its C * 9 columns: the position is decoded once per block and the
// column index needs only 32-bit divisions by constants
__global__ __launch_bounds__(256) void k_im2col3x3s2_rows(float *__restrict__ cols, const float *__restrict__ in,
                                                          int C, int H, int W, int64_t cs, int64_t chs, int64_t rs,
                                                          int Ho, int Wo) {
    const int P = C * 9;
    const int row = blockIdx.x;
    const int ow = row % Wo, oh = (row / Wo) % Ho, c = row / (Wo * Ho);
    const float *src = in + c * cs;
    float *dst = cols + (int64_t)row * P;
    for (int p = threadIdx.x; p < P; p += 256) {
        const int ic = p / 9, r9 = p - 9 * ic, ki = r9 / 3, kj = r9 - 3 * ki;
        const int ih = oh * 2 + ki - 1, iw = ow * 2 + kj - 1;
        float v = 0.0f;
        if (ih >= 0 && ih < H && iw >= 0 && iw < W) v = src[ic * chs + (int64_t)ih * rs + iw];
        dst[p] = v;
    }
}

// the same patches by output row strips: a block owns the Wo positions of one
// output row (chunk c, row oh) and walks the channels 32 at a time, staging
// the three input rows 2 oh - 1 .. 2 oh + 1 of those channels in LDS (zero
// columns on both sides, zero rows outside the image), so the input is read
// in contiguous rows once per strip instead of 3-float runs per position, and
// each position's 288 columns of the channel group go out as one contiguous run
constexpr int IM2COL_ICB = 32, IM2COL_XW = 128;
__global__ __launch_bounds__(256) void k_im2col3x3s2_strip(float *__restrict__ cols, const float *__restrict__ in,
                                                           int C, int H, int W, int64_t cs, int64_t chs, int64_t rs,
                                                           int Ho, int Wo) {
    // rows padded to an odd length so that the 9 taps of consecutive columns
    // fall in different LDS banks
    __shared__ float T[IM2COL_ICB][3][IM2COL_XW + 1];
    const int P = C * 9;
    const int c = blockIdx.x / Ho, oh = blockIdx.x % Ho;
    const float *src = in + c * cs;
    float *dst = cols + (int64_t)blockIdx.x * Wo * P;
    const int XW = W + 2;
    // the Wo x nq columns of one channel group; nq is a constant for full groups
    auto emit = [&](int icb, int nq) {
        for (int i = threadIdx.x; i < Wo * nq; i += 256) {
            const int ow = i / nq, q = i - ow * nq;
            const int icl = q / 9, r9 = q - 9 * icl, ki = r9 / 3, kj = r9 - 3 * ki;
            dst[(int64_t)ow * P + icb * 9 + q] = T[icl][ki][2 * ow + kj];
        }
    };
    // grid y splits the channel groups, so that short strips still fill the chip
    const int ngrp = (C + IM2COL_ICB - 1) / IM2COL_ICB, gpy = (ngrp + gridDim.y - 1) / gridDim.y;
    const int ic_end = min(C, (int)(blockIdx.y + 1) * gpy * IM2COL_ICB);
    for (int icb = blockIdx.y * gpy * IM2COL_ICB; icb < ic_end; icb += IM2COL_ICB) {
        const int nb = min(IM2COL_ICB, C - icb);
        __syncthreads();
        // eight loads in flight per thread before their LDS stores
        const int n = nb * 3 * XW;
        for (int i0 = threadIdx.x; i0 < n; i0 += 8 * 256) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = i0 + u * 256, ie = i < n ? i : 0;
                const int x = ie % XW, r = ie / XW, ki = r % 3, icl = r / 3;
                const int ih = 2 * oh + ki - 1, iw = x - 1;
                const bool ok = i < n && ih >= 0 && ih < H && iw >= 0 && iw < W;
                v[u] = src[ok ? (int64_t)(icb + icl) * chs + (int64_t)ih * rs + iw : 0];
                v[u] = ok ? v[u] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = i0 + u * 256;
                if (i < n) {
                    const int x = i % XW, r = i / XW;
                    T[r / 3][r % 3][x] = v[u];
                }
            }
        }
        __syncthreads();
        if (nb == IM2COL_ICB) emit(icb, IM2COL_ICB * 9);
        else emit(icb, nb * 9);
    }
}

hipError_t launch_im2col3x3s2(float *cols, const float *in, int n_chunks, int C, int H, int W, int64_t cs,
                              int64_t chs, int64_t rs, int Ho, int Wo, hipStream_t st) {
    const int64_t rows = (int64_t)n_chunks * Ho * Wo;
    if (C * 9 >= 256 && W + 2 <= IM2COL_XW && Wo == (W - 1) / 2 + 1 && (int64_t)n_chunks * Ho < (1ll << 31)) {
        // about 4096 blocks: strips x channel splits
        const int strips = n_chunks * Ho, ngrp = (C + IM2COL_ICB - 1) / IM2COL_ICB;
        const int cs_split = std::max(1, std::min(ngrp, (4096 + strips - 1) / strips));
        hipLaunchKernelGGL(k_im2col3x3s2_strip, dim3((unsigned)strips, (unsigned)cs_split), dim3(256), 0, st, cols, in, C,
                           H, W, cs, chs, rs, Ho, Wo);
        return hipGetLastError();
    }
    if (C * 9 >= 256 && rows < (1ll << 31)) {
        hipLaunchKernelGGL(k_im2col3x3s2_rows, dim3((unsigned)rows), dim3(256), 0, st, cols, in, C, H, W, cs, chs, rs,
                           Ho, Wo);
        return hipGetLastError();
    }
    const int64_t total = (int64_t)n_chunks * Ho * Wo * C * 9;
    const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL(k_im2col3x3s2, dim3(blocks), dim3(256), 0, st, cols, in, n_chunks, C, H, W, cs, chs, rs,
                       Ho, Wo);
    return hipGetLastError();
}

// First convolution of the stem (one input channel, 3x3, stride 2, pad 1) +
// bias + GELU computed directly (conv2d, mod.rs:1077-1154, then gelu): a
// block stages one chunk's padded input plane in LDS and produces CONV1_OCB
// output channels of it: a thread holds one position's 9 taps in registers
// and walks the block's channels.  Each output is the f32 FMA chain over the
// taps in im2col column order (ki, kj), plus the bias, then gelu at its index
// in the chunk's [C][Ho][Wo] output (the path choice of gelu_ref, hoisted per
// channel by GeluSpan).  Outputs go to out + c * C * Ho * Wo.
constexpr int CONV1_OCB = 16, CONV1_LDS = 13312;
__global__ __launch_bounds__(256) void k_conv1_direct(float *__restrict__ out, const float *__restrict__ in,
                                                      int64_t cs, int64_t rs, int H, int W,
                                                      const uint16_t *__restrict__ w, const float *__restrict__ bias,
                                                      int C, int Ho, int Wo, int nhwc) {
    __shared__ float X[CONV1_LDS];
    const int c = blockIdx.x, XW = W + 2;
    const float *src = in + c * cs;
    for (int i = threadIdx.x; i < (H + 2) * XW; i += 256) {
        const int r = i / XW, x = i - r * XW, ih = r - 1, iw = x - 1;
        X[i] = (ih >= 0 && ih < H && iw >= 0 && iw < W) ? src[(int64_t)ih * rs + iw] : 0.0f;
    }
    __syncthreads();
    const int plane = Ho * Wo;
    const int64_t n = (int64_t)C * plane;
    float *dst = out + (int64_t)c * n;
    // this block's channels: weights and gelu path choices (plane <= n / 16, C >= 16)
    const int oc0 = blockIdx.y * CONV1_OCB, noc = min(CONV1_OCB, C - oc0);
    __shared__ float wsh[CONV1_OCB][10];
    __shared__ int64_t gsh[CONV1_OCB][3];
    if (threadIdx.x < noc * 9) {
        const int o = threadIdx.x / 9, k = threadIdx.x % 9;
        wsh[o][k] = bf16_to_f32(w[(oc0 + o) * 9 + k]);
    } else if (threadIdx.x >= 160 && threadIdx.x < 160 + noc) {
        const int o = threadIdx.x - 160;
        const GeluSpan gs((int64_t)(oc0 + o) * plane, n);
        wsh[o][9] = bias[oc0 + o];
        gsh[o][0] = gs.b1; gsh[o][1] = gs.ts0; gsh[o][2] = gs.ts1;
    }
    __syncthreads();
    // each thread: one position's 9 taps in registers, then every channel of the block
    for (int sp = threadIdx.x; sp < plane; sp += 256) {
        const int oh = sp / Wo, ow = sp - oh * Wo;
        const float *xp = X + 2 * oh * XW + 2 * ow;
        float xv[9];
#pragma unroll
        for (int ki = 0; ki < 3; ki++)
#pragma unroll
            for (int kj = 0; kj < 3; kj++) xv[ki * 3 + kj] = xp[ki * XW + kj];
        auto value = [&](int o) {
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < 9; k++) acc = fmaf(xv[k], wsh[o][k], acc);
            const int64_t gi = (int64_t)(oc0 + o) * plane + sp;      // the reference's (channel-major) index
            const bool vec = gi < gsh[o][0] ? gi < gsh[o][1] : gi < gsh[o][2];
            return gelu_at(__fadd_rn(acc, wsh[o][9]), vec);
        };
        if (nhwc) {
            // channels last: this position's channels oc0 .. oc0 + noc - 1 are
            // one contiguous run (float4 stores; C and oc0 are multiples of 4)
            float *row = dst + (int64_t)sp * C + oc0;
            for (int o = 0; o < noc; o += 4)
                *reinterpret_cast<float4 *>(row + o) = make_float4(value(o), value(o + 1), value(o + 2), value(o + 3));
        } else {
            for (int o = 0; o < noc; o++) dst[(int64_t)(oc0 + o) * plane + sp] = value(o);
        }
    }
}

hipError_t launch_conv1_direct(float *out, const float *in, int n_chunks, int64_t cs, int64_t rs, int H, int W,
                               const uint16_t *w, const float *bias, int C, int Ho, int Wo, bool nhwc,
                               hipStream_t st) {
    if ((H + 2) * (W + 2) > CONV1_LDS || Ho != (H - 1) / 2 + 1 || Wo != (W - 1) / 2 + 1 || n_chunks <= 0 || C < 16)
        return hipErrorInvalidValue;
    if (nhwc && (C % 4 != 0 || (uintptr_t)out % 16 != 0)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)n_chunks, (unsigned)((C + CONV1_OCB - 1) / CONV1_OCB));
    hipLaunchKernelGGL(k_conv1_direct, grid, dim3(256), 0, st, out, in, cs, rs, H, W, w, bias, C, Ho, Wo,
                       nhwc ? 1 : 0);
    return hipGetLastError();
}

// w[o][c][t] -> out[o][t][c] (bf16): a convolution's weights with the K index
// (channel, tap) reordered to (tap, channel), the order of the channels-last
// implicit-im2col GEMM
__global__ __launch_bounds__(256) void k_taps_last(uint16_t *__restrict__ out, const uint16_t *__restrict__ in,
                                                   int O, int Cin, int T) {
    const int64_t total = (int64_t)O * Cin * T;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int c = (int)(i % Cin);
        const int64_t r = i / Cin;
        const int t = (int)(r % T);
        const int64_t o = r / T;
        out[i] = in[(o * Cin + c) * T + t];
    }
}

hipError_t launch_taps_last(uint16_t *out, const uint16_t *in, int O, int Cin, int T, hipStream_t st) {
    if (O <= 0 || Cin <= 0 || T <= 0) return hipErrorInvalidValue;
    const int64_t total = (int64_t)O * Cin * T;
    const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL(k_taps_last, dim3(blocks), dim3(256), 0, st, out, in, O, Cin, T);
    return hipGetLastError();
}

// [chunk][C][F][T] -> [chunk * T][C * F] with column ch * F + f (encoder.rs:265-277)
__global__ __launch_bounds__(256) void k_conv_reshape(float *__restrict__ out, const float *__restrict__ in,
                                                      int n_chunks, int C, int F, int T) {
    const int64_t total = (int64_t)n_chunks * C * F * T;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int col = (int)(i % (C * F));
        const int64_t row = i / (C * F);
        const int t = (int)(row % T);
        const int c = (int)(row / T);
        const int ch = col / F, f = col % F;
        out[i] = in[(((int64_t)c * C + ch) * F + f) * T + t];
    }
}

hipError_t launch_conv_reshape(float *out, const float *in, int n_chunks, int C, int F, int T, hipStream_t st) {
    const int64_t total = (int64_t)n_chunks * C * F * T;
    const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL(k_conv_reshape, dim3(blocks), dim3(256), 0, st, out, in, n_chunks, C, F, T);
    return hipGetLastError();
}

// prompt rows: row r < n_tok_head: embed[tok[r]]; then n_mid rows copied from
// mid; then the remaining token rows (transcribe.rs:106-169)
__global__ __launch_bounds__(256) void k_build_prompt(float *__restrict__ out, const uint16_t *__restrict__ embed,
                                                      const int *__restrict__ toks, int n_head, const float *mid,
                                                      int n_mid, int n_tail, int H) {
    const int r = blockIdx.x;
    float *o = out + (int64_t)r * H;
    if (r < n_head || r >= n_head + n_mid) {
        const int ti = r < n_head ? r : r - n_mid;
        const uint16_t *e = embed + (int64_t)toks[ti] * H;
        for (int i = threadIdx.x; i < H; i += 256) o[i] = bf16_to_f32(e[i]);
    } else {
        const float *m = mid + (int64_t)(r - n_head) * H;
        for (int i = threadIdx.x; i < H; i += 256) o[i] = m[i];
    }
    (void)n_tail;
}

// flags[r] = 1 when rows r of a and b differ in any bit (the row-equality test
// of the streaming prefill's prefix reuse, transcribe.rs:1095-1104)
__global__ __launch_bounds__(256) void k_row_diff(const float *__restrict__ a, const float *__restrict__ b,
                                                  int64_t H, int *__restrict__ flags) {
    __shared__ int any;
    const int64_t r = blockIdx.x;
    if (threadIdx.x == 0) any = 0;
    __syncthreads();
    const uint32_t *pa = reinterpret_cast<const uint32_t *>(a + r * H), *pb = reinterpret_cast<const uint32_t *>(b + r * H);
    int d = 0;
    for (int64_t i = threadIdx.x; i < H; i += 256) d |= pa[i] != pb[i];
    if (d) any = 1;
    __syncthreads();
    if (threadIdx.x == 0) flags[r] = any;
}

hipError_t launch_row_diff(const float *a, const float *b, int64_t rows, int64_t H, int *flags, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_row_diff, dim3((unsigned)rows), dim3(256), 0, st, a, b, H, flags);
    return hipGetLastError();
}

// idx[r] = the aligner's per-row argmax of x[r] (align.rs:312-321): a left
// scan that starts at column 0 and moves on only for a strictly greater value,
// i.e. the lowest column holding the maximum of the non-NaN values, and 0 when
// column 0 is NaN (nothing compares greater than it).  A lane scans a strided
// column set in increasing order; pairs merge by value, then lowest column.
__device__ inline void argmax_pick(float &v, int &i, float ov, int oi) {
    if (oi == INT_MAX) return;
    if (i == INT_MAX || ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}

__global__ __launch_bounds__(256) void k_argmax_f32_rows(const float *__restrict__ x, int64_t ld, int64_t cols,
                                                         int32_t *__restrict__ idx) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const float *row = x + blockIdx.x * ld;
    float v = 0.0f;
    int i = INT_MAX;
    for (int64_t c = threadIdx.x; c < cols; c += 256) {
        const float y = row[c];
        if (y == y && (i == INT_MAX || y > v)) { v = y; i = (int)c; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) argmax_pick(v, i, __shfl_xor(v, o), __shfl_xor(i, o));
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sv[w] = v; si[w] = i; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 4; k++) argmax_pick(v, i, sv[k], si[k]);
        const float c0 = row[0];
        idx[blockIdx.x] = (c0 != c0 || i == INT_MAX) ? 0 : i;
    }
}

hipError_t launch_argmax_f32_rows(const float *x, int64_t ld, int64_t rows, int64_t cols, int32_t *idx,
                                  hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_argmax_f32_rows, dim3((unsigned)rows), dim3(256), 0, st, x, ld, cols, idx);
    return hipGetLastError();
}

// dst[k] = src[rows[k]] for k < n, rows of H floats
__global__ __launch_bounds__(256) void k_gather_rows(float *__restrict__ dst, const float *__restrict__ src,
                                                     const int32_t *__restrict__ rows, int64_t H) {
    const float *s = src + (int64_t)rows[blockIdx.x] * H;
    float *d = dst + (int64_t)blockIdx.x * H;
    for (int64_t c = threadIdx.x; c < H; c += 256) d[c] = s[c];
}

hipError_t launch_gather_rows(float *dst, const float *src, const int32_t *rows, int64_t n, int64_t H,
                              hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_gather_rows, dim3((unsigned)n), dim3(256), 0, st, dst, src, rows, H);
    return hipGetLastError();
}

hipError_t launch_build_prompt(float *out, const uint16_t *embed, const int *toks, int n_head, const float *mid,
                               int n_mid, int n_tail, int H, hipStream_t st) {
    hipLaunchKernelGGL(k_build_prompt, dim3(n_head + n_mid + n_tail), dim3(256), 0, st, out, embed, toks, n_head,
                       mid, n_mid, n_tail, H);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Multi-row attention (flash-style online softmax, f32):
//   decoder prefill: causal over the KV cache, GQA (causal_attention with
//                    seq_q > 1, mod.rs:1539-1607)
//   encoder:         full attention inside fixed windows (bidirectional_attention,
//                    mod.rs:1386-1471)
// A block owns 32 query rows (QT queries x G heads of one KV head) and walks key
// tiles of 32; 8 threads per row.
// ---------------------------------------------------------------------------
// The rows [s0, s1) of the sequence that row q belongs to: the whole call, or
// with n_seg > 0 the last sequence starting at or before q (compile-time
// indices only, so the tables stay in the kernel arguments)
__device__ __forceinline__ void attn_sequence(const AttnRowsArgs &a, int q, int &s0, int &s1) {
    s0 = 0;
    s1 = min(a.n_q, a.n_k);
    if (a.n_seg > 0) {
#pragma unroll
        for (int j = 0; j < QASR_ATTN_MAX_SEG; j++)
            if (j < a.n_seg && a.seg_lo[j] <= q) {
                s0 = a.seg_lo[j];
                s1 = a.seg_hi[j];
            }
    }
}

template <int HD>
__global__ __launch_bounds__(256) void k_attn_rows(AttnRowsArgs a) {
    constexpr int R = 32, KT = 32, DP = HD / 8;
    __shared__ float Qs[R][HD + 4];
    __shared__ float Ks[KT][HD + 4];
    __shared__ float Vs[KT][HD + 4];
    __shared__ float Ps[R][KT + 1];
    const int t = threadIdx.x, r = t >> 3, sub = t & 7;
    const int G = a.G, QT = R / G;
    const int kvh = blockIdx.x, q0 = blockIdx.y * QT;
    const int qi = q0 + r / G, h = kvh * G + r % G;
    // the block's sequence (windowed calls; blocks never straddle two)
    int s0 = 0, s1 = a.n_q;
    if (a.window > 0) attn_sequence(a, q0, s0, s1);
    const bool row_ok = qi < a.n_q && qi < s1;
    // key range of this row
    int lo = 0, hi;
    if (a.window > 0) {
        lo = s0 + ((qi - s0) / a.window) * a.window;
        hi = min(lo + a.window, min(a.n_k, s1));
    } else {
        hi = min(a.q_offset + qi + 1, a.n_k);
    }
    if (!row_ok) { lo = 0; hi = 0; }
    // key range of the block
    const int qlast = min(q0 + QT, min(a.n_q, s1)) - 1;
    int blo, bhi;
    if (a.window > 0) {
        blo = s0 + ((q0 - s0) / a.window) * a.window;
        bhi = min(s0 + ((qlast - s0) / a.window) * a.window + a.window, min(a.n_k, s1));
    } else {
        blo = 0;
        bhi = min(a.q_offset + qlast + 1, a.n_k);
    }
    for (int i = t; i < R * HD; i += 256) {
        const int rr = i / HD, d = i % HD;
        const int qq = q0 + rr / G, hh = kvh * G + rr % G;
        Qs[rr][d] = qq < a.n_q ? a.q[(int64_t)qq * a.q_rs + hh * HD + d] : 0.0f;
    }
    float m = -INFINITY, l = 0.0f, o[DP];
#pragma unroll
    for (int i = 0; i < DP; i++) o[i] = 0.0f;
    const float *kb = a.k + (int64_t)kvh * a.k_hs, *vb = a.v + (int64_t)kvh * a.k_hs;
    for (int j0 = blo; j0 < bhi; j0 += KT) {
        __syncthreads();
        for (int i = t; i < KT * HD; i += 256) {
            const int kk = i / HD, d = i % HD;
            const int j = j0 + kk;
            const bool ok = j < bhi;
            const int64_t off = (int64_t)(ok ? j : j0) * a.k_rs + d;
            const float kv = kb[off], vv = vb[off];
            Ks[kk][d] = ok ? kv : 0.0f;
            Vs[kk][d] = ok ? vv : 0.0f;
        }
        __syncthreads();
        float s[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int kk = sub * 4 + c;
            float acc = 0.0f;
#pragma unroll 8
            for (int d = 0; d < HD; d++) acc = fmaf(Qs[r][d], Ks[kk][d], acc);
            const int j = j0 + kk;
            s[c] = (j >= lo && j < hi) ? __fmul_rn(acc, a.scale) : -INFINITY;
        }
        float tm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        tm = fmaxf(tm, __shfl_xor(tm, 1, 64));
        tm = fmaxf(tm, __shfl_xor(tm, 2, 64));
        tm = fmaxf(tm, __shfl_xor(tm, 4, 64));
        const float mn = fmaxf(m, tm);
        float corr = 1.0f, ps = 0.0f;
        if (mn != -INFINITY) {
            corr = m == -INFINITY ? 0.0f : expf(__fsub_rn(m, mn));
#pragma unroll
            for (int c = 0; c < 4; c++) {
                s[c] = s[c] == -INFINITY ? 0.0f : expf(__fsub_rn(s[c], mn));
                ps = __fadd_rn(ps, s[c]);
            }
        } else {
#pragma unroll
            for (int c = 0; c < 4; c++) s[c] = 0.0f;
        }
        ps = __fadd_rn(ps, __shfl_xor(ps, 1, 64));
        ps = __fadd_rn(ps, __shfl_xor(ps, 2, 64));
        ps = __fadd_rn(ps, __shfl_xor(ps, 4, 64));
        l = fmaf(l, corr, ps);
        m = mn;
#pragma unroll
        for (int c = 0; c < 4; c++) Ps[r][sub * 4 + c] = s[c];
        __syncthreads();
#pragma unroll
        for (int i = 0; i < DP; i++) o[i] = __fmul_rn(o[i], corr);
        for (int kk = 0; kk < KT; kk++) {
            const float p = Ps[r][kk];
#pragma unroll
            for (int i = 0; i < DP; i++) o[i] = fmaf(p, Vs[kk][sub * DP + i], o[i]);
        }
    }
    if (row_ok) {
        float *op = a.out + (int64_t)qi * a.o_rs + h * HD + sub * DP;
        const float inv = l > 0.0f ? __fdiv_rn(1.0f, l) : 0.0f;
#pragma unroll
        for (int i = 0; i < DP; i++) op[i] = __fmul_rn(o[i], inv);
    }
}

// ---------------------------------------------------------------------------
// The same multi-row attention on f32 MFMA (v_mfma_f32_16x16x4_f32, exact f32
// products, f32 accumulation).  A block owns 16 query rows of the G query
// heads of one KV head; its NW waves are (head g, key split ks), G x KS = NW,
// and wave (g, ks) takes the 16-key sub-tiles ks, ks + KS, ... of every
// KS x 16-key chunk staged in LDS, with an online softmax of its own; the KS
// states of a head are merged through LDS at the end.  The next chunk's K/V
// loads go out into registers before the current chunk's MFMA work.  With
// kv_div = 2 (and G = 1) a block owns one query head x and reads KV head x / 2,
// which gives the 8 waves of a 128-dim head 8 key splits.  Per sub-tile the wave
// forms S^T = K Q^T (16 keys x 16 queries; lane l holds keys 4 (l / 16) + i
// of query l % 16, the dot over d split as lane group l / 16 covering dims
// [l/16 HD/4, +HD/4)), so the softmax of a query reduces over the lane's 4
// values and two cross-group shuffles, and the probabilities already sit in
// the A-operand layout of O += P V (query l % 16, key 4 (l / 16) + i at step
// i).  The O rows a lane accumulates are queries 4 (l / 16) + j, whose
// rescale factors come from the lanes owning those queries.
// ---------------------------------------------------------------------------
// One block's work: query rows [q0, q0 + 16) of the KV head (pair) blockIdx.x.
template <int HD, int G, int NW>
__device__ __forceinline__ void attn_mfma_block(const AttnRowsArgs &a, int q0) {
    constexpr int KS = NW / G, CH = 16 * KS, NST = HD / 4, NT = HD / 16, LD = HD + 4;
    constexpr int NTH = NW * 64, SV = CH * (HD / 4) / NTH;   // float4 of K (and of V) staged per thread
    static_assert(CH * (HD / 4) % NTH == 0, "staging");
    // one LDS buffer: K and V chunks [CH][LD] during the loop, the waves' O rows after it
    static_assert(2 * CH * LD >= NW * 16 * HD, "merge buffer");
    __shared__ __attribute__((aligned(16))) float smem[2 * CH * LD];
    float (*Ks)[LD] = reinterpret_cast<float (*)[LD]>(smem);
    float (*Vs)[LD] = reinterpret_cast<float (*)[LD]>(smem + CH * LD);
    const int t = threadIdx.x, lane = t & 63;
    const int wid = __builtin_amdgcn_readfirstlane(t >> 6);
    const int g = wid / KS, ks = wid % KS;
    const int kvh = blockIdx.x;
    const int h = kvh * G + g;
    const int lq = lane & 15, lg = lane >> 4;
    // key range of this lane's query (for the S^T masks) and of the block
    const int qi = q0 + lq;
    // the block's sequence (windowed calls; blocks never straddle two)
    int s0 = 0, s1 = a.n_q;
    if (a.window > 0) attn_sequence(a, q0, s0, s1);
    int lo = 0, hi = 0;
    if (qi < a.n_q && qi < s1) {
        if (a.window > 0) {
            lo = s0 + ((qi - s0) / a.window) * a.window;
            hi = min(lo + a.window, min(a.n_k, s1));
        } else {
            hi = min(a.q_offset + qi + 1, a.n_k);
        }
    }
    const int qlast = min(q0 + 16, min(a.n_q, s1)) - 1;
    if (qlast < q0) return;                 // padding rows between two sequences
    int blo, bhi;
    if (a.window > 0) {
        blo = s0 + ((q0 - s0) / a.window) * a.window;
        bhi = min(s0 + ((qlast - s0) / a.window) * a.window + a.window, min(a.n_k, s1));
    } else {
        blo = 0;
        bhi = min(a.q_offset + qlast + 1, a.n_k);
    }
    // this lane's slice of q: dims [lg NST, lg NST + NST) of query qi, head h
    float qv[NST];
    {
        const float *qp = a.q + (int64_t)min(qi, a.n_q - 1) * a.q_rs + h * HD + lg * NST;
#pragma unroll
        for (int s = 0; s < NST; s += 4) {
            const float4 x = *reinterpret_cast<const float4 *>(qp + s);
            qv[s] = x.x; qv[s + 1] = x.y; qv[s + 2] = x.z; qv[s + 3] = x.w;
        }
    }
    f32x4 o[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) o[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;
    const int kv_head = a.kv_div > 1 ? kvh / a.kv_div : kvh;
    const float *kb = a.k + (int64_t)kv_head * a.k_hs, *vb = a.v + (int64_t)kv_head * a.k_hs;
    // K/V of a chunk pass through registers: the loads of chunk c0 + CH are
    // issued before the MFMA work on chunk c0, so their latency overlaps it.
    // Rows past the range repeat row blo (their scores are masked).
    f32x4 kx[SV], vx[SV];
#pragma unroll
    for (int u = 0; u < SV; u++) {
        const int i = t + u * NTH, kk = i / (HD / 4), d4 = (i % (HD / 4)) * 4;
        const int j = blo + kk < bhi ? blo + kk : blo;
        kx[u] = *reinterpret_cast<const f32x4 *>(kb + (int64_t)j * a.k_rs + d4);
        vx[u] = *reinterpret_cast<const f32x4 *>(vb + (int64_t)j * a.k_rs + d4);
    }
    for (int c0 = blo; c0 < bhi; c0 += CH) {
        __syncthreads();
        // stage keys [c0, c0 + CH)
#pragma unroll
        for (int u = 0; u < SV; u++) {
            const int i = t + u * NTH, kk = i / (HD / 4), d4 = (i % (HD / 4)) * 4;
            *reinterpret_cast<f32x4 *>(&Ks[kk][d4]) = kx[u];
            *reinterpret_cast<f32x4 *>(&Vs[kk][d4]) = vx[u];
        }
        __syncthreads();
        // next chunk (past the last one: rows blo again, unused)
#pragma unroll
        for (int u = 0; u < SV; u++) {
            const int i = t + u * NTH, kk = i / (HD / 4), d4 = (i % (HD / 4)) * 4;
            const int j = c0 + CH + kk < bhi ? c0 + CH + kk : blo;
            kx[u] = *reinterpret_cast<const f32x4 *>(kb + (int64_t)j * a.k_rs + d4);
            vx[u] = *reinterpret_cast<const f32x4 *>(vb + (int64_t)j * a.k_rs + d4);
        }
        const int kt = 16 * ks;                 // this wave's sub-tile of the chunk
        if (c0 + kt >= bhi) continue;
        // S^T[key kt + 4 lg + i][query lq]
        f32x4 st = {0.0f, 0.0f, 0.0f, 0.0f};
        const float *kr = &Ks[kt + lq][lg * NST];
#pragma unroll
        for (int s = 0; s < NST; s += 4) {
            const float4 kx = *reinterpret_cast<const float4 *>(kr + s);
            st = __builtin_amdgcn_mfma_f32_16x16x4f32(kx.x, qv[s], st, 0, 0, 0);
            st = __builtin_amdgcn_mfma_f32_16x16x4f32(kx.y, qv[s + 1], st, 0, 0, 0);
            st = __builtin_amdgcn_mfma_f32_16x16x4f32(kx.z, qv[s + 2], st, 0, 0, 0);
            st = __builtin_amdgcn_mfma_f32_16x16x4f32(kx.w, qv[s + 3], st, 0, 0, 0);
        }
        float sv[4], tm = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int j = c0 + kt + 4 * lg + i;
            sv[i] = (j >= lo && j < hi) ? __fmul_rn(st[i], a.scale) : -INFINITY;
            tm = fmaxf(tm, sv[i]);
        }
        tm = fmaxf(tm, __shfl_xor(tm, 16, 64));
        tm = fmaxf(tm, __shfl_xor(tm, 32, 64));
        const float mn = fmaxf(m, tm);
        const float corr = (m == -INFINITY) ? 0.0f : expf(__fsub_rn(m, mn));
        float ps = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            sv[i] = sv[i] == -INFINITY ? 0.0f : expf(__fsub_rn(sv[i], mn));
        }
        ps = __fadd_rn(__fadd_rn(sv[0], sv[1]), __fadd_rn(sv[2], sv[3]));
        ps = __fadd_rn(ps, __shfl_xor(ps, 16, 64));
        ps = __fadd_rn(ps, __shfl_xor(ps, 32, 64));
        l = fmaf(l, corr, ps);
        m = mn;
        // rescale the O rows this lane holds (queries 4 lg + j) by their owners' factors
        float cj[4];
#pragma unroll
        for (int j = 0; j < 4; j++) cj[j] = __shfl(corr, 4 * lg + j, 64);
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
            for (int j = 0; j < 4; j++) o[n][j] = __fmul_rn(o[n][j], cj[j]);
        // O += P V: step i pairs key kt + 4 lg + i of P (this lane's sv[i]) with V row kt + 4 lg + i
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float *vr = &Vs[kt + 4 * lg + i][lq];
#pragma unroll
            for (int n = 0; n < NT; n++) o[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(sv[i], vr[16 * n], o[n], 0, 0, 0);
        }
    }
    // merge the KS key splits of each head: (m, l) per query, O rows through LDS
    __syncthreads();
    float *Om = smem;                                   // [NW waves][16 rows][HD]
    __shared__ float Mm[NW][16], Ll[NW][16];
    if (lg == 0) { Mm[wid][lq] = m; Ll[wid][lq] = l; }
#pragma unroll
    for (int n = 0; n < NT; n++)
#pragma unroll
        for (int j = 0; j < 4; j++) Om[(wid * 16 + 4 * lg + j) * HD + 16 * n + lq] = o[n][j];
    __syncthreads();
    for (int i = t; i < G * 16 * HD; i += NTH) {
        const int gg = i / (16 * HD), r = (i / HD) % 16, d = i % HD;
        const int q = q0 + r;
        if (q >= a.n_q) continue;
        float M = -INFINITY;
#pragma unroll
        for (int k2 = 0; k2 < KS; k2++) M = fmaxf(M, Mm[gg * KS + k2][r]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int k2 = 0; k2 < KS; k2++) {
            const int w = gg * KS + k2;
            const float f = Mm[w][r] == -INFINITY ? 0.0f : expf(__fsub_rn(Mm[w][r], M));
            L = fmaf(Ll[w][r], f, L);
            O = fmaf(Om[(w * 16 + r) * HD + d], f, O);
        }
        a.out[(int64_t)q * a.o_rs + (kvh * G + gg) * HD + d] = L > 0.0f ? __fdiv_rn(O, L) : 0.0f;
    }
}

template <int HD, int G, int NW>
__global__ __launch_bounds__(NW * 64) void k_attn_mfma(AttnRowsArgs a) {
    // causal: tiles in reverse, so that the blocks with the most keys start first
    attn_mfma_block<HD, G, NW>(a, (a.window > 0 ? blockIdx.y : gridDim.y - 1 - blockIdx.y) * 16);
}

// Causal attention of several sequences in one launch (the multi-sequence
// prefill): block row y belongs to sequence j (blk[j] <= y < blk[j + 1]) and
// is that sequence's row block of a call of its own (the same q0, in the
// same reverse order), with the sequence's query / output rows, KV cache,
// key count and query offset.
template <int HD, int G, int NW>
__global__ __launch_bounds__(NW * 64) void k_attn_mfma_seqs(AttnSeqArgs s) {
    const int y = blockIdx.y;
    int b1 = s.blk[1];
    int64_t row = s.row[0];
    const float *k = s.k[0], *v = s.v[0];
    int nq = s.n_q[0], nk = s.n_k[0], qo = s.q_offset[0];
#pragma unroll
    for (int u = 1; u < QASR_ATTN_MAX_SEQ; u++)
        if (u < s.n && y >= s.blk[u]) {
            b1 = s.blk[u + 1];
            row = s.row[u];
            k = s.k[u];
            v = s.v[u];
            nq = s.n_q[u];
            nk = s.n_k[u];
            qo = s.q_offset[u];
        }
    AttnRowsArgs a = s.base;
    a.q += row * a.q_rs;
    a.out += row * a.o_rs;
    a.k = k;
    a.v = v;
    a.n_q = nq;
    a.n_k = nk;
    a.q_offset = qo;
    attn_mfma_block<HD, G, NW>(a, (b1 - 1 - y) * 16);
}

hipError_t launch_attn_rows_seqs(const AttnSeqArgs &s0, int n_kv_heads, int head_dim, hipStream_t st) {
    const AttnRowsArgs &a = s0.base;
    if (s0.n < 1 || s0.n > QASR_ATTN_MAX_SEQ || a.window > 0 || head_dim != 128 || a.G != 2)
        return hipErrorInvalidValue;
    AttnSeqArgs s = s0;
    s.base.kv_div = 1;
    s.blk[0] = 0;
    for (int j = 0; j < s.n; j++) {
        if (s.n_q[j] <= 0) return hipErrorInvalidValue;
        s.blk[j + 1] = s.blk[j] + (s.n_q[j] + 15) / 16;
    }
    // both query heads of a KV head in one block of 16 waves, 8 key splits
    // each: every head meets the key partition of launch_attn_rows' form for
    // these heads (one head per 8-wave block, 8 splits; the same bits), and
    // the block stages each K/V chunk once for the two heads
    const dim3 grid(n_kv_heads, s.blk[s.n]);
    hipLaunchKernelGGL((k_attn_mfma_seqs<128, 2, 16>), grid, dim3(1024), 0, st, s);
    return hipGetLastError();
}

hipError_t launch_attn_rows(const AttnRowsArgs &a, int n_kv_heads, int head_dim, hipStream_t st) {
    if (a.G <= 0 || 32 % a.G != 0 || a.n_q <= 0) return hipErrorInvalidValue;
    const bool aligned = a.q_rs % 4 == 0 && a.k_rs % 4 == 0 && a.k_hs % 4 == 0 && (uintptr_t)a.q % 16 == 0 &&
                         (uintptr_t)a.k % 16 == 0 && (uintptr_t)a.v % 16 == 0;
    if (aligned && (a.G == 1 || a.G == 2) && (head_dim == 128 || head_dim == 64)) {
        const dim3 grid(n_kv_heads, (a.n_q + 15) / 16);
        // 128-dim decoder heads (G = 2): one query head per block, its 8 waves
        // 8 key splits (KV head x / 2); measured 30.0 us for the 404-row prefill
        // against 32.5 with both heads of a KV head in one 8-wave block and 35.7
        // with 4 waves.  64-dim encoder heads: 4 waves (12.4 us against 13.6 at 8).
#define QAM(HDV, GV, NWV) hipLaunchKernelGGL((k_attn_mfma<HDV, GV, NWV>), grid, dim3(NWV * 64), 0, st, a);
        if (head_dim == 128 && a.G == 2) {
            AttnRowsArgs b = a;
            b.kv_div = 2;
            const dim3 grid1(n_kv_heads * 2, (a.n_q + 15) / 16);
            hipLaunchKernelGGL((k_attn_mfma<128, 1, 8>), grid1, dim3(512), 0, st, b);
        } else if (head_dim == 128) { QAM(128, 1, 8) }
        else if (a.G == 2) { QAM(64, 2, 4) }
        else { QAM(64, 1, 4) }
#undef QAM
        return hipGetLastError();
    }
    const dim3 grid(n_kv_heads, (a.n_q + 32 / a.G - 1) / (32 / a.G));
    if (head_dim == 128) hipLaunchKernelGGL(k_attn_rows<128>, grid, dim3(256), 0, st, a);
    else if (head_dim == 64) hipLaunchKernelGGL(k_attn_rows<64>, grid, dim3(256), 0, st, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// mel pieces (audio.rs:273-372)
// ---------------------------------------------------------------------------
// frames[t][n] = padded[t * 160 + n] * window[n], reflect padding of 200
__global__ __launch_bounds__(256) void k_mel_frames(float *__restrict__ fr, const float *__restrict__ x, int64_t ns,
                                                    const float *__restrict__ window, int nf) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)nf * 400) return;
    const int n = (int)(i % 400);
    const int64_t t = i / 400;
    const int64_t p = t * 160 + n;          // index into the padded signal
    float v;
    if (p < 200) {
        const int64_t s = 200 - p;
        v = s < ns ? x[s] : 0.0f;
    } else if (p < 200 + ns) {
        v = x[p - 200];
    } else {
        const int64_t s = ns - 2 - (p - 200 - ns);
        v = s >= 0 ? x[s] : 0.0f;
    }
    fr[i] = __fmul_rn(v, window[n]);
}

// powT[t][k] = re^2 + im^2 from re/im [k][t]
__global__ __launch_bounds__(256) void k_mel_power(float *__restrict__ pT, const float *__restrict__ re,
                                                   const float *__restrict__ im, int nf) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)nf * 201) return;
    const int k = (int)(i % 201);
    const int64_t t = i / 201;
    const float r = re[k * (int64_t)nf + t], m = im[k * (int64_t)nf + t];
    pT[i] = __fadd_rn(__fmul_rn(r, r), __fmul_rn(m, m));
}

// log10(max(v, 1e-10)) in place and per-block maxima
__global__ __launch_bounds__(256) void k_mel_log(float *__restrict__ mel, int64_t n, float *__restrict__ bmax) {
    __shared__ float red[4];
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    float v = -1e30f;
    if (i < n) {
        v = log10f(fmaxf(mel[i], 1e-10f));
        mel[i] = v;
    }
    v = wave_max_f32(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) bmax[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__global__ __launch_bounds__(256) void k_mel_norm(float *__restrict__ mel, int64_t n, const float *__restrict__ bmax,
                                                  int nb) {
    __shared__ float gm;
    if (threadIdx.x < 64) {
        float v = -1e30f;
        for (int b = threadIdx.x; b < nb; b += 64) v = fmaxf(v, bmax[b]);
        v = wave_max_f32(v);
        if (threadIdx.x == 0) gm = v;
    }
    __syncthreads();
    const float mn = __fsub_rn(gm, 8.0f);
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        mel[i] = __fdiv_rn(__fadd_rn(fmaxf(mel[i], mn), 4.0f), 4.0f);
}

hipError_t launch_mel_frames(float *fr, const float *x, int64_t ns, const float *window, int nf, hipStream_t st) {
    const int64_t n = (int64_t)nf * 400;
    hipLaunchKernelGGL(k_mel_frames, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, fr, x, ns, window, nf);
    return hipGetLastError();
}
hipError_t launch_mel_power(float *pT, const float *re, const float *im, int nf, hipStream_t st) {
    const int64_t n = (int64_t)nf * 201;
    hipLaunchKernelGGL(k_mel_power, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, pT, re, im, nf);
    return hipGetLastError();
}
hipError_t launch_mel_log_norm(float *mel, int64_t n, float *bmax, hipStream_t st) {
    const int nb = (int)((n + 255) / 256);
    hipLaunchKernelGGL(k_mel_log, dim3(nb), dim3(256), 0, st, mel, n, bmax);
    hipLaunchKernelGGL(k_mel_norm, dim3(std::min(nb, 1024)), dim3(256), 0, st, mel, n, bmax, nb);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// timing helper: one wave that idles for `ticks` of the 100 MHz constant clock
// (s_memrealtime).  Queued in front of a timed batch of launches, it holds the
// stream until the host has enqueued the whole batch, so the batch runs back to
// back.  The loop always ends: the clock is monotonic.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void k_delay(int64_t ticks) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while ((int64_t)(__builtin_amdgcn_s_memrealtime() - t0) < ticks) __builtin_amdgcn_s_sleep(64);
}

hipError_t launch_delay(int us, hipStream_t st) {
    if (us < 0 || us > 100000) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_delay, dim3(1), dim3(64), 0, st, (int64_t)us * 100);
    return hipGetLastError();
}

}  // namespace qasr
