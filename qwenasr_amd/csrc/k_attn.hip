// Decode-step attention and the small row-wise kernels around it.
#include "kernels.h"

namespace qasr {

template <typename T> __device__ __forceinline__ float ld_kv(const T *p);
template <> __device__ __forceinline__ float ld_kv<float>(const float *p) { return *p; }
template <> __device__ __forceinline__ float ld_kv<uint16_t>(const uint16_t *p) { return bf16_to_f32(*p); }
template <typename T> __device__ __forceinline__ T st_kv(float v);
template <> __device__ __forceinline__ float st_kv<float>(float v) { return v; }
template <> __device__ __forceinline__ uint16_t st_kv<uint16_t>(float v) { return f32_to_bf16_rne(v); }
// the f32 value a cache element of type T holds after storing v
template <typename T> __device__ __forceinline__ float round_kv(float v) { const T s = st_kv<T>(v); return ld_kv<T>(&s); }

// load 8 consecutive KV elements as f32
__device__ __forceinline__ void ld8(const float *p, float o[8]) {
    const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}
__device__ __forceinline__ void ld8(const uint16_t *p, float o[8]) {
    const uint4 a = *reinterpret_cast<const uint4 *>(p);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        o[2 * i] = __uint_as_float(w[i] << 16);
        o[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
}

// Sum over the 128 threads of a head (two waves) through LDS slots red[2h], red[2h+1].
__device__ __forceinline__ float head_sum128(float v, float *red) {
    v = wave_sum_f32(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return __fadd_rn(red[w & ~1], red[w | 1]);
}

// ---------------------------------------------------------------------------
// GQA decode attention, one layer, D = 128, G = Hq / Hkv query heads per KV
// head.  Restates causal_attention with seq_q = 1 (kernels/mod.rs:1492-1536):
// scores dot(q, k_j) * scale over j <= pos, softmax, sum_j p_j v_j, with q/k
// per-head RMSNorm (mod.rs:1214-1238) and NeoX RoPE (mod.rs:1780-1788) fused
// in front and the new K/V row written into the cache (decoder.rs:233-253).
// The context is split into n_split ranges (one block each); every block
// writes (max, sum, o) partials and the last block of a KV head merges them
// with the usual log-sum-exp rescaling.  Softmax is therefore evaluated in a
// different order than the reference's sequential online scan: results agree
// to f32 rounding, not bit for bit.
// ---------------------------------------------------------------------------
#define ATT_MAXC 256
#define ATT_MAXS 64

template <int G, typename KVT>
__global__ __launch_bounds__(256) void k_attn_decode(AttnDecodeArgs a) {
    constexpr int D = 128;
    static_assert(G * D == 256, "one thread per (query head, dim)");
    __shared__ float qs[G][D];
    __shared__ float knew[D], vnew[D];
    __shared__ float red[8];
    __shared__ float sc[G][ATT_MAXC];
    __shared__ float pv[2][G][D];
    __shared__ float mw[G][ATT_MAXS], lw[G][ATT_MAXS];
    __shared__ int last;
    const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
    const int n_split = a.n_split;
    const int kvh = blockIdx.x / n_split, split = blockIdx.x % n_split;
    const int Hkv = gridDim.x / n_split, Hq = Hkv * G;
    const int pos = a.state ? a.state[1] : a.pos;
    const int L = pos + 1;
    const int chunk = (L + n_split - 1) / n_split;
    const int j0 = split * chunk, j1 = min(L, j0 + chunk);
    const bool prep = a.q_norm != nullptr;     // raw projections: norm + rope + cache write
    const bool own_pos = prep && j0 <= pos && pos < j1;
    KVT *kc = reinterpret_cast<KVT *>(a.kcache) + (int64_t)kvh * a.head_stride;
    KVT *vc = reinterpret_cast<KVT *>(a.vcache) + (int64_t)kvh * a.head_stride;

    // ---- query heads of this group ---------------------------------------
    {
        const int gi = t / D, d = t % D;
        float v = a.qkv[(kvh * G + gi) * D + d];
        if (prep) {
            const float ss = head_sum128(__fmul_rn(v, v), red);
            const float r = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)D), a.eps)));
            v = __fmul_rn(__fmul_rn(v, r), a.q_norm[d]);
            qs[gi][d] = v;
            __syncthreads();
            const float *c = a.rope_cos + (int64_t)pos * D, *s = a.rope_sin + (int64_t)pos * D;
            const int h = D / 2;
            float o;
            if (d < h) o = __fadd_rn(__fmul_rn(v, c[d]), __fmul_rn(-qs[gi][d + h], s[d]));
            else o = __fadd_rn(__fmul_rn(v, c[d]), __fmul_rn(qs[gi][d - h], s[d]));
            __syncthreads();
            qs[gi][d] = o;
        } else {
            qs[gi][d] = v;
        }
    }
    // ---- new K/V row (the block whose range holds pos) --------------------
    if (own_pos) {
        const int d = t % D;
        float kv = a.qkv[Hq * D + kvh * D + d];
        const float ss = head_sum128(t < D ? __fmul_rn(kv, kv) : 0.0f, red);
        if (t < D) {
            const float r = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)D), a.eps)));
            kv = __fmul_rn(__fmul_rn(kv, r), a.k_norm[d]);
            knew[d] = kv;
        }
        __syncthreads();
        float o = 0.0f, vv = 0.0f;
        if (t < D) {
            const float *c = a.rope_cos + (int64_t)pos * D, *s = a.rope_sin + (int64_t)pos * D;
            const int h = D / 2;
            if (d < h) o = __fadd_rn(__fmul_rn(kv, c[d]), __fmul_rn(-knew[d + h], s[d]));
            else o = __fadd_rn(__fmul_rn(kv, c[d]), __fmul_rn(knew[d - h], s[d]));
            vv = a.qkv[Hq * D + Hkv * D + kvh * D + d];
            kc[(int64_t)pos * D + d] = st_kv<KVT>(o);
            vc[(int64_t)pos * D + d] = st_kv<KVT>(vv);
        }
        __syncthreads();
        if (t < D) {   // the values the cache now holds (a bf16 cache rounds)
            knew[d] = round_kv<KVT>(o);
            vnew[d] = round_kv<KVT>(vv);
        }
    }
    __syncthreads();

    // ---- scores: 16 lanes per position, 8 dims per lane --------------------
    const int sub = lane >> 4, dl = (lane & 15) * 8;
    float qv[G][8];
#pragma unroll
    for (int gi = 0; gi < G; gi++)
#pragma unroll
        for (int i = 0; i < 8; i++) qv[gi][i] = qs[gi][dl + i];
    for (int base = j0; base < j1; base += 16) {
        const int j = base + wid * 4 + sub;
        float kr[8];
        if (j < j1) {
            if (own_pos && j == pos) {
#pragma unroll
                for (int i = 0; i < 8; i++) kr[i] = knew[dl + i];
            } else {
                ld8(kc + (int64_t)j * D + dl, kr);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) kr[i] = 0.0f;
        }
#pragma unroll
        for (int gi = 0; gi < G; gi++) {
            float p = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++) p = fmaf(qv[gi][i], kr[i], p);
            p = group_sum_f32<16>(p);
            if ((lane & 15) == 0 && j < j1) sc[gi][j - j0] = __fmul_rn(p, a.scale);
        }
    }
    __syncthreads();
    // ---- softmax over this block's range ------------------------------------
    const int n = j1 > j0 ? j1 - j0 : 0;
    float mloc[G], lsum[G];
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
        float m = -INFINITY;
        for (int j = t; j < n; j += 256) m = fmaxf(m, sc[gi][j]);
        m = wave_max_f32(m);
        __syncthreads();
        if (lane == 0) red[wid] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        float s = 0.0f;
        for (int j = t; j < n; j += 256) {
            const float p = expf(__fsub_rn(sc[gi][j], m));
            sc[gi][j] = p;
            s = __fadd_rn(s, p);
        }
        s = wave_sum_f32(s);
        __syncthreads();
        if (lane == 0) red[4 + wid] = s;
        __syncthreads();
        mloc[gi] = m;
        lsum[gi] = __fadd_rn(__fadd_rn(red[4], red[5]), __fadd_rn(red[6], red[7]));
    }
    // ---- o = sum_j p_j v_j: thread (half, d) covers j = j0 + half + 2i ------
    {
        const int d = t % D, half = t / D;
        float acc[G];
#pragma unroll
        for (int gi = 0; gi < G; gi++) acc[gi] = 0.0f;
        for (int j = j0 + half; j < j1; j += 2) {
            const float vv = (own_pos && j == pos) ? vnew[d] : ld_kv<KVT>(vc + (int64_t)j * D + d);
#pragma unroll
            for (int gi = 0; gi < G; gi++) acc[gi] = fmaf(sc[gi][j - j0], vv, acc[gi]);
        }
#pragma unroll
        for (int gi = 0; gi < G; gi++) pv[half][gi][d] = acc[gi];
    }
    __syncthreads();
    float *part = a.part + ((int64_t)kvh * n_split + split) * G * (D + 2);
    {
        const int gi = t / D, d = t % D;
        st_agent(part + gi * (D + 2) + 2 + d, __fadd_rn(pv[0][gi][d], pv[1][gi][d]));
        if (d == 0) {
            st_agent(part + gi * (D + 2), n > 0 ? mloc[gi] : -INFINITY);
            st_agent(part + gi * (D + 2) + 1, n > 0 ? lsum[gi] : 0.0f);
        }
    }
    if (!arrive_last(a.counters + kvh, (unsigned)n_split, &last)) return;
    // ---- last block of this KV head: log-sum-exp merge of the n_split partials
    const float *pb = a.part + (int64_t)kvh * n_split * G * (D + 2);
    for (int i = t; i < n_split * G; i += 256) {
        const int s = i / G, gi = i % G;
        mw[gi][s] = ld_agent(pb + (s * G + gi) * (D + 2));
        lw[gi][s] = ld_agent(pb + (s * G + gi) * (D + 2) + 1);
    }
    __syncthreads();
    if (t < G) {
        float M = -INFINITY;
        for (int s = 0; s < n_split; s++) M = fmaxf(M, mw[t][s]);
        float lt = 0.0f;
        for (int s = 0; s < n_split; s++) {
            const float f = mw[t][s] == -INFINITY ? 0.0f : expf(__fsub_rn(mw[t][s], M));
            mw[t][s] = f;
            lt = fmaf(lw[t][s], f, lt);
        }
        lw[t][0] = lt;
    }
    __syncthreads();
    {
        const int gi = t / D, d = t % D;
        float ot = 0.0f;
        for (int s0 = 0; s0 < n_split; s0 += 8) {
            float ov[8];
#pragma unroll
            for (int i = 0; i < 8; i++)
                ov[i] = s0 + i < n_split ? ld_agent(pb + ((s0 + i) * G + gi) * (D + 2) + 2 + d) : 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (s0 + i < n_split) ot = fmaf(ov[i], mw[gi][s0 + i], ot);
        }
        const float lt = lw[gi][0];
        a.out[(kvh * G + gi) * D + d] = lt > 0.0f ? __fdiv_rn(ot, lt) : 0.0f;
    }
    if (t == 0) reset_counter(a.counters + kvh);
}

hipError_t launch_attn_decode(const AttnDecodeArgs &a, int n_heads, int n_kv_heads, int head_dim,
                              int kv_bf16, hipStream_t st) {
    if (head_dim != 128 || n_kv_heads <= 0 || n_heads != 2 * n_kv_heads) return hipErrorInvalidValue;
    if (a.n_split <= 0 || a.n_split > ATT_MAXS) return hipErrorInvalidValue;
    const dim3 grid(n_kv_heads * a.n_split);
    if (kv_bf16) hipLaunchKernelGGL((k_attn_decode<2, uint16_t>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((k_attn_decode<2, float>), grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// RMSNorm over rows (rms_norm, kernels/mod.rs:1191-1212, AVX order of
// avx.rs:377-415), one wave per row, hidden % 64 == 0.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rms_norm_rows(float *__restrict__ out, const float *__restrict__ x,
                                                       const float *__restrict__ w, int64_t seq, int H,
                                                       float eps) {
    extern __shared__ float lds[];
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int64_t row = (int64_t)blockIdx.x * 4 + wid;
    if (row >= seq) return;
    const float *xr = x + row * H;
    float *o = out + row * H;
    const int nslot = H >> 4;
    float *T = lds + wid * H;
    for (int s = lane; s < nslot; s += 64)
        for (int r = 0; r < 16; r++) T[r * nslot + s] = xr[16 * s + r];
    __builtin_amdgcn_wave_barrier();
    float acc = 0.0f;
    if (lane < 16) {
        const float *tr = T + lane * nslot;
        for (int i = 0; i < nslot; i++) acc = fmaf(tr[i], tr[i], acc);
    }
    const float ss = avx16_tree(acc);
    const float rinv = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)H), eps)));
    for (int i = lane; i < H; i += 64) o[i] = __fmul_rn(__fmul_rn(xr[i], rinv), w[i]);
}

hipError_t launch_rms_norm_rows(float *out, const float *x, const float *w, int64_t seq, int hidden,
                                float eps, hipStream_t st) {
    if (hidden % 64 != 0 || hidden > 4096) return hipErrorInvalidValue;
    const unsigned blocks = (unsigned)((seq + 3) / 4);
    hipLaunchKernelGGL(k_rms_norm_rows, dim3(blocks), dim3(256), 4 * hidden * sizeof(float), st, out, x,
                       w, seq, hidden, eps);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Per-head RMSNorm (rms_norm_per_head, kernels/mod.rs:1214-1238) and NeoX RoPE
// (apply_rope_neox, mod.rs:1738-1791) over [seq][heads][hd] rows, hd = 128:
// one wave per (row, head), two elements per lane (d and d + 64).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_head_norm_rope(float *__restrict__ x, const float *__restrict__ w,
                                                        const float *__restrict__ cos_t,
                                                        const float *__restrict__ sin_t, int64_t seq,
                                                        int heads, int64_t row_stride, float eps, int do_norm,
                                                        int do_rope) {
    constexpr int D = 128;
    const int lane = threadIdx.x & 63;
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= seq * heads) return;
    const int64_t s = item / heads;
    float *v = x + s * row_stride + (item % heads) * D;
    float x1 = v[lane], x2 = v[lane + 64];
    if (do_norm) {
        const float ss = wave_sum_f32(__fadd_rn(__fmul_rn(x1, x1), __fmul_rn(x2, x2)));
        const float r = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)D), eps)));
        x1 = __fmul_rn(__fmul_rn(x1, r), w[lane]);
        x2 = __fmul_rn(__fmul_rn(x2, r), w[lane + 64]);
    }
    if (do_rope) {
        const float *c = cos_t + s * D, *sn = sin_t + s * D;
        const float n1 = __fadd_rn(__fmul_rn(x1, c[lane]), __fmul_rn(-x2, sn[lane]));
        const float n2 = __fadd_rn(__fmul_rn(x2, c[lane + 64]), __fmul_rn(x1, sn[lane + 64]));
        x1 = n1; x2 = n2;
    }
    v[lane] = x1;
    v[lane + 64] = x2;
}

hipError_t launch_head_norm_rope_strided(float *x, int64_t row_stride, const float *w, const float *cos_t,
                                         const float *sin_t, int64_t seq, int heads, float eps, int do_norm,
                                         int do_rope, hipStream_t st) {
    const unsigned blocks = (unsigned)((seq * heads + 3) / 4);
    hipLaunchKernelGGL(k_head_norm_rope, dim3(blocks), dim3(256), 0, st, x, w, cos_t, sin_t, seq, heads, row_stride,
                       eps, do_norm, do_rope);
    return hipGetLastError();
}

hipError_t launch_head_norm_rope(float *x, const float *w, const float *cos_t, const float *sin_t,
                                 int64_t seq, int heads, int hd, float eps, int do_norm, int do_rope,
                                 hipStream_t st) {
    if (hd != 128) return hipErrorInvalidValue;
    return launch_head_norm_rope_strided(x, (int64_t)heads * hd, w, cos_t, sin_t, seq, heads, eps, do_norm,
                                         do_rope, st);
}

}  // namespace qasr
