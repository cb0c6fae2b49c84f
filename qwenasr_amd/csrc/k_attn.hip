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
//
// The context is split into n_split ranges (one block each).  A block streams
// its range in tiles of 32 positions through LDS: the first tile's loads are
// issued before the q/k prologue and each next tile is prefetched into
// registers while the current one is consumed, so the block pays about one
// memory round trip per tile.  Softmax is online within the block; every
// block publishes (max, sum, o) and the last block of a KV head merges them
// with log-sum-exp rescaling.  The order of operations differs from the
// reference's sequential scan: results agree to f32 rounding, not bit for bit.
// ---------------------------------------------------------------------------
#define ATT_MAXC 256
#define ATT_MAXS 64
#define ATT_TP 32

template <typename KVT> struct KvTile;
template <> struct KvTile<float> {      // 32 x 128 f32 = 1024 float4, 4 per thread
    static constexpr int N = 4;
    float4 k[N], v[N];
};
template <> struct KvTile<uint16_t> {   // 32 x 128 bf16 = 512 uint4, 2 per thread
    static constexpr int N = 2;
    uint4 k[N], v[N];
};

template <typename KVT>
__device__ __forceinline__ void tile_load(KvTile<KVT> &r, const KVT *kc, const KVT *vc, int j0, int j1, int skip) {
    constexpr int PER_ROW = sizeof(KVT) == 4 ? 32 : 16;     // 16-byte vectors per position
#pragma unroll
    for (int i = 0; i < KvTile<KVT>::N; i++) {
        const int idx = threadIdx.x + 256 * i;
        const int j = j0 + idx / PER_ROW, c = idx % PER_ROW;
        const bool ok = j < j1 && j != skip;
        const int jj = ok ? j : j0;
        if (sizeof(KVT) == 4) {
            const float4 kv = reinterpret_cast<const float4 *>(kc + (int64_t)jj * 128)[c];
            const float4 vv = reinterpret_cast<const float4 *>(vc + (int64_t)jj * 128)[c];
            reinterpret_cast<float4 *>(&r.k[i])[0] = kv;
            reinterpret_cast<float4 *>(&r.v[i])[0] = vv;
        } else {
            const uint4 kv = reinterpret_cast<const uint4 *>(kc + (int64_t)jj * 128)[c];
            const uint4 vv = reinterpret_cast<const uint4 *>(vc + (int64_t)jj * 128)[c];
            reinterpret_cast<uint4 *>(&r.k[i])[0] = kv;
            reinterpret_cast<uint4 *>(&r.v[i])[0] = vv;
        }
    }
}

template <typename KVT>
__device__ __forceinline__ void tile_store(const KvTile<KVT> &r, float (*Ks)[132], float (*Vs)[128]) {
    constexpr int PER_ROW = sizeof(KVT) == 4 ? 32 : 16;
#pragma unroll
    for (int i = 0; i < KvTile<KVT>::N; i++) {
        const int idx = threadIdx.x + 256 * i;
        const int p = idx / PER_ROW, c = idx % PER_ROW;
        if (sizeof(KVT) == 4) {
            const float4 kv = reinterpret_cast<const float4 *>(&r.k[i])[0];
            const float4 vv = reinterpret_cast<const float4 *>(&r.v[i])[0];
            *reinterpret_cast<float4 *>(&Ks[p][4 * c]) = kv;
            *reinterpret_cast<float4 *>(&Vs[p][4 * c]) = vv;
        } else {
            const uint4 kv = reinterpret_cast<const uint4 *>(&r.k[i])[0];
            const uint4 vv = reinterpret_cast<const uint4 *>(&r.v[i])[0];
            const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w}, vw[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                Ks[p][8 * c + 2 * e] = __uint_as_float(kw[e] << 16);
                Ks[p][8 * c + 2 * e + 1] = __uint_as_float(kw[e] & 0xFFFF0000u);
                Vs[p][8 * c + 2 * e] = __uint_as_float(vw[e] << 16);
                Vs[p][8 * c + 2 * e + 1] = __uint_as_float(vw[e] & 0xFFFF0000u);
            }
        }
    }
}

template <int G, typename KVT, bool MERGE>
__global__ __launch_bounds__(256) void k_attn_decode(AttnDecodeArgs a) {
    constexpr int D = 128, TP = ATT_TP;
    static_assert(G * D == 256, "one thread per (query head, dim)");
    __shared__ float Ks[TP][D + 4];
    __shared__ float Vs[TP][D];
    __shared__ float qs[G][D];
    __shared__ float knew[D], vnew[D];
    __shared__ float red[8];
    __shared__ float ps[G][TP];
    __shared__ float pv[2][G][D];
    __shared__ float mw[G][ATT_MAXS], lw[G][ATT_MAXS];
    __shared__ int last;
    const int t = threadIdx.x, lane = t & 63;
    const int n_split = a.n_split;
    const int kvh = blockIdx.x / n_split, split = blockIdx.x % n_split;
    const int Hkv = gridDim.x / n_split, Hq = Hkv * G;
    const int pos = a.state ? a.state[1] : a.pos;
    const int L = pos + 1;
    const int chunk = (L + n_split - 1) / n_split;
    const int j0 = split * chunk, j1 = min(L, j0 + chunk);
    const bool prep = a.q_norm != nullptr;     // raw projections: norm + rope + cache write
    const bool own_pos = prep && j0 <= pos && pos < j1;
    const int skip = own_pos ? pos : -1;
    KVT *kc = reinterpret_cast<KVT *>(a.kcache) + (int64_t)kvh * a.head_stride;
    KVT *vc = reinterpret_cast<KVT *>(a.vcache) + (int64_t)kvh * a.head_stride;
    const int gi = t / D, d = t % D;

    // ---- issue the small operand loads, then the first tile ---------------
    float qv = a.qkv[(kvh * G + gi) * D + d];
    float cv = 0.0f, sv = 0.0f, kraw = 0.0f, vraw = 0.0f;
    if (prep) {
        cv = a.rope_cos[(int64_t)pos * D + d];
        sv = a.rope_sin[(int64_t)pos * D + d];
    }
    if (own_pos && t < D) {
        kraw = a.qkv[Hq * D + kvh * D + d];
        vraw = a.qkv[Hq * D + Hkv * D + kvh * D + d];
    }
    KvTile<KVT> tr;
    if (j0 < j1) tile_load<KVT>(tr, kc, vc, j0, min(j1, j0 + TP), skip);

    // ---- query heads of this group: per-head RMSNorm + RoPE --------------
    if (prep) {
        const float ss = head_sum128(__fmul_rn(qv, qv), red);
        const float r = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)D), a.eps)));
        qv = __fmul_rn(__fmul_rn(qv, r), a.q_norm[d]);
        qs[gi][d] = qv;
        __syncthreads();
        const int h = D / 2;
        float o;
        if (d < h) o = __fadd_rn(__fmul_rn(qv, cv), __fmul_rn(-qs[gi][d + h], sv));
        else o = __fadd_rn(__fmul_rn(qv, cv), __fmul_rn(qs[gi][d - h], sv));
        __syncthreads();
        qs[gi][d] = o;
    } else {
        qs[gi][d] = qv;
    }
    // ---- new K/V row (the block whose range holds pos) --------------------
    if (own_pos) {
        const float ss = head_sum128(t < D ? __fmul_rn(kraw, kraw) : 0.0f, red);
        float kv = 0.0f;
        if (t < D) {
            const float r = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)D), a.eps)));
            kv = __fmul_rn(__fmul_rn(kraw, r), a.k_norm[d]);
            knew[d] = kv;
        }
        __syncthreads();
        float o = 0.0f;
        if (t < D) {
            const int h = D / 2;
            if (d < h) o = __fadd_rn(__fmul_rn(kv, cv), __fmul_rn(-knew[d + h], sv));
            else o = __fadd_rn(__fmul_rn(kv, cv), __fmul_rn(knew[d - h], sv));
            kc[(int64_t)pos * D + d] = st_kv<KVT>(o);
            vc[(int64_t)pos * D + d] = st_kv<KVT>(vraw);
        }
        __syncthreads();
        if (t < D) {   // the values the cache now holds (a bf16 cache rounds)
            knew[d] = round_kv<KVT>(o);
            vnew[d] = round_kv<KVT>(vraw);
        }
    }
    __syncthreads();

    // ---- stream the range in tiles -----------------------------------------
    // scores: thread t -> position p = t / 8, dims (t % 8) * 16 .. +16
    const int sp = t >> 3, sd = (t & 7) * 16;
    float qreg[G][16];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int i = 0; i < 16; i++) qreg[g][i] = qs[g][sd + i];
    float m_run[G], l_run[G], acc[G];
#pragma unroll
    for (int g = 0; g < G; g++) { m_run[g] = -INFINITY; l_run[g] = 0.0f; acc[g] = 0.0f; }
    const int hh = t / D;                    // PV: thread (hh, d) takes positions p = hh, hh + 2, ...
    for (int b = j0; b < j1; b += TP) {
        const int n = min(TP, j1 - b);
        tile_store<KVT>(tr, Ks, Vs);
        __syncthreads();
        if (own_pos && pos >= b && pos < b + n) {          // the new row comes from LDS
            if (t < D) { Ks[pos - b][t] = knew[t]; Vs[pos - b][t] = vnew[t]; }
            __syncthreads();
        }
        if (b + TP < j1) tile_load<KVT>(tr, kc, vc, b + TP, min(j1, b + 2 * TP), skip);   // prefetch
        float sc[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            float p = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) p = fmaf(qreg[g][i], Ks[sp][sd + i], p);
            p = group_sum_f32<8>(p);
            sc[g] = p;
        }
        if ((t & 7) == 0) {
#pragma unroll
            for (int g = 0; g < G; g++) ps[g][sp] = sp < n ? __fmul_rn(sc[g], a.scale) : -INFINITY;
        }
        __syncthreads();
        // online softmax update (every thread keeps the block-wide state of each head)
        float corr[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            float tm = -INFINITY;
            for (int p = 0; p < n; p++) tm = fmaxf(tm, ps[g][p]);
            const float mn = fmaxf(m_run[g], tm);
            corr[g] = m_run[g] == -INFINITY ? 0.0f : expf(__fsub_rn(m_run[g], mn));
            m_run[g] = mn;
        }
        __syncthreads();
        if (t < G * TP) {
            const int g = t / TP, p = t % TP;
            ps[g][p] = p < n ? expf(__fsub_rn(ps[g][p], m_run[g])) : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < G; g++) {
            float s = 0.0f;
            for (int p = 0; p < n; p++) s = __fadd_rn(s, ps[g][p]);
            l_run[g] = fmaf(l_run[g], corr[g], s);
            acc[g] = __fmul_rn(acc[g], corr[g]);
        }
        for (int p = hh; p < n; p += 2) {
            const float vv = Vs[p][d];
#pragma unroll
            for (int g = 0; g < G; g++) acc[g] = fmaf(ps[g][p], vv, acc[g]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int g = 0; g < G; g++) pv[hh][g][d] = acc[g];
    __syncthreads();
    float *part = a.part + ((int64_t)kvh * n_split + split) * G * (D + 2);
    const float o_part = __fadd_rn(pv[0][gi][d], pv[1][gi][d]);
    const float m_part = j1 > j0 ? m_run[gi] : -INFINITY, l_part = j1 > j0 ? l_run[gi] : 0.0f;
    if (!MERGE) {
        // the consumer (the o_proj kernel) merges; the kernel boundary publishes these
        part[gi * (D + 2) + 2 + d] = o_part;
        if (d == 0) {
            part[gi * (D + 2)] = m_part;
            part[gi * (D + 2) + 1] = l_part;
        }
        return;
    }
    st_agent(part + gi * (D + 2) + 2 + d, o_part);
    if (d == 0) {
        st_agent(part + gi * (D + 2), m_part);
        st_agent(part + gi * (D + 2) + 1, l_part);
    }
    if (!arrive_last(a.counters + kvh, (unsigned)n_split, &last)) return;
    // ---- last block of this KV head: log-sum-exp merge of the n_split partials
    const float *pb = a.part + (int64_t)kvh * n_split * G * (D + 2);
    for (int i = t; i < n_split * G; i += 256) {
        const int s = i / G, g = i % G;
        mw[g][s] = ld_agent(pb + (s * G + g) * (D + 2));
        lw[g][s] = ld_agent(pb + (s * G + g) * (D + 2) + 1);
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
                              int kv_bf16, hipStream_t st, bool merge) {
    if (head_dim != 128 || n_kv_heads <= 0 || n_heads != 2 * n_kv_heads) return hipErrorInvalidValue;
    if (a.n_split <= 0 || a.n_split > ATT_MAXS) return hipErrorInvalidValue;
    const dim3 grid(n_kv_heads * a.n_split);
    if (merge) {
        if (kv_bf16) hipLaunchKernelGGL((k_attn_decode<2, uint16_t, true>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((k_attn_decode<2, float, true>), grid, dim3(256), 0, st, a);
    } else {
        if (kv_bf16) hipLaunchKernelGGL((k_attn_decode<2, uint16_t, false>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((k_attn_decode<2, float, false>), grid, dim3(256), 0, st, a);
    }
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
