// Decode-step attention and the small row-wise kernels around it.
#include "kernels.h"
#include "mv_wave.h"

namespace qasr {

template <typename T> __device__ __forceinline__ float ld_kv(const T *p);
template <> __device__ __forceinline__ float ld_kv<float>(const float *p) { return *p; }
template <> __device__ __forceinline__ float ld_kv<uint16_t>(const uint16_t *p) { return bf16_to_f32(*p); }
template <typename T> __device__ __forceinline__ T st_kv(float v);
template <> __device__ __forceinline__ float st_kv<float>(float v) { return v; }
template <> __device__ __forceinline__ uint16_t st_kv<uint16_t>(float v) { return f32_to_bf16_rne(v); }
// the f32 value a cache element of type T holds after storing v
template <typename T> __device__ __forceinline__ float round_kv(float v) { const T s = st_kv<T>(v); return ld_kv<T>(&s); }

// ---------------------------------------------------------------------------
// GQA decode attention, one layer, D = 128, two query heads per KV head.
// Restates causal_attention with seq_q = 1 (kernels/mod.rs:1492-1536): scores
// dot(q, k_j) * scale over j <= pos, softmax, sum_j p_j v_j, with the q/k
// per-head RMSNorm (mod.rs:1214-1238) and NeoX RoPE (mod.rs:1780-1788) fused
// in front and the new K/V row written into the cache (decoder.rs:233-253).
//
// Work split: the context is cut into groups of 8 positions; block (KV head,
// split) owns a contiguous run of groups and each of its NW waves takes every
// NW-th group with an online-softmax state of its own, so the main loop has no
// block barrier.  Lane (pj = lane / 8, ds = lane % 8) holds 16 dimensions of
// position pj of the wave's current group: dims 32 i + 4 ds + e (i, e < 4) of
// an f32 cache, 64 i + 8 ds + e (i < 2, e < 8) of a bf16 cache.  Either way
// each load instruction covers whole 128-byte lines of 8 positions, and dims d
// and d + 64 (a RoPE pair) sit in the same lane as slots k and k + 8.  A score
// is a 16-term dot plus three xor shuffles; the softmax max and sum over the 8
// positions take three more.  Each lane accumulates p_j v_j of its own
// positions under the wave's running max; after the loop the lanes of a wave
// are summed, the waves' states merged in LDS (one barrier) and the result
// published as the block's partial (max, sum, o[128]).  The partials of a KV
// head are merged by log-sum-exp either by its last block to finish (MERGE) or
// by the o_proj kernel's prologue.  The order of operations differs from the
// reference's sequential scan: results agree to f32 rounding, not bit for bit.
// ---------------------------------------------------------------------------
#define ATT_MAXS 64

// 16 dimensions of one position in the lane layout of cache type T
template <typename T> struct KvSlice;
template <> struct KvSlice<float> {
    float4 v[4];
    static __device__ __forceinline__ int dim(int k, int ds) { return 32 * (k >> 2) + 4 * ds + (k & 3); }
    __device__ __forceinline__ void load(const float *row, int ds) {
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = reinterpret_cast<const float4 *>(row + dim(4 * i, ds))[0];
    }
    __device__ __forceinline__ void to_f32(float o[16]) const {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o[4 * i] = v[i].x; o[4 * i + 1] = v[i].y; o[4 * i + 2] = v[i].z; o[4 * i + 3] = v[i].w;
        }
    }
    static __device__ __forceinline__ void store(float *row, int ds, const float o[16]) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            reinterpret_cast<float4 *>(row + dim(4 * i, ds))[0] =
                make_float4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
    }
};
template <> struct KvSlice<uint16_t> {
    uint4 v[2];
    static __device__ __forceinline__ int dim(int k, int ds) { return 64 * (k >> 3) + 8 * ds + (k & 7); }
    __device__ __forceinline__ void load(const uint16_t *row, int ds) {
#pragma unroll
        for (int i = 0; i < 2; i++) v[i] = reinterpret_cast<const uint4 *>(row + dim(8 * i, ds))[0];
    }
    __device__ __forceinline__ void to_f32(float o[16]) const {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                o[8 * i + 2 * e] = __uint_as_float(w[e] << 16);
                o[8 * i + 2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
            }
        }
    }
    static __device__ __forceinline__ void store(uint16_t *row, int ds, const float o[16]) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; e++)
                w[e] = (uint32_t)f32_to_bf16_rne(o[8 * i + 2 * e]) |
                       ((uint32_t)f32_to_bf16_rne(o[8 * i + 2 * e + 1]) << 16);
            reinterpret_cast<uint4 *>(row + dim(8 * i, ds))[0] = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
};

// 16 f32 values of a [128] vector in the lane layout of cache type T
template <typename T>
__device__ __forceinline__ void ld16(const float *v, int ds, float o[16]) {
#pragma unroll
    for (int k = 0; k < 16; k += 4) {
        const float4 x = reinterpret_cast<const float4 *>(v + KvSlice<T>::dim(k, ds))[0];
        o[k] = x.x; o[k + 1] = x.y; o[k + 2] = x.z; o[k + 3] = x.w;
    }
}

// per-head RMSNorm then NeoX RoPE of one head's 16 lane slots (slot k + 8 is
// dim d + 64); the 8 lanes of a position together hold the head's 128 dims
__device__ __forceinline__ void norm_rope16(float x[16], const float w[16], const float c[16], const float s[16],
                                            float eps) {
    constexpr int D = 128;
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; k++) ss = fmaf(x[k], x[k], ss);
    ss = sum8(ss);
    const float r = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(div_by_count(ss, D), eps)));
#pragma unroll
    for (int k = 0; k < 16; k++) x[k] = __fmul_rn(__fmul_rn(x[k], r), w[k]);
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const float x1 = x[k], x2 = x[k + 8];
        x[k] = __fadd_rn(__fmul_rn(x1, c[k]), __fmul_rn(-x2, s[k]));
        x[k + 8] = __fadd_rn(__fmul_rn(x2, c[k + 8]), __fmul_rn(x1, s[k + 8]));
    }
}

// Online-softmax state of one wave for G query heads over the positions its
// lanes have seen: running max m, sum l, and o (16 dims per lane).
template <int G>
struct AttnAcc {
    float m[G], l[G], acc[G][16];
    __device__ __forceinline__ void init() {
#pragma unroll
        for (int g = 0; g < G; g++) {
            m[g] = -INFINITY;
            l[g] = 0.0f;
#pragma unroll
            for (int k = 0; k < 16; k++) acc[g][k] = 0.0f;
        }
    }
    // one group of 8 positions (this lane's position valid or not): scores,
    // the group max and sum over the 8 position lanes, rescale, accumulate
    __device__ __forceinline__ void consume(const float (&q)[G][16], const float (&kf)[16], const float (&vf)[16],
                                            bool valid, float scale) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            float s = 0.0f;
#pragma unroll
            for (int k = 0; k < 16; k++) s = fmaf(q[g][k], kf[k], s);
            s = sum8(s);
            s = valid ? __fmul_rn(s, scale) : -INFINITY;
            const float mn = fmaxf(m[g], max_x8(s));           // finite: a group has a valid position
            const float corr = m[g] == -INFINITY ? 0.0f : expf(__fsub_rn(m[g], mn));
            const float p = valid ? expf(__fsub_rn(s, mn)) : 0.0f;
            l[g] = fmaf(l[g], corr, sum_x8(p));
#pragma unroll
            for (int k = 0; k < 16; k++) acc[g][k] = fmaf(p, vf[k], __fmul_rn(acc[g][k], corr));
            m[g] = mn;
        }
    }
};

// Block partial of NW waves: the lanes of each wave summed, the waves' states
// merged through LDS (one barrier).  Threads t < G * 128 receive (m, l, o[d])
// of query head t / 128, dim t % 128.
template <typename KVT, int NW, int G>
__device__ __forceinline__ void attn_block_partial(AttnAcc<G> &st, float (*wm)[G], float (*wl)[G],
                                                   float (*wacc)[G][128], float &o_part, float &m_part,
                                                   float &l_part) {
    constexpr int D = 128;
    const int t = threadIdx.x, lane = t & 63, wid = t >> 6, pj = lane >> 3, ds = lane & 7;
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int k = 0; k < 16; k++) st.acc[g][k] = sum_x8(st.acc[g][k]);
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) { wm[wid][g] = st.m[g]; wl[wid][g] = st.l[g]; }
    }
    if (pj == 0) {
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int k = 0; k < 16; k++) wacc[wid][g][KvSlice<KVT>::dim(k, ds)] = st.acc[g][k];
    }
    __syncthreads();
    const int gq = (t >> 7) & 1, d = t & 127;
    o_part = 0.0f;
    m_part = -INFINITY;
    l_part = 0.0f;
    if (t < G * D) {
#pragma unroll
        for (int w = 0; w < NW; w++) m_part = fmaxf(m_part, wm[w][gq]);
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float f = wm[w][gq] == -INFINITY ? 0.0f : expf(__fsub_rn(wm[w][gq], m_part));
            o_part = fmaf(wacc[w][gq][d], f, o_part);
            l_part = fmaf(wl[w][gq], f, l_part);
        }
    }
}

// DEC: 0 operator mode (position argument, even split of the context);
// 1 decode step (device state, static partition, loads before the position
// arrives); 2 multi-stream decode step: k_qk_prep_rows has already normed and
// rotated q and written the new K/V row; the per-stream partition and
// position are read first, so that no row past a stream's context is fetched;
// 3 as 2 with one group in flight per wave (fewer registers, more resident
// blocks; the groups are consumed in the same order)
template <typename KVT, int NW, bool MERGE, int DEC>
__global__ __launch_bounds__(NW * 64) void k_attn_decode(AttnDecodeArgs a) {
    constexpr int D = 128, G = 2;
    using Sl = KvSlice<KVT>;
    __shared__ float wm[NW][G], wl[NW][G];
    __shared__ float wacc[NW][G][D];
    __shared__ float mw[G][ATT_MAXS], lw[G][ATT_MAXS];
    __shared__ int last;
    const int t = threadIdx.x, lane = t & 63;
    const int wid = __builtin_amdgcn_readfirstlane(t >> 6);
    const int pj = lane >> 3, ds = lane & 7;
    const int n_split = a.n_split;
    const int kvh = blockIdx.x / n_split, split = blockIdx.x % n_split;
    const int Hkv = gridDim.x / n_split, Hq = Hkv * G;
    constexpr bool prep = DEC == 1;                      // raw projections: norm + rope + cache write
    // stream of a multi-stream step (0 otherwise): its cache, q/k/v row,
    // position, RoPE rows and partials
    const int bs = (DEC >= 2 && a.stream_order) ? a.stream_order[blockIdx.y] : (int)blockIdx.y;
    KVT *kc = reinterpret_cast<KVT *>(a.kcache) + bs * a.batch_kv_stride + (int64_t)kvh * a.head_stride;
    KVT *vc = reinterpret_cast<KVT *>(a.vcache) + bs * a.batch_kv_stride + (int64_t)kvh * a.head_stride;
    const float *qkv = a.qkv + bs * a.batch_qkv_stride;
    float *partb = a.part + bs * a.batch_part_stride;

    // ---- loads, all issued before the first wait.  Decode-step mode (DEC):
    // the block owns groups [split gpb, (split + 1) gpb) (gpb per stream in a
    // multi-stream step) whatever the
    // position, so the first two groups of each wave are requested before the
    // position (device state) arrives; rows past the cache read row 0 and
    // everything past the context is masked later (the new K/V row's slot is
    // read too and replaced).  The RoPE rows of the position come from
    // rope_cur.  Operator mode: the position is an argument and the context is
    // split evenly.  Every load is unconditional (dummy addresses when unused):
    // a branch around a load makes the compiler wait for it at the join.
    Sl ka, va, kb, vb;
    float q[G][16];
    float cs[16], sn[16], qn[16], kn[16], vn[16], knw[16];
    int pos, g0, g1s;
    if constexpr (DEC >= 2) {
        if (a.select == 2 && a.gpb_dev[bs] <= QASR_STEP_MAX_GPB) return;   // k_attn_step_batch's stream
        // q first: the first group's scores wait for q and that group only
#pragma unroll
        for (int g = 0; g < G; g++) ld16<KVT>(qkv + (kvh * G + g) * D, ds, q[g]);
        pos = a.state[4 * bs + 1];
        const int gpb = a.gpb_dev[bs];
        g0 = split * gpb;
        g1s = g0 + gpb;
        const int max_rows = min((int)(a.head_stride / D), pos + 1);
        const int ja = 8 * (g0 + wid) + pj, jb = ja + 8 * NW;
        const int ra = ja < max_rows ? ja : 0, rb = jb < max_rows ? jb : 0;
        ka.load(kc + (int64_t)ra * D, ds);
        va.load(vc + (int64_t)ra * D, ds);
        if constexpr (DEC == 2) {
            kb.load(kc + (int64_t)rb * D, ds);
            vb.load(vc + (int64_t)rb * D, ds);
        }
    } else if constexpr (DEC == 1) {
        const int max_rows = (int)(a.head_stride / D), gpb = a.gpb;
        g0 = split * gpb;
        g1s = g0 + gpb;
        const int ja = 8 * (g0 + wid) + pj, jb = ja + 8 * NW;
        const int ra = ja < max_rows ? ja : 0, rb = jb < max_rows ? jb : 0;
        ka.load(kc + (int64_t)ra * D, ds);
        va.load(vc + (int64_t)ra * D, ds);
        kb.load(kc + (int64_t)rb * D, ds);
        vb.load(vc + (int64_t)rb * D, ds);
#pragma unroll
        for (int g = 0; g < G; g++) ld16<KVT>(qkv + (kvh * G + g) * D, ds, q[g]);
        ld16<KVT>(a.q_norm, ds, qn);
        ld16<KVT>(a.k_norm, ds, knw);
        ld16<KVT>(qkv + Hq * D + kvh * D, ds, kn);
        ld16<KVT>(qkv + Hq * D + Hkv * D + kvh * D, ds, vn);
        ld16<KVT>(a.rope_cur + 256 * bs, ds, cs);
        ld16<KVT>(a.rope_cur + 256 * bs + D, ds, sn);
        pos = a.state[4 * bs + 1];
    } else {
#pragma unroll
        for (int g = 0; g < G; g++) ld16<KVT>(qkv + (kvh * G + g) * D, ds, q[g]);
        pos = a.pos;
        const int n_grp = (pos + 8) >> 3;
        const int gpb = (n_grp + n_split - 1) / n_split;
        g0 = split * gpb;
        g1s = g0 + gpb;
        const int j0 = 8 * g0, j1 = min(pos + 1, 8 * min(n_grp, g1s));
        const int ja = 8 * (g0 + wid) + pj, jb = ja + 8 * NW;
        const int ra = ja < j1 ? ja : j0, rb = jb < j1 ? jb : j0;
        ka.load(kc + (int64_t)ra * D, ds);
        va.load(vc + (int64_t)ra * D, ds);
        kb.load(kc + (int64_t)rb * D, ds);
        vb.load(vc + (int64_t)rb * D, ds);
    }
    const int L = pos + 1;
    const int n_grp = (L + 7) >> 3;
    const int g1 = min(n_grp, g1s);
    const int j0 = 8 * g0, j1 = min(L, 8 * g1);
    const bool own_pos = prep && j0 <= pos && pos < j1;
    const int skip = own_pos ? pos : -1;
    // rows of group grp once the context is known: out-of-range and the new
    // position read row j0 (< j1 whenever the block has a group to stream)
    auto row_of = [&](int grp) {
        const int j = 8 * grp + pj;
        return (j < j1 && j != skip) ? j : j0;
    };
    __builtin_amdgcn_sched_barrier(0);

    // ---- query heads: per-head RMSNorm + RoPE; the new K/V row -------------
    if (prep) {
#pragma unroll
        for (int g = 0; g < G; g++) norm_rope16(q[g], qn, cs, sn, a.eps);
    }
    if (own_pos) {
        norm_rope16(kn, knw, cs, sn, a.eps);
#pragma unroll
        for (int k = 0; k < 16; k++) {     // the values the cache holds (a bf16 cache rounds)
            kn[k] = round_kv<KVT>(kn[k]);
            vn[k] = round_kv<KVT>(vn[k]);
        }
        if (wid == 0 && pj == 0) {
            Sl::store(kc + (int64_t)pos * D, ds, kn);
            Sl::store(vc + (int64_t)pos * D, ds, vn);
        }
    }

    // ---- stream this wave's groups (two in flight) -------------------------
    AttnAcc<G> acc;
    acc.init();
    const float scale = a.scale;
    auto consume = [&](const Sl &kt, const Sl &vt, int grp) {
        float kf[16], vf[16];
        kt.to_f32(kf);
        vt.to_f32(vf);
        const int j = 8 * grp + pj;
        if (j == skip) {
#pragma unroll
            for (int k = 0; k < 16; k++) { kf[k] = kn[k]; vf[k] = vn[k]; }
        }
        acc.consume(q, kf, vf, j < j1, scale);
    };
    auto load = [&](Sl &kt, Sl &vt, int grp) {
        const int j = row_of(grp);
        kt.load(kc + (int64_t)j * D, ds);
        vt.load(vc + (int64_t)j * D, ds);
    };
    // The refills are unconditional (past the run they read row j0 again): a
    // load under a branch leaves the buffer's registers with two definitions,
    // and the copy the compiler then makes at the loop edge waits for every
    // load in flight, the other buffer's included.
    if constexpr (DEC == 3) {
        for (int gi = g0 + wid; gi < g1; gi += NW) {
            consume(ka, va, gi);
            load(ka, va, gi + NW);
        }
    } else {
        for (int gi = g0 + wid; gi < g1; gi += 2 * NW) {
            consume(ka, va, gi);
            load(ka, va, gi + 2 * NW);
            const int gb = gi + NW;
            if (gb < g1) consume(kb, vb, gb);
            load(kb, vb, gb + 2 * NW);
        }
    }

    // ---- merge the lanes of each wave, then the waves of the block ----------
    const int gq = (t >> 7) & 1, d = t & 127;    // threads t < 256: (query head, dim)
    float o_part, m_part, l_part;
    attn_block_partial<KVT, NW, G>(acc, wm, wl, wacc, o_part, m_part, l_part);
    if (!MERGE) {
        // the consumer (the o_proj kernel or a merge kernel) merges; the kernel
        // boundary publishes these.  (m, l) of head h = G kvh + gq at
        // [(2 h + {0,1}) S + split]; o as part_o_index lays it out (the
        // multi-stream step: split index slowest, so the stores coalesce).
        if (t < G * D) {
            const int h = kvh * G + gq;
            const int64_t oi = DEC >= 2 ? part_o_index_slow(n_split, split, Hq, h * D + d)
                                        : part_o_index(n_split, split, Hq, h * D + d);
            partb[oi] = o_part;
            if (d == 0) {
                partb[(2 * h) * n_split + split] = m_part;
                partb[(2 * h + 1) * n_split + split] = l_part;
            }
        }
        return;
    }
    float *part = a.part + ((int64_t)kvh * n_split + split) * G * (D + 2);
    if (t < G * D) {
        st_agent(part + gq * (D + 2) + 2 + d, o_part);
        if (d == 0) {
            st_agent(part + gq * (D + 2), m_part);
            st_agent(part + gq * (D + 2) + 1, l_part);
        }
    }
    if (!arrive_last(a.counters + kvh, (unsigned)n_split, &last)) return;
    // ---- last block of this KV head: log-sum-exp merge of the n_split partials
    const float *pb = a.part + (int64_t)kvh * n_split * G * (D + 2);
    for (int i = t; i < n_split * G; i += NW * 64) {
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
    if (t < G * D) {
        float ot = 0.0f;
        for (int s0 = 0; s0 < n_split; s0 += 8) {
            float ov[8];
#pragma unroll
            for (int i = 0; i < 8; i++)
                ov[i] = s0 + i < n_split ? ld_agent(pb + ((s0 + i) * G + gq) * (D + 2) + 2 + d) : 0.0f;
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (s0 + i < n_split) ot = fmaf(ov[i], mw[gq][s0 + i], ot);
        }
        const float lt = lw[gq][0];
        a.out[(kvh * G + gq) * D + d] = lt > 0.0f ? __fdiv_rn(ot, lt) : 0.0f;
    }
    if (t == 0) reset_counter(a.counters + kvh);
}

// ---------------------------------------------------------------------------
// GQA decode attention of one decode step (the DEC = 1 case above, same
// inputs, partial format and numerics contract), laid out for a short
// dependent chain per wave.  A block serves ONE query head and one context
// split: grid = Hkv x 2 x n_split with the KV head fastest, so the two query
// heads of a KV head and all its splits go to one XCD (blocks go round-robin
// over the 8 XCDs) and read the same K/V rows through that XCD's L2, and twice
// as many CUs share the work as with both query heads in one block.  Lane l
// owns dims 2l and 2l + 1 of every position: a group's 8 K rows and 8 V rows
// are 16 loads of 8 (f32) or 4 (bf16) bytes per lane, each instruction
// covering whole rows.  Per group a lane forms 2-term partial dots for the 8
// positions, and one reduce-scatter over the wave (a permlane32 swap, a
// permlane16 swap and a row_ror:8 DPP step, then three DPP sums) leaves every
// lane one finished score: lanes are position slots, replicated 8 times.  The
// softmax over the wave's 8 x GPW positions takes 3 cross-lane steps; the
// probabilities go through LDS (8 floats per group, two 16-byte reads per
// lane), and since each lane already owns its dims, P V needs no cross-lane
// sum and no branch (positions past the context have probability 0 and their
// V operand is replaced by 0).  The RoPE pair (d, d + 64) sits in lanes l and
// l + 32 (one permlane32 swap).
// ---------------------------------------------------------------------------
template <typename T> struct KvPair;
template <> struct KvPair<float> {
    float2 v;
    __device__ __forceinline__ void load(const float *row, int lane) { v = reinterpret_cast<const float2 *>(row)[lane]; }
    __device__ __forceinline__ float x() const { return v.x; }
    __device__ __forceinline__ float y() const { return v.y; }
    __device__ __forceinline__ void set(float a, float b) { v = make_float2(a, b); }
    static __device__ __forceinline__ void store(float *row, int lane, float a, float b) {
        reinterpret_cast<float2 *>(row)[lane] = make_float2(a, b);
    }
};
template <> struct KvPair<uint16_t> {
    uint32_t v;
    __device__ __forceinline__ void load(const uint16_t *row, int lane) {
        v = reinterpret_cast<const uint32_t *>(row)[lane];
    }
    __device__ __forceinline__ float x() const { return __uint_as_float(v << 16); }
    __device__ __forceinline__ float y() const { return __uint_as_float(v & 0xFFFF0000u); }
    __device__ __forceinline__ void set(float a, float b) {
        v = (uint32_t)f32_to_bf16_rne(a) | ((uint32_t)f32_to_bf16_rne(b) << 16);
    }
    static __device__ __forceinline__ void store(uint16_t *row, int lane, float a, float b) {
        reinterpret_cast<uint32_t *>(row)[lane] = (uint32_t)f32_to_bf16_rne(a) | ((uint32_t)f32_to_bf16_rne(b) << 16);
    }
};

// full-wave sum, every lane receives it
__device__ __forceinline__ float wave_allsum(float v) { return sum_x8(sum8(v)); }

// the two halves of a swap: first operand's lanes 32-63 exchanged with the
// second's lanes 0-31 (and rows 1/3 with rows 0/2 for the 16-lane form)
__device__ __forceinline__ float swap32_add(float keep_lo, float keep_hi) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(keep_lo), __float_as_uint(keep_hi), false, false);
    return __fadd_rn(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float swap16_add(float keep_even, float keep_odd) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(keep_even), __float_as_uint(keep_odd), false, false);
    return __fadd_rn(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

// per-head RMSNorm + NeoX RoPE of one 128-dim head held as dims (2l, 2l + 1)
__device__ __forceinline__ float2 norm_rope2(float2 x, float2 w, float2 c, float2 s, float eps) {
    constexpr int D = 128;
    const float ss = wave_allsum(fmaf(x.y, x.y, __fmul_rn(x.x, x.x)));
    const float r = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(div_by_count(ss, D), eps)));
    x.x = __fmul_rn(__fmul_rn(x.x, r), w.x);
    x.y = __fmul_rn(__fmul_rn(x.y, r), w.y);
    // partner dims d +- 64 live in lane l ^ 32
    const auto px = __builtin_amdgcn_permlane32_swap(__float_as_uint(x.x), __float_as_uint(x.x), false, false);
    const auto py = __builtin_amdgcn_permlane32_swap(__float_as_uint(x.y), __float_as_uint(x.y), false, false);
    const bool lo = (threadIdx.x & 32) == 0;
    // one of the two results is this lane's own value, the other its partner's
    // (whichever way round the swap returns them; equal bits mean equal values)
    const float qx = __uint_as_float(px[0] == __float_as_uint(x.x) ? px[1] : px[0]);
    const float qy = __uint_as_float(py[0] == __float_as_uint(x.y) ? py[1] : py[0]);
    float2 o;
    if (lo) {   // x1 = own, x2 = partner
        o.x = __fadd_rn(__fmul_rn(x.x, c.x), __fmul_rn(-qx, s.x));
        o.y = __fadd_rn(__fmul_rn(x.y, c.y), __fmul_rn(-qy, s.y));
    } else {    // x2 = own, x1 = partner
        o.x = __fadd_rn(__fmul_rn(x.x, c.x), __fmul_rn(qx, s.x));
        o.y = __fadd_rn(__fmul_rn(x.y, c.y), __fmul_rn(qy, s.y));
    }
    return o;
}

// A wave holds its whole share of the block's run, groups g0 + wid + NW i
// for i < GPW (the host launches it only for runs of at most NW GPW groups):
// every group's scores, one max over all of them, then P V.  Rows the run
// leaves out are masked (scores -inf, probabilities 0, V operands 0).  The
// block of query head 0 of the KV head that holds the position writes the
// new K/V row; the other query head's block forms the same values for its
// own score and P V term.
//
// POLL (the attention blocks of k_qkv_attn, NW + 1 waves): q, the new k and
// the new v come from a.qkv_tag as (tag, value) pairs that blocks of the same
// launch store.  Wave NW only polls: it keeps two polls of its 6 pairs per
// lane in flight (its loads do not queue behind K/V rows, which complete in
// issue order), and once all carry this step's tag (state[4] x 32 + layer) it
// forms the normed, rotated q and k, writes the new K/V row and hands q, k, v
// to the K/V waves through LDS (one barrier).  A poll that has not matched
// after QASR_POLL_SPINS rounds sets *a.fault and goes on (the host reports
// the step as failed), so every wave ends.
#define QASR_POLL_SPINS (1 << 18)
//
// BATCH (k_attn_step_batch, the multi-stream step): grid row y is stream
// bs = stream_order[y]; each stream has its own cache slot, qkv row, position,
// RoPE rows, partials (split index slowest) and groups per block gpb_dev[bs]
// (its solo partition), and the waves load only their ceil(gpb / NW) groups
// (row 0 stands in for the rest, which the partition masks: they add exact
// zeros), so every stream gets the bits of the single-stream kernel run with
// its own GPW.
template <typename KVT, int NW, int GPW, bool POLL, bool BATCH = false>
__device__ __forceinline__ void attn_step_block(const AttnDecodeArgs &a, int blk, int nblk, int blk0 = 0) {
    constexpr int D = 128, G = 2;
    using Kp = KvPair<KVT>;
    unsigned long long *stamp = nullptr;
#ifdef QASR_STAMPS
    // fused launch: slots 0-7 by wave 0, 8 by the polling wave
    if (POLL && a.stamps) stamp = a.stamps + ((int64_t)a.layer * QASR_STAMP_BLOCKS + blockIdx.x) * QASR_STAMP_SLOTS;
    if ((threadIdx.x >> 6) == 0) QASR_STAMP(stamp, 0);
#endif
    (void)blk0;
    __shared__ float wm[NW], wl[NW];
    __shared__ float wacc[NW][D];
    __shared__ __attribute__((aligned(16))) float pw[NW][GPW][8];
    __shared__ float2 hq[POLL ? 64 : 1], hk[POLL ? 64 : 1], hv[POLL ? 64 : 1];
    const int t = threadIdx.x, lane = t & 63;
    const int wid = __builtin_amdgcn_readfirstlane(t >> 6);
    const int n_split = a.n_split;
    const int Hkv = nblk / (G * n_split), Hq = Hkv * G;
    const int kvh = blk % Hkv, gq = (blk / Hkv) % G, split = blk / (G * Hkv);
    const int h = kvh * G + gq;
    const int bs = BATCH ? (a.stream_order ? a.stream_order[blockIdx.y] : (int)blockIdx.y) : 0;
    KVT *kc = reinterpret_cast<KVT *>(a.kcache) + (BATCH ? bs * a.batch_kv_stride : 0) + (int64_t)kvh * a.head_stride;
    KVT *vc = reinterpret_cast<KVT *>(a.vcache) + (BATCH ? bs * a.batch_kv_stride : 0) + (int64_t)kvh * a.head_stride;
    const float *qkv = a.qkv + (BATCH ? bs * a.batch_qkv_stride : 0);
    float *part = a.part + (BATCH ? bs * a.batch_part_stride : 0);
    const float *rope_cur = a.rope_cur + (BATCH ? 256 * bs : 0);
    const int gpb = BATCH ? a.gpb_dev[bs] : a.gpb, g0 = split * gpb, g1s = g0 + gpb;
    const int gpw_own = BATCH ? (gpb + NW - 1) / NW : GPW;     // groups this stream's waves hold
    // rows loaded: the whole cache (the static partition needs no position),
    // or in a multi-stream step the stream's context (its position is loaded
    // with its partition anyway), so blocks and groups past it read row 0
    const int max_rows = BATCH ? min((int)(a.head_stride / D), a.state[4 * bs + 1] + 1) : (int)(a.head_stride / D);
    if (BATCH && 8 * g0 >= max_rows) {
        // a block wholly past the stream's context: an empty partial
        if (t < D) {
            part[part_o_index_slow(n_split, split, Hq, h * D + t)] = 0.0f;
            if (t == 0) {
                part[(2 * h) * n_split + split] = -INFINITY;
                part[(2 * h + 1) * n_split + split] = 0.0f;
            }
        }
        return;
    }

    // ---- every load before the first wait, the previous kernel's outputs
    // (q, the new k/v, the position) first, so that waiting for them does not
    // wait for the K/V rows (loads complete in issue order); the static
    // partition needs no device state, so the K rows, then the V rows, go out
    // before the position arrives (rows past the cache read row 0; everything
    // past the context is masked once the position is known)
    if (POLL && wid == NW) {
        // ---- the polling wave
        const float2 qn = reinterpret_cast<const float2 *>(a.q_norm)[lane];
        const float2 knw = reinterpret_cast<const float2 *>(a.k_norm)[lane];
        const float2 cs = reinterpret_cast<const float2 *>(rope_cur)[lane];
        const float2 sn = reinterpret_cast<const float2 *>(rope_cur + D)[lane];
        const int pos = a.state[1];
        const unsigned tag = (unsigned)a.state[4] * 32u + (unsigned)a.layer;
        const unsigned long long *tq = a.qkv_tag + h * D + 2 * lane;
        const unsigned long long *tk = a.qkv_tag + Hq * D + kvh * D + 2 * lane;
        const unsigned long long *tv = a.qkv_tag + Hq * D + Hkv * D + kvh * D + 2 * lane;
        auto issue = [&](unsigned long long (&u)[6]) {
            u[0] = ld_agent64(tq); u[1] = ld_agent64(tq + 1);
            u[2] = ld_agent64(tk); u[3] = ld_agent64(tk + 1);
            u[4] = ld_agent64(tv); u[5] = ld_agent64(tv + 1);
        };
        auto ready = [&](const unsigned long long (&u)[6]) {
            bool mine = true;
#pragma unroll
            for (int i = 0; i < 6; i++) mine &= (unsigned)(u[i] >> 32) == tag;
            return __all(mine) != 0;
        };
        // two polls in flight: the older one is checked while the newer one travels.
        // After a timed-out hand-off (the fault flag, cleared by the host when it
        // reports the failure) later launches do not wait again, and a wave that
        // has not matched its tags stores no K/V row.
        unsigned long long ua[6], ub[6], u[6];
        bool matched = ld_agent(a.fault) == 0;
        issue(ua);
        for (int spins = 0; matched; spins += 2) {
            __builtin_amdgcn_s_sleep(2);
            issue(ub);
            if (ready(ua)) {
#pragma unroll
                for (int i = 0; i < 6; i++) u[i] = ua[i];
                break;
            }
            __builtin_amdgcn_s_sleep(2);
            issue(ua);
            if (ready(ub)) {
#pragma unroll
                for (int i = 0; i < 6; i++) u[i] = ub[i];
                break;
            }
            if (spins >= QASR_POLL_SPINS) {
                if (lane == 0) st_agent(a.fault, 1);
                matched = false;
                break;
            }
        }
        if (!matched) {
#pragma unroll
            for (int i = 0; i < 6; i++) u[i] = 0;
        }
        QASR_STAMP(stamp, 8);
        float2 q = make_float2(__uint_as_float((unsigned)u[0]), __uint_as_float((unsigned)u[1]));
        float2 kn = make_float2(__uint_as_float((unsigned)u[2]), __uint_as_float((unsigned)u[3]));
        float2 vn = make_float2(__uint_as_float((unsigned)u[4]), __uint_as_float((unsigned)u[5]));
        const int g1 = min((pos + 8) >> 3, g1s);
        const bool own_pos = 8 * g0 <= pos && pos < min(pos + 1, 8 * g1);
        q = norm_rope2(q, qn, cs, sn, a.eps);
        if (own_pos) {
            kn = norm_rope2(kn, knw, cs, sn, a.eps);
            Kp kp, vp;
            kp.set(kn.x, kn.y);      // the values the cache holds (a bf16 cache rounds)
            vp.set(vn.x, vn.y);
            kn = make_float2(kp.x(), kp.y());
            vn = make_float2(vp.x(), vp.y());
            if (gq == 0 && matched) {
                Kp::store(kc + (int64_t)pos * D, lane, kn.x, kn.y);
                Kp::store(vc + (int64_t)pos * D, lane, vn.x, vn.y);
            }
        }
        hq[lane] = q;
        hk[lane] = kn;
        hv[lane] = vn;
        __syncthreads();          // q, k, v to the K/V waves
        __syncthreads();          // their merge
        return;
    }
    float2 q, kn, vn;
    if (!POLL) {
        q = reinterpret_cast<const float2 *>(qkv + h * D)[lane];
        kn = reinterpret_cast<const float2 *>(qkv + Hq * D + kvh * D)[lane];
        vn = reinterpret_cast<const float2 *>(qkv + Hq * D + Hkv * D + kvh * D)[lane];
    }
    const float2 qn = reinterpret_cast<const float2 *>(a.q_norm)[lane];
    const float2 knw = reinterpret_cast<const float2 *>(a.k_norm)[lane];
    const float2 cs = reinterpret_cast<const float2 *>(rope_cur)[lane];
    const float2 sn = reinterpret_cast<const float2 *>(rope_cur + D)[lane];
    const int pos = a.state[BATCH ? 4 * bs + 1 : 1];
    Kp kr[GPW][8], vr[GPW][8];
#pragma unroll
    for (int i = 0; i < GPW; i++)
#pragma unroll
        for (int p = 0; p < 8; p++) {
            const int j = 8 * (g0 + wid + NW * i) + p;
            kr[i][p].load(kc + (int64_t)(i < gpw_own && j < max_rows ? j : 0) * D, lane);
        }
#pragma unroll
    for (int i = 0; i < GPW; i++)
#pragma unroll
        for (int p = 0; p < 8; p++) {
            const int j = 8 * (g0 + wid + NW * i) + p;
            vr[i][p].load(vc + (int64_t)(i < gpw_own && j < max_rows ? j : 0) * D, lane);
        }
    __builtin_amdgcn_sched_barrier(0);
    if (wid == 0) QASR_STAMP(stamp, 1);
    if (POLL) {
        __syncthreads();          // q (normed, rotated), k, v from the polling wave
        q = hq[lane];
        kn = hk[lane];
        vn = hv[lane];
        if (wid == 0) QASR_STAMP(stamp, 2);
    }

    const int L = pos + 1;
    const int g1 = min((L + 7) >> 3, g1s);
    const int j1 = min(L, 8 * g1);
    const bool own_pos = 8 * g0 <= pos && pos < j1;

    // lane -> position slot of the reduce-scatter: bit 2 from the swap32
    // half, bit 1 from the swap16 half (told apart by running the same swaps
    // on indicators), bit 0 = lane bit 3 (row_ror:8)
    const float s32 = swap32_add(0.0f, 1.0f);
    const float s16 = swap16_add(0.0f, 1.0f);
    const int bit3 = (lane >> 3) & 1;
    const int my_p = (s32 > 1.0f ? 4 : 0) + (s16 > 1.0f ? 2 : 0) + bit3;

    // ---- q: per-head RMSNorm + RoPE; the new K/V row (POLL: done by the
    // polling wave) -----------------------------------------------------------
    if (!POLL) {
        q = norm_rope2(q, qn, cs, sn, a.eps);
        if (own_pos) {
            kn = norm_rope2(kn, knw, cs, sn, a.eps);
            Kp kp, vp;
            kp.set(kn.x, kn.y);      // the values the cache holds (a bf16 cache rounds)
            vp.set(vn.x, vn.y);
            kn = make_float2(kp.x(), kp.y());
            vn = make_float2(vp.x(), vp.y());
            if (wid == 0 && gq == 0) {
                Kp::store(kc + (int64_t)pos * D, lane, kn.x, kn.y);
                Kp::store(vc + (int64_t)pos * D, lane, vn.x, vn.y);
            }
        }
    }

    // ---- scores: 2-term partials, one reduce-scatter per group --------------
    float sc[GPW];
#pragma unroll
    for (int i = 0; i < GPW; i++) {
        const int jb = 8 * (g0 + wid + NW * i);
        float v8[8];
#pragma unroll
        for (int p = 0; p < 8; p++) {
            float kx = kr[i][p].x(), ky = kr[i][p].y();
            if (own_pos && jb + p == pos) { kx = kn.x; ky = kn.y; }
            v8[p] = fmaf(q.y, ky, __fmul_rn(q.x, kx));
        }
        float r1[4];
#pragma unroll
        for (int k = 0; k < 4; k++) r1[k] = swap32_add(v8[k], v8[k + 4]);
        float r2[2];
#pragma unroll
        for (int k = 0; k < 2; k++) r2[k] = swap16_add(r1[k], r1[k + 2]);
        float r3;
        {
            const float keep = bit3 ? r2[1] : r2[0], send = bit3 ? r2[0] : r2[1];
            r3 = __fadd_rn(keep, dpp_f32<QASR_DPP_ROW_ROR8>(send));
        }
        // the 8 lanes of a slot (lane bits 0-2) end with identical sums
        r3 = __fadd_rn(r3, dpp_f32<QASR_DPP_ROW_HALF_MIRROR>(r3));
        r3 = __fadd_rn(r3, dpp_f32<QASR_DPP_QP_1032>(r3));
        r3 = __fadd_rn(r3, dpp_f32<QASR_DPP_QP_2301>(r3));
        sc[i] = jb + my_p < j1 ? __fmul_rn(r3, a.scale) : -INFINITY;
    }
    if (wid == 0) QASR_STAMP(stamp, 3);

    // ---- softmax over this wave's positions --------------------------------
    float m = sc[0];
#pragma unroll
    for (int i = 1; i < GPW; i++) m = fmaxf(m, sc[i]);
    m = fmaxf(m, dpp_f32<QASR_DPP_ROW_ROR8>(m));
    m = xrow16_max(m);
    m = xhalf_max(m);
    float pr[GPW], l = 0.0f;
#pragma unroll
    for (int i = 0; i < GPW; i++) {
        pr[i] = m == -INFINITY ? 0.0f : expf(__fsub_rn(sc[i], m));
        l = __fadd_rn(l, pr[i]);
    }
    if ((lane & 7) == 0) {      // one lane per position slot
#pragma unroll
        for (int i = 0; i < GPW; i++) pw[wid][i][my_p] = pr[i];
    }
    l = __fadd_rn(l, dpp_f32<QASR_DPP_ROW_ROR8>(l));
    l = xrow16_sum(l);
    l = xhalf_sum(l);
    if (wid == 0) QASR_STAMP(stamp, 4);

    // ---- P V: probabilities from LDS (the wave's own writes) ----------------
    float ox = 0.0f, oy = 0.0f;
#pragma unroll
    for (int i = 0; i < GPW; i++) {
        float P[8];
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const float4 v4 = reinterpret_cast<const float4 *>(&pw[wid][i][0])[k];
            P[4 * k] = v4.x; P[4 * k + 1] = v4.y; P[4 * k + 2] = v4.z; P[4 * k + 3] = v4.w;
        }
        const int jb = 8 * (g0 + wid + NW * i);
        float gx = 0.0f, gy = 0.0f;
#pragma unroll
        for (int p = 0; p < 8; p++) {
            const bool live = jb + p < j1;
            float vx = live ? vr[i][p].x() : 0.0f, vy = live ? vr[i][p].y() : 0.0f;
            if (own_pos && jb + p == pos) { vx = vn.x; vy = vn.y; }
            gx = fmaf(P[p], vx, gx);
            gy = fmaf(P[p], vy, gy);
        }
        ox = __fadd_rn(ox, gx);
        oy = __fadd_rn(oy, gy);
    }
    if (wid == 0) QASR_STAMP(stamp, 5);

    // ---- merge the waves of the block (LDS, one barrier) --------------------
    if (lane == 0) { wm[wid] = m; wl[wid] = l; }
    reinterpret_cast<float2 *>(&wacc[wid][0])[lane] = make_float2(ox, oy);
    __syncthreads();
    if (wid == 0) QASR_STAMP(stamp, 6);
    if (t < D) {
        const int d = t;
        float m_part = -INFINITY, o_part = 0.0f, l_part = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) m_part = fmaxf(m_part, wm[w]);
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float f = wm[w] == -INFINITY ? 0.0f : expf(__fsub_rn(wm[w], m_part));
            o_part = fmaf(wacc[w][d], f, o_part);
            l_part = fmaf(wl[w], f, l_part);
        }
        part[BATCH ? part_o_index_slow(n_split, split, Hq, h * D + d) : part_o_index(n_split, split, Hq, h * D + d)] =
            o_part;
        if (d == 0) {
            part[(2 * h) * n_split + split] = m_part;
            part[(2 * h + 1) * n_split + split] = l_part;
        }
        if (wid == 0) QASR_STAMP(stamp, 7);
    }
}

template <typename KVT, int NW, int GPW>
__global__ __launch_bounds__(NW * 64) void k_attn_step(AttnDecodeArgs a) {
    attn_step_block<KVT, NW, GPW, false>(a, blockIdx.x, gridDim.x);
}

// ---------------------------------------------------------------------------
// Multi-stream form of k_attn_step (f32 cache): the same waves, lanes and
// arithmetic per query head, so every stream gets the bits of the
// single-stream kernel run alone on its context (its partition gpb_dev, its
// split count).  For throughput over many streams:
//  * a block serves both query heads of its KV head (k_attn_step gives each
//    its own block): it loads the K/V rows once and forms the two heads'
//    scores, softmaxes and P V side by side, each with the single-head
//    kernel's operations and order; the 4 waves' merge then runs one head per
//    128 threads;
//  * a wave's K groups (its share of the stream's partition, not the
//    launch's maximum) all go out at entry; its V groups go out once the
//    scores are formed, into the same registers, and arrive while the
//    softmax runs (101 VGPRs, 4 waves per SIMD at 4 groups per wave).
//    Measured on config 4 (us per layer): both heads per block with one
//    group of K, then of V, in flight 46.2; all groups in flight 43.3; one
//    head per block, one group in flight 54.3, or the whole run of K and V
//    in registers at once 69.9.
// Groups past the stream's context read row 0 (masked, adding exact zeros);
// blocks wholly past it store empty partials and leave.  Grid row y is
// stream stream_order[y]; grid column kvh + Hkv x split; partials go split
// index slowest.
// ---------------------------------------------------------------------------
template <int NW, int GPW>
__global__ __launch_bounds__(NW * 64) void k_attn_step_batch(AttnDecodeArgs a) {
    constexpr int D = 128, G = 2;
    using Kp = KvPair<float>;
    __shared__ float wm[G][NW], wl[G][NW];
    __shared__ float wacc[G][NW][D];
    __shared__ __attribute__((aligned(16))) float pw[G][NW][GPW][8];
    const int t = threadIdx.x, lane = t & 63;
    const int wid = __builtin_amdgcn_readfirstlane(t >> 6);
    const int n_split = a.n_split;
    const int Hkv = gridDim.x / n_split, Hq = Hkv * G;
    const int blk = blockIdx.x;
    const int kvh = blk % Hkv, split = blk / Hkv;
    const int h0 = kvh * G;                          // query heads h0 and h0 + 1
    const int bs = a.stream_order ? a.stream_order[blockIdx.y] : (int)blockIdx.y;
    float *kc = reinterpret_cast<float *>(a.kcache) + bs * a.batch_kv_stride + (int64_t)kvh * a.head_stride;
    float *vc = reinterpret_cast<float *>(a.vcache) + bs * a.batch_kv_stride + (int64_t)kvh * a.head_stride;
    const float *qkv = a.qkv + bs * a.batch_qkv_stride;
    float *part = a.part + bs * a.batch_part_stride;
    const float *rope_cur = a.rope_cur + 256 * bs;
    const int gpb = a.gpb_dev[bs], g0 = split * gpb, g1s = g0 + gpb;
    if (a.select == 1 && gpb > QASR_STEP_MAX_GPB) return;     // k_attn_decode's stream this step
    const int gpw_own = (gpb + NW - 1) / NW;
    const int pos = a.state[4 * bs + 1];
    const int max_rows = min((int)(a.head_stride / D), pos + 1);
    // thread t < 2 D stores head h0 + t / D's column t % D of an early partial
    auto early_partial = [&](float o, float m_v, float l_v) {
        if (t < G * D) {
            const int h = h0 + t / D, d = t % D;
            part[part_o_index_slow(n_split, split, Hq, h * D + d)] = o;
            if (d == 0) {
                part[(2 * h) * n_split + split] = m_v;
                part[(2 * h + 1) * n_split + split] = l_v;
            }
        }
    };
    if (gpw_own > GPW) {
        // a partition longer than this launch's waves hold (the host sizes GPW
        // from its per-position table): NaN partials and the fault flag the
        // host checks, never a silent drop of groups
        const float nan = __builtin_nanf("");
        early_partial(nan, nan, nan);
        if (t == 0 && a.fault) st_agent(a.fault, 1);
        return;
    }
    if (8 * g0 >= max_rows) {
        early_partial(0.0f, -INFINITY, 0.0f);        // a block wholly past the stream's context
        return;
    }
    auto row_of = [&](int i, int p) {
        const int j = 8 * (g0 + wid + NW * i) + p;
        return (int64_t)(i < gpw_own && j < max_rows ? j : 0) * D;
    };
    // q of both heads, the new k/v and the first K group
    float2 q[G];
#pragma unroll
    for (int g = 0; g < G; g++) q[g] = reinterpret_cast<const float2 *>(qkv + (h0 + g) * D)[lane];
    float2 kn = reinterpret_cast<const float2 *>(qkv + Hq * D + kvh * D)[lane];
    float2 vn = reinterpret_cast<const float2 *>(qkv + Hq * D + Hkv * D + kvh * D)[lane];
    const float2 qn = reinterpret_cast<const float2 *>(a.q_norm)[lane];
    const float2 knw = reinterpret_cast<const float2 *>(a.k_norm)[lane];
    const float2 cs = reinterpret_cast<const float2 *>(rope_cur)[lane];
    const float2 sn = reinterpret_cast<const float2 *>(rope_cur + D)[lane];
    Kp kr[GPW][8];
#pragma unroll
    for (int i = 0; i < GPW; i++)
        if (i < gpw_own) {                            // uniform
#pragma unroll
            for (int p = 0; p < 8; p++) kr[i][p].load(kc + row_of(i, p), lane);
        }
    __builtin_amdgcn_sched_barrier(0);

    const int L = pos + 1;
    const int g1 = min((L + 7) >> 3, g1s);
    const int j1 = min(L, 8 * g1);
    const bool own_pos = 8 * g0 <= pos && pos < j1;
    const float s32 = swap32_add(0.0f, 1.0f);
    const float s16 = swap16_add(0.0f, 1.0f);
    const int bit3 = (lane >> 3) & 1;
    const int my_p = (s32 > 1.0f ? 4 : 0) + (s16 > 1.0f ? 2 : 0) + bit3;
#pragma unroll
    for (int g = 0; g < G; g++) q[g] = norm_rope2(q[g], qn, cs, sn, a.eps);
    if (own_pos) {
        kn = norm_rope2(kn, knw, cs, sn, a.eps);
        if (wid == 0) {
            Kp::store(kc + (int64_t)pos * D, lane, kn.x, kn.y);
            Kp::store(vc + (int64_t)pos * D, lane, vn.x, vn.y);
        }
    }

    // ---- pass 1: scores --------------------------------------------------------
    float sc[G][GPW];
#pragma unroll
    for (int i = 0; i < GPW; i++) {
#pragma unroll
        for (int g = 0; g < G; g++) sc[g][i] = -INFINITY;
        if (i >= gpw_own) continue;                   // uniform
        const int jb = 8 * (g0 + wid + NW * i);
#pragma unroll
        for (int g = 0; g < G; g++) {
            float v8[8];
#pragma unroll
            for (int p = 0; p < 8; p++) {
                float kx = kr[i][p].x(), ky = kr[i][p].y();
                if (own_pos && jb + p == pos) { kx = kn.x; ky = kn.y; }
                v8[p] = fmaf(q[g].y, ky, __fmul_rn(q[g].x, kx));
            }
            float r1[4];
#pragma unroll
            for (int k = 0; k < 4; k++) r1[k] = swap32_add(v8[k], v8[k + 4]);
            float r2[2];
#pragma unroll
            for (int k = 0; k < 2; k++) r2[k] = swap16_add(r1[k], r1[k + 2]);
            float r3;
            {
                const float keep = bit3 ? r2[1] : r2[0], send = bit3 ? r2[0] : r2[1];
                r3 = __fadd_rn(keep, dpp_f32<QASR_DPP_ROW_ROR8>(send));
            }
            r3 = __fadd_rn(r3, dpp_f32<QASR_DPP_ROW_HALF_MIRROR>(r3));
            r3 = __fadd_rn(r3, dpp_f32<QASR_DPP_QP_1032>(r3));
            r3 = __fadd_rn(r3, dpp_f32<QASR_DPP_QP_2301>(r3));
            sc[g][i] = jb + my_p < j1 ? __fmul_rn(r3, a.scale) : -INFINITY;
        }
    }
    // every V group goes out while the softmax forms (into the K rows' registers)
    Kp vr[GPW][8];
#pragma unroll
    for (int i = 0; i < GPW; i++)
        if (i < gpw_own) {                            // uniform
#pragma unroll
            for (int p = 0; p < 8; p++) vr[i][p].load(vc + row_of(i, p), lane);
        }

    // ---- softmax over this wave's positions (the single-stream order) -------
    float m[G], l[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        float mg = sc[g][0];
#pragma unroll
        for (int i = 1; i < GPW; i++) mg = fmaxf(mg, sc[g][i]);
        mg = fmaxf(mg, dpp_f32<QASR_DPP_ROW_ROR8>(mg));
        mg = xrow16_max(mg);
        mg = xhalf_max(mg);
        float pr[GPW], lg = 0.0f;
#pragma unroll
        for (int i = 0; i < GPW; i++) {
            pr[i] = mg == -INFINITY ? 0.0f : expf(__fsub_rn(sc[g][i], mg));
            if (i < gpw_own) lg = __fadd_rn(lg, pr[i]);
        }
        if ((lane & 7) == 0) {
#pragma unroll
            for (int i = 0; i < GPW; i++) pw[g][wid][i][my_p] = pr[i];
        }
        lg = __fadd_rn(lg, dpp_f32<QASR_DPP_ROW_ROR8>(lg));
        lg = xrow16_sum(lg);
        lg = xhalf_sum(lg);
        m[g] = mg;
        l[g] = lg;
    }

    // ---- pass 2: P V ------------------------------------------------------------
    float ox[G] = {0.0f, 0.0f}, oy[G] = {0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < GPW; i++) {
        if (i >= gpw_own) continue;                   // uniform
        const int jb = 8 * (g0 + wid + NW * i);
#pragma unroll
        for (int g = 0; g < G; g++) {
            float P[8];
#pragma unroll
            for (int k = 0; k < 2; k++) {
                const float4 v4 = reinterpret_cast<const float4 *>(&pw[g][wid][i][0])[k];
                P[4 * k] = v4.x; P[4 * k + 1] = v4.y; P[4 * k + 2] = v4.z; P[4 * k + 3] = v4.w;
            }
            float gx = 0.0f, gy = 0.0f;
#pragma unroll
            for (int p = 0; p < 8; p++) {
                const bool live = jb + p < j1;
                float vx = live ? vr[i][p].x() : 0.0f, vy = live ? vr[i][p].y() : 0.0f;
                if (own_pos && jb + p == pos) { vx = vn.x; vy = vn.y; }
                gx = fmaf(P[p], vx, gx);
                gy = fmaf(P[p], vy, gy);
            }
            ox[g] = __fadd_rn(ox[g], gx);
            oy[g] = __fadd_rn(oy[g], gy);
        }
    }

    // ---- merge the waves of the block per head (LDS, one barrier) -----------
#pragma unroll
    for (int g = 0; g < G; g++) {
        if (lane == 0) { wm[g][wid] = m[g]; wl[g][wid] = l[g]; }
        reinterpret_cast<float2 *>(&wacc[g][wid][0])[lane] = make_float2(ox[g], oy[g]);
    }
    __syncthreads();
    if (t < G * D) {
        const int g = t / D, d = t % D, h = h0 + g;
        float m_part = -INFINITY, o_part = 0.0f, l_part = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) m_part = fmaxf(m_part, wm[g][w]);
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float f = wm[g][w] == -INFINITY ? 0.0f : expf(__fsub_rn(wm[g][w], m_part));
            o_part = fmaf(wacc[g][w][d], f, o_part);
            l_part = fmaf(wl[g][w], f, l_part);
        }
        part[part_o_index_slow(n_split, split, Hq, h * D + d)] = o_part;
        if (d == 0) {
            part[(2 * h) * n_split + split] = m_part;
            part[(2 * h + 1) * n_split + split] = l_part;
        }
    }
}

// ---------------------------------------------------------------------------
// One launch for a layer's RMSNorm + qkv matvec and its decode attention.
// Blocks [0, n_mv) are the qkv matvec (w8a8_wave with the layer-0 embedding
// gather when EMBED), each row published as a (tag, value) pair in a.qkv_tag;
// blocks [n_mv, grid) are k_attn_step's blocks, which issue their K/V loads at
// once and then poll the pairs of their query head and KV head.  Workgroups
// are dispatched in index order, so every matvec block has been dispatched
// before any attention block waits: the waits end whatever the occupancy.
// Tags are state[4] x 32 + layer: the LM-head merge advances state[4] once per
// step, so a pair left by an earlier step or layer never matches.  The
// values, and so the attention's outputs, are bit-identical to the two
// separate launches'.
// ---------------------------------------------------------------------------
template <typename KVT, int GPW, int NS, int R, bool EMBED>
__global__ __launch_bounds__(320) void k_qkv_attn(MvArgs m, AttnDecodeArgs a, int n_mv) {
    __shared__ float lds[4 * QASR_NORM_LDS(NS)];
    __shared__ __attribute__((aligned(16))) int qlds[NS * 256];
    // both branches read arguments spread over ~7 lines: one batch of misses
    kernarg_touch<(int)(sizeof(MvArgs) + sizeof(AttnDecodeArgs))>();
    if ((int)blockIdx.x < n_mv) {
        // waves 0-3 run the matvec; wave 4 only joins its one block barrier
        if ((threadIdx.x >> 6) == 4) {
            __syncthreads();
            return;
        }
        const unsigned tag = (unsigned)a.state[4] * 32u + (unsigned)a.layer;
        unsigned long long *stamp = nullptr;
#ifdef QASR_STAMPS
        if (a.stamps) stamp = a.stamps + ((int64_t)a.layer * QASR_STAMP_BLOCKS + blockIdx.x) * QASR_STAMP_SLOTS;
        if ((threadIdx.x >> 6) == 0) QASR_STAMP(stamp, 0);
#endif
        w8a8_wave<NS, R, MV_PLAIN, true, EMBED, true>(m, blockIdx.x, lds, qlds, a.qkv_tag, tag, stamp);
    } else {
        attn_step_block<KVT, 4, GPW, true>(a, blockIdx.x - n_mv, gridDim.x - n_mv, n_mv);
    }
}

hipError_t launch_qkv_attn(const MvArgs &m, const AttnDecodeArgs &a, int n_heads, int n_kv_heads, int head_dim,
                           int kv_bf16, bool embed, int rows_per_wave, hipStream_t st) {
    if (head_dim != 128 || n_kv_heads <= 0 || n_heads != 2 * n_kv_heads || a.n_split <= 0 || a.n_split > ATT_MAXS)
        return hipErrorInvalidValue;
    if (!a.qkv_tag || !a.fault || !a.q_norm || !a.k_norm || !a.rope_cur || !a.state || a.layer < 0 || a.layer >= 32)
        return hipErrorInvalidValue;
    if (a.gpw < 1 || a.gpw > 4 || a.gpb <= 0 || a.gpb > 4 * a.gpw || a.head_stride < 128 || a.batch > 1)
        return hipErrorInvalidValue;
    if (rows_per_wave != 4 || m.n_total != (n_heads + 2 * n_kv_heads) * head_dim || m.K % 64 != 0 ||
        m.n_total % (4 * rows_per_wave) != 0)
        return hipErrorInvalidValue;
    const int ns = (m.K + 1023) / 1024;
    if (ns != 1 && ns != 2) return hipErrorInvalidValue;
    const int n_mv = m.n_total / (4 * rows_per_wave);
    const dim3 grid(n_mv + n_kv_heads * 2 * a.n_split);
#define QASR_QA(KVT, GPW, NS)                                                                                     \
    if (embed) hipLaunchKernelGGL((k_qkv_attn<KVT, GPW, NS, 4, true>), grid, dim3(320), 0, st, m, a, n_mv);     \
    else hipLaunchKernelGGL((k_qkv_attn<KVT, GPW, NS, 4, false>), grid, dim3(320), 0, st, m, a, n_mv);
#define QASR_QA_G(KVT, NS)                                                                                        \
    switch (a.gpw) {                                                                                              \
        case 1: QASR_QA(KVT, 1, NS) break;                                                                        \
        case 2: QASR_QA(KVT, 2, NS) break;                                                                        \
        case 3: QASR_QA(KVT, 3, NS) break;                                                                        \
        default: QASR_QA(KVT, 4, NS) break;                                                                       \
    }
    if (kv_bf16) {
        if (ns == 1) { QASR_QA_G(uint16_t, 1) } else { QASR_QA_G(uint16_t, 2) }
    } else {
        if (ns == 1) { QASR_QA_G(float, 1) } else { QASR_QA_G(float, 2) }
    }
#undef QASR_QA_G
#undef QASR_QA
    return hipGetLastError();
}

// advances the decode epoch by one (a step whose LM-head merge did not run)
__global__ void k_epoch_advance(int *epoch) {
    if (threadIdx.x == 0) epoch[0] += 1;
}
hipError_t launch_epoch_advance(int *epoch, hipStream_t st) {
    hipLaunchKernelGGL(k_epoch_advance, dim3(1), dim3(64), 0, st, epoch);
    return hipGetLastError();
}

// Multi-stream decode prologue of the attention: per stream b, per-head
// RMSNorm + RoPE of the 16 query heads (in place in the qkv row) and of the new
// key, and the new K/V row written at the stream's position.  The lane layout,
// norm_rope16 and the cache rounding are the decode kernel's own (lanes
// (head, ds) as (pj, ds)), so the values are bit-identical to that kernel's
// fused prologue.  Grid: streams; 3 waves = 24 rows (16 q heads, 8 kv heads).
template <typename KVT>
__global__ __launch_bounds__(192) void k_qk_prep_rows(AttnDecodeArgs a, int Hkv) {
    constexpr int D = 128, G = 2;
    using Sl = KvSlice<KVT>;
    const int bs = blockIdx.x, t = threadIdx.x;
    if (a.select == 2 && a.gpb_dev[bs] <= QASR_STEP_MAX_GPB) return;   // prepared by k_attn_step_batch
    const int row = t >> 3, ds = t & 7, Hq = Hkv * G;
    float *qkv = const_cast<float *>(a.qkv) + bs * a.batch_qkv_stride;
    const bool isq = row < Hq;
    const int kvh = isq ? 0 : row - Hq;
    float x[16], w[16], cs[16], sn[16], v[16];
    ld16<KVT>(isq ? qkv + row * D : qkv + Hq * D + kvh * D, ds, x);
    ld16<KVT>(isq ? a.q_norm : a.k_norm, ds, w);
    ld16<KVT>(a.rope_cur + 256 * bs, ds, cs);
    ld16<KVT>(a.rope_cur + 256 * bs + D, ds, sn);
    ld16<KVT>(qkv + Hq * D + Hkv * D + kvh * D, ds, v);
    const int pos = a.state[4 * bs + 1];
    norm_rope16(x, w, cs, sn, a.eps);
    if (isq) {
#pragma unroll
        for (int k = 0; k < 16; k += 4)
            reinterpret_cast<float4 *>(qkv + row * D + KvSlice<KVT>::dim(k, ds))[0] =
                make_float4(x[k], x[k + 1], x[k + 2], x[k + 3]);
    } else {
        KVT *kc = reinterpret_cast<KVT *>(a.kcache) + bs * a.batch_kv_stride + (int64_t)kvh * a.head_stride;
        KVT *vc = reinterpret_cast<KVT *>(a.vcache) + bs * a.batch_kv_stride + (int64_t)kvh * a.head_stride;
        Sl::store(kc + (int64_t)pos * D, ds, x);
        Sl::store(vc + (int64_t)pos * D, ds, v);
    }
}

hipError_t launch_qk_prep_rows(const AttnDecodeArgs &a, int n_heads, int n_kv_heads, int head_dim, int kv_bf16,
                               hipStream_t st) {
    const int nb = a.batch > 1 ? a.batch : 1;
    if (head_dim != 128 || n_kv_heads != 8 || n_heads != 16 || !a.q_norm || !a.k_norm || !a.rope_cur || !a.state)
        return hipErrorInvalidValue;
    if (a.select != 0 && (a.select != 2 || !a.gpb_dev)) return hipErrorInvalidValue;
    if (kv_bf16) hipLaunchKernelGGL(k_qk_prep_rows<uint16_t>, dim3(nb), dim3(192), 0, st, a, n_kv_heads);
    else hipLaunchKernelGGL(k_qk_prep_rows<float>, dim3(nb), dim3(192), 0, st, a, n_kv_heads);
    return hipGetLastError();
}

hipError_t launch_attn_decode(const AttnDecodeArgs &a, int n_heads, int n_kv_heads, int head_dim,
                              int kv_bf16, hipStream_t st, bool merge) {
    if (head_dim != 128 || n_kv_heads <= 0 || n_heads != 2 * n_kv_heads) return hipErrorInvalidValue;
    if (a.n_split <= 0 || a.n_split > ATT_MAXS) return hipErrorInvalidValue;
    if (a.select < 0 || a.select > 2 || (a.select && !a.gpb_dev) || (a.select == 1 && a.gpw <= 0) ||
        (a.select == 2 && a.gpw > 0))
        return hipErrorInvalidValue;
    if (a.waves != 0 && a.waves != 4 && a.waves != 8) return hipErrorInvalidValue;
    // decode-step mode: every pointer of the fused prologue, the state and a static partition
    const bool dec = a.q_norm != nullptr;
    if (dec && (!a.k_norm || !a.rope_cur || !a.state || a.gpb <= 0 || a.head_stride < 128)) return hipErrorInvalidValue;
    const int nb = a.batch > 1 ? a.batch : 1;
    if (nb > 1 && (merge || !dec || !a.gpb_dev || nb > 65535)) return hipErrorInvalidValue;   // streams: separate merge
    if (a.gpb_dev && (merge || !dec || n_kv_heads != 8)) return hipErrorInvalidValue;   // prep block: 24 rows
    const dim3 grid(n_kv_heads * a.n_split, nb);
#define QASR_ATT(NW, DEC)                                                                           \
    if (merge) {                                                                                     \
        if (kv_bf16) hipLaunchKernelGGL((k_attn_decode<uint16_t, NW, true, DEC>), grid, dim3(NW * 64), 0, st, a); \
        else hipLaunchKernelGGL((k_attn_decode<float, NW, true, DEC>), grid, dim3(NW * 64), 0, st, a);            \
    } else {                                                                                         \
        if (kv_bf16) hipLaunchKernelGGL((k_attn_decode<uint16_t, NW, false, DEC>), grid, dim3(NW * 64), 0, st, a); \
        else hipLaunchKernelGGL((k_attn_decode<float, NW, false, DEC>), grid, dim3(NW * 64), 0, st, a);           \
    }
#define QASR_ATT_MS(NW)                                                                              \
    if (a.depth == 1) {                                                                              \
        if (kv_bf16) hipLaunchKernelGGL((k_attn_decode<uint16_t, NW, false, 3>), grid, dim3(NW * 64), 0, st, a); \
        else hipLaunchKernelGGL((k_attn_decode<float, NW, false, 3>), grid, dim3(NW * 64), 0, st, a);  \
    } else {                                                                                         \
        if (kv_bf16) hipLaunchKernelGGL((k_attn_decode<uint16_t, NW, false, 2>), grid, dim3(NW * 64), 0, st, a); \
        else hipLaunchKernelGGL((k_attn_decode<float, NW, false, 2>), grid, dim3(NW * 64), 0, st, a);  \
    }
    if (dec && !merge && a.gpw > 0 && a.gpb_dev) {
        // k_attn_step_batch (multi-stream step): grid (KV head x split, stream),
        // 4 waves of up to gpw groups; each stream's gpb_dev must be <= 4 gpw
        if (a.waves != 4 || a.gpw < 1 || a.gpw > 4 || kv_bf16 || nb > 65535) return hipErrorInvalidValue;
        const dim3 bgrid(n_kv_heads * a.n_split, nb);
#define QASR_ATT_BSTEP(GPW) hipLaunchKernelGGL((k_attn_step_batch<4, GPW>), bgrid, dim3(256), 0, st, a);
        if (a.gpw == 1) { QASR_ATT_BSTEP(1) } else if (a.gpw == 2) { QASR_ATT_BSTEP(2) }
        else if (a.gpw == 3) { QASR_ATT_BSTEP(3) } else { QASR_ATT_BSTEP(4) }
#undef QASR_ATT_BSTEP
        return hipGetLastError();
    }
    if (dec && !merge && a.gpw > 0) {
        // k_attn_step (single-stream step): one block per (query head, split),
        // 4 waves of gpw = 1..4 groups (the whole run: gpb <= 4 gpw)
        if (a.waves != 4 || a.gpw < 1 || a.gpw > 4 || a.gpb > 4 * a.gpw || a.gpb_dev || nb != 1)
            return hipErrorInvalidValue;
        const dim3 sgrid(n_kv_heads * 2 * a.n_split);
#define QASR_ATT_STEP(GPW)                                                                             \
        if (kv_bf16) hipLaunchKernelGGL((k_attn_step<uint16_t, 4, GPW>), sgrid, dim3(256), 0, st, a);  \
        else hipLaunchKernelGGL((k_attn_step<float, 4, GPW>), sgrid, dim3(256), 0, st, a);
        if (a.gpw == 1) { QASR_ATT_STEP(1) } else if (a.gpw == 2) { QASR_ATT_STEP(2) }
        else if (a.gpw == 3) { QASR_ATT_STEP(3) } else { QASR_ATT_STEP(4) }
#undef QASR_ATT_STEP
        return hipGetLastError();
    }
    if (a.gpb_dev) {
        if (a.waves == 4) { QASR_ATT_MS(4) } else { QASR_ATT_MS(8) }
    } else if (dec) {
        if (a.waves == 4) { QASR_ATT(4, 1) } else { QASR_ATT(8, 1) }
    } else {
        QASR_ATT(4, 0)
    }
#undef QASR_ATT_MS
#undef QASR_ATT
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// RMSNorm over rows (rms_norm, kernels/mod.rs:1191-1212, AVX order of
// avx.rs:377-415), one single-wave block per row, hidden % 64 == 0: lane l
// holds the 16-element slots s = l + 64 c in registers (float4 loads), the
// row goes through LDS transposed (T[r][s] = x[16 s + r]) so that lanes
// r < 16 run the reference's 16 sequential FMA chains, then the output is
// written from the registers.
// ---------------------------------------------------------------------------
template <int NS>
__global__ __launch_bounds__(64) void k_rms_norm_rows(float *__restrict__ out, const float *__restrict__ x,
                                                      const float *__restrict__ w, int H, float eps) {
    __shared__ float T[QASR_NORM_LDS(NS)];
    const int lane = threadIdx.x;
    const int64_t row = blockIdx.x;
    const float *xr = x + row * H;
    float *o = out + row * H;
    const int nslot = H >> 4, ts = nslot + QASR_NORM_PAD;
    float4 xv[NS][4], wv[NS][4];
#pragma unroll
    for (int c = 0; c < NS; c++) {
        const int sl = lane + 64 * c, se = sl < nslot ? sl : 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            xv[c][i] = reinterpret_cast<const float4 *>(xr + 16 * se)[i];
            wv[c][i] = reinterpret_cast<const float4 *>(w + 16 * se)[i];
        }
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
    float acc = 0.0f;
    if (lane < 16) {
        const float4 *t = reinterpret_cast<const float4 *>(T + lane * ts);
        for (int i = 0; i < (nslot >> 2); i++) {
            const float4 v = t[i];
            acc = fmaf(v.x, v.x, acc);
            acc = fmaf(v.y, v.y, acc);
            acc = fmaf(v.z, v.z, acc);
            acc = fmaf(v.w, v.w, acc);
        }
    }
    const float ss = avx16_tree(acc);
    const float rinv = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(div_by_count(ss, H), eps)));
#pragma unroll
    for (int c = 0; c < NS; c++) {
        const int sl = lane + 64 * c;
        if (sl < nslot) {
            float4 *op = reinterpret_cast<float4 *>(o + 16 * sl);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 a = xv[c][i], b = wv[c][i];
                op[i] = make_float4(__fmul_rn(__fmul_rn(a.x, rinv), b.x), __fmul_rn(__fmul_rn(a.y, rinv), b.y),
                                    __fmul_rn(__fmul_rn(a.z, rinv), b.z), __fmul_rn(__fmul_rn(a.w, rinv), b.w));
            }
        }
    }
}

hipError_t launch_rms_norm_rows(float *out, const float *x, const float *w, int64_t seq, int hidden,
                                float eps, hipStream_t st) {
    if (hidden % 64 != 0 || hidden > 4096) return hipErrorInvalidValue;
    if (seq <= 0) return hipSuccess;
    const dim3 grid((unsigned)seq);
    switch ((hidden + 1023) / 1024) {
        case 1: hipLaunchKernelGGL(k_rms_norm_rows<1>, grid, dim3(64), 0, st, out, x, w, hidden, eps); break;
        case 2: hipLaunchKernelGGL(k_rms_norm_rows<2>, grid, dim3(64), 0, st, out, x, w, hidden, eps); break;
        case 3: hipLaunchKernelGGL(k_rms_norm_rows<3>, grid, dim3(64), 0, st, out, x, w, hidden, eps); break;
        default: hipLaunchKernelGGL(k_rms_norm_rows<4>, grid, dim3(64), 0, st, out, x, w, hidden, eps); break;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Per-head RMSNorm (rms_norm_per_head, kernels/mod.rs:1214-1238) and NeoX RoPE
// (apply_rope_neox, mod.rs:1738-1791) over [seq][heads][hd] rows, hd = 128:
// one wave per (row, head), two elements per lane (d and d + 64).
// ---------------------------------------------------------------------------
// one head's two lane elements (d = lane, lane + 64): RMSNorm then NeoX RoPE
__device__ __forceinline__ void head_norm_rope2(float &x1, float &x2, const float *__restrict__ w,
                                                const float *__restrict__ c, const float *__restrict__ sn,
                                                float eps, bool do_norm, bool do_rope) {
    constexpr int D = 128;
    const int lane = threadIdx.x & 63;
    if (do_norm) {
        const float ss = wave_sum_f32(__fadd_rn(__fmul_rn(x1, x1), __fmul_rn(x2, x2)));
        const float r = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(div_by_count(ss, D), eps)));
        x1 = __fmul_rn(__fmul_rn(x1, r), w[lane]);
        x2 = __fmul_rn(__fmul_rn(x2, r), w[lane + 64]);
    }
    if (do_rope) {
        const float n1 = __fadd_rn(__fmul_rn(x1, c[lane]), __fmul_rn(-x2, sn[lane]));
        const float n2 = __fadd_rn(__fmul_rn(x2, c[lane + 64]), __fmul_rn(x1, sn[lane + 64]));
        x1 = n1; x2 = n2;
    }
}

// The prefill's per-head work after the qkv GEMM in one launch
// (decoder.rs:497-514): q heads normed and rotated in place; k heads normed,
// rotated and written to the KV cache with the v heads.  One wave per
// (row, head): waves [0, Hq) of a row take the q heads, [Hq, Hq + Hkv) the
// k/v heads.
__global__ __launch_bounds__(256) void k_prefill_qkv_post(PrefillPostArgs a) {
    constexpr int D = 128;
    const int lane = threadIdx.x & 63;
    const int per_row = a.Hq + a.Hkv;
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= a.S * per_row) return;
    const int64_t s = item / per_row;
    const int h = (int)(item % per_row);
    float *row = a.qkv + s * a.row_stride;
    const float *c = a.cos_t + s * D, *sn = a.sin_t + s * D;
    if (h < a.Hq) {
        float *v = row + h * D;
        float x1 = v[lane], x2 = v[lane + 64];
        head_norm_rope2(x1, x2, a.q_norm, c, sn, a.eps, true, true);
        v[lane] = x1;
        v[lane + 64] = x2;
    } else {
        const int kh = h - a.Hq;
        const float *kp = row + a.Hq * D + kh * D, *vp = row + (a.Hq + a.Hkv) * D + kh * D;
        float x1 = kp[lane], x2 = kp[lane + 64];
        const float v1 = vp[lane], v2 = vp[lane + 64];
        head_norm_rope2(x1, x2, a.k_norm, c, sn, a.eps, true, true);
        const int64_t dst = kh * a.head_stride + (a.start + s) * D;
        a.kc[dst + lane] = x1;
        a.kc[dst + lane + 64] = x2;
        a.vc[dst + lane] = v1;
        a.vc[dst + lane + 64] = v2;
    }
}

// k_prefill_qkv_post over several sequences: a wave's row picks its
// sequence's position, KV bases and head stride (compile-time table indices).
__global__ __launch_bounds__(256) void k_prefill_qkv_post_seqs(PrefillPostSeqArgs sa) {
    constexpr int D = 128;
    const PrefillPostArgs &a = sa.base;
    const int lane = threadIdx.x & 63;
    const int per_row = a.Hq + a.Hkv;
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= sa.row[sa.n] * per_row) return;
    const int64_t s = item / per_row;
    const int h = (int)(item % per_row);
    int64_t r0 = sa.row[0], start = sa.start[0], hs = sa.head_stride[0];
    float *kc = sa.kc[0], *vc = sa.vc[0];
#pragma unroll
    for (int u = 1; u < QASR_ATTN_MAX_SEQ; u++)
        if (u < sa.n && s >= sa.row[u]) {
            r0 = sa.row[u];
            start = sa.start[u];
            hs = sa.head_stride[u];
            kc = sa.kc[u];
            vc = sa.vc[u];
        }
    const int64_t pos = start + (s - r0);
    float *row = a.qkv + s * a.row_stride;
    const float *c = a.cos_t + pos * D, *sn = a.sin_t + pos * D;
    if (h < a.Hq) {
        float *v = row + h * D;
        float x1 = v[lane], x2 = v[lane + 64];
        head_norm_rope2(x1, x2, a.q_norm, c, sn, a.eps, true, true);
        v[lane] = x1;
        v[lane + 64] = x2;
    } else {
        const int kh = h - a.Hq;
        const float *kp = row + a.Hq * D + kh * D, *vp = row + (a.Hq + a.Hkv) * D + kh * D;
        float x1 = kp[lane], x2 = kp[lane + 64];
        const float v1 = vp[lane], v2 = vp[lane + 64];
        head_norm_rope2(x1, x2, a.k_norm, c, sn, a.eps, true, true);
        const int64_t dst = kh * hs + pos * D;
        kc[dst + lane] = x1;
        kc[dst + lane + 64] = x2;
        vc[dst + lane] = v1;
        vc[dst + lane + 64] = v2;
    }
}

hipError_t launch_prefill_qkv_post_seqs(const PrefillPostSeqArgs &a, hipStream_t st) {
    if (a.n < 1 || a.n > QASR_ATTN_MAX_SEQ) return hipErrorInvalidValue;
    const int64_t items = a.row[a.n] * (a.base.Hq + a.base.Hkv);
    if (items <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_prefill_qkv_post_seqs, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_prefill_qkv_post(const PrefillPostArgs &a, hipStream_t st) {
    const int64_t items = a.S * (a.Hq + a.Hkv);
    if (items <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_prefill_qkv_post, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, st, a);
    return hipGetLastError();
}

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
    head_norm_rope2(x1, x2, w, do_rope ? cos_t + s * D : nullptr, do_rope ? sin_t + s * D : nullptr, eps,
                    do_norm != 0, do_rope != 0);
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
