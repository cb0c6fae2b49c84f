// Shared device helpers for the qasr_hip kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define QASR_WAVE 64

namespace qasr {

// ---- wave reductions (all lanes receive the result) ------------------------
// DPP controls (GFX9 encoding): quad_perm [1,0,3,2] / [2,3,0,1], row_half_mirror,
// row_mirror, then row_bcast:15 into rows 1,3 and row_bcast:31 into rows 2,3;
// lane 63 ends with the full reduction.  Integer sums and max are exact in any
// order, so these need not follow any particular tree.
#define QASR_DPP_QP_1032 0xB1
#define QASR_DPP_QP_2301 0x4E
#define QASR_DPP_ROW_HALF_MIRROR 0x141
#define QASR_DPP_ROW_MIRROR 0x140
#define QASR_DPP_ROW_BCAST15 0x142
#define QASR_DPP_ROW_BCAST31 0x143
__device__ __forceinline__ int wave_sum_i32(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, QASR_DPP_QP_1032, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, QASR_DPP_QP_2301, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, QASR_DPP_ROW_HALF_MIRROR, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, QASR_DPP_ROW_MIRROR, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, QASR_DPP_ROW_BCAST15, 0xA, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, QASR_DPP_ROW_BCAST31, 0xC, 0xF, false);
    return __builtin_amdgcn_readlane(v, 63);
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_max_step(float v) {
    const int o = __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROW_MASK, 0xF, false);
    return fmaxf(v, __int_as_float(o));
}
__device__ __forceinline__ float wave_max_f32(float v) {
    v = dpp_max_step<QASR_DPP_QP_1032, 0xF>(v);
    v = dpp_max_step<QASR_DPP_QP_2301, 0xF>(v);
    v = dpp_max_step<QASR_DPP_ROW_HALF_MIRROR, 0xF>(v);
    v = dpp_max_step<QASR_DPP_ROW_MIRROR, 0xF>(v);
    v = dpp_max_step<QASR_DPP_ROW_BCAST15, 0xA>(v);
    v = dpp_max_step<QASR_DPP_ROW_BCAST31, 0xC>(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = __fadd_rn(v, __shfl_xor(v, o, QASR_WAVE));
    return v;
}
// ---- 8-lane reductions without LDS -----------------------------------------
// Lanes are viewed as 8 groups of 8 (group = lane / 8, member = lane % 8).
// sum8/max8 reduce over the members of a group (quad_perm [1,0,3,2], [2,3,0,1],
// then row_half_mirror, which pairs each quad with the other quad of its 8);
// sum_x8/max_x8 reduce over the groups at a fixed member (row_ror:8 pairs
// lanes i and i ^ 8 within a 16-lane row, v_permlane16_swap pairs rows 0/1 and
// 2/3, v_permlane32_swap pairs the wave's halves).  Every lane of a reduction
// set receives the same value.
#define QASR_DPP_ROW_ROR8 0x128
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float xrow16_sum(float v) {     // v[i] + v[i ^ 16]
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __fadd_rn(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float xhalf_sum(float v) {      // v[i] + v[i ^ 32]
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __fadd_rn(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float xrow16_max(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float xhalf_max(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float sum8(float v) {
    v = __fadd_rn(v, dpp_f32<QASR_DPP_QP_1032>(v));
    v = __fadd_rn(v, dpp_f32<QASR_DPP_QP_2301>(v));
    return __fadd_rn(v, dpp_f32<QASR_DPP_ROW_HALF_MIRROR>(v));
}
__device__ __forceinline__ float sum_x8(float v) {
    v = __fadd_rn(v, dpp_f32<QASR_DPP_ROW_ROR8>(v));
    return xhalf_sum(xrow16_sum(v));
}
__device__ __forceinline__ float max_x8(float v) {
    v = fmaxf(v, dpp_f32<QASR_DPP_ROW_ROR8>(v));
    return xhalf_max(xrow16_max(v));
}

// reduction over aligned groups of `width` lanes (width a power of two <= 64)
template <int WIDTH>
__device__ __forceinline__ float group_sum_f32(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v = __fadd_rn(v, __shfl_xor(v, o, QASR_WAVE));
    return v;
}

// IEEE round-to-nearest sqrt (what glibc sqrtf returns).  v_sqrt_f32 alone is
// only ~1 ulp accurate; the estimate s is corrected by comparing x against the
// products with its two neighbours, computed exactly with fma.
__device__ __forceinline__ float sqrt_rn(float x) {
    const bool tiny = x < 0x1.0p-96f;
    const float xs = tiny ? x * 0x1.0p+32f : x;
    float s = __builtin_amdgcn_sqrtf(xs);
    const float dn = __uint_as_float(__float_as_uint(s) - 1u);
    const float up = __uint_as_float(__float_as_uint(s) + 1u);
    const float r_dn = fmaf(-dn, s, xs);
    const float r_up = fmaf(-up, s, xs);
    s = r_dn <= 0.0f ? dn : s;
    s = r_up > 0.0f ? up : s;
    s = tiny ? s * 0x1.0p-16f : s;
    return (xs == 0.0f || xs == __builtin_inff() || xs != xs) ? __builtin_amdgcn_sqrtf(xs) * (tiny ? 0x1.0p-16f : 1.0f) : s;
}

// ---- cross-block hand-off ------------------------------------------------
// MI355X's L2 is private to each XCD, so a block that publishes data for a
// block on another XCD must get it past its own L2.  The producer stores with
// agent-scope relaxed atomics (write-through) and waits for their
// acknowledgement; arrive_last then orders them before its counter bump (an
// agent-scope release fence and an acq_rel increment), and the consumer, after
// the matching acquire, reads with agent-scope atomic loads (which miss its
// local L2).
// Phase stamps of the profiling build (-DQASR_STAMPS, libqasr_hip_stamps.so):
// lane 0 of the calling wave records the 100 MHz real-time counter in
// slot[idx].  The product build compiles them to nothing.
#ifdef QASR_STAMPS
#define QASR_STAMP(slot, idx)                                                         \
    do {                                                                              \
        if ((slot) && (threadIdx.x & 63) == 0) (slot)[idx] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define QASR_STAMP(slot, idx) \
    do {                      \
    } while (0)
#endif
#define QASR_STAMP_SLOTS 16
#define QASR_STAMP_BLOCKS 2048

// Reads one dword of every 64-byte line of the first NBYTES bytes of the
// kernel arguments in one batch and waits once: arguments read later hit the
// scalar cache.  For kernels whose argument reads the compiler would otherwise
// split into several dependent batches, each a memory round trip.
template <int NBYTES>
__device__ __forceinline__ void kernarg_touch() {
    static_assert(NBYTES <= 8 * 64, "at most 8 lines");
#if defined(__HIP_DEVICE_COMPILE__)
    typedef const uint32_t __attribute__((address_space(4))) *ka_ptr;   // the constant (kernarg) space
    const ka_ptr ka = (ka_ptr)__builtin_amdgcn_kernarg_segment_ptr();
    constexpr int L = (NBYTES + 63) / 64;
    uint32_t v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = i < L ? ka[16 * i] : 0u;
    // every value an operand of its own: the loads go out together, one wait
    asm volatile("" ::"s"(v[0]), "s"(v[1]), "s"(v[2]), "s"(v[3]), "s"(v[4]), "s"(v[5]), "s"(v[6]), "s"(v[7]));
#endif
}

// RMSNorm's LDS transpose (16 rows of the K/16 slots): rows padded by 4
// floats so that the 16 lanes reading one row each start on different banks;
// floats per wave for NS 1024-element slot groups
#define QASR_NORM_PAD 4
#define QASR_NORM_LDS(NS) (16 * (64 * (NS) + QASR_NORM_PAD))

__device__ __forceinline__ void st_agent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(int *p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ld_agent(const int *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long ld_agent64(const unsigned long long *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// wait until every memory operation this thread issued has completed
__device__ __forceinline__ void wait_all_mem() { __builtin_amdgcn_s_waitcnt(0); }
// Counter bump after the block's stores; true in the last block to arrive.
// Ordering: every thread waits for its own stores (the barrier does not wait
// for vector memory), thread 0 publishes them with an agent-scope release
// fence and an acq_rel bump, and the threads of the last block acquire at
// agent scope before they read what the other blocks wrote.
__device__ __forceinline__ bool arrive_last(unsigned *ctr, unsigned n_blocks, int *flag_lds) {
    wait_all_mem();
    __syncthreads();
    if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        *flag_lds = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == n_blocks - 1;
    }
    __syncthreads();
    const bool last = *flag_lds != 0;
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    return last;
}
__device__ __forceinline__ void reset_counter(unsigned *ctr) {
    __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
}

// f32 -> bf16 round-to-nearest-even (finite inputs)
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// (v).round().clamp(-127, 127) as i8 — Rust f32::round is round-half-away-from-zero.
__device__ __forceinline__ int round_clamp_i8(float f) {
    float r = roundf(f);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    return (int)r;
}

// Activation-quantization constants of quantize_f32_to_int8 (kernels/mod.rs:1795-1802).
__device__ __forceinline__ void act_scales(float max_abs, float *scale, float *inv) {
    *scale = max_abs > 0.0f ? __fdiv_rn(max_abs, 127.0f) : 1.0f;
    *inv = __fdiv_rn(127.0f, fmaxf(max_abs, 1e-10f));
}

__device__ __forceinline__ int pack4_i8(int a, int b, int c, int d) {
    return (a & 0xFF) | ((b & 0xFF) << 8) | ((c & 0xFF) << 16) | ((int)((unsigned)d << 24));
}

// hsum_ps tree of the reference (kernels/avx.rs:37-51) applied to 16 AVX-lane
// accumulators held in lanes 0..15: t_j = A_j + A_{j+8}; result
// ((t0+t4)+(t1+t5)) + ((t2+t6)+(t3+t7)); returned in every lane.  Each step
// is a DPP row shift (row_shl:N, lane i reads lane i + N of its 16-lane row)
// and one add, so lanes 0-7, 0-3, then 0 and 2 hold the tree's partial sums
// in the reference's order.
#define QASR_DPP_ROW_SHL(N) (0x100 + (N))
__device__ __forceinline__ float avx16_tree(float a) {
    const float t = __fadd_rn(a, dpp_f32<QASR_DPP_ROW_SHL(8)>(a));
    const float u = __fadd_rn(t, dpp_f32<QASR_DPP_ROW_SHL(4)>(t));
    const float v = __fadd_rn(u, dpp_f32<QASR_DPP_ROW_SHL(1)>(u));
    const float r = __fadd_rn(v, dpp_f32<QASR_DPP_ROW_SHL(2)>(v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r), 0));
}

// x / n rounded to nearest: for n a power of two the product with 2^-log2(n),
// which is exact (the same value, the same single rounding), else a division
__device__ __forceinline__ float div_by_count(float x, int n) {
    if ((n & (n - 1)) == 0) return __fmul_rn(x, __int_as_float((127 - __builtin_ctz((unsigned)n)) << 23));
    return __fdiv_rn(x, (float)n);
}

// gelu of the reference (avx.rs:536-563) for element `idx` of a buffer of n
// elements that gelu() splits into 16 per-thread chunks (mod.rs:1250-1289):
// the last n_chunk % 8 elements of each chunk take the scalar libm-tanh path.
// avx::fast_exp_avx (avx.rs:487-514); cvtps_epi32 rounds to nearest even
__device__ __forceinline__ float fast_exp_ref(float x) {
    float val = __fmul_rn(x, 1.442695041f);
    val = fminf(val, 126.0f);
    val = fmaxf(val, -126.0f);
    const int ip = (int)rintf(val);
    const float fp = __fsub_rn(val, (float)ip);
    const float ei = __uint_as_float((uint32_t)(ip + 127) << 23);
    const float f = __fmul_rn(fp, 0.6931471806f);
    float p = fmaf(1.0f / 120.0f, f, 1.0f / 24.0f);
    p = fmaf(p, f, 1.0f / 6.0f);
    p = fmaf(p, f, 0.5f);
    p = fmaf(p, f, 1.0f);
    p = fmaf(p, f, 1.0f);
    return __fmul_rn(ei, p);
}

// the two element paths of gelu (avx.rs:536-563): 8-wide fast_exp / scalar libm tanh
__device__ __forceinline__ float gelu_at(float v, bool vec) {
    if (vec) {
        const float v3 = __fmul_rn(__fmul_rn(v, v), v);
        const float inner = __fmul_rn(0.7978845608028654f, fmaf(0.044715f, v3, v));
        const float e2 = fast_exp_ref(__fmul_rn(2.0f, inner));
        const float t = __fsub_rn(1.0f, __fdiv_rn(2.0f, __fadd_rn(e2, 1.0f)));
        return __fmul_rn(0.5f, __fmul_rn(v, __fadd_rn(1.0f, t)));
    }
    const float x3 = __fmul_rn(__fmul_rn(v, v), v);
    const float inner = __fmul_rn(0.7978845608028654f, __fadd_rn(v, __fmul_rn(0.044715f, x3)));
    return __fmul_rn(__fmul_rn(0.5f, v), __fadd_rn(1.0f, tanhf(inner)));
}

__device__ __forceinline__ float gelu_ref(float v, int64_t idx, int64_t n) {
    bool vec = true;
    if (n > 4096 && n < (int64_t)1 << 31) {
        // the same arithmetic in 32 bits (a 64-bit division is a long software sequence)
        const uint32_t un = (uint32_t)n, ui = (uint32_t)idx, chunk = (un + 15) / 16;
        const uint32_t start = ui / chunk * chunk, len = min(chunk, un - start);
        vec = ui - start < len - len % 8;
    } else if (n > 4096) {
        const int64_t chunk = (n + 15) / 16;
        const int64_t c = idx / chunk, start = c * chunk;
        const int64_t len = min(chunk, n - start);
        vec = (idx - start) < len - (len % 8);
    } else {
        vec = idx < n - (n % 8);
    }
    return gelu_at(v, vec);
}

// gelu_ref's path choice for indices idx in [lo, lo + span) with span no larger
// than one per-thread chunk (so the range meets at most two chunks), computed
// once: vec(idx) = idx < b1 ? idx < ts0 : idx < ts1
struct GeluSpan {
    int64_t b1, ts0, ts1;
    __device__ __forceinline__ GeluSpan(int64_t lo, int64_t n) {
        if (n > 4096) {
            const int64_t chunk = (n + 15) / 16, s0 = lo / chunk * chunk;
            const int64_t len0 = min(chunk, n - s0), s1 = s0 + chunk, len1 = max((int64_t)0, min(chunk, n - s1));
            b1 = s1;
            ts0 = s0 + len0 - len0 % 8;
            ts1 = s1 + len1 - len1 % 8;
        } else {
            b1 = INT64_MAX;
            ts0 = ts1 = n - n % 8;
        }
    }
    __device__ __forceinline__ bool vec(int64_t idx) const { return idx < b1 ? idx < ts0 : idx < ts1; }
};

}  // namespace qasr
