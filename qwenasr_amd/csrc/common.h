// Shared device helpers for the qasr_hip kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define QASR_WAVE 64

namespace qasr {

// ---- wave reductions (all lanes receive the result) ------------------------
__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, QASR_WAVE);
    return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, QASR_WAVE));
    return v;
}
__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = __fadd_rn(v, __shfl_xor(v, o, QASR_WAVE));
    return v;
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
// ((t0+t4)+(t1+t5)) + ((t2+t6)+(t3+t7)); returned in every lane.
__device__ __forceinline__ float avx16_tree(float a) {
    float t = __fadd_rn(a, __shfl_down(a, 8, QASR_WAVE));
    float u = __fadd_rn(t, __shfl_down(t, 4, QASR_WAVE));
    float v = __fadd_rn(u, __shfl_down(u, 1, QASR_WAVE));
    float r = __fadd_rn(v, __shfl_down(v, 2, QASR_WAVE));
    return __shfl(r, 0, QASR_WAVE);
}

}  // namespace qasr
