// Device-side types and wavefront reductions for gfx950 (64-lane waves).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define HX_WAVE 64

// Butterfly over all 64 lanes; every lane ends with the full result.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, HX_WAVE);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, HX_WAVE));
    return v;
}

// Returns v as an fp32 register value the backend cannot see through. Without
// it, fp16(x_f32 * y) is selected as one v_fma_mixlo_f16, which rounds the
// exact product to fp16 once; the scalar contracts round to fp32 first.
__device__ __forceinline__ float f32_rounded(float v) {
    asm("" : "+v"(v));
    return v;
}

// tanh-form GELU (ACT2FN["gelu_pytorch_tanh"]) and exact erf GELU, in fp32.
__device__ __forceinline__ float gelu_tanh_f32(float x) {
    const float inner = 0.7978845608028654f * (x + 0.044715f * x * x * x);
    return 0.5f * x * (1.0f + tanhf(inner));
}

__device__ __forceinline__ float gelu_erf_f32(float x) {
    return 0.5f * x * (1.0f + erff(x * 0.7071067811865476f));
}

__device__ __forceinline__ float apply_act(float x, int act) {
    if (act == 1) return gelu_tanh_f32(x);
    if (act == 2) return gelu_erf_f32(x);
    return x;
}
