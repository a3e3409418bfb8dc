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

// Lane exchange within a 16-lane row through a DPP operand modifier (a VALU
// operand, no LDS round trip): 0xB1 / 0x4E swap lanes xor 1 / xor 2 within
// each quad, 0x141 mirrors each half-row (lane i <-> 7 - i), 0x140 each row
// (i <-> 15 - i).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF,
                                                                 false));
}

__device__ __forceinline__ float lane_f32(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over all 64 lanes (all active); every lane ends with the same bits:
// pairwise within quads, half-rows and rows (each step adds two equal-order
// partial sums, so both partners compute the same value), then the four row
// sums as (r0 + r1) + (r2 + r3).
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    return (lane_f32(v, 0) + lane_f32(v, 16)) + (lane_f32(v, 32) + lane_f32(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x141>(v));
    v = fmaxf(v, dpp_f32<0x140>(v));
    return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}

// Returns v as an fp32 register value the backend cannot see through. Without
// it, fp16(x_f32 * y) is selected as one v_fma_mixlo_f16, which rounds the
// exact product to fp16 once; the scalar contracts round to fp32 first.
__device__ __forceinline__ float f32_rounded(float v) {
    asm("" : "+v"(v));
    return v;
}

// tanh-form GELU (ACT2FN["gelu_pytorch_tanh"]) and exact erf GELU, in fp32.
// GELU, tanh form: 0.5 x (1 + tanh(u)) with u = sqrt(2/pi) (x + 0.044715 x^3).
// Since 1 + tanh(u) = 2 / (1 + exp(-2u)), this is x / (1 + exp(-2u)): one
// hardware exp2 and one reciprocal instead of a library tanh (a few fp32 ulps
// from the tanh form, far below the fp16 rounding of every consumer). Large
// negative x sends exp(-2u) to +inf and the result to -0; large positive x
// sends it to 0 and the result to x.
__device__ __forceinline__ float gelu_tanh_f32(float x) {
    const float m2u = -1.5957691216057308f * (x + 0.044715f * x * x * x);   // -2u
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(m2u * 1.4426950408889634f));
}

__device__ __forceinline__ float gelu_erf_f32(float x) {
    return 0.5f * x * (1.0f + erff(x * 0.7071067811865476f));
}

__device__ __forceinline__ float apply_act(float x, int act) {
    if (act == 1) return gelu_tanh_f32(x);
    if (act == 2) return gelu_erf_f32(x);
    return x;
}
