// LayerNorm row arithmetic shared by layernorm_fp16 and the W^T GEMM with a
// LayerNorm prologue, so both produce the same bits
// (kernels/layernorm_fp16/baseline.c:11-35: two-pass biased variance, then
// (x - mean) / sqrt(var + eps) * w + b, in fp32).
//
// A row is held by one 64-lane wave: lane L's chunk ch holds the VEC elements
// at [(ch * 64 + L) * VEC, +VEC); chunks past the row's end hold 0 and count as
// 0 in both sums. Contraction is off: every product and sum is rounded as
// written, whichever kernel inlines this.
#pragma once

#include "device.h"

template <int VEC, int NCH>
__device__ __forceinline__ void ln_row_stats(float (&v)[NCH][VEC], const bool (&ok)[NCH], int C,
                                             float eps, float &mean, float &inv) {
#pragma clang fp contract(off)
    float s = 0.0f;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
        for (int j = 0; j < VEC; ++j) s += v[ch][j];
    mean = wave_sum(s) / (float) C;
    float q = 0.0f;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            const float d = ok[ch] ? v[ch][j] - mean : 0.0f;
            v[ch][j] = d;
            q += d * d;
        }
    inv = 1.0f / sqrtf(wave_sum(q) / (float) C + eps);
}

// One output element from its centred value d = x - mean, as an fp32 value:
// ((d * inv) * w) + b with each product and the sum rounded to fp32 as
// written (kernels/layernorm_fp16/baseline.c:33 rounds three times; contraction
// is off, so no fused multiply-add). f32_rounded keeps the caller's fp16
// conversion a second, separate rounding of that fp32 result.
__device__ __forceinline__ float ln_apply(float d, float inv, float w, float b) {
#pragma clang fp contract(off)
    return f32_rounded(d * inv * w + b);
}
