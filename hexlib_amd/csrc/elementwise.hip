// Bandwidth kernels: add_fp16, scale_fp16, cast_f32_f16.
//
// One 16-byte vector (8 fp16 lanes) per thread per step, grid-stride, the
// sub-vector tail done by the first block. Each output is ONE float rounding
// of an exact or single-op fp32 result, so the result is bit-identical to the
// scalar contract: fp16(float(a)+float(b)) (kernels/add_fp16/kernel_api.h:12-22),
// fp16(float(x)*factor) (kernels/scale_fp16/kernel_api.h:11), fp16(x) round to
// nearest even (kernels/cast_f32_f16/kernel_api.h:11).
// The scale product passes through f32_rounded(): otherwise fp16(float(x) *
// factor) is selected as v_fma_mixlo_f16, which rounds the exact product once
// where the contract rounds to fp32 first and then to fp16 (they differ on
// ~3% of inputs for factor 0.7; FP-contraction pragmas do not prevent it).
// Algorithmic bytes per element: add 6, scale 4, cast 6.
#include "device.h"
#include "internal.h"

namespace {

constexpr int TPB = 256;
constexpr int UNROLL = 2;  // vectors in flight per thread per step

__global__ __launch_bounds__(TPB) void add_v8(const f16x8 *__restrict__ a,
                                              const f16x8 *__restrict__ b,
                                              f16x8 *__restrict__ y, long long nvec,
                                              const f16 *__restrict__ at,
                                              const f16 *__restrict__ bt,
                                              f16 *__restrict__ yt, int tail) {
#pragma clang fp contract(off)
    const long long stride = (long long) gridDim.x * TPB;
    for (long long i = (long long) blockIdx.x * TPB + threadIdx.x; i < nvec; i += stride) {
        const f16x8 va = a[i], vb = b[i];
        f16x8 r;
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = (f16) ((float) va[j] + (float) vb[j]);
        y[i] = r;
    }
    if (blockIdx.x == 0 && (int) threadIdx.x < tail)
        yt[threadIdx.x] = (f16) ((float) at[threadIdx.x] + (float) bt[threadIdx.x]);
}

__global__ __launch_bounds__(TPB) void add_s(const f16 *__restrict__ a, const f16 *__restrict__ b,
                                             f16 *__restrict__ y, long long n) {
#pragma clang fp contract(off)
    const long long stride = (long long) gridDim.x * TPB;
    for (long long i = (long long) blockIdx.x * TPB + threadIdx.x; i < n; i += stride)
        y[i] = (f16) ((float) a[i] + (float) b[i]);
}

__global__ __launch_bounds__(TPB) void scale_v8(const f16x8 *__restrict__ x, f16x8 *__restrict__ y,
                                                long long nvec, float factor,
                                                const f16 *__restrict__ xt, f16 *__restrict__ yt,
                                                int tail) {
#pragma clang fp contract(off)
    const long long stride = (long long) gridDim.x * TPB;
    for (long long i = (long long) blockIdx.x * TPB + threadIdx.x; i < nvec; i += stride) {
        const f16x8 v = x[i];
        f16x8 r;
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = (f16) f32_rounded((float) v[j] * factor);
        y[i] = r;
    }
    if (blockIdx.x == 0 && (int) threadIdx.x < tail)
        yt[threadIdx.x] = (f16) f32_rounded((float) xt[threadIdx.x] * factor);
}

__global__ __launch_bounds__(TPB) void scale_s(const f16 *__restrict__ x, f16 *__restrict__ y,
                                               long long n, float factor) {
#pragma clang fp contract(off)
    const long long stride = (long long) gridDim.x * TPB;
    for (long long i = (long long) blockIdx.x * TPB + threadIdx.x; i < n; i += stride)
        y[i] = (f16) f32_rounded((float) x[i] * factor);
}

__global__ __launch_bounds__(TPB) void cast_v8(const f32x4 *__restrict__ x, f16x8 *__restrict__ y,
                                               long long nvec, const float *__restrict__ xt,
                                               f16 *__restrict__ yt, int tail) {
#pragma clang fp contract(off)
    const long long stride = (long long) gridDim.x * TPB;
    for (long long i = (long long) blockIdx.x * TPB + threadIdx.x; i < nvec; i += stride) {
        const f32x4 lo = x[2 * i], hi = x[2 * i + 1];
        f16x8 r;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            r[j] = (f16) lo[j];
            r[j + 4] = (f16) hi[j];
        }
        y[i] = r;
    }
    if (blockIdx.x == 0 && (int) threadIdx.x < tail) yt[threadIdx.x] = (f16) xt[threadIdx.x];
}

__global__ __launch_bounds__(TPB) void cast_s(const float *__restrict__ x, f16 *__restrict__ y,
                                              long long n) {
#pragma clang fp contract(off)
    const long long stride = (long long) gridDim.x * TPB;
    for (long long i = (long long) blockIdx.x * TPB + threadIdx.x; i < n; i += stride)
        y[i] = (f16) x[i];
}

inline unsigned vec_grid(long long nvec) {
    return hx::blocks_for(nvec > 0 ? nvec : 1, TPB * UNROLL, 8192);
}

}  // namespace

extern "C" void add_fp16(const hexlib_hf *a, const hexlib_hf *b, hexlib_hf *y, int n) {
    if (n <= 0 || !a || !b || !y) return;
    auto A = reinterpret_cast<const f16 *>(a);
    auto B = reinterpret_cast<const f16 *>(b);
    auto Y = reinterpret_cast<f16 *>(y);
    if (hx::aligned(a, 16) && hx::aligned(b, 16) && hx::aligned(y, 16)) {
        const long long nvec = n / 8;
        const int tail = n % 8;
        HX_LAUNCH(add_v8, dim3(vec_grid(nvec)), dim3(TPB), 0,
                  reinterpret_cast<const f16x8 *>(A), reinterpret_cast<const f16x8 *>(B),
                  reinterpret_cast<f16x8 *>(Y), nvec, A + nvec * 8, B + nvec * 8, Y + nvec * 8,
                  tail);
    } else {
        HX_LAUNCH(add_s, dim3(hx::blocks_for(n, TPB, 8192)), dim3(TPB), 0, A, B, Y, (long long) n);
    }
}

extern "C" void scale_fp16(const hexlib_hf *x, hexlib_hf *y, int n, float factor) {
    if (n <= 0 || !x || !y) return;
    auto X = reinterpret_cast<const f16 *>(x);
    auto Y = reinterpret_cast<f16 *>(y);
    if (hx::aligned(x, 16) && hx::aligned(y, 16)) {
        const long long nvec = n / 8;
        HX_LAUNCH(scale_v8, dim3(vec_grid(nvec)), dim3(TPB), 0,
                  reinterpret_cast<const f16x8 *>(X), reinterpret_cast<f16x8 *>(Y), nvec, factor,
                  X + nvec * 8, Y + nvec * 8, n % 8);
    } else {
        HX_LAUNCH(scale_s, dim3(hx::blocks_for(n, TPB, 8192)), dim3(TPB), 0, X, Y, (long long) n,
                  factor);
    }
}

extern "C" void cast_f32_f16(const float *x, hexlib_hf *y, int n) {
    if (n <= 0 || !x || !y) return;
    auto Y = reinterpret_cast<f16 *>(y);
    if (hx::aligned(x, 16) && hx::aligned(y, 16)) {
        const long long nvec = n / 8;
        HX_LAUNCH(cast_v8, dim3(vec_grid(nvec)), dim3(TPB), 0, reinterpret_cast<const f32x4 *>(x),
                  reinterpret_cast<f16x8 *>(Y), nvec, x + nvec * 8, Y + nvec * 8, n % 8);
    } else {
        HX_LAUNCH(cast_s, dim3(hx::blocks_for(n, TPB, 8192)), dim3(TPB), 0, x, Y, (long long) n);
    }
}
