// Row reductions: softmax_fp16, layernorm_fp16, rmsnorm_fp16.
//
// One 64-lane wavefront per row, four rows per 256-thread block. The row is
// read ONCE into registers (up to 64 * VEC * NCH elements), reduced with an
// xor-butterfly across the wave, and written once -- so HBM traffic is the
// algorithmic minimum (2 B in + 2 B out per element, plus the parameters).
// Rows wider than the register budget take a looping variant that re-reads x.
//
// Arithmetic follows the scalar contracts in fp32, rounding only the stored
// value: softmax subtracts the row max before exp and divides last
// (kernels/softmax_fp16/kernel_api.h:18-22); layernorm uses the two-pass
// biased variance (kernels/layernorm_fp16/baseline.c:11-35); rmsnorm is
// x * (1/sqrt(mean(x^2) + eps)) * w (kernels/rmsnorm_fp16/kernel_api.h:9-12).
#include "device.h"
#include "internal.h"
#include "lnmath.h"

namespace {

constexpr int TPB = 256;
constexpr int ROWS_PER_BLOCK = TPB / HX_WAVE;

// Row-in-registers loader: chunk ch of lane L covers elements
// [(ch*64 + L)*VEC, +VEC). VEC > 1 requires C % VEC == 0 and aligned rows.
template <int VEC, int NCH>
struct RowRegs {
    float v[NCH][VEC];
    bool ok[NCH];

    __device__ __forceinline__ void load(const f16 *xr, int C, int lane, float fill) {
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
            const int base = (ch * HX_WAVE + lane) * VEC;
            ok[ch] = base < C;
            if constexpr (VEC == 8) {
                f16x8 t = ok[ch] ? *reinterpret_cast<const f16x8 *>(xr + base) : f16x8{};
#pragma unroll
                for (int j = 0; j < 8; ++j) v[ch][j] = ok[ch] ? (float) t[j] : fill;
            } else if constexpr (VEC == 4) {
                f16x4 t = ok[ch] ? *reinterpret_cast<const f16x4 *>(xr + base) : f16x4{};
#pragma unroll
                for (int j = 0; j < 4; ++j) v[ch][j] = ok[ch] ? (float) t[j] : fill;
            } else {
                v[ch][0] = ok[ch] ? (float) xr[base] : fill;
            }
        }
    }

    // f(value, ch, j) gives element j of chunk ch, in fp32.
    template <class F>
    __device__ __forceinline__ void store(f16 *yr, int lane, F f) const {
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
            if (!ok[ch]) continue;
            const int base = (ch * HX_WAVE + lane) * VEC;
            if constexpr (VEC == 8) {
                f16x8 t;
#pragma unroll
                for (int j = 0; j < 8; ++j) t[j] = (f16) f(v[ch][j], ch, j);
                *reinterpret_cast<f16x8 *>(yr + base) = t;
            } else if constexpr (VEC == 4) {
                f16x4 t;
#pragma unroll
                for (int j = 0; j < 4; ++j) t[j] = (f16) f(v[ch][j], ch, j);
                *reinterpret_cast<f16x4 *>(yr + base) = t;
            } else {
                yr[base] = (f16) f(v[ch][0], ch, 0);
            }
        }
    }
};

// Per-column parameters (LayerNorm/RMSNorm weight and bias) for the lane's
// elements, in the RowRegs order. Loaded together with the row, so their
// memory latency overlaps the row's instead of following the reductions.
// A chunk past the row end holds zeros and is never used.
template <int VEC, int NCH, class T>
struct ColRegs {
    T v[NCH][VEC];

    __device__ __forceinline__ void load(const T *__restrict__ p, const bool (&ok)[NCH], int lane) {
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
            const int base = (ch * HX_WAVE + lane) * VEC;
            if (ok[ch]) {
#pragma unroll
                for (int j = 0; j < VEC; ++j) v[ch][j] = p[base + j];
            } else {
#pragma unroll
                for (int j = 0; j < VEC; ++j) v[ch][j] = T(0);
            }
        }
    }
};

template <int VEC, int NCH>
__global__ __launch_bounds__(TPB) void softmax_regs(const f16 *__restrict__ x, f16 *__restrict__ y,
                                                    int R, int C) {
    const int lane = threadIdx.x & (HX_WAVE - 1);
    const long long row = (long long) blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
    if (row >= R) return;
    RowRegs<VEC, NCH> r;
    r.load(x + row * C, C, lane, -INFINITY);
    float m = -INFINITY;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
        for (int j = 0; j < VEC; ++j) m = fmaxf(m, r.v[ch][j]);
    m = wave_max(m);
    float s = 0.0f;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
            const float e = r.ok[ch] ? expf(r.v[ch][j] - m) : 0.0f;
            r.v[ch][j] = e;
            s += e;
        }
    s = wave_sum(s);
    r.store(y + row * C, lane, [s](float e, int, int) { return e / s; });
}

template <int VEC, int NCH>
__global__ __launch_bounds__(TPB) void layernorm_regs(const f16 *__restrict__ x,
                                                      const float *__restrict__ w,
                                                      const float *__restrict__ b,
                                                      f16 *__restrict__ y, int R, int C, float eps) {
    const int lane = threadIdx.x & (HX_WAVE - 1);
    const long long row = (long long) blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
    if (row >= R) return;
    RowRegs<VEC, NCH> r;
    r.load(x + row * C, C, lane, 0.0f);
    ColRegs<VEC, NCH, float> wr, br;
    wr.load(w, r.ok, lane);
    br.load(b, r.ok, lane);
    float mean, inv;
    ln_row_stats<VEC, NCH>(r.v, r.ok, C, eps, mean, inv);
    r.store(y + row * C, lane,
            [&](float d, int ch, int j) { return ln_apply(d, inv, wr.v[ch][j], br.v[ch][j]); });
}

template <int VEC, int NCH>
__global__ __launch_bounds__(TPB) void rmsnorm_regs(const f16 *__restrict__ x,
                                                    const f16 *__restrict__ w,
                                                    f16 *__restrict__ y, int R, int C, float eps) {
    const int lane = threadIdx.x & (HX_WAVE - 1);
    const long long row = (long long) blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
    if (row >= R) return;
    RowRegs<VEC, NCH> r;
    r.load(x + row * C, C, lane, 0.0f);
    ColRegs<VEC, NCH, f16> wr;
    wr.load(w, r.ok, lane);
    float q = 0.0f;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
        for (int j = 0; j < VEC; ++j) q += r.v[ch][j] * r.v[ch][j];
    const float inv = 1.0f / sqrtf(wave_sum(q) / (float) C + eps);
    r.store(y + row * C, lane, [&](float v, int ch, int j) { return v * inv * (float) wr.v[ch][j]; });
}

// ---- rows too wide for registers: re-read x from memory ------------------------
__global__ __launch_bounds__(TPB) void softmax_loop(const f16 *__restrict__ x, f16 *__restrict__ y,
                                                    int R, int C) {
    const int lane = threadIdx.x & (HX_WAVE - 1);
    const long long row = (long long) blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
    if (row >= R) return;
    const f16 *xr = x + row * C;
    f16 *yr = y + row * C;
    float m = -INFINITY;
    for (int c = lane; c < C; c += HX_WAVE) m = fmaxf(m, (float) xr[c]);
    m = wave_max(m);
    float s = 0.0f;
    for (int c = lane; c < C; c += HX_WAVE) s += expf((float) xr[c] - m);
    s = wave_sum(s);
    for (int c = lane; c < C; c += HX_WAVE) yr[c] = (f16) (expf((float) xr[c] - m) / s);
}

__global__ __launch_bounds__(TPB) void layernorm_loop(const f16 *__restrict__ x,
                                                      const float *__restrict__ w,
                                                      const float *__restrict__ b,
                                                      f16 *__restrict__ y, int R, int C, float eps) {
    const int lane = threadIdx.x & (HX_WAVE - 1);
    const long long row = (long long) blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
    if (row >= R) return;
    const f16 *xr = x + row * C;
    f16 *yr = y + row * C;
    float s = 0.0f;
    for (int c = lane; c < C; c += HX_WAVE) s += (float) xr[c];
    const float mean = wave_sum(s) / (float) C;
    float q = 0.0f;
    for (int c = lane; c < C; c += HX_WAVE) {
        const float d = (float) xr[c] - mean;
        q += d * d;
    }
    const float inv = 1.0f / sqrtf(wave_sum(q) / (float) C + eps);
    for (int c = lane; c < C; c += HX_WAVE) yr[c] = (f16) (((float) xr[c] - mean) * inv * w[c] + b[c]);
}

__global__ __launch_bounds__(TPB) void rmsnorm_loop(const f16 *__restrict__ x,
                                                    const f16 *__restrict__ w,
                                                    f16 *__restrict__ y, int R, int C, float eps) {
    const int lane = threadIdx.x & (HX_WAVE - 1);
    const long long row = (long long) blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
    if (row >= R) return;
    const f16 *xr = x + row * C;
    f16 *yr = y + row * C;
    float q = 0.0f;
    for (int c = lane; c < C; c += HX_WAVE) q += (float) xr[c] * (float) xr[c];
    const float inv = 1.0f / sqrtf(wave_sum(q) / (float) C + eps);
    for (int c = lane; c < C; c += HX_WAVE) yr[c] = (f16) ((float) xr[c] * inv * (float) w[c]);
}

// Picks (VEC, NCH) for a row width. VEC 8 when C % 8 == 0 and C >= 512 (one
// 16-byte access per lane), VEC 4 when C % 4 == 0, else 1; NCH is the fewest
// chunks covering C, capped at 8 -- beyond that the looping kernels run.
struct Shape {
    int vec, nch;
};

inline Shape pick(int C, bool aligned16) {
    int vec = 1;
    if (aligned16 && C % 8 == 0 && C >= 512) vec = 8;
    else if (aligned16 && C % 4 == 0) vec = 4;
    const int per = HX_WAVE * vec;
    int nch = (C + per - 1) / per;
    int p2 = 1;
    while (p2 < nch) p2 <<= 1;
    return {vec, p2 <= 8 ? p2 : 0};
}

#define HX_ROW_DISPATCH(KERNEL, LOOP, grid, ...)                                   \
    do {                                                                          \
        const Shape s = pick(C, rows_aligned);                                    \
        if (s.nch == 0) { HX_LAUNCH(LOOP, grid, dim3(TPB), 0, __VA_ARGS__); break; } \
        switch (s.vec * 16 + s.nch) {                                             \
        case 8 * 16 + 1: HX_LAUNCH((KERNEL<8, 1>), grid, dim3(TPB), 0, __VA_ARGS__); break; \
        case 8 * 16 + 2: HX_LAUNCH((KERNEL<8, 2>), grid, dim3(TPB), 0, __VA_ARGS__); break; \
        case 8 * 16 + 4: HX_LAUNCH((KERNEL<8, 4>), grid, dim3(TPB), 0, __VA_ARGS__); break; \
        case 8 * 16 + 8: HX_LAUNCH((KERNEL<8, 8>), grid, dim3(TPB), 0, __VA_ARGS__); break; \
        case 4 * 16 + 1: HX_LAUNCH((KERNEL<4, 1>), grid, dim3(TPB), 0, __VA_ARGS__); break; \
        case 4 * 16 + 2: HX_LAUNCH((KERNEL<4, 2>), grid, dim3(TPB), 0, __VA_ARGS__); break; \
        case 4 * 16 + 4: HX_LAUNCH((KERNEL<4, 4>), grid, dim3(TPB), 0, __VA_ARGS__); break; \
        case 4 * 16 + 8: HX_LAUNCH((KERNEL<4, 8>), grid, dim3(TPB), 0, __VA_ARGS__); break; \
        case 1 * 16 + 1: HX_LAUNCH((KERNEL<1, 1>), grid, dim3(TPB), 0, __VA_ARGS__); break; \
        case 1 * 16 + 2: HX_LAUNCH((KERNEL<1, 2>), grid, dim3(TPB), 0, __VA_ARGS__); break; \
        case 1 * 16 + 4: HX_LAUNCH((KERNEL<1, 4>), grid, dim3(TPB), 0, __VA_ARGS__); break; \
        case 1 * 16 + 8: HX_LAUNCH((KERNEL<1, 8>), grid, dim3(TPB), 0, __VA_ARGS__); break; \
        default: HX_LAUNCH(LOOP, grid, dim3(TPB), 0, __VA_ARGS__); break;         \
        }                                                                         \
    } while (0)

inline dim3 row_grid(int R) { return dim3((unsigned) ((R + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK)); }

}  // namespace

extern "C" void softmax_fp16(const hexlib_hf *x, hexlib_hf *y, int R, int C) {
    if (R <= 0 || C <= 0 || !x || !y) return;
    auto X = reinterpret_cast<const f16 *>(x);
    auto Y = reinterpret_cast<f16 *>(y);
    const bool rows_aligned = hx::aligned(x, 16) && hx::aligned(y, 16);
    HX_ROW_DISPATCH(softmax_regs, softmax_loop, row_grid(R), X, Y, R, C);
}

extern "C" void layernorm_fp16(const hexlib_hf *x, const float *w, const float *b, hexlib_hf *y,
                               int R, int C, float eps) {
    if (R <= 0 || C <= 0 || !x || !w || !b || !y) return;
    auto X = reinterpret_cast<const f16 *>(x);
    auto Y = reinterpret_cast<f16 *>(y);
    const bool rows_aligned = hx::aligned(x, 16) && hx::aligned(y, 16);
    HX_ROW_DISPATCH(layernorm_regs, layernorm_loop, row_grid(R), X, w, b, Y, R, C, eps);
}

extern "C" void rmsnorm_fp16(const hexlib_hf *x, const hexlib_hf *w, hexlib_hf *y, int R, int C,
                             float eps) {
    if (R <= 0 || C <= 0 || !x || !w || !y) return;
    auto X = reinterpret_cast<const f16 *>(x);
    auto W = reinterpret_cast<const f16 *>(w);
    auto Y = reinterpret_cast<f16 *>(y);
    const bool rows_aligned = hx::aligned(x, 16) && hx::aligned(y, 16);
    HX_ROW_DISPATCH(rmsnorm_regs, rmsnorm_loop, row_grid(R), X, W, Y, R, C, eps);
}
