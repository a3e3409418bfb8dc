// Data-movement and rotation kernels: transpose_th / transpose_bth,
// transpose_hd, patchify, rope_2d.
//
// The three permutations are bit-exact by construction (pure copies). RoPE
// evaluates each product and the sum separately rounded in fp32 (FMA
// contraction switched off in that kernel), matching the scalar contract
// operation for operation (kernels/rope_2d_fp16/baseline.c:31-36).
//
// Algorithmic bytes per element moved: transposes 4 (fp16 in + out),
// patchify 8 (fp32 in + out), rope 4 + the two fp32 tables read once per
// token (8 B per (token, d)).
#include "device.h"
#include "internal.h"

namespace {

constexpr int TPB = 256;

// ---- [B,T,H,D] -> [B,H,T,D] ----------------------------------------------
// Output-ordered: consecutive threads write consecutive 16-byte chunks; each
// input run of D elements is contiguous, so reads are whole runs too.
__global__ __launch_bounds__(TPB) void tr_bth_v8(const f16x8 *__restrict__ x,
                                                 f16x8 *__restrict__ y, int T, int H, int dv,
                                                 long long total) {
    const long long stride = (long long) gridDim.x * TPB;
    for (long long o = (long long) blockIdx.x * TPB + threadIdx.x; o < total; o += stride) {
        long long r = o;
        const int c = (int) (r % dv); r /= dv;
        const int t = (int) (r % T); r /= T;
        const int h = (int) (r % H);
        const long long b = r / H;
        y[o] = x[((b * T + t) * H + h) * dv + c];
    }
}

__global__ __launch_bounds__(TPB) void tr_bth_s(const f16 *__restrict__ x, f16 *__restrict__ y,
                                                int T, int H, int D, long long total) {
    const long long stride = (long long) gridDim.x * TPB;
    for (long long o = (long long) blockIdx.x * TPB + threadIdx.x; o < total; o += stride) {
        long long r = o;
        const int d = (int) (r % D); r /= D;
        const int t = (int) (r % T); r /= T;
        const int h = (int) (r % H);
        const long long b = r / H;
        y[o] = x[((b * T + t) * H + h) * D + d];
    }
}

// ---- [B,T,D] -> [B,D,T] : 64x64 tiles through LDS ---------------------------
// The read side walks rows of D, the write side rows of T; the LDS tile
// (padded to an odd word stride) turns the strided half into a bank-spread
// column read. Full tiles use 16-byte global accesses on both sides.
constexpr int TT = 64;

__global__ __launch_bounds__(TPB) void tr_hd_tile(const f16 *__restrict__ x, f16 *__restrict__ y,
                                                  int T, int D, int vec) {
    __shared__ f16 tile[TT][TT + 2];
    const int b = blockIdx.z;
    const int t0 = blockIdx.y * TT, d0 = blockIdx.x * TT;
    const f16 *xb = x + (long long) b * T * D;
    f16 *yb = y + (long long) b * T * D;
    const int r = threadIdx.x >> 2, c0 = (threadIdx.x & 3) * 16;
    const bool full = vec && (t0 + TT <= T) && (d0 + TT <= D) && ((D & 7) == 0) && ((T & 7) == 0);
    if (full) {
        const f16x8 *src = reinterpret_cast<const f16x8 *>(xb + (long long) (t0 + r) * D + d0 + c0);
        const f16x8 v0 = src[0], v1 = src[1];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            tile[r][c0 + j] = v0[j];
            tile[r][c0 + 8 + j] = v1[j];
        }
    } else {
        const int t = t0 + r;
        for (int j = 0; j < 16; ++j) {
            const int d = d0 + c0 + j;
            tile[r][c0 + j] = (t < T && d < D) ? xb[(long long) t * D + d] : (f16) 0;
        }
    }
    __syncthreads();
    // write row d = d0 + r, columns t0 + c0 .. +15
    if (full) {
        f16x8 v0, v1;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v0[j] = tile[c0 + j][r];
            v1[j] = tile[c0 + 8 + j][r];
        }
        f16x8 *dst = reinterpret_cast<f16x8 *>(yb + (long long) (d0 + r) * T + t0 + c0);
        dst[0] = v0;
        dst[1] = v1;
    } else {
        const int d = d0 + r;
        for (int j = 0; j < 16; ++j) {
            const int t = t0 + c0 + j;
            if (d < D && t < T) yb[(long long) d * T + t] = tile[c0 + j][r];
        }
    }
}

// ---- patchify ----------------------------------------------------------------
// out[token][feat] = img[b*C + c][t][h][w] with token (per image) in merge-block
// order ((bh*Bw + bw)*m + mh)*m + mw and feat = ((c*T + t)*p + ph)*p + pw
// (kernels/patchify_fp32/kernel_api.h:18-38). Output-ordered; with p % 4 == 0
// each thread moves one 16-byte run of 4 consecutive pw.
struct PatchGeom {
    int C, T, H, W, p, m, gh, gw, batch;
};

template <int V>
__global__ __launch_bounds__(TPB) void patchify_k(const float *__restrict__ img,
                                                  float *__restrict__ out, PatchGeom g,
                                                  long long total) {
    const int feat = g.C * g.T * g.p * g.p;
    const int fv = feat / V;
    const int ntok = g.gh * g.gw;
    const int Bw = g.gw / g.m;
    const long long stride = (long long) gridDim.x * TPB;
    for (long long o = (long long) blockIdx.x * TPB + threadIdx.x; o < total; o += stride) {
        const long long row = o / fv;
        const int f = (int) (o % fv) * V;
        const int b = (int) (row / ntok);
        const int tok = (int) (row % ntok);
        const int mw = tok % g.m, mh = (tok / g.m) % g.m;
        const int blk = tok / (g.m * g.m);
        const int bw = blk % Bw, bh = blk / Bw;
        const int gy = bh * g.m + mh, gx = bw * g.m + mw;
        const int pw = f % g.p, ph = (f / g.p) % g.p;
        const int ct = f / (g.p * g.p);  // c*T + t
        const long long src = (((long long) b * g.C * g.T + ct) * g.H + (long long) gy * g.p + ph) * g.W
                              + (long long) gx * g.p + pw;
        if constexpr (V == 4) {
            reinterpret_cast<f32x4 *>(out)[o] = *reinterpret_cast<const f32x4 *>(img + src);
        } else {
            out[o] = img[src];
        }
    }
}

// ---- rope_2d -------------------------------------------------------------------
// y[t,h,i]      = x[t,h,i]*cos[t,i] - x[t,h,i+half]*sin[t,i]
// y[t,h,i+half] = x[t,h,i+half]*cos[t,i+half] + x[t,h,i]*sin[t,i+half]
// One thread per (t, h, 4 consecutive i) when half % 4 == 0.
template <int V>
__global__ __launch_bounds__(TPB) void rope_k(const f16 *__restrict__ x,
                                              const float *__restrict__ cs,
                                              const float *__restrict__ sn, f16 *__restrict__ y,
                                              int T, int H, int D, long long xld, long long yld,
                                              long long total) {
#pragma clang fp contract(off)
    const int half = D / 2;
    const int hv = half / V;
    const long long stride = (long long) gridDim.x * TPB;
    for (long long o = (long long) blockIdx.x * TPB + threadIdx.x; o < total; o += stride) {
        const int i = (int) (o % hv) * V;
        const long long th = o / hv;  // t*H + h
        const int t = (int) (th / H);
        const int hh = (int) (th % H);
        const f16 *xr = x + t * xld + (long long) hh * D;
        f16 *yr = y + t * yld + (long long) hh * D;
        const float *cr = cs + (long long) t * D;
        const float *sr = sn + (long long) t * D;
        float x0[V], x1[V], c0[V], c1[V], s0[V], s1[V];
        if constexpr (V == 4) {
            const f16x4 a = *reinterpret_cast<const f16x4 *>(xr + i);
            const f16x4 bb = *reinterpret_cast<const f16x4 *>(xr + i + half);
            const f32x4 ca = *reinterpret_cast<const f32x4 *>(cr + i);
            const f32x4 cb = *reinterpret_cast<const f32x4 *>(cr + i + half);
            const f32x4 sa = *reinterpret_cast<const f32x4 *>(sr + i);
            const f32x4 sb = *reinterpret_cast<const f32x4 *>(sr + i + half);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x0[j] = (float) a[j]; x1[j] = (float) bb[j];
                c0[j] = ca[j]; c1[j] = cb[j]; s0[j] = sa[j]; s1[j] = sb[j];
            }
        } else {
            x0[0] = (float) xr[i]; x1[0] = (float) xr[i + half];
            c0[0] = cr[i]; c1[0] = cr[i + half]; s0[0] = sr[i]; s1[0] = sr[i + half];
        }
        f16 y0[V], y1[V];
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const float p0 = x0[j] * c0[j];
            const float q0 = x1[j] * s0[j];
            const float p1 = x1[j] * c1[j];
            const float q1 = x0[j] * s1[j];
            y0[j] = (f16) (p0 - q0);
            y1[j] = (f16) (p1 + q1);
        }
        if constexpr (V == 4) {
            f16x4 u, w;
#pragma unroll
            for (int j = 0; j < 4; ++j) { u[j] = y0[j]; w[j] = y1[j]; }
            *reinterpret_cast<f16x4 *>(yr + i) = u;
            *reinterpret_cast<f16x4 *>(yr + i + half) = w;
        } else {
            yr[i] = y0[0];
            yr[i + half] = y1[0];
        }
    }
}

inline unsigned grid_for(long long total) { return hx::blocks_for(total, TPB, 16384); }

}  // namespace

extern "C" void transpose_bth_fp16(const hexlib_hf *x, hexlib_hf *y, int B, int T, int H, int D) {
    if (B <= 0 || T <= 0 || H <= 0 || D <= 0 || !x || !y) return;
    auto X = reinterpret_cast<const f16 *>(x);
    auto Y = reinterpret_cast<f16 *>(y);
    const long long n = (long long) B * T * H * D;
    if (D % 8 == 0 && hx::aligned(x, 16) && hx::aligned(y, 16)) {
        const long long total = n / 8;
        HX_LAUNCH(tr_bth_v8, dim3(grid_for(total)), dim3(TPB), 0,
                  reinterpret_cast<const f16x8 *>(X), reinterpret_cast<f16x8 *>(Y), T, H, D / 8,
                  total);
    } else {
        HX_LAUNCH(tr_bth_s, dim3(grid_for(n)), dim3(TPB), 0, X, Y, T, H, D, n);
    }
}

extern "C" void transpose_th_fp16(const hexlib_hf *x, hexlib_hf *y, int T, int H, int D) {
    transpose_bth_fp16(x, y, 1, T, H, D);
}

extern "C" void transpose_hd_fp16(const hexlib_hf *x, hexlib_hf *y, int B, int T, int D) {
    if (B <= 0 || T <= 0 || D <= 0 || !x || !y || B > 65535) return;
    const int vec_ok = hx::aligned(x, 16) && hx::aligned(y, 16);
    dim3 grid((D + TT - 1) / TT, (T + TT - 1) / TT, B);
    if (grid.y > 65535) return;
    HX_LAUNCH(tr_hd_tile, grid, dim3(TPB), 0, reinterpret_cast<const f16 *>(x),
              reinterpret_cast<f16 *>(y), T, D, vec_ok);
}

extern "C" void patchify_fp32_batched(const float *img, float *out, int BC, int T, int H, int W,
                                      int patch, int merge, int grid_h, int grid_w, int batch) {
    if (batch <= 0) batch = 1;
    if (BC <= 0 || T <= 0 || H <= 0 || W <= 0 || patch <= 0 || merge <= 0 || grid_h <= 0 ||
        grid_w <= 0 || !img || !out)
        return;
    if (BC % batch || grid_h * patch != H || grid_w * patch != W || grid_h % merge ||
        grid_w % merge)
        return;
    PatchGeom g{BC / batch, T, H, W, patch, merge, grid_h, grid_w, batch};
    const long long n = (long long) batch * grid_h * grid_w * g.C * T * patch * patch;
    if (patch % 4 == 0 && W % 4 == 0 && hx::aligned(img, 16) && hx::aligned(out, 16)) {
        HX_LAUNCH(patchify_k<4>, dim3(grid_for(n / 4)), dim3(TPB), 0, img, out, g, n / 4);
    } else {
        HX_LAUNCH(patchify_k<1>, dim3(grid_for(n)), dim3(TPB), 0, img, out, g, n);
    }
}

extern "C" void patchify_fp32(const float *img, float *out, int C, int T, int H, int W, int patch,
                              int merge, int grid_h, int grid_w) {
    patchify_fp32_batched(img, out, C, T, H, W, patch, merge, grid_h, grid_w, 1);
}

namespace {
// rope over T tokens of H heads of D, token rows xld / yld halves apart.
void rope_launch(const hexlib_hf *x, const float *costab, const float *sintab, hexlib_hf *y,
                 int T, int H, int D, long long xld, long long yld) {
    auto X = reinterpret_cast<const f16 *>(x);
    auto Y = reinterpret_cast<f16 *>(y);
    const int half = D / 2;
    if (half % 4 == 0 && xld % 4 == 0 && yld % 4 == 0 && hx::aligned(x, 8) && hx::aligned(y, 8) &&
        hx::aligned(costab, 16) && hx::aligned(sintab, 16)) {
        const long long total = (long long) T * H * (half / 4);
        HX_LAUNCH(rope_k<4>, dim3(grid_for(total)), dim3(TPB), 0, X, costab, sintab, Y, T, H, D, xld, yld,
                  total);
    } else {
        const long long total = (long long) T * H * half;
        HX_LAUNCH(rope_k<1>, dim3(grid_for(total)), dim3(TPB), 0, X, costab, sintab, Y, T, H, D, xld, yld,
                  total);
    }
}
}  // namespace

extern "C" void rope_2d_fp16(const hexlib_hf *x, const float *costab, const float *sintab,
                             hexlib_hf *y, int T, int H, int D) {
    if (T <= 0 || H <= 0 || D <= 0 || (D & 1) || !x || !costab || !sintab || !y) return;
    rope_launch(x, costab, sintab, y, T, H, D, (long long) H * D, (long long) H * D);
}

extern "C" void rope_2d_qk_fp16(const hexlib_hf *qkv, const float *costab, const float *sintab,
                                hexlib_hf *qk, int rows, int H, int D) {
    if (rows <= 0 || H <= 0 || D <= 0 || (D & 1) || !qkv || !costab || !sintab || !qk) return;
    // q's H heads then k's H heads are 2H consecutive heads of each qkv row
    rope_launch(qkv, costab, sintab, qk, rows, 2 * H, D, 3LL * H * D, 2LL * H * D);
}
