// Fused multi-head attention, forward: out = softmax(scale * q k^T) v per
// (image, head), for the encoder's full (non-causal) attention. It replaces the
// reference's chain scale -> transpose_hd -> matmul -> softmax -> matmul and the
// transposes around it (hexlib/models/vit.py:185-193); the op is an extension
// with no kernel_api.h counterpart.
//
// Layout: q, k, v and out are [rows = batch * T, H, D] fp16, the layout rope_2d
// and the linears produce (token-major, heads interleaved), so no transpose is
// needed on either side.
//
// Numerics: q.k in fp32 (MFMA accumulate), scaled in fp32; a running max and
// sum per query (online softmax, exp2 of log2e-scaled scores); the unnormalised
// probabilities are rounded to fp16 for the P.V product, accumulated in fp32;
// the output is divided by the fp32 sum and rounded to fp16 once.
//
// Structure: one 64-lane wave per 32 queries of one (image, head); keys walk in
// tiles of 32. Both products run on v_mfma_f32_32x32x16_f16 (lane l supplies
// row l % 32 of A and column l % 32 of B, 8 consecutive k at 8 * (l / 32);
// result element i of lane l is D[(i/4)*8 + (l/32)*4 + i%4][l % 32]):
//   S^T = K Q^T   A = K rows (keys), B = Q^T columns (queries): lane l then
//                 holds 16 scores of ONE query (l % 32), so the row max / sum
//                 are in-lane plus one exchange with lane l ^ 32.
//   O^T = V^T P^T A = V^T rows (d), B = P^T: the B operand is the lane's own
//                 16 probabilities, provided A's k index means the same key.
// To make that true the K rows are loaded in a permuted key order: S^T row r
// holds key kperm(r), chosen so that P's k index 8h + j of chunk c is key
// 16c + 8h + j; the V^T operand then reads 8 consecutive keys. V^T is formed
// through LDS ([D][40] halves, 80-byte rows: the 16 rows one ds_read_b128
// phase touches fall in 16 distinct bank groups).
#include <cmath>

#include "device.h"
#include "internal.h"

namespace {

constexpr int QT = 32;          // queries per wave
constexpr int KT = 32;          // keys per tile
constexpr int VT_STRIDE = 40;   // halves per LDS row of V^T

__device__ __forceinline__ int kperm(int r) {
    return 16 * (r >> 4) + 8 * ((r >> 2) & 1) + 4 * ((r >> 3) & 1) + (r & 3);
}

template <int D>
__global__ __launch_bounds__(64) void attn_fwd(const f16 *__restrict__ q, const f16 *__restrict__ k,
                                               const f16 *__restrict__ v, f16 *__restrict__ o,
                                               int T, int H, float scale_log2e) {
    constexpr int KC = D / 16;   // 16-wide d chunks of q.k
    constexpr int DT = D / 32;   // 32-row tiles of O^T
    constexpr int VCH = D / 8;   // 16-byte chunks per V row
    __shared__ __attribute__((aligned(16))) f16 vt[D * VT_STRIDE];

    const int bh = blockIdx.y;
    const int b = bh / H, h = bh % H;
    const long long ld = (long long) H * D;   // token stride
    const long long base = (long long) b * T * ld + (long long) h * D;
    const f16 *qb = q + base, *kb = k + base, *vb = v + base;
    f16 *ob = o + base;
    const int lane = threadIdx.x, hl = lane >> 5, c32 = lane & 31;
    const int q0 = blockIdx.x * QT;

    // B operand of S^T: query column c32, d = 16 kk + 8 hl .. +8
    f16x8 qf[KC];
    {
        const int qi = min(q0 + c32, T - 1);
#pragma unroll
        for (int kk = 0; kk < KC; ++kk)
            qf[kk] = *reinterpret_cast<const f16x8 *>(qb + qi * ld + 16 * kk + 8 * hl);
    }
    const int krow_key = kperm(c32);   // key (within the tile) this lane's K row holds

    f32x16 oacc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) oacc[t] = f32x16{};
    float m = -INFINITY, l = 0.f;

    for (int kt = 0; kt < T; kt += KT) {
        // K operand (A of S^T): row c32 = key kt + kperm(c32), d = 16 kk + 8 hl
        f16x8 kf[KC];
        {
            const int key = min(kt + krow_key, T - 1);   // rows past T are masked below
#pragma unroll
            for (int kk = 0; kk < KC; ++kk)
                kf[kk] = *reinterpret_cast<const f16x8 *>(kb + key * ld + 16 * kk + 8 * hl);
        }
        // V tile -> LDS as V^T[d][key]; keys past T are zero (their p is 0,
        // and 0 * garbage could be NaN)
#pragma unroll
        for (int t = 0; t < KT * VCH / 64; ++t) {
            const int e = lane + 64 * t;
            const int vk = e / VCH, d0 = (e % VCH) * 8;
            const int key = kt + vk;
            const f16x8 vv = key < T ? *reinterpret_cast<const f16x8 *>(vb + key * ld + d0) : f16x8{};
#pragma unroll
            for (int j = 0; j < 8; ++j) vt[(d0 + j) * VT_STRIDE + vk] = vv[j];
        }

        f32x16 s = f32x16{};
#pragma unroll
        for (int kk = 0; kk < KC; ++kk) s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[kk], qf[kk], s, 0, 0, 0);

        // element i of this lane is key kt + 16 (i / 8) + 8 hl + i % 8
        float tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int key = kt + 16 * (i >> 3) + 8 * hl + (i & 7);
            s[i] = key < T ? s[i] * scale_log2e : -INFINITY;
            tmax = fmaxf(tmax, s[i]);
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float m_new = fmaxf(m, tmax);     // finite: key kt < T is always valid
        const float alpha = exp2f(m - m_new);
        f16x8 pb[2];
        float psum = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float p = exp2f(s[i] - m_new);
            psum += p;
            pb[i >> 3][i & 7] = (f16) p;
        }
        l = l * alpha + psum;
        m = m_new;
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) oacc[t][i] *= alpha;

        __syncthreads();   // V^T tile written
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                const f16x8 va = *reinterpret_cast<const f16x8 *>(vt + (t * 32 + c32) * VT_STRIDE + 16 * c + 8 * hl);
                oacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[c], oacc[t], 0, 0, 0);
            }
        __syncthreads();   // V^T tile consumed before the next one is written
    }

    l += __shfl_xor(l, 32);
    const float inv = 1.0f / l;
    const int qi = q0 + c32;
    if (qi >= T) return;
    // oacc[t][i] = O^T[d = 32 t + (i/4)*8 + 4 hl + i%4][query qi]
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            f16x4 out;
#pragma unroll
            for (int e = 0; e < 4; ++e) out[e] = (f16) (oacc[t][4 * g + e] * inv);
            *reinterpret_cast<f16x4 *>(ob + qi * ld + 32 * t + 8 * g + 4 * hl) = out;
        }
}

}  // namespace

extern "C" void attention_fp16(const hexlib_hf *q, const hexlib_hf *k, const hexlib_hf *v,
                               hexlib_hf *out, int rows, int H, int D, int batch, float scale) {
    if (!q || !k || !v || !out || rows <= 0 || H <= 0 || batch <= 0 || rows % batch) return;
    if (D != 32 && D != 64) return;
    if (!hx::aligned(q, 16) || !hx::aligned(k, 16) || !hx::aligned(v, 16) || !hx::aligned(out, 8)) return;
    const int T = rows / batch;
    if ((long long) batch * H > 65535) return;
    const dim3 grid((unsigned) ((T + QT - 1) / QT), (unsigned) (batch * H));
    const float sl2e = scale * 1.4426950408889634f;
    const auto *Q = reinterpret_cast<const f16 *>(q);
    const auto *K = reinterpret_cast<const f16 *>(k);
    const auto *V = reinterpret_cast<const f16 *>(v);
    auto *O = reinterpret_cast<f16 *>(out);
    if (D == 64) HX_LAUNCH(attn_fwd<64>, grid, dim3(64), 0, Q, K, V, O, T, H, sl2e);
    else HX_LAUNCH(attn_fwd<32>, grid, dim3(64), 0, Q, K, V, O, T, H, sl2e);
}
