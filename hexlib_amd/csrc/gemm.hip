// fp16 GEMMs on CDNA4 MFMA: matmul_fp16 (batched), matmul_epilogue_f16w_fp16
// (W [K,N]), matmul_epilogue_f16wt_fp16 (W^T [N,K]), matmul_epilogue_fp16
// (q4_0 blocked along N -- the reference kernel ABI) and
// matmul_epilogue_q4k_fp16 (q4_0 grouped along K of W^T).
//
// Numerics (kernels/matmul_fp16/kernel_api.h:18-29, kernels/matmul_epilogue_fp16/
// kernel_api.h:16-27, baseline.c:34-97): fp16 x fp16 products accumulated in
// fp32 by v_mfma_f32_32x32x16_f16; a q4_0 weight is dequantized to
// fp16(d * (q - 8)) before it is multiplied (the reference kernel's rounding);
// then the fp32 bias is added, the activation applied in fp32 and the result
// rounded to fp16 once. Split-K partial sums are reduced in a fixed order, so
// results are identical run to run.
//
// Structure. A 256-thread workgroup (4 waves, 2 x 2) owns a BM x BN output tile
// and walks its K range in BK = 64 slices staged in LDS with K contiguous per
// row ([m][k] and [n][k], rows padded to 144 B so a 16-lane ds_read_b128 phase
// touches every bank once). The next slice's global loads are issued into
// registers before the current slice's MFMAs and written to the other LDS
// buffer afterwards: one barrier per slice. B arrives in one of five layouts
// and is converted to [n][k] on its way into LDS:
//   B_Q8K q8_0 [N][K/32] 34-B blocks -- dequantize, 16-byte LDS writes
//   B_KN  fp16 [K, N]                -- 16-byte loads along n, 2-byte LDS scatter
//   B_NK  fp16 [N, K] (W^T)          -- 16-byte loads and 16-byte LDS writes
//   B_Q4N q4_0 [K][N/32] 18-B blocks -- dequantize, 2-byte LDS scatter
//   B_Q4K q4_0 [N][K/32] 18-B blocks -- dequantize, 16-byte LDS writes
//
// MFMA roles are swapped: the weight fragment is the instruction's A operand
// and the activation fragment its B operand, so the 32x32 result is C^T and
// lane l holds, for output row m = l % 32, four runs of 4 consecutive output
// columns -- stored as 8-byte vectors. (Operand layout of
// v_mfma_f32_32x32x16_f16: lane l supplies row l % 32 of A and column l % 32
// of B, each as 8 consecutive k at offset 8 * (l / 32); result element i of
// lane l is D[(i/4)*8 + (l/32)*4 + i%4][l % 32].)
//
// Split-K (small M): gridDim.z = batch * splits; split s writes its fp32
// partial tile to a library workspace and `splitk_reduce` sums the splits in
// order 0..S-1, adds bias, applies the activation and rounds.
#include <atomic>
#include <type_traits>
#include <mutex>
#include <vector>

#include "device.h"
#include "lnmath.h"
#include "internal.h"

namespace {

constexpr int TPB = 256;
constexpr int BK = 64;
constexpr int LDS_STRIDE = BK + 8;  // halves per LDS row (144 B)
constexpr int MAX_SPLITS = 16;      // split-K factor limit (splitk_reduce unrolls to it)

enum BMode { B_KN = 0, B_NK = 1, B_Q4N = 2, B_Q4K = 3, B_Q8K = 4 };

struct GemmArgs {
    const f16 *A;
    long long lda, sA;          // row stride, batch stride (elements)
    const void *B;
    long long ldb, sB;          // fp16: elements; q4: bytes per block row / batch stride bytes
    const float *bias;
    f16 *C;
    long long ldc, sC;
    int M, N, K, act;
    int splits, k_per_split;    // split-K: K range [s*k_per_split, min(K, (s+1)*k_per_split))
    float *ws;                  // split-K workspace [batch][splits][M][N] fp32
    const f16 *R;               // residual [M, N] (row stride ldr) added after rounding, or null
    long long ldr;
    // rope on output columns [0, rope_cols) in heads of rope_d, or null; the tables are
    // stored transposed, [rope_d, M], so the 32 rows of an MFMA output column read 32
    // consecutive floats; the weight rows of each rope head are stored pair-interleaved
    // (see rope_store4)
    const float *rcos, *rsin;
    int rope_cols, rope_d;
    // LayerNorm of A's rows (over all K) applied before the product, or null:
    // out = epilogue(LN(A) @ B), LN(A) rounded to fp16 as layernorm_fp16 stores it
    const float *ln_w, *ln_b;
    float ln_eps;
    // folded LayerNorm (gemm_nk_kw<..., LNF>): A is the LayerNorm's raw input x,
    // B its weight-scaled W'^T, and bias holds 2N floats, c2 then c1 (see
    // gemm_nk_kw); the row statistics are taken from the A tiles in the ring
    float lnf_eps;
};

__device__ __forceinline__ bool hx_aligned8(const void *p) {
    return (reinterpret_cast<uintptr_t>(p) & 7) == 0;
}

// Rope in the epilogue (rope columns only). The weight rows of each rope head
// are stored pair-interleaved: computed column 2i of a head is the head's
// feature i and column 2i + 1 its feature i + D/2, so a lane's 4 consecutive
// columns n .. n + 3 (n % 4 == 0, D % 4 == 0) hold the two rotation pairs
// (i0, i0 + D/2) and (i0 + 1, i0 + 1 + D/2), i0 = (n % D) / 2. Each value is
// first rounded to fp16 (the linear's stored output), rotated in fp32 with the
// products and the sum rounded separately, rounded to fp16 again (rope_2d_fp16's
// arithmetic, kernels/rope_2d_fp16/baseline.c), and stored de-interleaved at
// features (i0, i0 + 1) and (i0 + D/2, i0 + 1 + D/2) of the head.
struct RopeQuad {
    int lo, hi;   // output features of pair i0 (lo, lo + 1 holds pair i0 + 1) and of its partners
    int t;        // table column of pair i0
};

__device__ __forceinline__ RopeQuad rope_quad(int n, int rope_d) {
    const int lc = n % rope_d, i0 = lc >> 1;
    return {n - lc + i0, n - lc + i0 + (rope_d >> 1), i0};
}

// c0 = cos[t], cos[t + 1]; c1 = cos[t + D/2], cos[t + 1 + D/2]; s0, s1 likewise
__device__ __forceinline__ void rope_store4(f16 *crow, RopeQuad q, const float v[4], float2 c0, float2 c1,
                                            float2 s0, float2 s1) {
#pragma clang fp contract(off)
    f16x2 lo, hi;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const float x0 = (float) (f16) v[2 * u], x1 = (float) (f16) v[2 * u + 1];
        const float ca = u ? c0.y : c0.x, sa = u ? s0.y : s0.x;
        const float cb = u ? c1.y : c1.x, sb = u ? s1.y : s1.x;
        const float p0 = x0 * ca, q0 = x1 * sa, p1 = x1 * cb, q1 = x0 * sb;
        lo[u] = (f16) f32_rounded(p0 - q0);
        hi[u] = (f16) f32_rounded(p1 + q1);
    }
    *reinterpret_cast<f16x2 *>(crow + q.lo) = lo;
    *reinterpret_cast<f16x2 *>(crow + q.hi) = hi;
}

// One output's epilogue: act(acc + bias) rounded to fp16 and, with a residual
// r, fp16(float(r) + float(that)) -- matmul_epilogue then add_fp16, each
// rounded as the reference stores it (the sum is materialised in fp32 first,
// so the compiler cannot fuse it into the fp16 conversion).
__device__ __forceinline__ f16 epi(float v, int act, bool has_r, f16 r) {
    // the activation's fp32 result is materialised before the fp16 rounding,
    // so no form fuses the last multiply into the conversion (one rounding
    // instead of the reference's two)
    const f16 h = (f16) f32_rounded(apply_act(v, act));
    if (!has_r) return h;
    return (f16) f32_rounded((float) r + (float) h);
}

// The same with the activation and the residual fixed at compile time: an
// unrolled epilogue over 16 outputs then holds no branch per output (the
// runtime form costs about 1.5 us per launch in the batch-1 GEMMs' epilogue).
template <int ACT>
__device__ __forceinline__ float act_t(float x) {
    if constexpr (ACT == 1) return gelu_tanh_f32(x);
    else if constexpr (ACT == 2) return gelu_erf_f32(x);
    else return x;
}

template <int ACT, bool RES>
__device__ __forceinline__ f16 epi_t(float v, f16 r) {
    const f16 h = (f16) f32_rounded(act_t<ACT>(v));
    if constexpr (!RES) return h;
    else return (f16) f32_rounded((float) r + (float) h);
}


// The unvectorised store of up to 4 consecutive outputs (ragged N, unaligned
// rows); out of line so the tiled kernels' unrolled epilogues stay small.
__device__ __noinline__ void store_tail(f16 *dst, int cnt, int act, const f16 *r, float v0, float v1,
                                        float v2, float v3) {
    const float v[4] = {v0, v1, v2, v3};
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (e < cnt) dst[e] = epi(v[e], act, r, r ? r[e] : (f16) 0);
}

// One 32x32 output block's plain epilogue (the lane holds row m, columns
// nb + 8 g + 4 (lane / 32) .. + 3 in MFMA order) with the activation and the
// residual fixed at compile time; kw_store dispatches on the runtime values.
// The bias of one 32-column block, columns nb .. nb + 31 (nb wave-uniform), read
// through the constant address space: uniform addresses become scalar loads,
// issued at kernel start and tracked apart from the vector loads of the ring.
struct BlockBias {
    float v[32];
};

__device__ __forceinline__ BlockBias load_block_bias(const GemmArgs &p, int nb) {
    typedef const __attribute__((address_space(4))) float cfloat;
    BlockBias b;
    const int nbu = __builtin_amdgcn_readfirstlane(nb);
    if (p.bias && nbu + 32 <= p.N) {
        const cfloat *src = reinterpret_cast<const cfloat *>(reinterpret_cast<uintptr_t>(p.bias + nbu));
#pragma unroll
        for (int k = 0; k < 32; ++k) b.v[k] = src[k];
    } else {
#pragma unroll
        for (int k = 0; k < 32; ++k) b.v[k] = (p.bias && nbu + k < p.N) ? p.bias[nbu + k] : 0.0f;
    }
    return b;
}

// The residual of one 32x32 block (the lane's 4 groups of 4 columns), loaded
// at kernel start, before the ring's first copies, so its latency is spent
// under the K loop; zero where the vector store does not apply.
struct BlockRes {
    f16x4 r[4];
};

template <int NG = 4>
__device__ __forceinline__ BlockRes load_block_res(const GemmArgs &p, int m, int nb, int lane, bool vec_store) {
    BlockRes t{};
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int n = nb + g * 8 + (lane >> 5) * 4;
        t.r[g] = p.R && vec_store && m < p.M && n + 3 < p.N
                     ? *reinterpret_cast<const f16x4 *>(p.R + (long long) m * p.ldr + n) : f16x4{};
    }
    return t;
}

// NG: the 8-column groups stored (3: the first 24 columns of a 32 x 24 tile).
template <int ACT, bool RES, int NG = 4>
__device__ __forceinline__ void kw_store_t(const GemmArgs &p, int m, int nb, int lane, const f32x16 &sum,
                                           bool vec_store, const BlockBias &bb, const BlockRes &br) {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int n = nb + g * 8 + (lane >> 5) * 4;
        float bv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[e] = (lane >> 5) ? bb.v[g * 8 + 4 + e] : bb.v[g * 8 + e];
        f16 *dst = p.C + (long long) m * p.ldc + n;
        if (vec_store && n + 3 < p.N) {
            f16x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = epi_t<ACT, RES>(sum[g * 4 + e] + bv[e], br.r[g][e]);
            *reinterpret_cast<f16x4 *>(dst) = o;
        } else {
            store_tail(dst, p.N - n, p.act, p.R ? p.R + m * p.ldr + n : nullptr, sum[g * 4] + bv[0],
                       sum[g * 4 + 1] + bv[1], sum[g * 4 + 2] + bv[2], sum[g * 4 + 3] + bv[3]);
        }
    }
}

// Calls f(integral_constant<int, ACT>, integral_constant<bool, RES>) for the
// runtime activation (0..2) and residual.
template <typename F>
__device__ __forceinline__ void dispatch_epi(int act, bool res, F &&f) {
    using A0 = std::integral_constant<int, 0>;
    using A1 = std::integral_constant<int, 1>;
    using A2 = std::integral_constant<int, 2>;
    using R0 = std::integral_constant<bool, false>;
    using R1 = std::integral_constant<bool, true>;
    if (act == 1) {
        if (res) f(A1{}, R1{});
        else f(A1{}, R0{});
    } else if (act == 2) {
        if (res) f(A2{}, R1{});
        else f(A2{}, R0{});
    } else {
        if (res) f(A0{}, R1{});
        else f(A0{}, R0{});
    }
}


// The plain epilogue of one whole 32x32 block (nb + 32 <= N, 16-byte aligned
// rows) staged through a wave-private LDS tile (rows of 40 halves): each lane
// computes its 16 outputs in MFMA order into the tile, then the wave stores
// the block as 16-byte row segments, four lanes per 64-byte row. Taken by
// the 64x64 tile, whose four waves each store a block (the folded fc1 at
// batch 1: 6.67 -> 6.49 us); the 32x32 tile's one storing wave keeps the
// direct 8-byte stores, which measured faster there.
template <int ACT, bool RES>
__device__ __forceinline__ void kw_store_staged_t(const GemmArgs &p, int mb, int nb, int lane, const f32x16 &sum,
                                                  const BlockBias &bb, const BlockRes &br, f16 *tile) {
    constexpr int TS = 40;
    const int r = lane & 31;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        float bv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[e] = (lane >> 5) ? bb.v[g * 8 + 4 + e] : bb.v[g * 8 + e];
        f16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = epi_t<ACT, RES>(sum[g * 4 + e] + bv[e], br.r[g][e]);
        *reinterpret_cast<f16x4 *>(tile + r * TS + g * 8 + (lane >> 5) * 4) = o;
    }
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int row = it * 16 + (lane >> 2), c = (lane & 3) * 8;
        const f16x8 v = *reinterpret_cast<const f16x8 *>(tile + row * TS + c);
        if (mb + row < p.M) *reinterpret_cast<f16x8 *>(p.C + (long long) (mb + row) * p.ldc + nb + c) = v;
    }
}

__device__ __forceinline__ void kw_store_staged(const GemmArgs &p, int mb, int nb, int lane, const f32x16 &sum,
                                                const BlockBias &bb, const BlockRes &br, f16 *tile) {
    dispatch_epi(p.act, p.R != nullptr, [&](auto act_c, auto res_c) {
        kw_store_staged_t<decltype(act_c)::value, decltype(res_c)::value>(p, mb, nb, lane, sum, bb, br, tile);
    });
}

template <int NG = 4>
__device__ __forceinline__ void kw_store(const GemmArgs &p, int m, int nb, int lane, const f32x16 &sum,
                                         bool vec_store, const BlockBias &bb, const BlockRes &br) {
    const bool res = p.R != nullptr;
    if (p.act == 1) {
        if (res) kw_store_t<1, true, NG>(p, m, nb, lane, sum, vec_store, bb, br);
        else kw_store_t<1, false, NG>(p, m, nb, lane, sum, vec_store, bb, br);
    } else if (p.act == 2) {
        if (res) kw_store_t<2, true, NG>(p, m, nb, lane, sum, vec_store, bb, br);
        else kw_store_t<2, false, NG>(p, m, nb, lane, sum, vec_store, bb, br);
    } else {
        if (res) kw_store_t<0, true, NG>(p, m, nb, lane, sum, vec_store, bb, br);
        else kw_store_t<0, false, NG>(p, m, nb, lane, sum, vec_store, bb, br);
    }
}


__device__ __forceinline__ f16 q4_val(float d, int q) { return (f16) (d * (float) (q - 8)); }

__device__ __forceinline__ void load_q4_block(const uint8_t *p, float &d, uint32_t qs[4]) {
    const uint16_t *h = reinterpret_cast<const uint16_t *>(p);
    d = (float) __builtin_bit_cast(f16, h[0]);
#pragma unroll
    for (int i = 0; i < 4; ++i) qs[i] = (uint32_t) h[1 + 2 * i] | ((uint32_t) h[2 + 2 * i] << 16);
}

// Half a q8_0 block (16 int8 at byte 2 + 16 * half, 2-byte aligned) and its scale.
__device__ __forceinline__ void load_q8_half(const uint8_t *p, int half, float &d, uint32_t qs[4]) {
    const uint16_t *h = reinterpret_cast<const uint16_t *>(p);
    d = (float) __builtin_bit_cast(f16, h[0]);
#pragma unroll
    for (int i = 0; i < 4; ++i) qs[i] = (uint32_t) h[1 + 8 * half + 2 * i] | ((uint32_t) h[2 + 8 * half + 2 * i] << 16);
}

// q * d rounded once to fp16 (the product of an int8 and an fp16 is exact in fp32).
__device__ __forceinline__ f16 q8_val(float d, const uint32_t qs[4], int j) {
    return (f16) (d * (float) (int8_t) ((qs[j >> 2] >> ((j & 3) * 8)) & 0xFF));
}

__device__ __forceinline__ int nib(const uint32_t qs[4], int j, int shift) {
    return (int) ((qs[j >> 2] >> ((j & 3) * 8 + shift)) & 0xF);
}

template <int BM, int BN, int MODE, bool AVEC, bool BVEC>
struct Gemm {
    static constexpr int TM = BM / 64;   // 32-row MFMA tiles per wave along M
    static constexpr int TN = BN / 64;
    static constexpr int A_VECS = BM * BK / 8 / TPB;
    static constexpr int B_VECS = BN * BK / 8 / TPB;
    static constexpr int Q4N_ITEMS_ALL = BK * (BN / 32) * 2;   // (k, block, half)
    static constexpr int Q4K_ITEMS_ALL = BN * (BK / 32) * 2;   // (n, block, half)
    static constexpr int Q4N_ITEMS = (Q4N_ITEMS_ALL + TPB - 1) / TPB;
    static constexpr int Q4K_ITEMS = (Q4K_ITEMS_ALL + TPB - 1) / TPB;
    static constexpr int B_ITEMS = MODE == B_Q4N ? Q4N_ITEMS : (MODE == B_Q4K || MODE == B_Q8K) ? Q4K_ITEMS : B_VECS;
    static constexpr bool Q4 = MODE == B_Q4N || MODE == B_Q4K || MODE == B_Q8K;   // block-quantized B

    struct Regs {
        f16x8 a[A_VECS];
        f16x8 b[Q4 ? 1 : B_ITEMS];
        float qd[Q4 ? B_ITEMS : 1];
        uint32_t qs[Q4 ? B_ITEMS : 1][4];
    };

    static __device__ __forceinline__ void load_a(const GemmArgs &p, const f16 *A, int m0, int k0,
                                                  int kend, Regs &r) {
#pragma unroll
        for (int i = 0; i < A_VECS; ++i) {
            const int v = threadIdx.x + i * TPB;
            const int row = v / (BK / 8), kc = (v % (BK / 8)) * 8;
            const int m = m0 + row, k = k0 + kc;
            if constexpr (AVEC) {
                r.a[i] = (m < p.M && k < kend) ? *reinterpret_cast<const f16x8 *>(A + m * p.lda + k)
                                               : f16x8{};
            } else {
                f16x8 t;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    t[j] = (m < p.M && k + j < kend) ? A[m * p.lda + k + j] : (f16) 0;
                r.a[i] = t;
            }
        }
    }

    static __device__ __forceinline__ void load_b(const GemmArgs &p, const void *Bv, int n0, int k0,
                                                  int kend, Regs &r) {
        if constexpr (MODE == B_KN) {
            const f16 *B = reinterpret_cast<const f16 *>(Bv);
#pragma unroll
            for (int i = 0; i < B_VECS; ++i) {
                const int v = threadIdx.x + i * TPB;
                const int kr = v / (BN / 8), nc = (v % (BN / 8)) * 8;
                const int k = k0 + kr, n = n0 + nc;
                if constexpr (BVEC) {
                    r.b[i] = (k < kend && n < p.N) ? *reinterpret_cast<const f16x8 *>(B + k * p.ldb + n)
                                                   : f16x8{};
                } else {
                    f16x8 t;
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        t[j] = (k < kend && n + j < p.N) ? B[k * p.ldb + n + j] : (f16) 0;
                    r.b[i] = t;
                }
            }
        } else if constexpr (MODE == B_NK) {
            const f16 *B = reinterpret_cast<const f16 *>(Bv);
#pragma unroll
            for (int i = 0; i < B_VECS; ++i) {
                const int v = threadIdx.x + i * TPB;
                const int row = v / (BK / 8), kc = (v % (BK / 8)) * 8;
                const int n = n0 + row, k = k0 + kc;
                if constexpr (BVEC) {
                    r.b[i] = (n < p.N && k < kend) ? *reinterpret_cast<const f16x8 *>(B + n * p.ldb + k)
                                                   : f16x8{};
                } else {
                    f16x8 t;
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        t[j] = (n < p.N && k + j < kend) ? B[n * p.ldb + k + j] : (f16) 0;
                    r.b[i] = t;
                }
            }
        } else if constexpr (MODE == B_Q4N) {
            const uint8_t *W = reinterpret_cast<const uint8_t *>(Bv);
#pragma unroll
            for (int i = 0; i < Q4N_ITEMS; ++i) {
                const int it = threadIdx.x + i * TPB;
                const int blk = it >> 1;
                const int kr = blk / (BN / 32), nb = blk % (BN / 32);
                const int k = k0 + kr, n = n0 + nb * 32;
                r.qd[i] = 0.0f;
                r.qs[i][0] = r.qs[i][1] = r.qs[i][2] = r.qs[i][3] = 0x88888888u;  // q = 8 -> 0
                if (it < Q4N_ITEMS_ALL && k < kend && n < p.N)
                    load_q4_block(W + (long long) k * p.ldb + (long long) (n / 32) * 18, r.qd[i], r.qs[i]);
            }
        } else if constexpr (MODE == B_Q4K) {
            const uint8_t *W = reinterpret_cast<const uint8_t *>(Bv);
#pragma unroll
            for (int i = 0; i < Q4K_ITEMS; ++i) {
                const int it = threadIdx.x + i * TPB;
                const int blk = it >> 1;
                const int nr = blk / (BK / 32), kb = blk % (BK / 32);
                const int n = n0 + nr, k = k0 + kb * 32;
                r.qd[i] = 0.0f;
                r.qs[i][0] = r.qs[i][1] = r.qs[i][2] = r.qs[i][3] = 0x88888888u;
                if (it < Q4K_ITEMS_ALL && n < p.N && k < kend)
                    load_q4_block(W + (long long) n * p.ldb + (long long) (k / 32) * 18, r.qd[i], r.qs[i]);
            }
        } else {
            // q8_0 along K of W^T: item = (n, block, half), 16 int8 each
            const uint8_t *W = reinterpret_cast<const uint8_t *>(Bv);
#pragma unroll
            for (int i = 0; i < Q4K_ITEMS; ++i) {
                const int it = threadIdx.x + i * TPB;
                const int blk = it >> 1, half = it & 1;
                const int nr = blk / (BK / 32), kb = blk % (BK / 32);
                const int n = n0 + nr, k = k0 + kb * 32;
                r.qd[i] = 0.0f;
                r.qs[i][0] = r.qs[i][1] = r.qs[i][2] = r.qs[i][3] = 0u;
                if (it < Q4K_ITEMS_ALL && n < p.N && k < kend)
                    load_q8_half(W + (long long) n * p.ldb + (long long) (k / 32) * 34, half, r.qd[i], r.qs[i]);
            }
        }
    }

    static __device__ __forceinline__ void store(f16 *As, f16 *Bs, const Regs &r) {
#pragma unroll
        for (int i = 0; i < A_VECS; ++i) {
            const int v = threadIdx.x + i * TPB;
            const int row = v / (BK / 8), kc = (v % (BK / 8)) * 8;
            *reinterpret_cast<f16x8 *>(As + row * LDS_STRIDE + kc) = r.a[i];
        }
        if constexpr (MODE == B_KN) {
#pragma unroll
            for (int i = 0; i < B_VECS; ++i) {
                const int v = threadIdx.x + i * TPB;
                const int kr = v / (BN / 8), nc = (v % (BN / 8)) * 8;
#pragma unroll
                for (int j = 0; j < 8; ++j) Bs[(nc + j) * LDS_STRIDE + kr] = r.b[i][j];
            }
        } else if constexpr (MODE == B_NK) {
#pragma unroll
            for (int i = 0; i < B_VECS; ++i) {
                const int v = threadIdx.x + i * TPB;
                const int row = v / (BK / 8), kc = (v % (BK / 8)) * 8;
                *reinterpret_cast<f16x8 *>(Bs + row * LDS_STRIDE + kc) = r.b[i];
            }
        } else if constexpr (MODE == B_Q4N) {
#pragma unroll
            for (int i = 0; i < Q4N_ITEMS; ++i) {
                const int it = threadIdx.x + i * TPB;
                if (it >= Q4N_ITEMS_ALL) continue;
                const int blk = it >> 1, half = it & 1;
                const int kr = blk / (BN / 32), nb = blk % (BN / 32);
                // byte j: low nibble = element j, high nibble = element j + 16
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    Bs[(nb * 32 + half * 16 + j) * LDS_STRIDE + kr] = q4_val(r.qd[i], nib(r.qs[i], j, half * 4));
            }
        } else {
#pragma unroll
            for (int i = 0; i < Q4K_ITEMS; ++i) {
                const int it = threadIdx.x + i * TPB;
                if (it >= Q4K_ITEMS_ALL) continue;
                const int blk = it >> 1, half = it & 1;
                const int nr = blk / (BK / 32), kb = blk % (BK / 32);
                f16x8 lo, hi;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if constexpr (MODE == B_Q8K) {
                        lo[j] = q8_val(r.qd[i], r.qs[i], j);
                        hi[j] = q8_val(r.qd[i], r.qs[i], j + 8);
                    } else {
                        lo[j] = q4_val(r.qd[i], nib(r.qs[i], j, half * 4));
                        hi[j] = q4_val(r.qd[i], nib(r.qs[i], j + 8, half * 4));
                    }
                }
                f16 *dst = Bs + nr * LDS_STRIDE + kb * 32 + half * 16;
                *reinterpret_cast<f16x8 *>(dst) = lo;
                *reinterpret_cast<f16x8 *>(dst + 8) = hi;
            }
        }
    }

    // Must inline into the kernel: as a called function it gets a ~1 KB
    // scratch frame per lane and runs an order of magnitude slower.
    static __device__ __forceinline__ void run(const GemmArgs &p) {
        __shared__ __attribute__((aligned(16))) f16 As[2][BM * LDS_STRIDE];
        __shared__ __attribute__((aligned(16))) f16 Bs[2][BN * LDS_STRIDE];

        const int bz = blockIdx.z / p.splits;
        const int split = blockIdx.z % p.splits;
        const f16 *A = p.A + (long long) bz * p.sA;
        const void *B;
        if constexpr (MODE == B_KN || MODE == B_NK)
            B = reinterpret_cast<const f16 *>(p.B) + (long long) bz * p.sB;
        else
            B = reinterpret_cast<const uint8_t *>(p.B) + (long long) bz * p.sB;
        const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * (BN / 2);
        const int kbeg = split * p.k_per_split;
        const int kend = min(p.K, kbeg + p.k_per_split);

        f32x16 acc[TN][TM];
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int i = 0; i < TM; ++i) acc[j][i] = f32x16{};

        const int KT = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
        Regs r;
        if (KT > 0) {
            load_a(p, A, m0, kbeg, kend, r);
            load_b(p, B, n0, kbeg, kend, r);
            store(As[0], Bs[0], r);
        }
        __syncthreads();

        for (int kt = 0; kt < KT; ++kt) {
            const int cur = kt & 1;
            if (kt + 1 < KT) {
                load_a(p, A, m0, kbeg + (kt + 1) * BK, kend, r);
                load_b(p, B, n0, kbeg + (kt + 1) * BK, kend, r);
            }
            const f16 *as = As[cur];
            const f16 *bs = Bs[cur];
#pragma unroll
            for (int ks = 0; ks < BK; ks += 16) {
                f16x8 wf[TN], xf[TM];
                const int kk = ks + (lane >> 5) * 8;
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    wf[j] = *reinterpret_cast<const f16x8 *>(bs + (wn + j * 32 + (lane & 31)) * LDS_STRIDE + kk);
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    xf[i] = *reinterpret_cast<const f16x8 *>(as + (wm + i * 32 + (lane & 31)) * LDS_STRIDE + kk);
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int i = 0; i < TM; ++i)
                        acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[j], xf[i], acc[j][i], 0, 0, 0);
            }
            if (kt + 1 < KT) store(As[cur ^ 1], Bs[cur ^ 1], r);
            __syncthreads();
        }

        // acc[j][i][e]: n = n0 + wn + j*32 + (e/4)*8 + (lane/32)*4 + e%4, m = m0 + wm + i*32 + lane%32
        if (p.splits > 1) {
            float *ws = p.ws + ((long long) bz * p.splits + split) * (long long) p.M * p.N;
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const int m = m0 + wm + i * 32 + (lane & 31);
                    if (m >= p.M) continue;
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int n = n0 + wn + j * 32 + g * 8 + (lane >> 5) * 4;
                        float *dst = ws + (long long) m * p.N + n;
                        if (n + 3 < p.N && (p.N & 3) == 0) {
                            *reinterpret_cast<f32x4 *>(dst) =
                                f32x4{acc[j][i][g * 4], acc[j][i][g * 4 + 1], acc[j][i][g * 4 + 2], acc[j][i][g * 4 + 3]};
                        } else {
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                if (n + e < p.N) dst[e] = acc[j][i][g * 4 + e];
                        }
                    }
                }
            return;
        }

        f16 *C = p.C + (long long) bz * p.sC;
        const bool vec_store = (p.ldc & 3) == 0 && hx_aligned8(C) &&
                               (!p.R || ((p.ldr & 3) == 0 && hx_aligned8(p.R)));
        dispatch_epi(p.act, p.R != nullptr, [&](auto act_c, auto res_c) {
        constexpr int ACT = decltype(act_c)::value;
        constexpr bool RES = decltype(res_c)::value;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = n0 + wn + j * 32 + g * 8 + (lane >> 5) * 4;
                float bv[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) bv[e] = (p.bias && n + e < p.N) ? p.bias[n + e] : 0.0f;
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const int m = m0 + wm + i * 32 + (lane & 31);
                    if (m >= p.M) continue;
                    f16 *dst = C + (long long) m * p.ldc + n;
                    if (vec_store && n + 3 < p.N) {
                        const f16x4 r4 = RES ? *reinterpret_cast<const f16x4 *>(p.R + m * p.ldr + n) : f16x4{};
                        f16x4 o;
#pragma unroll
                        for (int e = 0; e < 4; ++e) o[e] = epi_t<ACT, RES>(acc[j][i][g * 4 + e] + bv[e], r4[e]);
                        *reinterpret_cast<f16x4 *>(dst) = o;
                    } else {
                        store_tail(dst, p.N - n, p.act, p.R ? p.R + m * p.ldr + n : nullptr,
                                   acc[j][i][g * 4] + bv[0], acc[j][i][g * 4 + 1] + bv[1],
                                   acc[j][i][g * 4 + 2] + bv[2], acc[j][i][g * 4 + 3] + bv[3]);
                    }
                }
            }
        }
        });
    }
};

template <int BM, int BN, int MODE, bool AVEC, bool BVEC>
__global__ __launch_bounds__(TPB) void gemm_kernel(GemmArgs p) {
    Gemm<BM, BN, MODE, AVEC, BVEC>::run(p);
}

// ---- W^T fast path: multi-stage direct-to-LDS pipeline -------------------------
//
// For B_NK with K % 64 == 0 (every encoder GEMM): each K slice of A and B is
// copied HBM -> LDS by global_load_lds_dwordx4 (lane i of a wave writes 16 B at
// the wave's LDS base + 16 i), so a ring of STAGES slices can be in flight
// without holding any of it in registers. LDS rows are 128 B (64 halves),
// unpadded; 16-byte chunk c of row r is stored in slot c ^ ((r >> 1) & 7) --
// the swizzle is applied by choosing which chunk each lane loads, and it makes
// the 16 rows one ds_read_b128 phase touches land in 16 distinct bank groups.
// Rows past M or N are loaded from a clamped (valid) row and never stored.
constexpr int DS_ROW = 64;  // halves per LDS row (128 B)

__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }

template <int ROWS, int NW>
__device__ __forceinline__ void lds_copy_slice(const f16 *__restrict__ base, long long ld, int row0,
                                               int rows_valid, int k0, f16 *lds) {
    // ROWS x 64 halves: ROWS/8 wave-instructions, dealt round-robin to the NW waves.
    static_assert(ROWS % (8 * NW) == 0, "slice rows must split evenly over the waves");
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < ROWS / (8 * NW); ++j) {
        const int rg = j * NW + wave;                // 8-row group
        const int r = rg * 8 + (lane >> 3);          // row within the slice
        const int slot = lane & 7;
        const int c = slot ^ swz(r);
        int gr = row0 + r;
        gr = gr < rows_valid ? gr : rows_valid - 1;  // clamp: never read out of bounds
        const f16 *src = base + (long long) gr * ld + k0 + c * 8;
        // Issued through asm so the compiler does not treat the copy as an
        // LDS store aliasing every later ds_read (it would wait vmcnt(0) and
        // drain the ring); the kernel's explicit vmcnt waits order it instead.
        const uint32_t dst = (uint32_t) (uintptr_t) (__attribute__((address_space(3))) f16 *) (lds + rg * 8 * DS_ROW);
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                     :
                     : "v"(src), "s"(__builtin_amdgcn_readfirstlane(dst))
                     : "memory", "m0");
    }
}

// s_waitcnt encoding (gfx9): vmcnt in [3:0] and [15:14]; expcnt/lgkmcnt left at max.
#define HX_WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4) | (0xF << 8))

// The LayerNorm prologue keeps A's whole row block resident in LDS: K <= 768.
constexpr int LN_KT = 12;

// Normalises the resident A row block in place: each wave takes BM / NW rows,
// with layernorm_fp16's lane mapping (VEC 8, NCH chunks) and arithmetic, and
// writes LN(x) rounded to fp16 back over x. Rows go in groups of RG: all of a
// group's reads, then its RG independent reductions (their shuffle chains
// overlap), then its writes. Rows past M hold a clamped copy of row M - 1 and
// are normalised harmlessly.
template <int BM, int NW, int NCH>
__device__ __forceinline__ void ln_rows_in_lds(f16 (*sA)[BM * DS_ROW], const GemmArgs &p) {
    constexpr int RG = 4;
    static_assert((BM / NW) % RG == 0, "row groups must split the wave's rows");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float g[NCH][8], b[NCH][8];
    bool ok[NCH];
    int off[NCH];   // the chunk's slice and 16-byte column, before the row's swizzle
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
        const int k0 = (ch * 64 + lane) * 8;
        ok[ch] = k0 < p.K;
        off[ch] = ok[ch] ? k0 : 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            g[ch][j] = ok[ch] ? p.ln_w[k0 + j] : 0.0f;
            b[ch][j] = ok[ch] ? p.ln_b[k0 + j] : 0.0f;
        }
    }
    for (int r0 = wave * (BM / NW); r0 < (wave + 1) * (BM / NW); r0 += RG) {
        float v[RG][NCH][8];
        f16 *at[RG][NCH];
#pragma unroll
        for (int q = 0; q < RG; ++q) {
            const int r = r0 + q;
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch) {
                const int c = (off[ch] & 63) >> 3;
                at[q][ch] = sA[off[ch] >> 6] + r * DS_ROW + ((c ^ swz(r)) << 3);
                const f16x8 t = ok[ch] ? *reinterpret_cast<const f16x8 *>(at[q][ch]) : f16x8{};
#pragma unroll
                for (int j = 0; j < 8; ++j) v[q][ch][j] = ok[ch] ? (float) t[j] : 0.0f;
            }
        }
        float mean[RG], inv[RG];
#pragma unroll
        for (int q = 0; q < RG; ++q) ln_row_stats<8, NCH>(v[q], ok, p.K, p.ln_eps, mean[q], inv[q]);
#pragma unroll
        for (int q = 0; q < RG; ++q)
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch) {
                if (!ok[ch]) continue;
                f16x8 t;
#pragma unroll
                for (int j = 0; j < 8; ++j) t[j] = (f16) ln_apply(v[q][ch][j], inv[q], g[ch][j], b[ch][j]);
                *reinterpret_cast<f16x8 *>(at[q][ch]) = t;
            }
    }
}

// lgkmcnt(0) with vmcnt and expcnt left at max: this wave's LDS writes are done.
#define HX_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4))

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef short v8i16 __attribute__((ext_vector_type(8)));

// The weight operand of one 32-column block from a [K][N] weight slice held
// in LDS as it is stored: BN / 64 tiles of [64 k][64 n] (DS_ROW rows, 16-byte
// chunks XOR-swizzled by k row). The MFMA wants, per lane, 8 consecutive k of
// column n = ncol + lane % 32: two ds_read_b64_tr_b16, each giving 4 k. Within
// a 16-lane group lane 4a + b receives element b of the 8 bytes lanes a, a + 4,
// a + 8, a + 12 address, so lane s addresses k row 4u + s / 4 (of the lane's
// 8) at columns 4 (s % 4) .. + 3 of its 16-column group.
__device__ __forceinline__ f16x8 kn_frag(const f16 *bs, int ncol, int q, int lane) {
    const f16 *tile = bs + (ncol >> 6) * (64 * DS_ROW);
    const int nn = (ncol & 63) + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const int k0 = 16 * q + 8 * (lane >> 5) + ((lane & 15) >> 2);
    v4i16 h[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int row = k0 + 4 * u;
        h[u] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16 *) (tile + row * DS_ROW + (((nn >> 3) ^ swz(row)) << 3) + (nn & 7)));
    }
    return __builtin_bit_cast(f16x8, (v8i16){h[0][0], h[0][1], h[0][2], h[0][3], h[1][0], h[1][1], h[1][2], h[1][3]});
}

// The 32-column [K][N] sub-slice of the K-across-waves kernel: 64 k rows of
// 32 halves (64 B), unswizzled. One wave-instruction copies 16 rows (four
// lanes a row, 16 B each, landing contiguously as global_load_lds_dwordx4
// places them); the four waves take 16 rows each. Rows k0 .. k0 + 63 and
// columns n0 .. n0 + 31 must lie inside the weight (K % 256 == 0, N % 32 == 0).
constexpr int KN32_ROW = 32;

__device__ __forceinline__ void lds_copy_kn32(const f16 *__restrict__ base, long long ld, int k0, int n0, f16 *lds) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = wave * 16 + (lane >> 2);
    const f16 *src = base + (long long) (k0 + r) * ld + n0 + (lane & 3) * 8;
    const uint32_t dst = (uint32_t) (uintptr_t) (__attribute__((address_space(3))) f16 *) (lds + wave * 16 * KN32_ROW);
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(src), "s"(__builtin_amdgcn_readfirstlane(dst))
                 : "memory", "m0");
}

// kn_frag's fragment (columns 0 .. 31, k step q) from that 32-column layout.
__device__ __forceinline__ f16x8 kn32_frag(const f16 *bs, int q, int lane) {
    const int nn = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const int k0 = 16 * q + 8 * (lane >> 5) + ((lane & 15) >> 2);
    v4i16 h[2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
        h[u] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4i16 *) (bs + (k0 + 4 * u) * KN32_ROW + nn));
    return __builtin_bit_cast(f16x8, (v8i16){h[0][0], h[0][1], h[0][2], h[0][3], h[1][0], h[1][1], h[1][2], h[1][3]});
}

// WM x WN waves; each owns a (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA tiles.
// LN: A's row block is loaded whole, layer-normalised in LDS, and only B
// streams through the ring (BM = 64, K <= 64 * LN_KT, 512 <= K).
// KN: the weight is [K][N] (matmul_fp16, matmul_epilogue_f16w), copied into
// the ring as stored (N % 64 == 0) and read through kn_frag.
// LNF (the 64x64 pipelined form only, one split): a LayerNorm over A's rows
// folded into the product as gemm_nk_kw's LNF form does it -- bias holds
// [c2 | c1]; the two waves of a wave row read the same A fragments, so wave
// column 0 sums x and column 1 sums x^2 (v_dot2_f32_f16); the sums meet in
// LDS after the loop and the epilogue applies rstd (acc - mean c1).
template <int BM, int BN, int STAGES, int WM = 2, int WN = 2, bool ROPE = false, bool LN = false, bool KN = false,
          bool LNF = false>
__global__ __launch_bounds__(64 * WM * WN) void gemm_nk_lds(GemmArgs p) {
    constexpr int NW = WM * WN;
    constexpr int TM = BM / (32 * WM), TN = BN / (32 * WN);
    // wave-instructions per ring slice per wave
    constexpr int LOADS = (LN ? BN : BM + BN) / (8 * NW);
    static_assert(STAGES >= 2 && LOADS * (STAGES - 2) <= 63, "vmcnt holds at most 63");
    static_assert(!LN || (BM / (8 * NW)) * LN_KT + LOADS * (STAGES - 1) <= 63, "vmcnt holds at most 63");
    // one 32x32 block per wave: the software-pipelined loop (see below)
    constexpr bool PIPE = TM == 1 && TN == 1 && !LN;
    static_assert(!PIPE || LOADS * (STAGES - 1) <= 63, "vmcnt holds at most 63");
    static_assert(!LNF || (PIPE && WN == 2 && !KN), "the folded LayerNorm takes the pipelined 2x2-wave form");
    __shared__ __attribute__((aligned(16))) f16 sA[LN ? LN_KT : STAGES][BM * DS_ROW];
    __shared__ __attribute__((aligned(16))) f16 sB[STAGES][BN * DS_ROW];
    // LNF: sum x (wave column 0) and sum x^2 (column 1) per [tile row][lane / 32]
    __shared__ float2 lnf_sums[LNF ? BM * 2 : 1];
    float lnf_acc = 0.0f;

    const int bz = blockIdx.z / p.splits;
    const int split = blockIdx.z % p.splits;
    const f16 *A = p.A + (long long) bz * p.sA;
    const f16 *B = reinterpret_cast<const f16 *>(p.B) + (long long) bz * p.sB;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave / WN) * (BM / WM), wn = (wave % WN) * (BN / WN);
    const int kbeg = split * p.k_per_split;
    const int kend = min(p.K, kbeg + p.k_per_split);
    const int KT = kend > kbeg ? (kend - kbeg) / BK : 0;   // K range is a multiple of 64

    f32x16 acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[j][i] = f32x16{};

    // The plain epilogue's bias, loaded before the K loop so its latency is
    // hidden (one column block per wave only: more would cost occupancy).
    constexpr bool BIAS_EARLY = TN == 1 && !ROPE;
    float bearly[BIAS_EARLY ? 4 : 1][4];
    float c1early[BIAS_EARLY && LNF ? 4 : 1][4];   // LNF: c1 (bias + N) likewise
    if constexpr (BIAS_EARLY) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int n = n0 + wn + g * 8 + (lane >> 5) * 4;
#pragma unroll
            for (int e = 0; e < 4; ++e) bearly[g][e] = (p.bias && p.splits == 1 && n + e < p.N) ? p.bias[n + e] : 0.0f;
            if constexpr (LNF) {
#pragma unroll
                for (int e = 0; e < 4; ++e) c1early[g][e] = n + e < p.N ? p.bias[p.N + n + e] : 0.0f;
            }
        }
    }

    static_assert(!KN || (BN % 64 == 0 && !ROPE && !LN), "the [K][N] weight comes in 64-column tiles");
    auto issue = [&](int kt, int st) {
        if constexpr (!LN) lds_copy_slice<BM, NW>(A, p.lda, m0, p.M, kbeg + kt * BK, sA[st]);
        if constexpr (KN) {
            // 64 k rows x 64 columns per tile; a tile wholly past N (N % 64 == 0)
            // re-reads the last one, in bounds, for columns never stored
#pragma unroll
            for (int h = 0; h < BN / 64; ++h)
                lds_copy_slice<64, NW>(B, p.ldb, kbeg + kt * BK, p.K, min(n0 + 64 * h, p.N - 64), sB[st] + h * (64 * DS_ROW));
        } else {
            lds_copy_slice<BN, NW>(B, p.ldb, n0, p.N, kbeg + kt * BK, sB[st]);
        }
    };

    if constexpr (LN) {
        // the whole A row block first, then the ring's first B slices; wait for
        // A only, normalise it in place, and publish it before the main loop
        for (int kt = 0; kt < KT; ++kt) lds_copy_slice<BM, NW>(A, p.lda, m0, p.M, kt * BK, sA[kt]);
#pragma unroll
        for (int s = 0; s < STAGES - 1; ++s)
            if (s < KT) issue(s, s);
        if (KT >= STAGES - 1) HX_WAIT_VMCNT(LOADS * (STAGES - 1));
        else HX_WAIT_VMCNT(0);
        __builtin_amdgcn_s_barrier();
        if (p.K > 512) ln_rows_in_lds<BM, NW, 2>(sA, p);
        else ln_rows_in_lds<BM, NW, 1>(sA, p);
        HX_WAIT_LGKM0();
        __builtin_amdgcn_s_barrier();
    } else if constexpr (!PIPE) {
#pragma unroll
        for (int s = 0; s < STAGES - 1; ++s)
            if (s < KT) issue(s, s);
    }

    if constexpr (PIPE) {
        // One 32x32 block per wave: the ring holds one more slice in flight, and
        // slice kt + 1's fragments are read from LDS while slice kt's MFMAs run
        // (two register sets). Slot kt % STAGES is refilled with slice
        // kt + STAGES once every wave has read it (the barrier after its MFMAs
        // were issued: their operands had arrived). Same MFMA order as below.
        struct Frags {
            f16x8 w[BK / 16], x[BK / 16];
        };
        const int rb = wn + (lane & 31), ra = wm + (lane & 31);
        auto read = [&](int kt, Frags &f) {
            const int slot = kt % STAGES;
            const f16 *as = sA[slot], *bs = sB[slot];
#pragma unroll
            for (int q = 0; q < BK / 16; ++q) {
                const int c = 2 * q + (lane >> 5);
                if constexpr (KN) f.w[q] = kn_frag(bs, wn, q, lane);
                else f.w[q] = *reinterpret_cast<const f16x8 *>(bs + rb * DS_ROW + ((c ^ swz(rb)) << 3));
                f.x[q] = *reinterpret_cast<const f16x8 *>(as + ra * DS_ROW + ((c ^ swz(ra)) << 3));
            }
        };
        auto step = [&](int kt, const Frags &cur, Frags &nxt) {
#pragma unroll
            for (int q = 0; q < BK / 16; ++q)
                acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur.w[q], cur.x[q], acc[0][0], 0, 0, 0);
            if constexpr (LNF) {
                const f16x2 one2 = {(f16) 1.0f, (f16) 1.0f};
                const bool sq = __builtin_amdgcn_readfirstlane(wave % WN) != 0;
#pragma unroll
                for (int q = 0; q < BK / 16; ++q)
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const f16x2 pr = {cur.x[q][2 * u], cur.x[q][2 * u + 1]};
                        lnf_acc = __builtin_amdgcn_fdot2(pr, sq ? pr : one2, lnf_acc, false);
                    }
            }
            __builtin_amdgcn_sched_barrier(0);
            if (kt + 1 < KT) {
                // slice kt + 1 is complete for this wave once at most the slices
                // issued after it remain outstanding
                if (kt + STAGES <= KT) HX_WAIT_VMCNT(LOADS * (STAGES - 2));
                else HX_WAIT_VMCNT(0);
                __builtin_amdgcn_s_barrier();
                if (kt + STAGES < KT) issue(kt + STAGES, kt % STAGES);
                read(kt + 1, nxt);
            }
        };
#pragma unroll
        for (int s = 0; s < STAGES; ++s)
            if (s < KT) issue(s, s);
        if (KT >= STAGES) HX_WAIT_VMCNT(LOADS * (STAGES - 1));
        else HX_WAIT_VMCNT(0);
        __builtin_amdgcn_s_barrier();
        Frags f0, f1;
        if (KT > 0) read(0, f0);
        for (int kt = 0; kt < KT; kt += 2) {
            step(kt, f0, f1);
            if (kt + 1 < KT) step(kt + 1, f1, f0);
        }
    } else
    for (int kt0 = 0; kt0 < KT; kt0 += STAGES) {
#pragma unroll
        for (int st = 0; st < STAGES; ++st) {
            const int kt = kt0 + st;
            if (kt >= KT) break;
            // this wave's copies of slice kt are done once at most the later
            // in-flight slices remain outstanding
            if (kt + STAGES - 1 <= KT) HX_WAIT_VMCNT(LOADS * (STAGES - 2));
            else HX_WAIT_VMCNT(0);
            // A bare barrier, not __syncthreads(): its release fence would wait
            // for every in-flight copy (vmcnt 0) and drain the ring. Slice kt's
            // copies are complete per wave (the wait above) and slice kt-1's
            // LDS reads completed before the MFMAs that consumed them.
            __builtin_amdgcn_s_barrier();
            if (kt + STAGES - 1 < KT) issue(kt + STAGES - 1, (st + STAGES - 1) % STAGES);
            const f16 *as = LN ? sA[kt] : sA[st];
            const f16 *bs = sB[st];
            // QB k-steps of 16 at a time: all their LDS reads are issued before
            // the first of their MFMAs (the scheduling barrier keeps them there),
            // so one LDS latency covers QB steps instead of each step waiting on
            // its own reads. The MFMA order is the plain k, j, i order.
            constexpr int QB = TM + TN <= 2 ? 4 : 2;
#pragma unroll
            for (int q0 = 0; q0 < BK / 16; q0 += QB) {
                f16x8 wf[QB][TN], xf[QB][TM];
#pragma unroll
                for (int q = 0; q < QB; ++q) {
                    const int c = 2 * (q0 + q) + (lane >> 5);   // 16-byte chunk of this lane's 8 k
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        const int r = wn + j * 32 + (lane & 31);
                        if constexpr (KN) wf[q][j] = kn_frag(bs, wn + j * 32, q0 + q, lane);
                        else wf[q][j] = *reinterpret_cast<const f16x8 *>(bs + r * DS_ROW + ((c ^ swz(r)) << 3));
                    }
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        const int r = wm + i * 32 + (lane & 31);
                        xf[q][i] = *reinterpret_cast<const f16x8 *>(as + r * DS_ROW + ((c ^ swz(r)) << 3));
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int q = 0; q < QB; ++q)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
#pragma unroll
                        for (int i = 0; i < TM; ++i)
                            acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[q][j], xf[q][i], acc[j][i], 0, 0, 0);
            }
        }
    }

    // epilogue: identical to Gemm::run's
    if (p.splits > 1) {
        float *ws = p.ws + ((long long) bz * p.splits + split) * (long long) p.M * p.N;
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int m = m0 + wm + i * 32 + (lane & 31);
                if (m >= p.M) continue;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int n = n0 + wn + j * 32 + g * 8 + (lane >> 5) * 4;
                    float *dst = ws + (long long) m * p.N + n;
                    if (n + 3 < p.N && (p.N & 3) == 0) {
                        *reinterpret_cast<f32x4 *>(dst) =
                            f32x4{acc[j][i][g * 4], acc[j][i][g * 4 + 1], acc[j][i][g * 4 + 2], acc[j][i][g * 4 + 3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (n + e < p.N) dst[e] = acc[j][i][g * 4 + e];
                    }
                }
            }
        return;
    }
    f16 *C = p.C + (long long) bz * p.sC;
    // LNF: this lane's row (wm + lane % 32) mean and rstd, from the two wave
    // columns' sums of both lane halves, in a fixed order
    float lnf_mean = 0.0f, lnf_inv = 1.0f;
    if constexpr (LNF) {
        const int ra = wm + (lane & 31);
        reinterpret_cast<float *>(lnf_sums)[(ra * 2 + (lane >> 5)) * 2 + wave % WN] = lnf_acc;
        HX_WAIT_LGKM0();
        __builtin_amdgcn_s_barrier();
        const float2 a = lnf_sums[ra * 2], b = lnf_sums[ra * 2 + 1];
        lnf_mean = (a.x + b.x) / (float) p.K;
        const float var = fmaxf((a.y + b.y) / (float) p.K - lnf_mean * lnf_mean, 0.0f);
        lnf_inv = 1.0f / sqrtf(var + p.lnf_eps);
    }
    // the value of accumulator element e of group g (column n + e; f: the bias
    // index, the output feature) after the folded LayerNorm's correction
    auto lnf = [&](float v, int f) {
        if constexpr (LNF) return lnf_inv * (v - lnf_mean * p.bias[p.N + f]);
        else return v;
    };
    // the plain epilogue's: group g, element e of column n + e (c1 prefetched
    // with the bias where it was)
    auto lnf_plain = [&](float v, int g, int e, int n) {
        if constexpr (LNF && BIAS_EARLY) return lnf_inv * (v - lnf_mean * c1early[g][e]);
        else return lnf(v, n + e);
    };
    if constexpr (ROPE) {
        // the rope entry point guarantees N % 4 == 0, rope_d % 4 == 0, ldc == N,
        // an 8-byte aligned C, one batch and no residual: every group
        // of 4 columns is in range as a whole and lies in one head or wholly past
        // the rope heads. The bias and table loads of GB groups are issued before
        // the first of their rotations, so their latencies overlap.
        dispatch_epi(p.act, false, [&](auto act_c, auto) {
        constexpr int ACT = decltype(act_c)::value;
        const int half = p.rope_d >> 1;
        // column groups per load batch: 4 for one row block; 1 for more, which keeps
        // the 128x128 tile under 192 VGPRs and so at 2 waves per SIMD
        constexpr int GB = TM == 1 ? 4 : 1;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
#pragma unroll
            for (int gb = 0; gb < 4; gb += GB) {
                RopeQuad q[GB];
                bool rope[GB];
                float bv[GB][4];
                float2 c0[GB][TM], c1[GB][TM], s0[GB][TM], s1[GB][TM];
#pragma unroll
                for (int h = 0; h < GB; ++h) {
                    const int n = n0 + wn + j * 32 + (gb + h) * 8 + (lane >> 5) * 4;
                    rope[h] = n < p.rope_cols;
                    q[h] = rope[h] ? rope_quad(n, p.rope_d) : RopeQuad{n, n + 1, 0};
                    const int f[4] = {q[h].lo, rope[h] ? q[h].hi : n + 1, q[h].lo + (rope[h] ? 1 : 2),
                                      rope[h] ? q[h].hi + 1 : n + 3};
#pragma unroll
                    for (int e = 0; e < 4; ++e) bv[h][e] = (p.bias && n < p.N) ? p.bias[f[e]] : 0.0f;
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        const int m = min(m0 + wm + i * 32 + (lane & 31), p.M - 1);
                        if (rope[h]) {
                            const long long ld = p.M, o = (long long) q[h].t * ld + m, oh = o + half * ld;
                            c0[h][i] = float2{p.rcos[o], p.rcos[o + ld]};
                            c1[h][i] = float2{p.rcos[oh], p.rcos[oh + ld]};
                            s0[h][i] = float2{p.rsin[o], p.rsin[o + ld]};
                            s1[h][i] = float2{p.rsin[oh], p.rsin[oh + ld]};
                        }
                    }
                }
#pragma unroll
                for (int h = 0; h < GB; ++h) {
                    const int g = gb + h;
                    const int n = n0 + wn + j * 32 + g * 8 + (lane >> 5) * 4;
                    if (n >= p.N) continue;
#pragma unroll
                    for (int i = 0; i < TM; ++i) {
                        const int m = m0 + wm + i * 32 + (lane & 31);
                        if (m >= p.M) continue;
                        f16 *crow = C + (long long) m * p.ldc;
                        const int f[4] = {q[h].lo, rope[h] ? q[h].hi : n + 1, q[h].lo + (rope[h] ? 1 : 2),
                                          rope[h] ? q[h].hi + 1 : n + 3};
                        if (rope[h]) {
                            float v[4];
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                v[e] = f32_rounded(act_t<ACT>(lnf(acc[j][i][g * 4 + e], f[e]) + bv[h][e]));
                            rope_store4(crow, q[h], v, c0[h][i], c1[h][i], s0[h][i], s1[h][i]);
                        } else {
                            f16x4 o;
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                o[e] = epi_t<ACT, false>(lnf(acc[j][i][g * 4 + e], f[e]) + bv[h][e], (f16) 0);
                            *reinterpret_cast<f16x4 *>(crow + n) = o;
                        }
                    }
                }
            }
        }
        });
        return;
    }
    const bool vec_store = (p.ldc & 3) == 0 && hx_aligned8(C) && (!p.R || ((p.ldr & 3) == 0 && hx_aligned8(p.R)));
    dispatch_epi(p.act, p.R != nullptr, [&](auto act_c, auto res_c) {
    constexpr int ACT = decltype(act_c)::value;
    constexpr bool RES = decltype(res_c)::value;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int n = n0 + wn + j * 32 + g * 8 + (lane >> 5) * 4;
            float bv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                bv[e] = BIAS_EARLY ? bearly[BIAS_EARLY ? g : 0][e] : (p.bias && n + e < p.N) ? p.bias[n + e] : 0.0f;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int m = m0 + wm + i * 32 + (lane & 31);
                if (m >= p.M) continue;
                f16 *dst = C + (long long) m * p.ldc + n;
                if (vec_store && n + 3 < p.N) {
                    const f16x4 r4 = RES ? *reinterpret_cast<const f16x4 *>(p.R + m * p.ldr + n) : f16x4{};
                    f16x4 o;
#pragma unroll
                    for (int e = 0; e < 4; ++e) o[e] = epi_t<ACT, RES>(lnf_plain(acc[j][i][g * 4 + e], g, e, n) + bv[e], r4[e]);
                    *reinterpret_cast<f16x4 *>(dst) = o;
                } else {
                    float t[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) t[e] = n + e < p.N ? lnf_plain(acc[j][i][g * 4 + e], g, e, n) + bv[e] : 0.0f;
                    store_tail(dst, p.N - n, p.act, p.R ? p.R + m * p.ldr + n : nullptr, t[0], t[1], t[2], t[3]);
                }
            }
        }
    }
    });
}

// ---- W^T small-M path: K split across the waves, 256-deep stages --------------
//
// For few rows and a long K (fc2 at batch 1: 256x3072x768) the 64x64 tiles
// need split-K and a second, reducing launch to fill the chip. Here a
// 256-thread workgroup owns a T x T output tile (T = 32: 192 workgroups for
// fc2) and walks K in KW_BK = 256-deep stages, each copied HBM->LDS by
// global_load_lds as four 64-wide sub-slices of A and B rows (the swizzled
// [row][64] layout of gemm_nk_lds), into a small ring. Wave w multiplies
// sub-slice w of every stage into its own accumulators for the whole tile, so
// every LDS fragment is read once per workgroup and a K of 768 takes three
// barriers. The four partial tiles are summed through LDS in wave order 0..3
// (fixed, so results are identical run to run) and the epilogue applies
// bias, activation, one rounding and the optional residual. Requires
// K % KW_BK == 0 and 16-byte aligned rows.
constexpr int KW_BK = 256;

// What one lane needs to store its 4 groups of a block with the rope: the
// groups' rope quads, bias values and table entries. Loaded apart from the
// store so a kernel can issue the loads early (gemm_nk_kw issues them before
// its first stage's copies).
struct RopeBlock {
    RopeQuad q[4];
    bool rope[4];
    float bv[4][4];
    float2 c0[4], c1[4], s0[4], s1[4];
};

// The 16 per-column values a lane needs for its 4 groups of 4 accumulator
// columns of the 32-column block at nb (column nb + 8 g + 4 (lane / 32) + e),
// from `src` indexed by output feature: a rope head's pair-interleaved columns
// hold features lo, hi, lo + 1, hi + 1 (rope_quad). A plain block (32
// consecutive features) is read with wave-uniform scalar loads, tracked apart
// from the vector loads of the ring (the folded fc1 at batch 1: 6.97 -> 6.67
// us against per-lane loads); a rope block keeps per-lane loads (scalar
// windows measured slower there).
__device__ __forceinline__ void load_block_cols(const GemmArgs &p, const float *src, int nb, int lane,
                                                float (&out)[16]) {
    typedef const __attribute__((address_space(4))) float cfloat;
    const int nbu = __builtin_amdgcn_readfirstlane(nb);
    const int hi = lane >> 5;
    const bool rope_blk = p.rcos && nbu < p.rope_cols;
    if (!rope_blk && nbu + 32 <= p.N) {
        const cfloat *c = reinterpret_cast<const cfloat *>(reinterpret_cast<uintptr_t>(src + nbu));
        float w[32];
#pragma unroll
        for (int k = 0; k < 32; ++k) w[k] = c[k];
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int e = 0; e < 4; ++e) out[g * 4 + e] = hi ? w[g * 8 + 4 + e] : w[g * 8 + e];
        return;
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int n = nb + g * 8 + hi * 4;
        int f[4] = {n, n + 1, n + 2, n + 3};
        if (p.rcos && n < p.rope_cols) {
            const RopeQuad q = rope_quad(n, p.rope_d);
            f[0] = q.lo;
            f[1] = q.hi;
            f[2] = q.lo + 1;
            f[3] = q.hi + 1;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) out[g * 4 + e] = n + e < p.N ? src[f[e]] : 0.0f;
    }
}

template <int RD>
__device__ __forceinline__ RopeBlock rope_block_load(const GemmArgs &p, int m, int nb, int lane) {
    const int rope_d = RD ? RD : p.rope_d;   // RD: the head width fixed at compile time (0: runtime)
    const int half = rope_d >> 1;
    const int mc = min(m, p.M - 1);
    RopeBlock rb;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int n = nb + g * 8 + (lane >> 5) * 4;
        rb.rope[g] = n < p.rope_cols;
        rb.q[g] = rb.rope[g] ? rope_quad(n, rope_d) : RopeQuad{n, n + 1, 0};
        const int f[4] = {rb.q[g].lo, rb.rope[g] ? rb.q[g].hi : n + 1, rb.q[g].lo + (rb.rope[g] ? 1 : 2),
                          rb.rope[g] ? rb.q[g].hi + 1 : n + 3};
#pragma unroll
        for (int e = 0; e < 4; ++e) rb.bv[g][e] = (p.bias && n < p.N) ? p.bias[f[e]] : 0.0f;
        rb.c0[g] = rb.c1[g] = rb.s0[g] = rb.s1[g] = float2{0.0f, 0.0f};
        if (rb.rope[g]) {
            const long long ld = p.M, o = (long long) rb.q[g].t * ld + mc, oh = o + half * ld;
            rb.c0[g] = float2{p.rcos[o], p.rcos[o + ld]};
            rb.c1[g] = float2{p.rcos[oh], p.rcos[oh + ld]};
            rb.s0[g] = float2{p.rsin[o], p.rsin[o + ld]};
            rb.s1[g] = float2{p.rsin[oh], p.rsin[oh + ld]};
        }
    }
    return rb;
}

template <int ACT>
__device__ __forceinline__ void rope_block_store(const GemmArgs &p, int m, int nb, int lane, const f32x16 &v,
                                                 const RopeBlock &rb) {
    if (m >= p.M) return;
    f16 *crow = p.C + (long long) m * p.ldc;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int n = nb + g * 8 + (lane >> 5) * 4;
        if (n >= p.N) continue;
        if (rb.rope[g]) {
            float x[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = f32_rounded(act_t<ACT>(v[g * 4 + e] + rb.bv[g][e]));
            rope_store4(crow, rb.q[g], x, rb.c0[g], rb.c1[g], rb.s0[g], rb.s1[g]);
        } else {
            f16x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = epi_t<ACT, false>(v[g * 4 + e] + rb.bv[g][e], (f16) 0);
            *reinterpret_cast<f16x4 *>(crow + n) = o;
        }
    }
}

// One 32x32 output block's rope epilogue (the lane holds row m, columns
// nb + 8 g + 4 (lane / 32) .. + 3 in MFMA order): the same arithmetic as
// gemm_nk_lds's rope epilogue, with every bias and table load issued first.
// The encoder's head width (64) gets its own form: the column-to-pair mapping
// then takes shifts and masks instead of integer divisions.
__device__ __forceinline__ RopeBlock load_block_rope(const GemmArgs &p, int m, int nb, int lane) {
    return p.rope_d == 64 ? rope_block_load<64>(p, m, nb, lane) : rope_block_load<0>(p, m, nb, lane);
}


// The rope epilogue of one 32x32 block staged through a wave-private LDS tile
// (rows of 40 halves) and stored as 16-byte row segments, four lanes per row:
// the same values as rope_block_store. A rope block (64-wide heads, N % 8,
// 16-byte aligned rows) holds output features lo0 .. lo0 + 15 and
// lo0 + 32 .. lo0 + 47 (lo0 = hb + (nb - hb) / 2), staged as one 32-half row;
// a plain block its 32 columns.
template <int ACT>
__device__ __forceinline__ void rope_block_store_staged(const GemmArgs &p, int mb, int nb, int lane,
                                                        const f32x16 &v, const RopeBlock &rb, f16 *tile) {
#pragma clang fp contract(off)
    constexpr int TS = 40;
    const int r = lane & 31, hi = lane >> 5;
    const bool rope_blk = nb < p.rope_cols;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        if (rope_blk) {
            float x[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = f32_rounded(act_t<ACT>(v[g * 4 + e] + rb.bv[g][e]));
            f16x2 lo, hv;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const float x0 = (float) (f16) x[2 * u], x1 = (float) (f16) x[2 * u + 1];
                const float ca = u ? rb.c0[g].y : rb.c0[g].x, sa = u ? rb.s0[g].y : rb.s0[g].x;
                const float cb = u ? rb.c1[g].y : rb.c1[g].x, sb = u ? rb.s1[g].y : rb.s1[g].x;
                const float p0 = x0 * ca, q0 = x1 * sa, p1 = x1 * cb, q1 = x0 * sb;
                lo[u] = (f16) f32_rounded(p0 - q0);
                hv[u] = (f16) f32_rounded(p1 + q1);
            }
            *reinterpret_cast<f16x2 *>(tile + r * TS + g * 4 + hi * 2) = lo;
            *reinterpret_cast<f16x2 *>(tile + r * TS + 16 + g * 4 + hi * 2) = hv;
        } else {
            f16x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = epi_t<ACT, false>(v[g * 4 + e] + rb.bv[g][e], (f16) 0);
            *reinterpret_cast<f16x4 *>(tile + r * TS + g * 8 + hi * 4) = o;
        }
    }
    const int hb = nb & ~63, lo0 = hb + ((nb - hb) >> 1);
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int row = it * 16 + (lane >> 2), c = lane & 3;
        const f16x8 val = *reinterpret_cast<const f16x8 *>(tile + row * TS + c * 8);
        const int col = rope_blk ? (c < 2 ? lo0 + c * 8 : lo0 + 32 + (c - 2) * 8) : nb + c * 8;
        if (mb + row < p.M) *reinterpret_cast<f16x8 *>(p.C + (long long) (mb + row) * p.ldc + col) = val;
    }
}

__device__ __forceinline__ void store_block_rope(const GemmArgs &p, int m, int nb, int lane, const f32x16 &v,
                                                 const RopeBlock &rb) {
    if (p.act == 1) rope_block_store<1>(p, m, nb, lane, v, rb);
    else if (p.act == 2) rope_block_store<2>(p, m, nb, lane, v, rb);
    else rope_block_store<0>(p, m, nb, lane, v, rb);
}

// The folded LayerNorm's c1 (bias[N + n]) for the lane's 16 accumulator
// columns of the 32-column block at nb: column nb + 8 g + 4 (lane / 32) + e,
// or, for a rope head's pair-interleaved columns, the output feature that
// column holds (the bias's own index, as rope_block_load takes it).
__device__ __forceinline__ void load_block_c1(const GemmArgs &p, int nb, int lane, float (&c1)[16]) {
    load_block_cols(p, p.bias + p.N, nb, lane, c1);
}

// T x T tile (T = 32: one 32x32 block, 3 stages; T = 64: 2x2 blocks per wave,
// 2 stages -- 128 KB of LDS). With T = 64 wave w stores block w after the
// reduction; with T = 32 wave 0 stores.
// KN: the weight is [K][N]: with T = 64 (N % 64 == 0) each sub-slice is its
// [64 k][64 n] tile as stored, read through kn_frag; with T = 32 (N % 32 == 0)
// its [64 k][32 n] tile, through kn32_frag.
// QB: the weight is block-quantized W^T, [N][K/32] blocks of an fp16 scale
// and 32 codes, 2-byte aligned -- QB = 8: q8_0 (32 int8, 34 bytes), QB = 4:
// q4_0 grouped along K (16 bytes of nibbles, 18 bytes). Each stage's blocks are
// loaded into registers while the previous stage is multiplied, then
// dequantized (fp16(d * q), fp16(d * (q - 8))) into the same LDS layout the
// fp16 copies fill.
// LNF: a LayerNorm over A's rows (all K) folded into the product. With
// W'[n][k] = fp16(ln_w[k] W[n][k]), c1[n] = sum_k W'[n][k] and
// c2[n] = bias[n] + sum_k ln_b[k] W[n][k] (prepared on the host),
//   LN(x) W^T + bias = rstd (x W'^T - mean c1) + c2,
// so the ring multiplies the raw x, and each wave also sums x and x^2 over the
// fragments it reads (v_dot2_f32_f16: two halves per instruction, products
// exact in fp32). The four waves' sums give the row's mean and one-pass
// variance in fp32 after the loop; the epilogue applies
// rstd (acc - mean c1[n]) before the bias (c2) and the activation.
// TN: the tile's output columns -- T, or 24 with T = 32 (plain fp16 W^T only):
// the MFMAs keep their 32 columns, the last 8 multiplying copies of the tile's
// row 23 of W^T (the copy clamps there), and the epilogue stores 24. Where
// 32 x 32 tiles leave CUs idle (N = 768 at 256 rows: 192 tiles) 32 x 24 fills
// a round of 256 with 12.5% fewer bytes per workgroup.
template <int T, bool ROPE = false, bool KN = false, int QB = 0, bool LNF = false, int TN = T>
__global__ __launch_bounds__(TPB) void gemm_nk_kw(GemmArgs p) {
    static_assert(!KN || !ROPE, "no rope epilogue on the [K][N] weight");
    static_assert(QB == 0 || ((QB == 8 || QB == 4) && (!KN || QB == 4) && (!ROPE || (QB == 8 && !KN))),
                  "quantized weights: q8_0 / q4_0 blocks along K of W^T, or q4_0 blocks along N of [K][N]; "
                  "the rope epilogue with q8_0 blocks along K (rows pair-interleaved like the fp16 W^T)");
    static_assert(!LNF || (T == 64 && !KN && QB == 0), "the folded LayerNorm takes the 64x64 W^T form");
    static_assert(TN == T || (T == 32 && TN == 24 && !ROPE && !KN && QB == 0 && !LNF),
                  "the 32 x 24 tile: plain fp16 W^T");
    constexpr int NG = TN == T ? 4 : TN / 8;   // 8-column groups stored per 32-column block
    constexpr bool Q8 = QB != 0;                 // a block-quantized weight (either format)
    constexpr int QBYTES = QB == 8 ? 34 : 18;
    constexpr int NB = T / 32;                 // 32-row blocks per tile side
    constexpr int STAGES = T == 32 ? 3 : 2;
    constexpr int LOADS = 4 * 2 * (T / 32);     // wave-instructions per stage: 4 sub-slices x (A + B) x T/32
    static_assert(LOADS * (STAGES - 1) <= 63, "vmcnt holds at most 63");
    static_assert(STAGES * 4 * 2 * T * DS_ROW * 2 >= 4 * NB * NB * 16 * 64 * 4, "reduction fits in the ring");
    // a [K][N] sub-slice is 64 k rows: of 64 columns (T = 64) or 32 (T = 32)
    constexpr int SB = KN ? 64 * (T == 64 ? DS_ROW : KN32_ROW) : T * DS_ROW;
    __shared__ __attribute__((aligned(16))) f16 sA[STAGES][4][T * DS_ROW];
    __shared__ __attribute__((aligned(16))) f16 sB[STAGES][4][SB];
    const f16 *A = p.A;
    const f16 *B = reinterpret_cast<const f16 *>(p.B);
    const int m0 = blockIdx.y * T, n0 = blockIdx.x * TN;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int KT = p.K / KW_BK;
    const int nrows = TN == T ? p.N : min(p.N, n0 + TN);   // W^T rows copied, the rest clamped to the last

    auto issue = [&](int kt, int st) {
#pragma unroll
        for (int sub = 0; sub < 4; ++sub) {
            lds_copy_slice<T, 4>(A, p.lda, m0, p.M, kt * KW_BK + sub * 64, sA[st][sub]);
            if constexpr (Q8) continue;
            else if constexpr (KN && T == 32) lds_copy_kn32(B, p.ldb, kt * KW_BK + sub * 64, n0, sB[st][sub]);
            else if constexpr (KN) lds_copy_slice<64, 4>(B, p.ldb, kt * KW_BK + sub * 64, p.K, n0, sB[st][sub]);
            else lds_copy_slice<T, 4>(B, p.ldb, n0, nrows, kt * KW_BK + sub * 64, sB[st][sub]);
        }
    };
    // blocks along K of W^T: a stage is T rows x 8 blocks; along N of [K][N]
    // (KN): 256 k x T / 32 blocks. Thread t takes blocks t + 256 u.
    constexpr int NQ = Q8 ? T * 8 / TPB : 1;
    struct Q8Regs {
        float d[NQ];
        uint32_t qs[NQ][8];
    };
    auto q8_load = [&](int kt, Q8Regs &q) {
        const uint8_t *Bq = reinterpret_cast<const uint8_t *>(p.B);
#pragma unroll
        for (int u = 0; u < NQ; ++u) {
            const int b = threadIdx.x + TPB * u, row = b >> 3, kb = b & 7;
            if constexpr (KN && T == 32) {   // block (k, n0 / 32), k = kt * 256 + b
                load_q4_block(Bq + (long long) (kt * KW_BK + b) * p.ldb + (n0 / 32) * 18, q.d[u], q.qs[u]);
                continue;
            }
            if constexpr (KN) {   // block (k, n0 / 32 + (b & 1)), k = kt * 256 + b / 2
                load_q4_block(Bq + (long long) (kt * KW_BK + (b >> 1)) * p.ldb + (n0 / 32 + (b & 1)) * 18, q.d[u],
                              q.qs[u]);
                continue;
            }
            const uint8_t *src = Bq + (long long) min(n0 + row, p.N - 1) * p.ldb + (kt * 8 + kb) * QBYTES;
            if constexpr (QB == 8) {
                load_q8_half(src, 0, q.d[u], q.qs[u]);
                float d1;
                load_q8_half(src, 1, d1, q.qs[u] + 4);
            } else {
                load_q4_block(src, q.d[u], q.qs[u]);
            }
        }
    };
    auto q8_store = [&](int st, const Q8Regs &q) {
#pragma unroll
        for (int u = 0; u < NQ; ++u) {
            const int b = threadIdx.x + TPB * u, row = b >> 3, kb = b & 7;
            if constexpr (KN && T == 32) {
                // the block's 32 values are row k = b of the 32-column sub-slice b / 64
                f16 *drow = sB[st][b >> 6] + (b & 63) * KN32_ROW;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    f16x8 v;
#pragma unroll
                    for (int j = 0; j < 8; ++j) v[j] = q4_val(q.d[u], nib(q.qs[u], (c * 8 + j) & 15, ((c * 8 + j) >> 4) * 4));
                    *reinterpret_cast<f16x8 *>(drow + c * 8) = v;
                }
                continue;
            }
            if constexpr (KN) {
                // the block's 32 values are n = n0 + 32 (b & 1) + j of row k:
                // four 8-column chunks of that k row of the [64 k][64 n] sub-slice
                const int kr = (b >> 1) & 63, nb = b & 1;
                f16 *drow = sB[st][(b >> 1) >> 6] + kr * DS_ROW;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    f16x8 v;
#pragma unroll
                    for (int j = 0; j < 8; ++j) v[j] = q4_val(q.d[u], nib(q.qs[u], (c * 8 + j) & 15, ((c * 8 + j) >> 4) * 4));
                    *reinterpret_cast<f16x8 *>(drow + (((nb * 4 + c) ^ swz(kr)) << 3)) = v;
                }
                continue;
            }
            f16 *dst = sB[st][kb >> 1] + row * DS_ROW;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                f16x8 v;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if constexpr (QB == 8) v[j] = q8_val(q.d[u], q.qs[u] + 4 * (c >> 1), (c & 1) * 8 + j);
                    else v[j] = q4_val(q.d[u], nib(q.qs[u], (c * 8 + j) & 15, ((c * 8 + j) >> 4) * 4));
                }
                *reinterpret_cast<f16x8 *>(dst + ((((kb & 1) * 4 + c) ^ swz(row)) << 3)) = v;
            }
        }
    };
    // the plain epilogue's bias (scalar loads) and residual for this wave's
    // output block, issued now, ahead of the ring's first copies
    BlockBias bbias{};
    BlockRes bres{};
    // the rope epilogue's bias and tables for the block this wave stores (block
    // `wave`), likewise issued before the ring
    RopeBlock rblk{};
    if constexpr (ROPE) {
        if (wave < NB * NB)
            rblk = load_block_rope(p, m0 + (wave / NB) * 32 + (lane & 31), n0 + (wave % NB) * 32, lane);
    }
    // LNF: c1 of the lane's 16 output columns (bias + N, indexed as the bias is)
    float lc1[16] = {};
    if constexpr (LNF) {
        if (wave < NB * NB) load_block_c1(p, n0 + (wave % NB) * 32, lane, lc1);
    }
    if constexpr (!ROPE) {
        bbias = load_block_bias(p, n0 + (wave % NB) * 32);
        if (p.R && wave < NB * NB) {
            const bool vs = (p.ldc & 3) == 0 && hx_aligned8(p.C) && (p.ldr & 3) == 0 && hx_aligned8(p.R);
            bres = load_block_res<NG>(p, m0 + (wave / NB) * 32 + (lane & 31), n0 + (wave % NB) * 32, lane, vs);
        }
    }
    f32x16 acc[NB][NB];   // [column block j][row block i]
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int i = 0; i < NB; ++i) acc[j][i] = f32x16{};
    // With a 2-slot ring both slots are filled before the loop and slot
    // (kt - 1) % 2 is refilled after the barrier of iteration kt (every wave
    // has multiplied stage kt - 1: its MFMAs were issued, so their LDS reads
    // had completed). With 3 slots two stages go out first (a third up front
    // only delays the first) and stage kt + 2 follows the barrier of
    // iteration kt. The two loops are kept apart: merging them into one with
    // an iteration-0 case measured 6% slower for the 3-slot form.
    constexpr bool FULL = STAGES == 2;
#pragma unroll
    for (int s = 0; s < (FULL ? STAGES : STAGES - 1); ++s)
        if (s < KT) issue(s, s);
    const int r = lane & 31;
    // LNF: this lane's sums of x and x^2 over the A fragments it reads (row
    // h * 32 + r, the k chunks of parity lane / 32 of this wave's sub-slices)
    float xs[NB] = {}, xq[NB] = {};
    auto mma_stage = [&](int st) {
        const f16 *as = sA[st][wave], *bs = sB[st][wave];
#pragma unroll
        for (int q = 0; q < BK / 16; ++q) {
            const int c = 2 * q + (lane >> 5);
            f16x8 wf[NB], xf[NB];
#pragma unroll
            for (int h = 0; h < NB; ++h) {
                const int rr = h * 32 + r;
                if constexpr (KN && T == 32) wf[h] = kn32_frag(bs, q, lane);
                else if constexpr (KN) wf[h] = kn_frag(bs, h * 32, q, lane);
                else wf[h] = *reinterpret_cast<const f16x8 *>(bs + rr * DS_ROW + ((c ^ swz(rr)) << 3));
                xf[h] = *reinterpret_cast<const f16x8 *>(as + rr * DS_ROW + ((c ^ swz(rr)) << 3));
            }
#pragma unroll
            for (int j = 0; j < NB; ++j)
#pragma unroll
                for (int i = 0; i < NB; ++i) acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[j], xf[i], acc[j][i], 0, 0, 0);
            if constexpr (LNF) {
                const f16x2 one2 = {(f16) 1.0f, (f16) 1.0f};
#pragma unroll
                for (int h = 0; h < NB; ++h)
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const f16x2 pr = {xf[h][2 * u], xf[h][2 * u + 1]};
                        xs[h] = __builtin_amdgcn_fdot2(pr, one2, xs[h], false);
                        xq[h] = __builtin_amdgcn_fdot2(pr, pr, xq[h], false);
                    }
            }
        }
    };
    if constexpr (Q8) {
        // the prologue above sent stage 0's A (and with 2 slots stage 1's); here
        // stage 0's weight is loaded and dequantized. Each iteration waits for
        // everything (stage kt's A copies, every wave's stage-kt dequantized
        // writes), sends stage kt + 1's A to its slot and loads its q8_0 blocks,
        // multiplies stage kt, then dequantizes stage kt + 1 into its slot --
        // free, since every wave has passed this iteration's barrier after
        // multiplying stage kt + 1 - STAGES.
        Q8Regs qx, qy;
        q8_load(0, qx);
        if (KT <= 3) {
            q8_store(0, qx);
            for (int kt = 0; kt < KT; ++kt) {
                const int st = kt % STAGES;
                HX_WAIT_VMCNT(0);
                HX_WAIT_LGKM0();
                __builtin_amdgcn_s_barrier();
                if (kt + 1 < KT) {
                    if (kt + 1 >= (FULL ? STAGES : STAGES - 1)) issue(kt + 1, (kt + 1) % STAGES);   // else the prologue sent it
                    q8_load(kt + 1, qx);
                }
                mma_stage(st);
                if (kt + 1 < KT) q8_store((kt + 1) % STAGES, qx);
            }
        } else {
            // Longer K: the blocks are loaded a stage earlier than they are
            // dequantized -- stage s in register set s % 2, stage kt + 2's
            // blocks sent in iteration kt ahead of stage kt + 1's A copies --
            // so the wait at the top of iteration kt + 1, needed for those
            // copies anyway, has them in registers before stage kt + 2 is
            // dequantized at its end (256 x 3072 x 768 q8_0: 13.5 us
            // against 14.2; at K = 768 the form above measured faster).
            q8_load(1, qy);
            q8_store(0, qx);
            auto step = [&](int kt, Q8Regs &cur, const Q8Regs &nxt) {   // cur: stage kt (done), nxt: kt + 1
                const int st = kt % STAGES;
                HX_WAIT_VMCNT(0);
                HX_WAIT_LGKM0();
                __builtin_amdgcn_s_barrier();
                if (kt + 2 < KT) q8_load(kt + 2, cur);
                if (kt + 1 < KT && kt + 1 >= (FULL ? STAGES : STAGES - 1))
                    issue(kt + 1, (kt + 1) % STAGES);   // else the prologue sent it
                mma_stage(st);
                if (kt + 1 < KT) q8_store((kt + 1) % STAGES, nxt);
            };
            for (int kt = 0; kt < KT; kt += 2) {
                step(kt, qx, qy);
                if (kt + 1 < KT) step(kt + 1, qy, qx);
            }
        }
    } else {
    for (int kt = 0; kt < KT; ++kt) {
        const int st = kt % STAGES;
        // stage kt's copies are done (this wave) once at most the later ones remain
        if constexpr (FULL) {
            if (kt == 0 && KT >= 2) HX_WAIT_VMCNT(LOADS);
            else HX_WAIT_VMCNT(0);
        } else {
            if (kt + STAGES - 1 <= KT) HX_WAIT_VMCNT(LOADS * (STAGES - 2));
            else HX_WAIT_VMCNT(0);
        }
        __builtin_amdgcn_s_barrier();   // and every wave's; stage kt - 1's reads are done
        if constexpr (FULL) {
            if (kt > 0 && kt + 1 < KT) issue(kt + 1, (kt + 1) % 2);
        } else {
            if (kt + STAGES - 1 < KT) issue(kt + STAGES - 1, (kt + STAGES - 1) % STAGES);
        }
        mma_stage(st);
    }
    }
    // combine the waves' partial tiles: [wave][block][e/4][lane][4] floats over
    // the ring. The q8_0 forms keep each wave's partial of the block it
    // stores (block `wave`) in registers and write only the others: same sum,
    // same order (the batch-1 q8_0 plan 0.690 -> 0.677 ms; the q4_0 plan lost
    // 0.6% and the fp16 plan 0.3% with it, so those forms write all four)
    constexpr bool KEEP_OWN = QB == 8;
    HX_WAIT_VMCNT(0);
    __builtin_amdgcn_s_barrier();
    float *red = reinterpret_cast<float *>(&sA[0][0][0]);
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            if (KEEP_OWN && i * NB + j == wave) continue;
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4)
                *reinterpret_cast<f32x4 *>(red + (((wave * NB * NB + i * NB + j) * 4 + e4) * 64 + lane) * 4) =
                    f32x4{acc[j][i][4 * e4], acc[j][i][4 * e4 + 1], acc[j][i][4 * e4 + 2], acc[j][i][4 * e4 + 3]};
        }
    // LNF: each lane's (sum x, sum x^2) pairs, [wave][row block][lane], in the
    // drained B ring (the partial tiles fill the A ring)
    float2 *lst = reinterpret_cast<float2 *>(&sB[0][0][0]);
    if constexpr (LNF) {
#pragma unroll
        for (int h = 0; h < NB; ++h) lst[(wave * NB + h) * 64 + lane] = float2{xs[h], xq[h]};
    }
    HX_WAIT_LGKM0();
    __builtin_amdgcn_s_barrier();
    if (wave >= NB * NB) return;
    const int blk = wave;                          // block (i, j) = (blk / NB, blk % NB)
    f32x16 own{};
    if constexpr (KEEP_OWN) {
        own = acc[0][0];
        if constexpr (NB == 2) {
            if (blk == 1) own = acc[1][0];
            else if (blk == 2) own = acc[0][1];
            else if (blk == 3) own = acc[1][1];
        }
    }
    // summed in wave order 0..3 from zero, the own partial in its place
    f32x16 sum = f32x16{};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        if (KEEP_OWN && v == blk) {
#pragma unroll
            for (int e = 0; e < 16; ++e) sum[e] += own[e];
            continue;
        }
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
            const f32x4 t = *reinterpret_cast<const f32x4 *>(red + (((v * NB * NB + blk) * 4 + e4) * 64 + lane) * 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) sum[4 * e4 + e] += t[e];
        }
    }
    // lane l holds output row l % 32 of the block, columns 8 g + 4 (l / 32) .. + 3
    const int m = m0 + (blk / NB) * 32 + r;
    if constexpr (LNF) {
        // the row's sums, in a fixed order (wave 0..3, then the two lanes of the row)
        float sx = 0.0f, sq = 0.0f;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float2 a = lst[(v * NB + blk / NB) * 64 + r], b = lst[(v * NB + blk / NB) * 64 + r + 32];
            sx += a.x + b.x;
            sq += a.y + b.y;
        }
        const float mean = sx / (float) p.K;
        const float var = fmaxf(sq / (float) p.K - mean * mean, 0.0f);
        const float inv = 1.0f / sqrtf(var + p.lnf_eps);
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int e = 0; e < 4; ++e) sum[g * 4 + e] = inv * (sum[g * 4 + e] - mean * lc1[g * 4 + e]);
    }
    if constexpr (ROPE) {   // the rope entry point's guarantees: N % 4, rope_d % 4, ldc == N, no residual
        const int nb = n0 + (blk % NB) * 32;
        if (p.rope_d == 64 && p.N % 8 == 0 && nb + 32 <= p.N && (reinterpret_cast<uintptr_t>(p.C) & 15) == 0) {
            f16 *tile = &sB[1][wave][0];
            const int mb = m0 + (blk / NB) * 32;
            if (p.act == 1) rope_block_store_staged<1>(p, mb, nb, lane, sum, rblk, tile);
            else if (p.act == 2) rope_block_store_staged<2>(p, mb, nb, lane, sum, rblk, tile);
            else rope_block_store_staged<0>(p, mb, nb, lane, sum, rblk, tile);
            return;
        }
        store_block_rope(p, m, nb, lane, sum, rblk);
        return;
    }
    f16 *C = p.C;
    const bool vec_store = (p.ldc & 3) == 0 && hx_aligned8(C) && (!p.R || ((p.ldr & 3) == 0 && hx_aligned8(p.R)));
    if constexpr (NB == 2) {
        if (vec_store && (p.ldc & 7) == 0 && (reinterpret_cast<uintptr_t>(C) & 15) == 0 &&
            n0 + (blk % NB) * 32 + 32 <= p.N) {
            kw_store_staged(p, m0 + (blk / NB) * 32, n0 + (blk % NB) * 32, lane, sum, bbias, bres, &sB[1][wave][0]);
            return;
        }
    }
    if (m >= p.M) return;
    kw_store<NG>(p, m, n0 + (blk % NB) * 32, lane, sum, vec_store, bbias, bres);
}

// ---- W^T large-M path: big wave tiles, fragment reads under the MFMAs ----------
//
// For many rows (the encoder at batch 32: M = 8192) the tiled kernel's waves
// are bound by LDS fragment reads and their latency, not by the MFMAs: a wave
// reads TM + TN fragments per 16-deep k step for TM x TN MFMAs and, one wave
// per SIMD, waits for them before it multiplies. Here each of the 4 waves
// (2 x 2) owns a (BM / 2) x (BN / 2) sub-tile -- 128 x 128 in the 256 x 256
// tile -- and step q + 1's fragments are read while step q's MFMAs run: two
// register sets, the reads interleaved one by one between the MFMAs. The K ring
// is gemm_nk_lds's direct-to-LDS ring (64-wide slices, STAGES deep); its one
// barrier per slice sits before the slice's last k step, whose MFMAs then
// cover the next slice's first reads. Workgroups are renumbered so that each
// XCD (the hardware deals workgroup b to XCD b % 8) takes one contiguous run of
// the row-major tile order, so the workgroups sharing an A row block share one
// L2. One batch, no split: K % 64 == 0, 16-byte aligned rows.
constexpr int XCDS = 8;

// Scheduling groups for one k step: an LDS read then an MFMA, NR times, then
// the step's remaining NM - NR MFMAs -- the reads go out early in the step.
template <int G, int NR, int NM>
__device__ __forceinline__ void interleave_reads() {
    static_assert(NM >= NR, "at least one MFMA per read");
    if constexpr (G < NR) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, G < NR - 1 ? 1 : NM - (NR - 1), 0);
        interleave_reads<G + 1, NR, NM>();
    }
}

// The rope forms' head width: the encoder's (rope_d = 64).
constexpr int BIG_RD = 64;

// The rope forms' epilogue (BM = 128, BN = 128 or 192: two or three heads per
// tile). Per pass i (the 64 tile rows of 32-row block i of both wave rows) the
// waves write their fp32 blocks to the staging rows; then each thread takes
// one staged row and BN / 32 8-feature output chunks (the lanes of a wave: 16
// rows x 4 consecutive chunks, so a row's stores are 64 contiguous bytes). A
// rope chunk's 8 output features i .. i + 7 of one half of a head come from
// computed columns 2i .. 2i + 15 (the pair-interleaved weight rows) and table
// columns t = i .. i + 7 (lo half) or i + D/2 .. (hi half), which the thread
// gathers into registers when the K loop is done (big_rope_tables); a chunk past
// the rope heads is stored plainly. The arithmetic is rope_store4's (each value
// rounded to fp16, products and sum rounded separately, rounded again), so the
// result is bit-identical to the other rope epilogues. Host guarantees:
// rope_d == 64, N % 8 == 0, ldc % 8 == 0, 16-byte aligned C, no residual.
// The table values this thread's epilogue uses, gathered after the K loop:
// in pass i it writes row (wave * 16 + lane % 16) of the pass's 64 and the
// 8-feature chunks c = lane / 16 + 4 k, whose features sit at
// f % 64 = 8 (c % 8), that is 8 cq in even k's chunks (the low half of a head,
// table columns 8 cq .. + 7) and 8 cq + 32 in odd k's (the high half, columns
// 8 cq + 32 .. + 7). tt[i][half][cos | sin][u]; a row past M reads 0.
template <int BM, int TM>
__device__ __forceinline__ void big_rope_tables(const GemmArgs &p, int m0, int wave, int lane,
                                                float (&tt)[TM][2][2][8]) {
    const int row = wave * 16 + (lane & 15), cq = lane >> 4;
    const long long ld = p.M;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int m = m0 + (row >> 5) * (BM / 2) + i * 32 + (row & 31);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int tab = 0; tab < 2; ++tab)
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    tt[i][h][tab][u] = m < p.M ? (tab ? p.rsin : p.rcos)[(long long) (8 * cq + 32 * h + u) * ld + m]
                                               : 0.0f;
    }
}

// The folded LayerNorm's statistics of the large-tile kernel, after the K
// loop: sum x (from wave column 0) and sum x^2 (wave column 1) of each lane's
// rows, as float2 [tile row][lane / 32], written in the first epilogue pass
// after its first barrier (the ring is free then) and read after its second.
template <int BM, int TM>
__device__ __forceinline__ void big_lnf_put(float2 *lst, int wave, int lane, const float (&xs)[TM],
                                            const float (&xq)[TM]) {
    constexpr int WN = 2;
    const int wm = (wave / WN) * (BM / 2), r = lane & 31;
    float *dst = reinterpret_cast<float *>(lst);
#pragma unroll
    for (int i = 0; i < TM; ++i) dst[((wm + i * 32 + r) * 2 + (lane >> 5)) * 2 + wave % WN] = wave % WN ? xq[i] : xs[i];
}

// mean and rstd of tile row tr from those pairs: fp32, one-pass variance
// clamped at 0, as the K-across-waves form takes them
__device__ __forceinline__ void big_lnf_row(const GemmArgs &p, const float2 *lst, int tr, float &mean, float &inv) {
    const float2 a = lst[tr * 2], b = lst[tr * 2 + 1];
    mean = (a.x + b.x) / (float) p.K;
    const float var = fmaxf((a.y + b.y) / (float) p.K - mean * mean, 0.0f);
    inv = 1.0f / sqrtf(var + p.lnf_eps);
}

template <int ACT, int BM, int BN, int TM, int TN, int EROW, bool LNF>
__device__ __forceinline__ void big_rope_epilogue(const GemmArgs &p, const f32x16 (&acc)[TN][TM], float *stage,
                                                  int m0, int n0, int wave, int lane, const float (&tt)[TM][2][2][8],
                                                  float bias_own, float c1_own, const float (&xs)[TM],
                                                  const float (&xq)[TM]) {
#pragma clang fp contract(off)
    constexpr int WN = 2, HALF = BIG_RD / 2;
    float *bias_s = stage + 64 * EROW;                     // [BN], by output feature
    float *c1_s = bias_s + BN;                             // LNF: [BN] c1, by output feature
    float2 *lst = reinterpret_cast<float2 *>(c1_s + BN);   // LNF: [BM][2] row sums
    const int tid = threadIdx.x, r = lane & 31;
    // bias by output feature, staged once (visible after the first pass's barrier)
    if (tid < BN) bias_s[tid] = bias_own;
    if constexpr (LNF) {
        if (tid < BN) c1_s[tid] = c1_own;
    }
    const int row = wave * 16 + (lane & 15);               // this thread's staged row
    const int cq = lane >> 4;                              // its chunks: cq, cq + 4, cq + 8, ...
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        // 1. staging writes
        __builtin_amdgcn_s_barrier();              // the ring's (or the last pass's) reads are done
        if constexpr (LNF) {
            if (i == 0) big_lnf_put<BM, TM>(lst, wave, lane, xs, xq);
        }
        const int srow = (wave / WN) * 32 + r;
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<f32x4 *>(stage + srow * EROW + (wave % WN) * (BN / 2) + j * 32 + g * 8 +
                                           (lane >> 5) * 4) =
                    f32x4{acc[j][i][g * 4], acc[j][i][g * 4 + 1], acc[j][i][g * 4 + 2], acc[j][i][g * 4 + 3]};
        HX_WAIT_LGKM0();
        __builtin_amdgcn_s_barrier();
        // 2. one row, four chunks
        const int m = m0 + (row >> 5) * (BM / 2) + i * 32 + (row & 31);
        if (m >= p.M) continue;
        // LNF: the row's mean and rstd; column c's value becomes rstd (v - mean c1[c])
        float lmean = 0.0f, linv = 1.0f;
        if constexpr (LNF) big_lnf_row(p, lst, (row >> 5) * (BM / 2) + i * 32 + (row & 31), lmean, linv);
        auto lnf = [&](float v, int f) {
            if constexpr (LNF) return linv * (v - lmean * c1_s[f]);
            else return v;
        };
        f16 *crow = p.C + (long long) m * p.ldc;
        const float *srow_p = stage + row * EROW;
#pragma unroll
        for (int k = 0; k < BN / 32; ++k) {
            const int c = cq + 4 * k, f0 = c * 8, n = n0 + f0;  // output features n .. n + 7
            if (n >= p.N) continue;
            f16x8 o;
            if (n < p.rope_cols) {
                const int lf = f0 % BIG_RD, hb = f0 - lf;            // feature in head, head start (tile)
                const bool hi = lf >= HALF;
                const int i0 = hi ? lf - HALF : lf;                  // pair index of the first feature
                const float *src = srow_p + hb + 2 * i0;             // computed columns 2 i0 .. 2 i0 + 15
                float v[16];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const f32x4 a4 = *reinterpret_cast<const f32x4 *>(src + 4 * q);
                    v[4 * q] = a4[0]; v[4 * q + 1] = a4[1]; v[4 * q + 2] = a4[2]; v[4 * q + 3] = a4[3];
                }
                // table columns lf .. lf + 7: this thread's gathered half k % 2
                const float(&ct)[8] = tt[i][k & 1][0];
                const float(&st)[8] = tt[i][k & 1][1];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    // computed column 2 (i0 + u) is feature i0 + u, 2 (i0 + u) + 1 is feature i0 + u + D/2
                    const float x0 =
                        (float) (f16) f32_rounded(act_t<ACT>(lnf(v[2 * u], hb + i0 + u) + bias_s[hb + i0 + u]));
                    const float x1 = (float) (f16) f32_rounded(
                        act_t<ACT>(lnf(v[2 * u + 1], hb + i0 + u + HALF) + bias_s[hb + i0 + u + HALF]));
                    const float cv = ct[u], sv = st[u];
                    if (hi) {
                        const float p1 = x1 * cv, q1 = x0 * sv;
                        o[u] = (f16) f32_rounded(p1 + q1);
                    } else {
                        const float p0 = x0 * cv, q0 = x1 * sv;
                        o[u] = (f16) f32_rounded(p0 - q0);
                    }
                }
            } else {
                const f32x4 a0 = *reinterpret_cast<const f32x4 *>(srow_p + f0);
                const f32x4 a1 = *reinterpret_cast<const f32x4 *>(srow_p + f0 + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    o[e] = epi_t<ACT, false>(lnf(a0[e], f0 + e) + bias_s[f0 + e], (f16) 0);
                    o[e + 4] = epi_t<ACT, false>(lnf(a1[e], f0 + 4 + e) + bias_s[f0 + 4 + e], (f16) 0);
                }
            }
            *reinterpret_cast<f16x8 *>(crow + n) = o;
        }
    }
}

// LNF: a LayerNorm over A's rows folded into the product, as gemm_nk_kw's
// LNF form: bias holds [c2 | c1], every wave sums x and x^2 over the A
// fragments its MFMAs use (two halves per v_dot2_f32_f16; the waves of wave
// columns 0 and 1 read the same rows, so column 0 sums x and column 1 x^2),
// and the epilogue applies rstd (acc - mean c1) before the bias.
template <int BM, int BN, int STAGES, bool ROPE = false, bool LNF = false>
__global__ __launch_bounds__(TPB) void gemm_nk_big(GemmArgs p, int gx, int ntiles) {
    constexpr int NW = 4, WN = 2;
    constexpr int TM = BM / 64, TN = BN / 64;     // 32x32 blocks per wave
    constexpr int LOADS = (BM + BN) / (8 * NW);    // wave-instructions per ring slice
    constexpr int NR = TM + TN, NM = TM * TN;      // fragment reads and MFMAs per k step
    static_assert(STAGES >= 2 && LOADS * (STAGES - 1) <= 63, "vmcnt holds at most 63");
    static_assert(!ROPE || (BM == 128 && (BN == 128 || BN == 192)), "the rope forms are 128 x 128 and 128 x 192");
    constexpr int EROW = BN + 4;                   // floats per staged row
    constexpr int RING_BYTES = STAGES * (BM + BN) * DS_ROW * 2;
    constexpr int STAGE_BYTES = 64 * EROW * 4;
    // bias (and c1) staged by output feature: the rope form's bias and LNF c1,
    // the plain form's LNF c1 (one value per thread held through the loop, not
    // eight: the 128 x 192 form's registers stay within two waves per SIMD)
    constexpr int BIAS_BYTES = ROPE ? (LNF ? 2 : 1) * BN * 4 : (LNF ? BN * 4 : 0);
    constexpr int LNF_BYTES = LNF ? BM * 2 * 8 : 0;                  // row sums [BM][2] float2
    constexpr int EPI_BYTES = STAGE_BYTES + BIAS_BYTES + LNF_BYTES;
    constexpr int LDS_BYTES = RING_BYTES > EPI_BYTES ? RING_BYTES : EPI_BYTES;
    // one buffer: the A ring, then the B ring; the epilogue reuses all of it
    __shared__ __attribute__((aligned(16))) f16 lds[LDS_BYTES / 2];
    auto sA = [&](int st) { return lds + st * (BM * DS_ROW); };
    auto sB = [&](int st) { return lds + STAGES * (BM * DS_ROW) + st * (BN * DS_ROW); };

    // XCD-contiguous numbering: a bijection of [0, ntiles) whatever the dealing
    const int b = blockIdx.x, q8 = ntiles / XCDS, r8 = ntiles % XCDS, x = b % XCDS, l = b / XCDS;
    const int t = (x < r8 ? x * (q8 + 1) : r8 * (q8 + 1) + (x - r8) * q8) + l;
    const int m0 = (t / gx) * BM, n0 = (t % gx) * BN;
    const f16 *A = p.A;
    const f16 *B = reinterpret_cast<const f16 *>(p.B);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave / WN) * (BM / 2), wn = (wave % WN) * (BN / 2);
    const int KT = p.K / BK;

    // The epilogue's column chunk and bias (see below), loaded before the K loop.
    constexpr int CPR = BN / 8, RPI = TPB / CPR;  // chunks per row, rows per sweep
    float *stage = reinterpret_cast<float *>(lds);
    const int tid = threadIdx.x, c8 = (tid % CPR) * 8, sr0 = tid / CPR, n = n0 + c8;
    const bool cols = tid < RPI * CPR && n < p.N;
    f32x4 b0 = {}, b1 = {};
    if (!ROPE && p.bias && cols) {
        b0 = *reinterpret_cast<const f32x4 *>(p.bias + n);
        b1 = *reinterpret_cast<const f32x4 *>(p.bias + n + 4);
    }
    // the rope form's bias and the LNF c1 (thread t: column n0 + t), loaded now
    float bias_own = 0.0f, c1_own = 0.0f;
    if constexpr (ROPE) bias_own = (tid < BN && p.bias && n0 + tid < p.N) ? p.bias[n0 + tid] : 0.0f;
    if constexpr (LNF) c1_own = (tid < BN && n0 + tid < p.N) ? p.bias[p.N + n0 + tid] : 0.0f;
    float xs[TM] = {}, xq[TM] = {};   // LNF: this lane's row sums (rows wm + 32 i + lane % 32)
    f32x16 acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[j][i] = f32x16{};

    struct Frags {
        f16x8 w[TN], x[TM];
    };
    auto issue = [&](int kt, int st) {
        lds_copy_slice<BM, NW>(A, p.lda, m0, p.M, kt * BK, sA(st));
        lds_copy_slice<BN, NW>(B, p.ldb, n0, p.N, kt * BK, sB(st));
    };
    // every row this lane reads has the same swizzle: wm, wn and 32 j are multiples of 16
    const int r = lane & 31, sw = swz(r);
    auto read = [&](int st, int q, Frags &f) {
        const int c = (2 * q + (lane >> 5)) ^ sw;
#pragma unroll
        for (int j = 0; j < TN; ++j)
            f.w[j] = *reinterpret_cast<const f16x8 *>(sB(st) + (wn + j * 32 + r) * DS_ROW + (c << 3));
#pragma unroll
        for (int i = 0; i < TM; ++i)
            f.x[i] = *reinterpret_cast<const f16x8 *>(sA(st) + (wm + i * 32 + r) * DS_ROW + (c << 3));
    };
    // one k step's MFMAs (from cur) with a later step's reads (into nxt) dealt between them
    auto step = [&](const Frags &cur, Frags &nxt, int st, int q) {
        read(st, q, nxt);
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int i = 0; i < TM; ++i)
                acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur.w[j], cur.x[i], acc[j][i], 0, 0, 0);
        interleave_reads<0, NR, NM>();
        if constexpr (LNF) {
            // the two waves of a wave row read the same A rows: column 0 sums x,
            // column 1 sums x^2 (a wave-uniform branch), half the VALU each
            const f16x2 one2 = {(f16) 1.0f, (f16) 1.0f};
            if (__builtin_amdgcn_readfirstlane(wave % WN) == 0) {
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const f16x2 pr = {cur.x[i][2 * u], cur.x[i][2 * u + 1]};
                        xs[i] = __builtin_amdgcn_fdot2(pr, one2, xs[i], false);
                    }
            } else {
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const f16x2 pr = {cur.x[i][2 * u], cur.x[i][2 * u + 1]};
                        xq[i] = __builtin_amdgcn_fdot2(pr, pr, xq[i], false);
                    }
            }
        }
    };

#pragma unroll
    for (int s = 0; s < STAGES; ++s)
        if (s < KT) issue(s, s);
    if (KT >= STAGES) HX_WAIT_VMCNT(LOADS * (STAGES - 1));
    else HX_WAIT_VMCNT(0);
    __builtin_amdgcn_s_barrier();
    // Fragments are read two k steps ahead (four register sets): step q's
    // MFMAs run while step q + 2's fragments arrive. The slice's barrier sits
    // after step 1, once this wave's reads of the slot (steps 2 and 3, issued
    // during steps 0 and 1) are done; steps 2 and 3 then read the next slice's
    // steps 0 and 1.
    Frags f0, f1, f2, f3;
    read(0, 0, f0);
    read(0, 1, f1);
    for (int kt = 0; kt < KT; ++kt) {
        const int st = kt % STAGES;
        step(f0, f2, st, 2);
        step(f1, f3, st, 3);
        if (kt + 1 < KT) {
            // this wave's reads of slot st are done, and (after the barrier) every
            // wave's; slice kt + 1 has landed once at most the later slices remain
            HX_WAIT_LGKM0();
            if (kt + STAGES <= KT) HX_WAIT_VMCNT(LOADS * (STAGES - 2));
            else HX_WAIT_VMCNT(0);
            __builtin_amdgcn_s_barrier();
            if (kt + STAGES < KT) issue(kt + STAGES, st);
        }
        // the last slice's reads here fetch a stale slot and are never used: one
        // MFMA path through the loop keeps the accumulators in place
        step(f2, f0, (kt + 1) % STAGES, 0);
        step(f3, f1, (kt + 1) % STAGES, 1);
    }

    // Epilogue through LDS (the ring is free now), one 32-row block of every
    // wave at a time: the waves write their fp32 blocks, then each thread takes
    // a fixed 8-column chunk of every RPI-th staged row -- bias (loaded once),
    // activation, rounding, the optional residual (prefetched one row ahead),
    // one 16-byte store. The rows are padded by 4 floats so the 32 rows of a
    // block's writes fall in distinct banks. The host guarantees N % 8 == 0,
    // ldc % 8 == 0 and 16-byte aligned C, R and bias.
    HX_WAIT_VMCNT(0);
    f16 *C = p.C;
    if constexpr (ROPE) {
        // The tables are gathered here, after the K loop, where the fragment
        // registers are free: held through the loop they raised the 128 x 192
        // form to 302 registers, one workgroup per CU. Their latency runs
        // under the first pass's staging writes.
        float tt[TM][2][2][8];
        big_rope_tables<BM, TM>(p, m0, wave, lane, tt);
        // the activation fixed at compile time: a runtime switch per output
        // would split the unrolled epilogue into a branch per element
        dispatch_epi(p.act, false, [&](auto act_c, auto) {
            big_rope_epilogue<decltype(act_c)::value, BM, BN, TM, TN, EROW, LNF>(p, acc, stage, m0, n0, wave, lane,
                                                                                 tt, bias_own, c1_own, xs, xq);
        });
        return;
    }
    float *c1_s = stage + 64 * EROW;                                  // LNF: [BN] c1
    float2 *lst = reinterpret_cast<float2 *>(c1_s + BN);              // LNF: [BM][2] row sums
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        __builtin_amdgcn_s_barrier();              // the ring's (or the last pass's) reads are done
        if constexpr (LNF) {
            if (i == 0) {
                big_lnf_put<BM, TM>(lst, wave, lane, xs, xq);
                if (tid < BN) c1_s[tid] = c1_own;
            }
        }
        const int srow = (wave / WN) * 32 + r;     // staged row: 32 rows per wave row
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<f32x4 *>(stage + srow * EROW + wn + j * 32 + g * 8 + (lane >> 5) * 4) =
                    f32x4{acc[j][i][g * 4], acc[j][i][g * 4 + 1], acc[j][i][g * 4 + 2], acc[j][i][g * 4 + 3]};
        HX_WAIT_LGKM0();
        __builtin_amdgcn_s_barrier();
        if (!cols) continue;
        // staged rows 0..31 are block i of wave row 0, 32..63 of wave row 1
        auto row_of = [&](int sr) { return m0 + (sr >> 5) * (BM / 2) + i * 32 + (sr & 31); };
        auto resid = [&](int sr) {
            const int m = row_of(sr);
            return p.R && sr < 64 && m < p.M ? *reinterpret_cast<const f16x8 *>(p.R + (long long) m * p.ldr + n)
                                             : f16x8{};
        };
        dispatch_epi(p.act, p.R != nullptr, [&](auto act_c, auto res_c) {
            constexpr int ACT = decltype(act_c)::value;
            constexpr bool RES = decltype(res_c)::value;
            f16x8 rn = RES ? resid(sr0) : f16x8{};
            for (int sr = sr0; sr < 64; sr += RPI) {
                const f16x8 r8 = rn;
                if constexpr (RES) rn = resid(sr + RPI);
                const int m = row_of(sr);
                if (m >= p.M) continue;
                f32x4 v0 = *reinterpret_cast<const f32x4 *>(stage + sr * EROW + c8);
                f32x4 v1 = *reinterpret_cast<const f32x4 *>(stage + sr * EROW + c8 + 4);
                if constexpr (LNF) {
                    float mean, inv;
                    big_lnf_row(p, lst, (sr >> 5) * (BM / 2) + i * 32 + (sr & 31), mean, inv);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v0[e] = inv * (v0[e] - mean * c1_s[c8 + e]);
                        v1[e] = inv * (v1[e] - mean * c1_s[c8 + 4 + e]);
                    }
                }
                f16x8 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    o[e] = epi_t<ACT, RES>(v0[e] + b0[e], r8[e]);
                    o[e + 4] = epi_t<ACT, RES>(v1[e] + b1[e], r8[e + 4]);
                }
                *reinterpret_cast<f16x8 *>(C + (long long) m * p.ldc + n) = o;
            }
        });
    }
}

// ---- W^T small-M path: register operands, K split across the waves -------------
//
// For small M (the encoder at batch 1: M = 256) the tiled kernels leave most
// CUs idle and each wave's single accumulator makes its MFMAs a dependent
// chain. Here a 256-thread workgroup owns a (32 TM) x (32 TN) output tile and
// its 4 waves split K: wave w takes 64-wide K slices w, w + 4, ... Each lane loads
// its MFMA operands straight from global memory (16 bytes = 8 consecutive k of
// one row, exactly the v_mfma_f32_32x32x16_f16 operand), the next slice's
// loads issued before the current slice is multiplied; no LDS staging and no
// barrier in the loop. The waves' fp32 partial tiles are summed through LDS in
// wave order 0..3 (fixed, so results are identical run to run), then bias,
// activation, rounding and the optional residual are applied as in the other
// epilogues. Requires K % 64 == 0 and 16-byte aligned rows.
template <int TM, int TN>
struct SkinnySlice {
    f16x8 a[TM][4];    // activation rows 32 i + l % 32, k = 16 st + 8 (l / 32) .. +8
    f16x8 b[TN][4];    // weight rows 32 j + l % 32
};

template <int TM, int TN>
__global__ __launch_bounds__(TPB) void gemm_nk_skinny(GemmArgs p) {
    constexpr int BM = 32 * TM, BN = 32 * TN;
    __shared__ float part[4][BM][BN + 1];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, hl = lane >> 5, r = lane & 31;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int KT = p.K / BK;
    const f16 *A = p.A;
    const f16 *B = reinterpret_cast<const f16 *>(p.B);
    // rows past M / N are loaded from a clamped (valid) row and never stored
    const f16 *arow[TM];
    const f16 *brow[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) arow[i] = A + (long long) min(m0 + 32 * i + r, p.M - 1) * p.lda + 8 * hl;
#pragma unroll
    for (int j = 0; j < TN; ++j) brow[j] = B + (long long) min(n0 + 32 * j + r, p.N - 1) * p.ldb + 8 * hl;

    auto load = [&](int kt, SkinnySlice<TM, TN> &sl) {
        const int k0 = kt * BK;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
#pragma unroll
            for (int i = 0; i < TM; ++i) sl.a[i][st] = *reinterpret_cast<const f16x8 *>(arow[i] + k0 + 16 * st);
#pragma unroll
            for (int j = 0; j < TN; ++j) sl.b[j][st] = *reinterpret_cast<const f16x8 *>(brow[j] + k0 + 16 * st);
        }
    };

    f32x16 acc[TN][TM];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[j][i] = f32x16{};
    SkinnySlice<TM, TN> cur, nxt;
    int kt = wave;
    if (kt < KT) load(kt, cur);
    for (; kt < KT; kt += 4) {
        if (kt + 4 < KT) load(kt + 4, nxt);
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur.b[j][st], cur.a[i][st], acc[j][i], 0, 0, 0);
        cur = nxt;
    }

    // acc[j][i][e] = partial C[m0 + 32 i + r][n0 + 32 j + (e/4)*8 + 4 hl + e%4]
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                part[wave][32 * i + r][32 * j + (e >> 2) * 8 + 4 * hl + (e & 3)] = acc[j][i][e];
    __syncthreads();

    // BM rows x BN columns, 4 consecutive columns per thread
    const bool vec = (p.ldc & 3) == 0 && hx_aligned8(p.C) && (!p.R || ((p.ldr & 3) == 0 && hx_aligned8(p.R)));
    for (int e = threadIdx.x; e < BM * (BN / 4); e += TPB) {
        const int row = e / (BN / 4), c0 = (e % (BN / 4)) * 4;
        const int m = m0 + row, n = n0 + c0;
        if (m >= p.M || n >= p.N) continue;
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            v[q] = ((part[0][row][c0 + q] + part[1][row][c0 + q]) + part[2][row][c0 + q]) + part[3][row][c0 + q];
        f16 *dst = p.C + (long long) m * p.ldc + n;
        if (vec && n + 3 < p.N) {
            const f16x4 r4 = p.R ? *reinterpret_cast<const f16x4 *>(p.R + (long long) m * p.ldr + n) : f16x4{};
            f16x4 o;
#pragma unroll
            for (int q = 0; q < 4; ++q) o[q] = epi(v[q] + (p.bias ? p.bias[n + q] : 0.0f), p.act, p.R, r4[q]);
            *reinterpret_cast<f16x4 *>(dst) = o;
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (n + q < p.N)
                    dst[q] = epi(v[q] + (p.bias ? p.bias[n + q] : 0.0f), p.act, p.R,
                                 p.R ? p.R[(long long) m * p.ldr + n + q] : (f16) 0);
        }
    }
}

// Sums S fp32 partials in order 0..S-1, adds bias, applies the activation and
// rounds once; 4 consecutive outputs per thread.
__global__ __launch_bounds__(TPB) void splitk_reduce(const float *__restrict__ ws,
                                                     const float *__restrict__ bias,
                                                     f16 *__restrict__ C, long long ldc, long long sC,
                                                     int M, int N, int splits, int act, int batch,
                                                     const f16 *__restrict__ R, long long ldr) {
    const long long per = (long long) M * N;
    const long long quads = (per + 3) / 4;
    const long long total = quads * batch;
    const long long stride = (long long) gridDim.x * TPB;
    for (long long q = (long long) blockIdx.x * TPB + threadIdx.x; q < total; q += stride) {
        const int bz = (int) (q / quads);
        const long long idx = (q % quads) * 4;
        const float *src = ws + (long long) bz * splits * per;
        float s[4] = {0.f, 0.f, 0.f, 0.f};
        if ((N & 3) == 0) {
            // all partial loads are issued before the first add (splits <= MAX_SPLITS)
            f32x4 v[MAX_SPLITS];
#pragma unroll
            for (int sp = 0; sp < MAX_SPLITS; ++sp)
                if (sp < splits) v[sp] = *reinterpret_cast<const f32x4 *>(src + sp * per + idx);
#pragma unroll
            for (int sp = 0; sp < MAX_SPLITS; ++sp)
                if (sp < splits) {
                    s[0] += v[sp][0]; s[1] += v[sp][1]; s[2] += v[sp][2]; s[3] += v[sp][3];
                }
        } else {
            for (int sp = 0; sp < splits; ++sp) {
                const float *p = src + sp * per + idx;
                for (int e = 0; e < 4; ++e)
                    if (idx + e < per) s[e] += p[e];
            }
        }
        for (int e = 0; e < 4; ++e) {
            const long long o = idx + e;
            if (o >= per) break;
            const int m = (int) (o / N), n = (int) (o % N);
            const float b = bias ? bias[n] : 0.0f;
            C[(long long) bz * sC + (long long) m * ldc + n] =
                epi(s[e] + b, act, R, R ? R[(long long) m * ldr + n] : (f16) 0);
        }
    }
}

// splitk_reduce for the rope epilogue (N % 4 == 0, rope_d % 4 == 0, one batch,
// no residual, tables [rope_d, M]): the same fixed-order sum, then each 4-column group of a rope
// head is rotated and stored de-interleaved as the tiled kernel's rope
// epilogue does (rope_store4); groups past the rope heads are stored plainly.
__global__ __launch_bounds__(TPB) void splitk_reduce_rope(const float *__restrict__ ws,
                                                          const float *__restrict__ bias,
                                                          f16 *__restrict__ C, int M, int N, int splits,
                                                          int act, const float *__restrict__ rcos,
                                                          const float *__restrict__ rsin, int rope_cols,
                                                          int rope_d) {
    const long long per = (long long) M * N;
    const long long quads = per / 4;
    const long long stride = (long long) gridDim.x * TPB;
    for (long long q = (long long) blockIdx.x * TPB + threadIdx.x; q < quads; q += stride) {
        const long long idx = q * 4;
        f32x4 v[MAX_SPLITS];
#pragma unroll
        for (int sp = 0; sp < MAX_SPLITS; ++sp)
            if (sp < splits) v[sp] = *reinterpret_cast<const f32x4 *>(ws + sp * per + idx);
        float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int sp = 0; sp < MAX_SPLITS; ++sp)
            if (sp < splits) {
                s[0] += v[sp][0]; s[1] += v[sp][1]; s[2] += v[sp][2]; s[3] += v[sp][3];
            }
        const int m = (int) (idx / N), n = (int) (idx % N);
        f16 *crow = C + (long long) m * N;
        if (n < rope_cols) {
            const RopeQuad r = rope_quad(n, rope_d);
            const int f[4] = {r.lo, r.hi, r.lo + 1, r.hi + 1};
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = f32_rounded(apply_act(s[e] + (bias ? bias[f[e]] : 0.0f), act));
            const long long ld = M, t = (long long) r.t * ld + m, th = t + (rope_d >> 1) * ld;
            rope_store4(crow, r, o, float2{rcos[t], rcos[t + ld]}, float2{rcos[th], rcos[th + ld]},
                        float2{rsin[t], rsin[t + ld]}, float2{rsin[th], rsin[th + ld]});
        } else {
            f16x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = epi(s[e] + (bias ? bias[n + e] : 0.0f), act, false, (f16) 0);
            *reinterpret_cast<f16x4 *>(crow + n) = o;
        }
    }
}

// ---- host side ------------------------------------------------------------------

struct Tile {
    int bm, bn;
};

// Chooses the tile and split count. Cost = (rounds of workgroups over the
// 256 CUs x 2 resident workgroups each -- both tiles' kernels run at 2 waves
// per SIMD) x (tile area / per-tile efficiency) x (K slices per split + a
// per-tile pipeline fill), plus a fixed cost for the reduction launch when K
// is split. Split-K only while the split grid still fits in one round. The
// constants come from a sweep of every tile, split and path over the
// encoder's GEMM shapes on MI355X (within 1% of the best configuration on
// average).
void plan_tiles(long long M, long long N, long long K, int batch, Tile &t, int &splits) {
    struct Cand { Tile t; double eff, fill; };
    static const Cand cands[] = {{{128, 128}, 1.0, 20.0}, {{64, 64}, 0.2, 0.0}};
    constexpr int SLOTS = 256 * 2;
    constexpr double SPLIT_COST = 20000.0;   // the reduction kernel, in the same units
    constexpr int MIN_SPLIT_SLICES = 8;      // shorter K ranges are latency-bound: no gain
    const long long kt = (K + BK - 1) / BK;
    double best = 1e300;
    t = {64, 64};
    splits = 1;
    for (const Cand &c : cands) {
        const long long tiles = ((M + c.t.bm - 1) / c.t.bm) * ((N + c.t.bn - 1) / c.t.bn) * batch;
        for (int s = 1; s <= MAX_SPLITS; s *= 2) {
            if (s > 1 && (kt / s < MIN_SPLIT_SLICES || tiles * s > SLOTS)) break;
            const long long per = (kt + s - 1) / s;
            const long long ss = (kt + per - 1) / per;
            const long long rounds = (tiles * ss + SLOTS - 1) / SLOTS;
            const double area = (double) c.t.bm * c.t.bn;
            const double cost = (double) rounds * area * ((double) per + c.fill) / c.eff +
                                (ss > 1 ? SPLIT_COST : 0.0);
            if (cost < best) {
                best = cost;
                t = c.t;
                splits = (int) ss;
            }
        }
    }
}

template <int BM, int BN, int MODE>
void launch_tile(const GemmArgs &p, int batch, bool avec, bool bvec) {
    dim3 grid((unsigned) ((p.N + BN - 1) / BN), (unsigned) ((p.M + BM - 1) / BM),
              (unsigned) (batch * p.splits));
    if (avec && bvec) HX_LAUNCH((gemm_kernel<BM, BN, MODE, true, true>), grid, dim3(TPB), 0, p);
    else if (avec) HX_LAUNCH((gemm_kernel<BM, BN, MODE, true, false>), grid, dim3(TPB), 0, p);
    else if (bvec) HX_LAUNCH((gemm_kernel<BM, BN, MODE, false, true>), grid, dim3(TPB), 0, p);
    else HX_LAUNCH((gemm_kernel<BM, BN, MODE, false, false>), grid, dim3(TPB), 0, p);
}

// Tuning override (hexlib_gpu_gemm_override): a tile and/or split count that
// replaces the heuristic's choice for every later GEMM in the process.
std::atomic<int> g_ov_bm{0}, g_ov_bn{0}, g_ov_splits{0}, g_ov_path{0};

// The small-M kernel trades data reuse for no LDS staging and no barriers: it
// wins only where the whole GEMM is a few K slices over few columns (a sweep
// of the encoder's shapes on MI355X: 256x768x768 5.7 us vs 7.9 us tiled; wider
// N or longer K are faster tiled).
bool skinny_auto(int M, int N, int K) { return M <= 256 && N <= 1024 && K <= 1024; }

// The K-across-waves kernels, when their one-per-CU workgroups fit one round
// (a sweep on MI355X): 32x32 up to 256 rows (256x3072x768 8.8 us vs 11.8
// split-K; 256x768x768 4.8 vs 5.2 small-M kernel), else 64x64 (256x768x3072
// 7.1 vs 8.2 tiled; 784x3072x768 16.5 vs 18.9). Returns the tile, or 0.
int kw_auto(int M, int N) {
    const long long t32 = (long long) ((M + 31) / 32) * ((N + 31) / 32);
    const long long t64 = (long long) ((M + 63) / 64) * ((N + 63) / 64);
    if (M <= 256 && t32 <= 256) return 32;
    return t64 <= 256 ? 64 : 0;
}

// The [K][N] K-across-waves tile (fp16 or N-blocked q4_0; N % 32 == 0): 64
// (N % 64 == 0) or 32 as kw_auto picks, or forced with path 4 (tile 64x64:
// the 64-column form, else the 32-column one); 0 for neither.
int kw_kn_tile(int path, int M, int N) {
    if (path == 4) return g_ov_bm.load() == 64 ? (N % 64 == 0 ? 64 : 0) : 32;
    if (path != 0) return 0;
    const int t = kw_auto(M, N);
    return t == 64 && N % 64 == 0 ? 64 : t == 32 ? 32 : 0;
}

// Within the 32-row K-across-waves choice: 32 x 24 tiles where 32 x 32 leaves
// CUs of the round idle and 32 x 24 still fits it.
bool kw24_auto(int M, int N) {
    const long long rows = (M + 31) / 32, t32 = rows * ((N + 31) / 32), t24 = rows * ((N + 23) / 24);
    return t32 < 256 && t24 <= 256 && t24 > t32;
}

// The large-tile kernel for tile bm x bn with a ring of `stages` slices;
// false when that form is not built (the rope epilogue exists for the forms
// the automatic choice uses).
bool launch_big(const GemmArgs &p, Tile t, int stages) {
    const int gx = (p.N + t.bn - 1) / t.bn, gy = (p.M + t.bm - 1) / t.bm;
    const long long nt = (long long) gx * gy;
    if (nt > 0x7fffffffLL) return false;
    const dim3 grid((unsigned) nt), block(TPB);
    const int n = (int) nt;
#define HX_BIG(BM_, BN_, S_)                                                              \
    if (t.bm == BM_ && t.bn == BN_ && stages == S_) {                                     \
        if (p.rcos) return false;                                                         \
        HX_LAUNCH((gemm_nk_big<BM_, BN_, S_>), grid, block, 0, p, gx, n);                 \
        return true;                                                                      \
    }
#define HX_BIG_ROPE(BM_, BN_, S_)                                                         \
    if (t.bm == BM_ && t.bn == BN_ && stages == S_) {                                     \
        if (p.rcos) HX_LAUNCH((gemm_nk_big<BM_, BN_, S_, true>), grid, block, 0, p, gx, n); \
        else HX_LAUNCH((gemm_nk_big<BM_, BN_, S_>), grid, block, 0, p, gx, n);            \
        return true;                                                                      \
    }
    HX_BIG(256, 256, 2)
    HX_BIG(256, 192, 2)
    HX_BIG(128, 256, 2)
    HX_BIG(128, 256, 3)
    HX_BIG_ROPE(128, 192, 2)
    HX_BIG(128, 192, 3)
    HX_BIG(256, 128, 2)
    HX_BIG(256, 128, 3)
    HX_BIG_ROPE(128, 128, 2)
    HX_BIG(128, 128, 3)
#undef HX_BIG
#undef HX_BIG_ROPE
    return false;
}

// The large-tile kernel's tile for an M x N product, or {0, 0} for the other
// paths. From a sweep of every form on MI355X at the encoder's batch-32 shapes
// (M = 8192, GELU epilogue, N(0, 1) operands): the 128 x 192 tile with a
// 2-slice ring (80 KB of LDS, two workgroups per CU) is the fastest plain
// linear wherever N % 192 == 0 -- 8192 x 768 x 3072 54.4 us against 56.3 for
// 128 x 128, 8192 x 3072 x 768 46.9 against 49.2, 8192 x 768 x 2304 41.3
// against 46.0. With the residual epilogue it is slower (8192 x 768 x 768 in
// the plan: 22.5 us against 19.7; its 24 chunks per row leave 16 threads of
// each sweep idle), so that form takes 128 x 128. The rope epilogue takes
// 128 x 192 since its table gather moved after the K loop (236 registers, two
// workgroups per CU; gathered before the loop it needed 302, one workgroup per
// CU, and lost to 128 x 128): the q/k/v + rope linear 40.8 us against 45.3,
// the batch-32 plan 2.66 ms against 2.72. Both wherever the grid fills at
// least one round of 256 workgroups; with fewer tiles (784 rows, 2048 x 3072 x
// 1024) the other paths are faster.
Tile big_auto(int M, int N, bool no_residual) {
    const long long t192 = (long long) ((M + 127) / 128) * ((N + 191) / 192);
    if (no_residual && N % 192 == 0 && t192 >= 256) return Tile{128, 192};
    const long long tiles = (long long) ((M + 127) / 128) * ((N + 127) / 128);
    return tiles >= 256 ? Tile{128, 128} : Tile{0, 0};
}

// The rope epilogue on the direct-to-LDS kernel, one split. It is its own
// instantiation, so it costs the plain kernels no registers; there is no
// 256x128 rope form (its 32 unrolled rope stores push the accumulators to
// scratch), that tile runs as 128x128.
void launch_lds_rope(const GemmArgs &p, Tile t) {
    if (t.bm >= 128) t = {128, 128};
    const dim3 grid((unsigned) ((p.N + t.bn - 1) / t.bn), (unsigned) ((p.M + t.bm - 1) / t.bm), 1);
    if (t.bm == 128) HX_LAUNCH((gemm_nk_lds<128, 128, 2, 2, 2, true>), grid, dim3(TPB), 0, p);
    else if (t.bm == 32) HX_LAUNCH((gemm_nk_lds<32, 64, 4, 1, 2, true>), grid, dim3(128), 0, p);
    else if (t.bn == 32) HX_LAUNCH((gemm_nk_lds<64, 32, 4, 2, 1, true>), grid, dim3(128), 0, p);
    else HX_LAUNCH((gemm_nk_lds<64, 64, 4, 2, 2, true>), grid, dim3(TPB), 0, p);
}

// Up to 16 rows on K-grouped quantized weights (QB = 4: q4_0, QB = 8: q8_0):
// v_mfma_f32_16x16x32_f16 tiles, one 32-k block per MFMA. A workgroup owns 16
// output columns and NW waves split K into contiguous runs of blocks. Lane l
// holds the MFMA operands of row / column l % 16 at k = 8 (l / 16) .. + 7: for
// the weight that is 8 codes of one block of row n of W^T -- q4_0: bytes
// 8 (c & 1) .. + 7 of the nibbles, low nibbles for c < 2, high otherwise (block
// element e is byte e & 15's nibble e / 16); q8_0: bytes 8 c .. + 7 -- loaded
// with the block's scale and dequantized to fp16(d * (q - 8)) or fp16(d * q), as
// every other path does. PF blocks per wave are in flight. The waves' 16 x 16
// fp32 partial tiles are summed through LDS in wave order, then bias and
// activation (`epi`). Needs K % 32 == 0 and 16-byte aligned A rows; rows past M
// and columns past N are read from a clamped row and never stored.
// SPLIT: K is split over gridDim.y workgroups as well, each taking
// p.k_per_split of it and storing its fp32 partial tile to p.ws [split][M][N]
// for splitk_reduce (bias, activation) -- where N gives too few workgroups.
template <int QB, int NW, bool SPLIT = false>
__global__ __launch_bounds__(64 * NW) void gemm_q16(GemmArgs p) {
    constexpr int QBYTES = QB == 8 ? 34 : 18, PF = 8;
    __shared__ float red[NW][64][4];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, rr = lane & 15, c = lane >> 4;
    const int n0 = blockIdx.x * 16, n = n0 + rr;
    const int kb_lo = SPLIT ? blockIdx.y * (p.k_per_split / 32) : 0;
    const int KB = SPLIT ? min(p.K / 32, kb_lo + p.k_per_split / 32) : p.K / 32;
    const int per = (KB - kb_lo + NW - 1) / NW, b0 = kb_lo + wave * per, nb = max(0, min(per, KB - b0));
    const uint16_t *wrow = reinterpret_cast<const uint16_t *>(reinterpret_cast<const uint8_t *>(p.B) +
                                                              (long long) min(n, p.N - 1) * p.ldb);
    const f16 *arow = p.A + (long long) min(rr, p.M - 1) * p.lda + 8 * c;
    const float bias = p.bias ? p.bias[min(n, p.N - 1)] : 0.0f;
    // 16-bit word offsets within a block: the scale, then the lane's 8 code bytes
    constexpr int BW = QBYTES / 2;
    const int qw = 1 + (QB == 8 ? 4 * c : 4 * (c & 1));
    struct Blk {
        f16x8 a;
        uint32_t q[2];
        uint16_t d;
    };
    auto load = [&](int b, Blk &x) {
        const uint16_t *w = wrow + (long long) b * BW;
        x.d = w[0];
        x.q[0] = (uint32_t) w[qw] | ((uint32_t) w[qw + 1] << 16);
        x.q[1] = (uint32_t) w[qw + 2] | ((uint32_t) w[qw + 3] << 16);
        x.a = *reinterpret_cast<const f16x8 *>(arow + 32 * b);
    };
    f32x4 acc = {};
    Blk buf[PF];
#pragma unroll
    for (int u = 0; u < PF; ++u)
        if (u < nb) load(b0 + u, buf[u]);
    const int sh = QB == 8 ? 0 : 4 * (c >> 1);
    for (int s0 = 0; s0 < nb; s0 += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const int sidx = s0 + u;
            if (sidx >= nb) break;
            const float d = (float) __builtin_bit_cast(f16, buf[u].d);
            f16x8 wv;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t byte = (buf[u].q[j >> 2] >> (8 * (j & 3))) & 0xFF;
                if constexpr (QB == 8) wv[j] = (f16) (d * (float) (int8_t) byte);
                else wv[j] = q4_val(d, (int) ((byte >> sh) & 0xF));
            }
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(buf[u].a, wv, acc, 0, 0, 0);
            if (sidx + PF < nb) load(b0 + sidx + PF, buf[u]);
        }
    }
    // lane l holds D[4 (l / 16) + i][l % 16] = out[m][n0 + l % 16]
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][lane][i] = acc[i];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += red[w][lane][i];
        const int m = 4 * c + i;
        if (m >= p.M || n >= p.N) continue;
        if constexpr (SPLIT) p.ws[((long long) blockIdx.y * p.M + m) * p.N + n] = v;
        else p.C[(long long) m * p.ldc + n] = epi(v + bias, p.act, p.R, p.R ? p.R[(long long) m * p.ldr + n] : (f16) 0);
    }
}

// Few-row GEMM on K-grouped quantized weights (QB = 4: q4_0, 18-byte blocks;
// QB = 8: q8_0, 34-byte blocks): one wave per output column n. The wave's
// lanes walk the K/32 blocks of row n of W^T (one contiguous run of bytes),
// dequantize each weight as the tiled kernels do, fp16(d * (q - 8)) or
// fp16(d * q), and multiply it by A's rows in fp32 (the fp16 x fp16 product is
// exact in fp32, as in the MFMA); an xor-butterfly sums the lanes. Up to
// GEMV_M rows: there a 32-row MFMA tile is mostly empty and the launch is
// bound by the weight stream. Needs K % 32 == 0, A rows 16-byte aligned.
constexpr int GEMV_M = 4;

template <int QB>
__global__ __launch_bounds__(TPB) void gemv_q(GemmArgs p) {
    constexpr int BLK = QB == 4 ? 18 : 34;
    const int lane = threadIdx.x & (HX_WAVE - 1);
    const int n = blockIdx.x * (TPB / HX_WAVE) + (threadIdx.x >> 6);
    if (n >= p.N) return;
    const uint8_t *W = static_cast<const uint8_t *>(p.B) + (long long) n * p.ldb;
    const int kb_n = p.K / 32;
    float acc[GEMV_M] = {};
    for (int kb = lane; kb < kb_n; kb += HX_WAVE) {
        f16 w[32];
        if constexpr (QB == 4) {
            float d;
            uint32_t qs[4];
            load_q4_block(W + (long long) kb * BLK, d, qs);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                w[j] = q4_val(d, nib(qs, j, 0));
                w[j + 16] = q4_val(d, nib(qs, j, 4));
            }
        } else {
            float d;
            uint32_t q0[4], q1[4];
            load_q8_half(W + (long long) kb * BLK, 0, d, q0);
            load_q8_half(W + (long long) kb * BLK, 1, d, q1);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                w[j] = q8_val(d, q0, j);
                w[j + 16] = q8_val(d, q1, j);
            }
        }
#pragma unroll
        for (int m = 0; m < GEMV_M; ++m) {
            if (m >= p.M) break;
            const f16x8 *a = reinterpret_cast<const f16x8 *>(p.A + (long long) m * p.lda + kb * 32);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const f16x8 x = a[c];
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[m] += (float) w[c * 8 + j] * (float) x[j];
            }
        }
    }
    const float bias = p.bias ? p.bias[n] : 0.0f;
#pragma unroll
    for (int m = 0; m < GEMV_M; ++m) {
        if (m >= p.M) break;
        const float v = wave_sum(acc[m]);
        if (lane == 0) {
            const f16 r = p.R ? p.R[(long long) m * p.ldr + n] : (f16) 0;
            p.C[(long long) m * p.ldc + n] = epi(v + bias, p.act, p.R, r);
        }
    }
}

// The LayerNorm-prologue form: 64x64 tiles, one split (every workgroup reads
// its whole A row block anyway).
void launch_ln(const GemmArgs &p) {
    const dim3 grid((unsigned) ((p.N + 63) / 64), (unsigned) ((p.M + 63) / 64), 1);
    HX_LAUNCH((gemm_nk_lds<64, 64, 4, 2, 2, false, true>), grid, dim3(TPB), 0, p);
}

template <int MODE>
void launch(GemmArgs p, int batch, bool avec, bool bvec) {
    const int path = g_ov_path.load();
    p.splits = 1;
    p.k_per_split = p.K;
    p.ws = nullptr;
    // small M: the register-operand kernel (K split across its waves, no split-K launch)
    const bool skinny_ok = MODE == B_NK && batch == 1 && p.K % BK == 0 && p.lda % 8 == 0 &&
                           p.ldb % 8 == 0 && avec && bvec && (p.M + 31) / 32 <= 65535 && !p.rcos;
    const bool kw_ok = MODE == B_NK && batch == 1 && p.K % KW_BK == 0 && p.lda % 8 == 0 && p.ldb % 8 == 0 &&
                       avec && bvec && (p.M + 31) / 32 <= 65535 && !p.ln_w;
    // the large-tile kernel: its epilogue stores 8-column chunks (and, with the
    // rope, takes 64-wide heads in whole 8-column chunks of rope columns, no
    // residual)
    const bool big_ok = MODE == B_NK && batch == 1 && p.K % BK == 0 && p.lda % 8 == 0 && p.ldb % 8 == 0 &&
                        avec && bvec && !p.ln_w && p.N % 8 == 0 && p.ldc % 8 == 0 &&
                        ((uintptr_t) p.C & 15) == 0 && (!p.bias || ((uintptr_t) p.bias & 15) == 0) &&
                        (!p.R || (p.ldr % 8 == 0 && ((uintptr_t) p.R & 15) == 0)) &&
                        (!p.rcos || (p.rope_d == BIG_RD && p.rope_cols % 8 == 0 && !p.R));
    if (big_ok && (path == 5 || path == 0)) {
        const Tile bt = path == 5 ? Tile{g_ov_bm.load(), g_ov_bn.load()} : big_auto(p.M, p.N, !p.R);
        const int stages = path == 5 && g_ov_splits.load() ? g_ov_splits.load() : 2;
        if (bt.bm && launch_big(p, bt, stages)) return;
    }
    // the [K][N] weight at few rows: the K-across-waves kernel's [K][N] forms
    // with the tile the W^T rule picks -- 64x64 (256 x 768 x 2304: 5.6 us
    // against 7.4 on the tiled ring) or the 32-column tile where it picks 32x32
    // (N % 32 == 0; 256 x 3072 x 768 8.9 us against 12.1 tiled and 13.1 on
    // the 64x64 form, 256 x 768 x 768 4.1 against 5.5 on the 64x64 form)
    const bool kw_kn_ok = MODE == B_KN && batch == 1 && p.K % KW_BK == 0 && p.N % 32 == 0 && p.lda % 8 == 0 &&
                          p.ldb % 8 == 0 && avec && bvec && (p.M + 31) / 32 <= 65535;
    const int kw_kn = kw_kn_ok ? kw_kn_tile(path, p.M, p.N) : 0;
    if (kw_kn == 64) {
        const dim3 grid((unsigned) ((p.N + 63) / 64), (unsigned) ((p.M + 63) / 64));
        HX_LAUNCH((gemm_nk_kw<64, false, true>), grid, dim3(TPB), 0, p);
        return;
    }
    if (kw_kn == 32) {
        HX_LAUNCH((gemm_nk_kw<32, false, true>), dim3((unsigned) (p.N / 32), (unsigned) ((p.M + 31) / 32)), dim3(TPB),
                  0, p);
        return;
    }
    // q8_0 and K-grouped q4_0 weights at few rows: the K-across-waves kernel
    // with the weight dequantized into LDS (path 1 keeps the register-staged
    // kernel). Up to K = 3072 (a sweep on MI355X: 256 x 768 x 2304 q8_0 8.2 us
    // against 12.0, cfg 5's 2048 x 2048 q4_0 at M = 1 10.0 against 12.1); at
    // K = 4864 the register-staged kernel's split-K is faster (13.3 against 19.7).
    // q8_0 and K-grouped q4_0 weights at a few rows: one wave per output column
    // (automatic route only; the forced paths keep their kernels). Measured on
    // MI355X at M = 1, q4_0: 896 x 4864 4.5 us against 13.5, 2048 x 2048 3.5
    // against 10.0; at M = 4 it is still ahead for K >= 896 (896 x 4864 8.5
    // against 13.6) and behind at K = 768 (5.9 against 5.4).
    if constexpr (MODE == B_Q8K || MODE == B_Q4K) {
        // the 16-row MFMA kernel: on the automatic route past gemv_q's rows,
        // where its 16-column workgroups fill a round of CUs (cfg 5's
        // 896 x 4864 at M = 16: 5.7 us against 13.3) and, with K split over
        // workgroups, where they are fewer than 64 (4864 x 896: 10.8 against
        // 13.8); in between (2048 x 2048: 128) the other routes measured as
        // fast or faster
        const int q16_gx = (p.N + 15) / 16;
        const bool q16_auto = p.M > GEMV_M && (q16_gx >= 256 || q16_gx < 64);
        if ((path == 7 || (path == 0 && q16_auto)) && batch == 1 && p.M <= 16 && p.K % 32 == 0 && p.lda % 8 == 0 &&
            avec && !p.rcos && !p.ln_w) {
            constexpr int QBM = MODE == B_Q8K ? 8 : 4;
            const int gx = (p.N + 15) / 16;
            const int nw = path == 7 && g_ov_splits.load() ? g_ov_splits.load() : 8;
            // fewer than a round of workgroups: split K over up to 8 of them,
            // at least 8 blocks per wave-run of each
            int ks = gx >= 256 ? 1 : min(8, (256 + gx - 1) / gx);
            ks = max(1, min(ks, p.K / 32 / 16));
            float *ws = nullptr;
            if (ks > 1) {
                const int kb = (p.K / 32 + ks - 1) / ks;
                p.k_per_split = kb * 32;
                ks = (p.K / 32 + kb - 1) / kb;
                const size_t bytes = (size_t) ks * p.M * p.N * sizeof(float);
                ws = hx::dry_run() ? nullptr : hx::workspace(bytes);
                if (hx::dry_run()) hx::reserve_workspace(bytes);
                if (!ws && hx::FixedWorkspace::refused()) return;
                if (!ws && !hx::dry_run()) ks = 1;
                p.ws = ws;
            }
            if (ks > 1) {
                const dim3 grid((unsigned) gx, (unsigned) ks);
                HX_LAUNCH((gemm_q16<QBM, 8, true>), grid, dim3(512), 0, p);
                HX_LAUNCH(splitk_reduce, dim3(hx::blocks_for(((long long) p.M * p.N + 3) / 4, TPB, 4096)), dim3(TPB),
                          0, (const float *) p.ws, p.bias, p.C, p.ldc, 0LL, p.M, p.N, ks, p.act, 1, p.R, p.ldr);
                return;
            }
            const dim3 grid((unsigned) gx);
            if (nw == 4) HX_LAUNCH((gemm_q16<QBM, 4>), grid, dim3(256), 0, p);
            else if (nw == 16) HX_LAUNCH((gemm_q16<QBM, 16>), grid, dim3(1024), 0, p);
            else HX_LAUNCH((gemm_q16<QBM, 8>), grid, dim3(512), 0, p);
            return;
        }
        if (path == 0 && batch == 1 && (p.M <= 2 || (p.M <= GEMV_M && p.K >= 896)) && p.K % 32 == 0 &&
            p.lda % 8 == 0 && avec && !p.rcos && !p.ln_w) {
            constexpr int WPB = TPB / HX_WAVE;
            HX_LAUNCH((gemv_q<MODE == B_Q8K ? 8 : 4>), dim3((unsigned) ((p.N + WPB - 1) / WPB)), dim3(TPB), 0, p);
            return;
        }
    }
    // q4_0 blocked along N (the reference ABI, [K][N/32] blocks) at few rows: the
    // K-across-waves kernel's [K][N] forms, each stage's blocks dequantized into
    // the ring in the layout its fp16 copies fill, with the fp16 rule's tile:
    // 256 x 3072 x 768 13.9 us on the 32-column tile against 17.3 on the
    // register-staged kernel and 23.7 on the 64x64 form; 256 x 768 x 768 5.6
    // against 8.0 (64x64) and 13.3.
    const bool kw_q4n_ok = MODE == B_Q4N && batch == 1 && p.K % KW_BK == 0 && p.N % 32 == 0 && p.lda % 8 == 0 &&
                           avec && (p.M + 31) / 32 <= 65535 && !p.rcos && !p.ln_w && path != 1;
    const int kw_q4n = kw_q4n_ok ? kw_kn_tile(path, p.M, p.N) : 0;
    if (kw_q4n == 64) {
        HX_LAUNCH((gemm_nk_kw<64, false, true, 4>), dim3((unsigned) (p.N / 64), (unsigned) ((p.M + 63) / 64)),
                  dim3(TPB), 0, p);
        return;
    }
    if (kw_q4n == 32) {
        HX_LAUNCH((gemm_nk_kw<32, false, true, 4>), dim3((unsigned) (p.N / 32), (unsigned) ((p.M + 31) / 32)),
                  dim3(TPB), 0, p);
        return;
    }
    const bool kw_q_ok = (MODE == B_Q8K || MODE == B_Q4K) && batch == 1 && p.K % KW_BK == 0 && p.lda % 8 == 0 &&
                         avec && (p.M + 31) / 32 <= 65535 && !p.rcos && !p.ln_w && path != 1;
    if (kw_q_ok) {
        constexpr int QBM = MODE == B_Q8K ? 8 : 4;
        const int kq = path == 4 ? (g_ov_bm.load() == 64 ? 64 : 32) : (path == 0 && p.K <= 3072 ? kw_auto(p.M, p.N) : 0);
        if (kq == 64) {
            HX_LAUNCH((gemm_nk_kw<64, false, false, QBM>), dim3((unsigned) ((p.N + 63) / 64), (unsigned) ((p.M + 63) / 64)),
                      dim3(TPB), 0, p);
            return;
        }
        if (kq == 32) {
            HX_LAUNCH((gemm_nk_kw<32, false, false, QBM>), dim3((unsigned) ((p.N + 31) / 32), (unsigned) ((p.M + 31) / 32)),
                      dim3(TPB), 0, p);
            return;
        }
    }
    int kw = 0;
    if (kw_ok && path == 4) kw = g_ov_bm.load() == 64 ? 64 : 32;
    else if (kw_ok && path == 0) kw = kw_auto(p.M, p.N);
    if (kw && p.rcos) kw = 64;   // the rope epilogue exists in the 64x64 form
    if (kw == 64) {
        const dim3 grid((unsigned) ((p.N + 63) / 64), (unsigned) ((p.M + 63) / 64));
        if (p.rcos) HX_LAUNCH((gemm_nk_kw<64, true>), grid, dim3(TPB), 0, p);
        else HX_LAUNCH((gemm_nk_kw<64>), grid, dim3(TPB), 0, p);
        return;
    }
    if (kw == 32) {
        const bool t24 = path == 4 ? g_ov_bn.load() == 24 : kw24_auto(p.M, p.N);
        if (t24) {
            HX_LAUNCH((gemm_nk_kw<32, false, false, 0, false, 24>),
                      dim3((unsigned) ((p.N + 23) / 24), (unsigned) ((p.M + 31) / 32)), dim3(TPB), 0, p);
            return;
        }
        const dim3 grid((unsigned) ((p.N + 31) / 32), (unsigned) ((p.M + 31) / 32));
        HX_LAUNCH((gemm_nk_kw<32>), grid, dim3(TPB), 0, p);
        return;
    }
    if (skinny_ok && (path == 3 || (path == 0 && skinny_auto(p.M, p.N, p.K)))) {
        int bm = g_ov_bm.load(), bn = g_ov_bn.load();
        if (path != 3 || bm == 0) bm = bn = 32;
        const dim3 grid((unsigned) ((p.N + bn - 1) / bn), (unsigned) ((p.M + bm - 1) / bm));
        if (bm == 32 && bn == 32) HX_LAUNCH((gemm_nk_skinny<1, 1>), grid, dim3(TPB), 0, p);
        else if (bm == 32) HX_LAUNCH((gemm_nk_skinny<1, 2>), grid, dim3(TPB), 0, p);
        else if (bn == 32) HX_LAUNCH((gemm_nk_skinny<2, 1>), grid, dim3(TPB), 0, p);
        else HX_LAUNCH((gemm_nk_skinny<2, 2>), grid, dim3(TPB), 0, p);
        return;
    }
    Tile t;
    int splits;
    plan_tiles(p.M, p.N, p.K, batch, t, splits);
    // path 5's tile and ring depth belong to the large-tile kernel: a shape it
    // cannot take runs with the heuristic's choice
    if (const int bm = g_ov_bm.load(); bm && path != 5) t = {bm, g_ov_bn.load()};
    if (t.bm == 32 && t.bn == 32) t = {64, 64};   // the skinny-only tile, on a shape it cannot take
    if (const int s = g_ov_splits.load(); s && path != 5) splits = s;
    if (splits > 1) {
        const int kt = (p.K + BK - 1) / BK;
        const int per = (kt + splits - 1) / splits;
        splits = (kt + per - 1) / per;
        const size_t bytes = (size_t) batch * splits * (size_t) p.M * p.N * sizeof(float);
        float *ws = hx::dry_run() ? nullptr : hx::workspace(bytes);
        if (hx::dry_run()) hx::reserve_workspace(bytes);
        // a caller-fixed workspace too small for this split: launch nothing
        if (!ws && hx::FixedWorkspace::refused()) return;
        if (ws || hx::dry_run()) {
            p.splits = splits;
            p.k_per_split = per * BK;
            p.ws = ws;
        }
    }
    bool lds_direct = MODE == B_NK && p.K % BK == 0 && p.lda % 8 == 0 && p.ldb % 8 == 0 &&
                      avec && bvec && p.k_per_split % BK == 0;
    // the [K][N] weight through the same ring (64-column tiles, transpose
    // reads), except a one-slice K over more than a round of workgroups,
    // where the register-staged kernel measured faster (384 x 256x64x256:
    // 33 us against 48)
    const long long kn_wgs = (long long) ((p.M + t.bm - 1) / t.bm) * ((p.N + t.bn - 1) / t.bn) * batch * p.splits;
    const bool kn_direct = MODE == B_KN && p.K % BK == 0 && p.N % 64 == 0 && p.lda % 8 == 0 && p.ldb % 8 == 0 &&
                           avec && bvec && p.k_per_split % BK == 0 && path != 1 && (p.K > BK || kn_wgs <= 512);
    if (path == 1 && !p.rcos) lds_direct = false;   // the rope epilogue exists on this kernel only
    if (p.rcos && !lds_direct) return;                 // unreachable: the rope entry point checks its preconditions
    if (lds_direct && p.rcos && p.splits == 1) {
        launch_lds_rope(p, t);
    } else if (kn_direct) {
        if (t.bn < 64) t = {64, 64};   // no 32-column [K][N] form
        dim3 grid((unsigned) ((p.N + t.bn - 1) / t.bn), (unsigned) ((p.M + t.bm - 1) / t.bm),
                  (unsigned) (batch * p.splits));
        if (t.bm == 256) HX_LAUNCH((gemm_nk_lds<256, 128, 3, 2, 2, false, false, true>), grid, dim3(TPB), 0, p);
        else if (t.bm == 128) HX_LAUNCH((gemm_nk_lds<128, 128, 2, 2, 2, false, false, true>), grid, dim3(TPB), 0, p);
        else if (t.bm == 32) HX_LAUNCH((gemm_nk_lds<32, 64, 4, 1, 2, false, false, true>), grid, dim3(128), 0, p);
        else HX_LAUNCH((gemm_nk_lds<64, 64, 4, 2, 2, false, false, true>), grid, dim3(TPB), 0, p);
    } else if (lds_direct) {
        dim3 grid((unsigned) ((p.N + t.bn - 1) / t.bn), (unsigned) ((p.M + t.bm - 1) / t.bm),
                  (unsigned) (batch * p.splits));
        if (t.bm == 256) HX_LAUNCH((gemm_nk_lds<256, 128, 3>), grid, dim3(TPB), 0, p);
        else if (t.bm == 128) HX_LAUNCH((gemm_nk_lds<128, 128, 2>), grid, dim3(TPB), 0, p);
        else if (t.bm == 32) HX_LAUNCH((gemm_nk_lds<32, 64, 4, 1, 2>), grid, dim3(128), 0, p);
        else if (t.bn == 32) HX_LAUNCH((gemm_nk_lds<64, 32, 4, 2, 1>), grid, dim3(128), 0, p);
        else HX_LAUNCH((gemm_nk_lds<64, 64, 4>), grid, dim3(TPB), 0, p);
    } else if (t.bm < 64 || t.bn < 64) launch_tile<64, 64, MODE>(p, batch, avec, bvec);
    else if (t.bm == 256) launch_tile<256, 128, MODE>(p, batch, avec, bvec);
    else if (t.bm == 128) launch_tile<128, 128, MODE>(p, batch, avec, bvec);
    else launch_tile<64, 64, MODE>(p, batch, avec, bvec);
    if (p.splits > 1 && p.rcos) {
        HX_LAUNCH(splitk_reduce_rope, dim3(hx::blocks_for((long long) p.M * p.N / 4, TPB, 4096)), dim3(TPB), 0,
                  (const float *) p.ws, p.bias, p.C, p.M, p.N, p.splits, p.act, p.rcos, p.rsin, p.rope_cols,
                  p.rope_d);
    } else if (p.splits > 1) {
        const long long quads = ((long long) p.M * p.N + 3) / 4 * batch;
        HX_LAUNCH(splitk_reduce, dim3(hx::blocks_for(quads, TPB, 4096)), dim3(TPB), 0,
                  (const float *) p.ws, p.bias, p.C, p.ldc, p.sC, p.M, p.N, p.splits, p.act, batch, p.R, p.ldr);
    }
}


bool dims_ok(int M, int K, int N, int batch) {
    return M > 0 && K > 0 && N > 0 && batch > 0 && batch <= 65535 && (M + 63) / 64 <= 65535;
}

GemmArgs args(const hexlib_hf *a, long long lda, long long sA, const void *b, long long ldb,
              long long sB, const float *bias, hexlib_hf *c, long long ldc, long long sC, int M,
              int N, int K, int act) {
    GemmArgs p{};
    p.A = reinterpret_cast<const f16 *>(a);
    p.lda = lda;
    p.sA = sA;
    p.B = b;
    p.ldb = ldb;
    p.sB = sB;
    p.bias = bias;
    p.C = reinterpret_cast<f16 *>(c);
    p.ldc = ldc;
    p.sC = sC;
    p.M = M;
    p.N = N;
    p.K = K;
    p.act = act;
    return p;
}

}  // namespace

extern "C" int hexlib_gpu_gemm_override(int bm, int bn, int splits, int path) {
    const bool tile_ok = path == 5 ? (bm == 128 || bm == 256) && (bn == 128 || bn == 192 || bn == 256)
                                   : (bm == 0 && bn == 0) || (bm == 256 && bn == 128) ||
                                         (bm == 128 && bn == 128) || (bm == 64 && bn == 64) ||
                                         (bm == 32 && bn == 64) || (bm == 64 && bn == 32) ||
                                         (path == 3 && bm == 32 && bn == 32) || (path == 4 && bm == 32 && bn == 24);
    if (!tile_ok || splits < 0 || splits > MAX_SPLITS || path < 0 || path > 7 || path == 6 ||
        (path == 7 && (bm || bn || (splits && splits != 4 && splits != 8 && splits != 16))) ||
        (path == 5 && splits > 3))
        return HEXLIB_DSP_ERR_INVAL_PARAMS;
    g_ov_bm = bm;
    g_ov_bn = bn;
    g_ov_splits = splits;
    g_ov_path = path;
    return HEXLIB_DSP_OK;
}

extern "C" void matmul_fp16(const hexlib_hf *A, const hexlib_hf *B, hexlib_hf *C, int Bn, int M,
                            int K, int N) {
    if (!A || !B || !C || !dims_ok(M, K, N, Bn)) return;
    launch<B_KN>(args(A, K, (long long) M * K, B, N, (long long) K * N, nullptr, C, N,
                      (long long) M * N, M, N, K, 0),
                 Bn, K % 8 == 0 && hx::aligned(A, 16), N % 8 == 0 && hx::aligned(B, 16));
}

extern "C" void matmul_epilogue_f16w_fp16(const hexlib_hf *a, const hexlib_hf *w, const float *bias,
                                          hexlib_hf *out, int M, int K, int N, int act) {
    if (!a || !w || !out || !dims_ok(M, K, N, 1) || act < 0 || act > 2) return;
    launch<B_KN>(args(a, K, 0, w, N, 0, bias, out, N, 0, M, N, K, act), 1,
                 K % 8 == 0 && hx::aligned(a, 16), N % 8 == 0 && hx::aligned(w, 16));
}

extern "C" void matmul_epilogue_f16wt_fp16(const hexlib_hf *a, const hexlib_hf *wt, const float *bias,
                                           hexlib_hf *out, int M, int K, int N, int act) {
    if (!a || !wt || !out || !dims_ok(M, K, N, 1) || act < 0 || act > 2) return;
    launch<B_NK>(args(a, K, 0, wt, K, 0, bias, out, N, 0, M, N, K, act), 1,
                 K % 8 == 0 && hx::aligned(a, 16), K % 8 == 0 && hx::aligned(wt, 16));
}

// ---- the no-allocation form of matmul_epilogue_f16wt_fp16 ----------------------
// For callers that cannot allocate (code under graph capture, tight serving
// loops): the split-K partials live in this file-scope device array -- one
// copy per GPU, held until the process ends -- instead of the library's
// grow-only workspace. Host code never uses the array's name as an address:
// each device's address comes from hipGetSymbolAddress on that device's first
// call. Every call on one GPU shares that GPU's array; calls that overlap in
// time on one GPU (different streams, or two graphs replaying at once) race on
// it. The partials are written in full before they are read, so nothing needs
// clearing between calls.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t) 16 << 20;
static __device__ __align__(256) float scratch[NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace {
std::mutex g_scratch_mu;
float *g_scratch_ptr[16] = {};

// This device's address of `scratch`, looked up once per device (with that
// device current); nullptr (and the HIP error noted) if the lookup fails.
float *noalloc_scratch() {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= 16) return nullptr;
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch_ptr[d]) {
        void *ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            hx::note(e != hipSuccess ? e : hipErrorInvalidSymbol);
            return nullptr;
        }
        g_scratch_ptr[d] = static_cast<float *>(ptr);
    }
    return g_scratch_ptr[d];
}
}  // namespace

extern "C" int matmul_epilogue_f16wt_noalloc_fp16(const hexlib_hf *a, const hexlib_hf *wt, const float *bias,
                                                  hexlib_hf *out, int M, int K, int N, int act) {
    if (!a || !wt || !out || !dims_ok(M, K, N, 1) || act < 0 || act > 2) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    float *ws = noalloc_scratch();
    if (!ws) return HEXLIB_DSP_ERR_INTERNAL;
    bool refused;
    {
        hx::FixedWorkspace fixed(ws, NOALLOC_SCRATCH_BYTES);
        launch<B_NK>(args(a, K, 0, wt, K, 0, bias, out, N, 0, M, N, K, act), 1,
                     K % 8 == 0 && hx::aligned(a, 16), K % 8 == 0 && hx::aligned(wt, 16));
        refused = hx::FixedWorkspace::refused();
    }
    return refused ? HEXLIB_DSP_ERR_VTCM_TOO_SMALL : HEXLIB_DSP_OK;
}

extern "C" void matmul_epilogue_f16wt_res_fp16(const hexlib_hf *a, const hexlib_hf *wt, const float *bias,
                                               const hexlib_hf *resid, hexlib_hf *out, int M, int K, int N,
                                               int act) {
    if (!a || !wt || !resid || !out || !dims_ok(M, K, N, 1) || act < 0 || act > 2) return;
    GemmArgs p = args(a, K, 0, wt, K, 0, bias, out, N, 0, M, N, K, act);
    p.R = reinterpret_cast<const f16 *>(resid);
    p.ldr = N;
    launch<B_NK>(p, 1, K % 8 == 0 && hx::aligned(a, 16), K % 8 == 0 && hx::aligned(wt, 16));
}

extern "C" void matmul_epilogue_f16wt_rope_fp16(const hexlib_hf *a, const hexlib_hf *wt, const float *bias,
                                                const float *costab, const float *sintab, hexlib_hf *out,
                                                int M, int K, int N, int act, int rope_heads, int rope_dim) {
    if (!a || !wt || !out || !costab || !sintab || !dims_ok(M, K, N, 1) || act < 0 || act > 2) return;
    const long long rope_cols = 2LL * rope_heads * rope_dim;
    // the direct-to-LDS kernel's preconditions (its epilogue implements the rope)
    if (rope_heads <= 0 || rope_dim <= 0 || rope_dim % 4 || rope_cols > N || N % 4 || K % BK || K % 8 ||
        !hx::aligned(a, 16) || !hx::aligned(wt, 16) || !hx::aligned(out, 8))
        return;
    GemmArgs p = args(a, K, 0, wt, K, 0, bias, out, N, 0, M, N, K, act);
    p.rcos = costab;
    p.rsin = sintab;
    p.rope_cols = (int) rope_cols;
    p.rope_d = rope_dim;
    launch<B_NK>(p, 1, true, true);
}

// A LayerNorm folded into the W^T linear that consumes it (one launch, no
// normalised activation stored): x is the LayerNorm's input, wt the
// weight-scaled W'^T and bias2 = [c2 | c1] (2N floats), see gemm_nk_kw's LNF.
// Preconditions of the K-across-waves form: K % 256 == 0, 16-byte aligned x
// and wt; the rope form adds the rope entry point's.
static bool lnf_ok(const hexlib_hf *x, const hexlib_hf *wt, const float *bias2, const hexlib_hf *out, int M, int K,
            int N, int act) {
    return x && wt && bias2 && out && dims_ok(M, K, N, 1) && act >= 0 && act <= 2 && K % KW_BK == 0 &&
           hx::aligned(x, 16) && hx::aligned(wt, 16);
}

// Many rows (the large-tile kernel's tile fills a round of CUs): its LNF form,
// on the 128 x 192 or 128 x 128 tile big_auto picks, where its epilogue's
// preconditions hold (N % 8 == 0, 16-byte aligned output and bias2; the rope
// form 64-wide heads). Returns false to leave the launch to the K-across-waves
// form.
static bool launch_big_lnf(const GemmArgs &p) {
    const Tile t = big_auto(p.M, p.N, true);
    if (!t.bm || p.N % 8 || p.ldc % 8 || !hx::aligned(p.C, 16) || !hx::aligned(p.bias, 16)) return false;
    if (p.rcos && (p.rope_d != BIG_RD || p.rope_cols % 8)) return false;
    const int gx = (p.N + t.bn - 1) / t.bn, gy = (p.M + t.bm - 1) / t.bm;
    const long long nt = (long long) gx * gy;
    if (nt > 0x7fffffffLL) return false;
    const dim3 grid((unsigned) nt), block(TPB);
    const int n = (int) nt;
    if (t.bn == 192) {
        if (p.rcos) HX_LAUNCH((gemm_nk_big<128, 192, 2, true, true>), grid, block, 0, p, gx, n);
        else HX_LAUNCH((gemm_nk_big<128, 192, 2, false, true>), grid, block, 0, p, gx, n);
    } else {
        if (p.rcos) HX_LAUNCH((gemm_nk_big<128, 128, 2, true, true>), grid, block, 0, p, gx, n);
        else HX_LAUNCH((gemm_nk_big<128, 128, 2, false, true>), grid, block, 0, p, gx, n);
    }
    return true;
}

// Between the two: where the K-across-waves form's 64x64 tiles (one workgroup
// per CU) need more than a round of CUs, the tiled 64x64 form (two per CU),
// as the unfolded linear takes it there (448x448 at batch 1: 784 rows).
static bool launch_lds_lnf(const GemmArgs &p) {
    const long long tiles = (long long) ((p.M + 63) / 64) * ((p.N + 63) / 64);
    if (tiles <= 256) return false;
    const dim3 grid((unsigned) ((p.N + 63) / 64), (unsigned) ((p.M + 63) / 64), 1);
    if (p.rcos) HX_LAUNCH((gemm_nk_lds<64, 64, 4, 2, 2, true, false, false, true>), grid, dim3(TPB), 0, p);
    else HX_LAUNCH((gemm_nk_lds<64, 64, 4, 2, 2, false, false, false, true>), grid, dim3(TPB), 0, p);
    return true;
}

extern "C" void lnfold_matmul_epilogue_f16wt_fp16(const hexlib_hf *x, const hexlib_hf *wt, const float *bias2,
                                                  hexlib_hf *out, int M, int K, int N, int act, float eps) {
    if (!lnf_ok(x, wt, bias2, out, M, K, N, act)) return;
    GemmArgs p = args(x, K, 0, wt, K, 0, bias2, out, N, 0, M, N, K, act);
    p.lnf_eps = eps;
    p.splits = 1;
    p.k_per_split = K;
    if (launch_big_lnf(p) || launch_lds_lnf(p)) return;
    const dim3 grid((unsigned) ((N + 63) / 64), (unsigned) ((M + 63) / 64));
    HX_LAUNCH((gemm_nk_kw<64, false, false, 0, true>), grid, dim3(TPB), 0, p);
}

extern "C" void lnfold_matmul_epilogue_f16wt_rope_fp16(const hexlib_hf *x, const hexlib_hf *wt, const float *bias2,
                                                       const float *costab, const float *sintab, hexlib_hf *out,
                                                       int M, int K, int N, int act, int rope_heads, int rope_dim,
                                                       float eps) {
    if (!lnf_ok(x, wt, bias2, out, M, K, N, act) || !costab || !sintab) return;
    const long long rope_cols = 2LL * rope_heads * rope_dim;
    if (rope_heads <= 0 || rope_dim <= 0 || rope_dim % 4 || rope_cols > N || N % 4 || !hx::aligned(out, 8)) return;
    GemmArgs p = args(x, K, 0, wt, K, 0, bias2, out, N, 0, M, N, K, act);
    p.rcos = costab;
    p.rsin = sintab;
    p.rope_cols = (int) rope_cols;
    p.rope_d = rope_dim;
    p.lnf_eps = eps;
    p.splits = 1;
    p.k_per_split = K;
    if (launch_big_lnf(p) || launch_lds_lnf(p)) return;
    const dim3 grid((unsigned) ((N + 63) / 64), (unsigned) ((M + 63) / 64));
    HX_LAUNCH((gemm_nk_kw<64, true, false, 0, true>), grid, dim3(TPB), 0, p);
}

// LayerNorm over K then the W^T linear, in one launch. Preconditions of the
// prologue: 512 <= K <= 64 * LN_KT, K % 64 == 0, 16-byte aligned x and wt.
bool ln_ok(const hexlib_hf *x, const float *ln_w, const float *ln_b, const hexlib_hf *wt, int K) {
    return x && ln_w && ln_b && wt && K >= 512 && K <= 64 * LN_KT && K % 64 == 0 && hx::aligned(x, 16) &&
           hx::aligned(wt, 16);
}

extern "C" void layernorm_matmul_epilogue_f16wt_fp16(const hexlib_hf *x, const float *ln_w,
                                                     const float *ln_b, const hexlib_hf *wt,
                                                     const float *bias, hexlib_hf *out, int M, int K,
                                                     int N, int act, float eps) {
    if (!out || !dims_ok(M, K, N, 1) || act < 0 || act > 2 || !ln_ok(x, ln_w, ln_b, wt, K)) return;
    GemmArgs p = args(x, K, 0, wt, K, 0, bias, out, N, 0, M, N, K, act);
    p.splits = 1;
    p.k_per_split = K;
    p.ln_w = ln_w;
    p.ln_b = ln_b;
    p.ln_eps = eps;
    launch_ln(p);
}

extern "C" void matmul_epilogue_fp16(const hexlib_hf *a, const unsigned char *w, const float *bias,
                                     hexlib_hf *out, int M, int K, int N, int act) {
    if (!a || !w || !out || !dims_ok(M, K, N, 1) || N % 32 || act < 0 || act > 2) return;
    if (!hx::aligned(w, 2)) return;
    launch<B_Q4N>(args(a, K, 0, w, (long long) (N / 32) * 18, 0, bias, out, N, 0, M, N, K, act), 1,
                  K % 8 == 0 && hx::aligned(a, 16), false);
}

extern "C" void matmul_epilogue_q8k_fp16(const hexlib_hf *a, const unsigned char *wt,
                                         const float *bias, hexlib_hf *out, int M, int K, int N,
                                         int act) {
    if (!a || !wt || !out || !dims_ok(M, K, N, 1) || K % 32 || act < 0 || act > 2) return;
    if (!hx::aligned(wt, 2)) return;
    launch<B_Q8K>(args(a, K, 0, wt, (long long) (K / 32) * 34, 0, bias, out, N, 0, M, N, K, act), 1,
                  K % 8 == 0 && hx::aligned(a, 16), false);
}

extern "C" void matmul_epilogue_q4k_fp16(const hexlib_hf *a, const unsigned char *wt,
                                         const float *bias, hexlib_hf *out, int M, int K, int N,
                                         int act) {
    if (!a || !wt || !out || !dims_ok(M, K, N, 1) || K % 32 || act < 0 || act > 2) return;
    if (!hx::aligned(wt, 2)) return;
    launch<B_Q4K>(args(a, K, 0, wt, (long long) (K / 32) * 18, 0, bias, out, N, 0, M, N, K, act), 1,
                  K % 8 == 0 && hx::aligned(a, 16), false);
}

// The q8_0 (K-grouped W^T) form of matmul_epilogue_f16wt_rope_fp16: the rows
// of W^T pair-interleaved within each rope head before quantization (rows are
// quantized independently, so that is the same blocks as the original rows,
// reordered), dequantized into the K-across-waves kernel's ring; the rope
// epilogue as the fp16 form's. Requires K % 256 == 0.
extern "C" void matmul_epilogue_q8k_rope_fp16(const hexlib_hf *a, const unsigned char *wt, const float *bias,
                                              const float *costab, const float *sintab, hexlib_hf *out, int M,
                                              int K, int N, int act, int rope_heads, int rope_dim) {
    if (!a || !wt || !out || !costab || !sintab || !dims_ok(M, K, N, 1) || act < 0 || act > 2) return;
    const long long rope_cols = 2LL * rope_heads * rope_dim;
    if (rope_heads <= 0 || rope_dim <= 0 || rope_dim % 4 || rope_cols > N || N % 4 || K % KW_BK ||
        !hx::aligned(a, 16) || !hx::aligned(wt, 2) || !hx::aligned(out, 8))
        return;
    GemmArgs p = args(a, K, 0, wt, (long long) (K / 32) * 34, 0, bias, out, N, 0, M, N, K, act);
    p.rcos = costab;
    p.rsin = sintab;
    p.rope_cols = (int) rope_cols;
    p.rope_d = rope_dim;
    const dim3 grid((unsigned) ((N + 63) / 64), (unsigned) ((M + 63) / 64));
    HX_LAUNCH((gemm_nk_kw<64, true, false, 8>), grid, dim3(TPB), 0, p);
}

// The quantized-weight linears with the residual add that consumes them in
// the epilogue (act(acc + bias) rounded to fp16, then fp16(resid + that)), as
// matmul_epilogue_f16wt_res_fp16 does for fp16 weights: every route these
// weights take (one wave per column, the 16-row MFMA form and its split-K
// reduce, the K-across-waves and register-staged kernels) applies it.
extern "C" void matmul_epilogue_res_fp16(const hexlib_hf *a, const unsigned char *w, const float *bias,
                                         const hexlib_hf *resid, hexlib_hf *out, int M, int K, int N, int act) {
    if (!a || !w || !resid || !out || !dims_ok(M, K, N, 1) || N % 32 || act < 0 || act > 2) return;
    if (!hx::aligned(w, 2)) return;
    GemmArgs p = args(a, K, 0, w, (long long) (N / 32) * 18, 0, bias, out, N, 0, M, N, K, act);
    p.R = reinterpret_cast<const f16 *>(resid);
    p.ldr = N;
    launch<B_Q4N>(p, 1, K % 8 == 0 && hx::aligned(a, 16), false);
}

extern "C" void matmul_epilogue_q8k_res_fp16(const hexlib_hf *a, const unsigned char *wt, const float *bias,
                                             const hexlib_hf *resid, hexlib_hf *out, int M, int K, int N,
                                             int act) {
    if (!a || !wt || !resid || !out || !dims_ok(M, K, N, 1) || K % 32 || act < 0 || act > 2) return;
    if (!hx::aligned(wt, 2)) return;
    GemmArgs p = args(a, K, 0, wt, (long long) (K / 32) * 34, 0, bias, out, N, 0, M, N, K, act);
    p.R = reinterpret_cast<const f16 *>(resid);
    p.ldr = N;
    launch<B_Q8K>(p, 1, K % 8 == 0 && hx::aligned(a, 16), false);
}

extern "C" void matmul_epilogue_q4k_res_fp16(const hexlib_hf *a, const unsigned char *wt, const float *bias,
                                             const hexlib_hf *resid, hexlib_hf *out, int M, int K, int N,
                                             int act) {
    if (!a || !wt || !resid || !out || !dims_ok(M, K, N, 1) || K % 32 || act < 0 || act > 2) return;
    if (!hx::aligned(wt, 2)) return;
    GemmArgs p = args(a, K, 0, wt, (long long) (K / 32) * 18, 0, bias, out, N, 0, M, N, K, act);
    p.R = reinterpret_cast<const f16 *>(resid);
    p.ldr = N;
    launch<B_Q4K>(p, 1, K % 8 == 0 && hx::aligned(a, 16), false);
}
