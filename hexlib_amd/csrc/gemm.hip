// fp16 GEMMs on CDNA4 MFMA: matmul_fp16 (batched), matmul_epilogue_f16w_fp16,
// matmul_epilogue_fp16 (q4_0 blocked along N -- the reference kernel ABI) and
// matmul_epilogue_q4k_fp16 (q4_0 grouped along K of W^T).
//
// Numerics (kernels/matmul_fp16/kernel_api.h:18-29, kernels/matmul_epilogue_fp16/
// kernel_api.h:16-27, baseline.c:34-97): fp16 x fp16 products accumulated in
// fp32 by v_mfma_f32_32x32x16_f16; a q4_0 weight is dequantized to
// fp16(d * (q - 8)) before it is multiplied (the reference kernel's own
// rounding); then bias (fp32) is added, the activation applied in fp32, and
// the result rounded to fp16 once.
//
// Structure. A 256-thread workgroup (4 waves, 2 x 2) owns a BM x BN output tile
// and walks K in BK = 32 slices. Each slice of A and B is staged in LDS with K
// contiguous per row ([m][k] and [n][k]), so every MFMA operand fragment is one
// 16-byte ds_read. The next slice's global loads are issued into registers
// before the current slice's MFMAs, then written to the other LDS buffer:
// one barrier per slice. The B operand arrives in one of four layouts and is
// converted to [n][k] on its way into LDS:
//   B_KN  fp16 [K, N] row-major     -- 16-byte loads along n, 2-byte LDS scatter
//   B_NK  fp16 [N, K] (W^T)         -- 16-byte loads along k, 16-byte LDS writes
//   B_Q4N q4_0 [K][N/32] 18-byte blocks (32 n at one k) -- dequant + scatter
//   B_Q4K q4_0 [N][K/32] 18-byte blocks (32 k at one n) -- dequant + 16-byte writes
// Wave tile (BM/2) x (BN/2) as (BM/64) x (BN/64) MFMA 32x32 tiles.
//
// MFMA operand layout (v_mfma_f32_32x32x16_f16, 64 lanes): lane l supplies row
// (l % 32) of the A fragment and column (l % 32) of the B fragment, each as 8
// consecutive k at offset 8 * (l / 32); A and B use the same k assignment, so
// the contraction is correct for any k permutation within the 16. Result
// element i of lane l is C[(i/4)*8 + (l/32)*4 + i%4][l % 32].
#include "device.h"
#include "internal.h"

namespace {

constexpr int TPB = 256;
constexpr int BK = 32;
constexpr int LDS_STRIDE = BK + 8;  // halves per LDS row: 80 B keeps 16-byte alignment

enum BMode { B_KN = 0, B_NK = 1, B_Q4N = 2, B_Q4K = 3 };

struct GemmArgs {
    const f16 *A;
    long long lda, sA;          // row stride, batch stride (elements)
    const void *B;
    long long ldb, sB;          // fp16: elements; q4: bytes per block row, batch stride bytes
    const float *bias;
    f16 *C;
    long long ldc, sC;
    int M, N, K, act;
};

__device__ __forceinline__ f16 q4_val(float d, int q) { return (f16) (d * (float) (q - 8)); }

// Loads 18-byte q4_0 block (2-byte aligned) into d and 16 code bytes.
__device__ __forceinline__ void load_q4_block(const uint8_t *p, float &d, uint32_t qs[4]) {
    const uint16_t *h = reinterpret_cast<const uint16_t *>(p);
    d = (float) __builtin_bit_cast(f16, h[0]);
#pragma unroll
    for (int i = 0; i < 4; ++i) qs[i] = (uint32_t) h[1 + 2 * i] | ((uint32_t) h[2 + 2 * i] << 16);
}

template <int BM, int BN, int MODE, bool AVEC, bool BVEC>
struct Gemm {
    static constexpr int TM = BM / 64;   // 32x32 tiles per wave along M
    static constexpr int TN = BN / 64;
    static constexpr int A_VECS = BM * BK / 8 / TPB;   // 16-byte vectors of A per thread
    static constexpr int B_VECS = BN * BK / 8 / TPB;
    // q4 work items per thread: (block, half) pairs
    static constexpr int Q4N_ITEMS = (BK * (BN / 32) * 2 + TPB - 1) / TPB;
    static constexpr int Q4K_ITEMS = (BN * (BK / 32) * 2 + TPB - 1) / TPB;
    static constexpr int B_ITEMS = (MODE == B_Q4N) ? Q4N_ITEMS : (MODE == B_Q4K) ? Q4K_ITEMS : B_VECS;

    struct Regs {
        f16x8 a[A_VECS];
        f16x8 b[B_ITEMS > 0 ? B_ITEMS : 1];
        float qd[B_ITEMS > 0 ? B_ITEMS : 1];
        uint32_t qs[B_ITEMS > 0 ? B_ITEMS : 1][4];
    };

    // ---- global -> registers ----
    static __device__ __forceinline__ void load_a(const GemmArgs &p, const f16 *A, int m0, int k0,
                                                  Regs &r) {
#pragma unroll
        for (int i = 0; i < A_VECS; ++i) {
            const int v = threadIdx.x + i * TPB;
            const int row = v / (BK / 8), kc = (v % (BK / 8)) * 8;
            const int m = m0 + row, k = k0 + kc;
            if constexpr (AVEC) {
                r.a[i] = (m < p.M && k < p.K) ? *reinterpret_cast<const f16x8 *>(A + m * p.lda + k)
                                              : f16x8{};
            } else {
                f16x8 t;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    t[j] = (m < p.M && k + j < p.K) ? A[m * p.lda + k + j] : (f16) 0;
                r.a[i] = t;
            }
        }
    }

    static __device__ __forceinline__ void load_b(const GemmArgs &p, const void *Bv, int n0, int k0,
                                                  Regs &r) {
        if constexpr (MODE == B_KN) {
            const f16 *B = reinterpret_cast<const f16 *>(Bv);
#pragma unroll
            for (int i = 0; i < B_VECS; ++i) {
                const int v = threadIdx.x + i * TPB;
                const int kr = v / (BN / 8), nc = (v % (BN / 8)) * 8;
                const int k = k0 + kr, n = n0 + nc;
                if constexpr (BVEC) {
                    r.b[i] = (k < p.K && n < p.N) ? *reinterpret_cast<const f16x8 *>(B + k * p.ldb + n)
                                                  : f16x8{};
                } else {
                    f16x8 t;
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        t[j] = (k < p.K && n + j < p.N) ? B[k * p.ldb + n + j] : (f16) 0;
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
                    r.b[i] = (n < p.N && k < p.K) ? *reinterpret_cast<const f16x8 *>(B + n * p.ldb + k)
                                                  : f16x8{};
                } else {
                    f16x8 t;
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        t[j] = (n < p.N && k + j < p.K) ? B[n * p.ldb + k + j] : (f16) 0;
                    r.b[i] = t;
                }
            }
        } else if constexpr (MODE == B_Q4N) {
            // Tile = BK rows (k) x BN/32 blocks. Item = (k, block, half).
            const uint8_t *W = reinterpret_cast<const uint8_t *>(Bv);
#pragma unroll
            for (int i = 0; i < Q4N_ITEMS; ++i) {
                const int it = threadIdx.x + i * TPB;
                const int blk = it >> 1;
                const int kr = blk / (BN / 32), nb = blk % (BN / 32);
                const int k = k0 + kr, n = n0 + nb * 32;
                r.qd[i] = 0.0f;
                r.qs[i][0] = r.qs[i][1] = r.qs[i][2] = r.qs[i][3] = 0x88888888u;  // q = 8 -> 0
                if (it < BK * (BN / 32) * 2 && k < p.K && n < p.N)
                    load_q4_block(W + (long long) k * p.ldb + (long long) (n / 32) * 18, r.qd[i], r.qs[i]);
            }
        } else {  // B_Q4K: tile = BN rows (n) x BK/32 blocks. Item = (n, block, half).
            const uint8_t *W = reinterpret_cast<const uint8_t *>(Bv);
#pragma unroll
            for (int i = 0; i < Q4K_ITEMS; ++i) {
                const int it = threadIdx.x + i * TPB;
                const int blk = it >> 1;
                const int nr = blk / (BK / 32), kb = blk % (BK / 32);
                const int n = n0 + nr, k = k0 + kb * 32;
                r.qd[i] = 0.0f;
                r.qs[i][0] = r.qs[i][1] = r.qs[i][2] = r.qs[i][3] = 0x88888888u;
                if (it < BN * (BK / 32) * 2 && n < p.N && k < p.K)
                    load_q4_block(W + (long long) n * p.ldb + (long long) (k / 32) * 18, r.qd[i], r.qs[i]);
            }
        }
    }

    // ---- registers -> LDS ([m][k] and [n][k]) ----
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
                if (it >= BK * (BN / 32) * 2) continue;
                const int blk = it >> 1, half = it & 1;
                const int kr = blk / (BN / 32), nb = blk % (BN / 32);
                const int shift = half * 4;
                // byte j: low nibble = element j, high nibble = element j + 16
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int q = (int) ((r.qs[i][j >> 2] >> ((j & 3) * 8 + shift)) & 0xF);
                    Bs[(nb * 32 + half * 16 + j) * LDS_STRIDE + kr] = q4_val(r.qd[i], q);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < Q4K_ITEMS; ++i) {
                const int it = threadIdx.x + i * TPB;
                if (it >= BN * (BK / 32) * 2) continue;
                const int blk = it >> 1, half = it & 1;
                const int nr = blk / (BK / 32), kb = blk % (BK / 32);
                const int shift = half * 4;
                f16x8 lo, hi;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    lo[j] = q4_val(r.qd[i], (int) ((r.qs[i][j >> 2] >> ((j & 3) * 8 + shift)) & 0xF));
                    hi[j] = q4_val(r.qd[i],
                                   (int) ((r.qs[i][(j + 8) >> 2] >> (((j + 8) & 3) * 8 + shift)) & 0xF));
                }
                f16 *dst = Bs + nr * LDS_STRIDE + kb * 32 + half * 16;
                *reinterpret_cast<f16x8 *>(dst) = lo;
                *reinterpret_cast<f16x8 *>(dst + 8) = hi;
            }
        }
    }

    static __device__ void run(const GemmArgs &p) {
        __shared__ __attribute__((aligned(16))) f16 As[2][BM * LDS_STRIDE];
        __shared__ __attribute__((aligned(16))) f16 Bs[2][BN * LDS_STRIDE];

        const int bz = blockIdx.z;
        const f16 *A = p.A + (long long) bz * p.sA;
        const void *B;
        if constexpr (MODE == B_KN || MODE == B_NK)
            B = reinterpret_cast<const f16 *>(p.B) + (long long) bz * p.sB;
        else
            B = reinterpret_cast<const uint8_t *>(p.B) + (long long) bz * p.sB;
        const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * (BN / 2);

        f32x16 acc[TM][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = f32x16{};

        const int KT = (p.K + BK - 1) / BK;
        Regs r;
        load_a(p, A, m0, 0, r);
        load_b(p, B, n0, 0, r);
        store(As[0], Bs[0], r);
        __syncthreads();

        for (int kt = 0; kt < KT; ++kt) {
            const int cur = kt & 1;
            if (kt + 1 < KT) {
                load_a(p, A, m0, (kt + 1) * BK, r);
                load_b(p, B, n0, (kt + 1) * BK, r);
            }
            const f16 *as = As[cur];
            const f16 *bs = Bs[cur];
#pragma unroll
            for (int ks = 0; ks < BK; ks += 16) {
                f16x8 af[TM], bf[TN];
                const int kk = ks + (lane >> 5) * 8;
#pragma unroll
                for (int i = 0; i < TM; ++i)
                    af[i] = *reinterpret_cast<const f16x8 *>(as + (wm + i * 32 + (lane & 31)) * LDS_STRIDE + kk);
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    bf[j] = *reinterpret_cast<const f16x8 *>(bs + (wn + j * 32 + (lane & 31)) * LDS_STRIDE + kk);
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
            if (kt + 1 < KT) store(As[cur ^ 1], Bs[cur ^ 1], r);
            __syncthreads();
        }

        f16 *C = p.C + (long long) bz * p.sC;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn + j * 32 + (lane & 31);
            const float bv = (p.bias && col < p.N) ? p.bias[col] : 0.0f;
#pragma unroll
            for (int i = 0; i < TM; ++i) {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int row = m0 + wm + i * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3);
                    if (row < p.M && col < p.N)
                        C[(long long) row * p.ldc + col] = (f16) apply_act(acc[i][j][e] + bv, p.act);
                }
            }
        }
    }
};

template <int BM, int BN, int MODE, bool AVEC, bool BVEC>
__global__ __launch_bounds__(TPB) void gemm_kernel(GemmArgs p) {
    Gemm<BM, BN, MODE, AVEC, BVEC>::run(p);
}

template <int BM, int BN, int MODE>
void launch_tile(const GemmArgs &p, int batch, bool avec, bool bvec) {
    dim3 grid((unsigned) ((p.N + BN - 1) / BN), (unsigned) ((p.M + BM - 1) / BM), (unsigned) batch);
    if (avec && bvec) HX_LAUNCH((gemm_kernel<BM, BN, MODE, true, true>), grid, dim3(TPB), 0, p);
    else if (avec) HX_LAUNCH((gemm_kernel<BM, BN, MODE, true, false>), grid, dim3(TPB), 0, p);
    else if (bvec) HX_LAUNCH((gemm_kernel<BM, BN, MODE, false, true>), grid, dim3(TPB), 0, p);
    else HX_LAUNCH((gemm_kernel<BM, BN, MODE, false, false>), grid, dim3(TPB), 0, p);
}

template <int MODE>
void launch(const GemmArgs &p, int batch, bool avec, bool bvec) {
    // 128x128 tiles once there are enough of them to cover the 256 CUs;
    // 64x64 tiles otherwise (4x the workgroups for small M or N).
    const long long big = (long long) ((p.M + 127) / 128) * ((p.N + 127) / 128) * batch;
    if (big >= 256) launch_tile<128, 128, MODE>(p, batch, avec, bvec);
    else launch_tile<64, 64, MODE>(p, batch, avec, bvec);
}

bool dims_ok(int M, int K, int N, int batch) {
    return M > 0 && K > 0 && N > 0 && batch > 0 && batch <= 65535 && (M + 63) / 64 <= 65535;
}

}  // namespace

extern "C" void matmul_fp16(const hexlib_hf *A, const hexlib_hf *B, hexlib_hf *C, int Bn, int M,
                            int K, int N) {
    if (!A || !B || !C || !dims_ok(M, K, N, Bn)) return;
    GemmArgs p{reinterpret_cast<const f16 *>(A), K, (long long) M * K, B, N, (long long) K * N,
               nullptr, reinterpret_cast<f16 *>(C), N, (long long) M * N, M, N, K, 0};
    launch<B_KN>(p, Bn, K % 8 == 0 && hx::aligned(A, 16), N % 8 == 0 && hx::aligned(B, 16));
}

extern "C" void matmul_epilogue_f16w_fp16(const hexlib_hf *a, const hexlib_hf *w, const float *bias,
                                          hexlib_hf *out, int M, int K, int N, int act) {
    if (!a || !w || !out || !dims_ok(M, K, N, 1) || act < 0 || act > 2) return;
    GemmArgs p{reinterpret_cast<const f16 *>(a), K, 0, w, N, 0, bias,
               reinterpret_cast<f16 *>(out), N, 0, M, N, K, act};
    launch<B_KN>(p, 1, K % 8 == 0 && hx::aligned(a, 16), N % 8 == 0 && hx::aligned(w, 16));
}

extern "C" void matmul_epilogue_fp16(const hexlib_hf *a, const unsigned char *w, const float *bias,
                                     hexlib_hf *out, int M, int K, int N, int act) {
    if (!a || !w || !out || !dims_ok(M, K, N, 1) || N % 32 || act < 0 || act > 2) return;
    if (!hx::aligned(w, 2)) return;
    GemmArgs p{reinterpret_cast<const f16 *>(a), K, 0, w, (long long) (N / 32) * 18, 0, bias,
               reinterpret_cast<f16 *>(out), N, 0, M, N, K, act};
    launch<B_Q4N>(p, 1, K % 8 == 0 && hx::aligned(a, 16), false);
}

extern "C" void matmul_epilogue_q4k_fp16(const hexlib_hf *a, const unsigned char *wt,
                                         const float *bias, hexlib_hf *out, int M, int K, int N,
                                         int act) {
    if (!a || !wt || !out || !dims_ok(M, K, N, 1) || K % 32 || act < 0 || act > 2) return;
    if (!hx::aligned(wt, 2)) return;
    GemmArgs p{reinterpret_cast<const f16 *>(a), K, 0, wt, (long long) (K / 32) * 18, 0, bias,
               reinterpret_cast<f16 *>(out), N, 0, M, N, K, act};
    launch<B_Q4K>(p, 1, K % 8 == 0 && hx::aligned(a, 16), false);
}
