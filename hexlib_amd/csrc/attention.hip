// Fused multi-head attention, forward: out = softmax(scale * q k^T) v per
// (image, head), for the encoder's full (non-causal) attention. It replaces the
// reference's chain scale -> transpose_hd -> matmul -> softmax -> matmul and the
// transposes around it (hexlib/models/vit.py:185-193); the op is an extension
// with no kernel_api.h counterpart.
//
// Layout: q, k, v and out are [rows = batch * T, H, D] fp16, the layout rope_2d
// and the linears produce (token-major, heads interleaved), so no transpose is
// needed on either side. attention_qk_v_fp16 takes q and k from a
// [rows, 2, H, D] tensor (rope_2d_qk_fp16's output) and v from the fused
// [rows, 3, H, D] projection, by row stride.
//
// Numerics: q.k in fp32 (MFMA accumulate), scaled in fp32 inside the exponent;
// a running max and sum per query (online softmax, exp2 of log2e-scaled
// scores, the max raised lazily: see softmax_step); the unnormalised
// probabilities are rounded to fp16 for the P.V product, accumulated in fp32;
// the output is divided by the fp32 sum and rounded to fp16 once.
//
// Structure: a workgroup of WAVES (4, or 8 when the grid would leave CUs idle)
// waves owns 32 queries of one (image, head);
// wave w takes key tiles w, w + WAVES, ... (32 keys each), with the next
// tile's K and V loads issued before the current tile is computed, and keeps
// its own running max, sum and output. The waves' partial results are merged
// through LDS at the end (rescaled by exp2 of the max differences). Both
// products run on v_mfma_f32_32x32x16_f16 (lane l supplies row l % 32 of A and
// column l % 32 of B, 8 consecutive k at 8 * (l / 32); result element i of
// lane l is D[(i/4)*8 + (l/32)*4 + i%4][l % 32]):
//   S^T = K Q^T   A = K rows (keys), B = Q^T columns (queries): lane l then
//                 holds 16 scores of ONE query (l % 32), so the row max / sum
//                 are in-lane plus one exchange with lane l ^ 32.
//   O^T = V^T P^T A = V^T rows (d), B = P^T: the B operand is the lane's own
//                 16 probabilities, provided A's k index means the same key.
// To make that true S^T row r holds key kperm(r), chosen so that P's k index
// 8h + j of chunk c is key 16c + 8h + j: the K tile goes to a wave-private
// LDS tile as loaded (8 lanes per key row, so a load touches 8 rows, not the
// 32 of the operand layout) and the operand reads row kperm(r) of it. The
// V^T operand then needs 8 consecutive keys of one d. The V
// tile goes to a wave-private LDS tile as loaded ([key][d], 16-byte writes,
// 192-byte rows) and each V^T operand is two ds_read_b64_tr_b16: within each
// 16-lane group, lane 4a + b receives element b of the 8 bytes that lanes a,
// a + 4, a + 8, a + 12 address, so lanes addressing 4 consecutive d of 4
// consecutive keys deliver to each lane 4 keys of one d. LDS operations of one
// wave complete in order, so the wave-private tile needs no
// barrier; the only workgroup barrier is before the merge, which every wave
// reaches.
#include <atomic>
#include <cmath>

#include "device.h"
#include "internal.h"

namespace {

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef short v8i16 __attribute__((ext_vector_type(8)));

constexpr int QT = 32;          // queries per wave
constexpr int KT = 32;          // keys per tile
// halves per LDS row of the V tile: the 4 rows x 64 bytes a 32-lane
// transpose-read phase touches fall in 4 distinct 16-bank windows (192-byte
// rows for D = 64; D = 32 rows are 64 bytes and need no padding)
template <int D>
constexpr int v_stride() { return D == 64 ? 96 : D; }
constexpr int CUS = 256;        // MI355X compute units

__device__ __forceinline__ int kperm(int r) {
    return 16 * (r >> 4) + 8 * ((r >> 2) & 1) + 4 * ((r >> 3) & 1) + (r & 3);
}

template <int D>
struct KvTile {
    f16x8 k[D / 16];       // this lane's 16-byte pieces of the K tile
    f16x8 v[D / 16];       // this lane's 16-byte pieces of the V tile
};

template <int D>
__device__ __forceinline__ void load_tile(const f16 *__restrict__ kb, long long ldk, const f16 *__restrict__ vb,
                                          long long ldv, int T, int kt, int lane, KvTile<D> &t) {
    constexpr int VCH = D / 8;
    // K as V: 8 lanes per 128-byte key row, so one load touches 8 rows (the
    // MFMA operand layout would touch 32); rows past T repeat row T - 1 and
    // are masked after the product
#pragma unroll
    for (int i = 0; i < D / 16; ++i) {
        const int e = lane + 64 * i;
        const int key = min(kt + e / VCH, T - 1);
        t.k[i] = *reinterpret_cast<const f16x8 *>(kb + key * ldk + (e % VCH) * 8);
    }
#pragma unroll
    for (int i = 0; i < D / 16; ++i) {
        const int e = lane + 64 * i;
        const int vkey = kt + e / VCH;
        // keys past T load as zero: their p is 0, and 0 * garbage could be NaN
        t.v[i] = vkey < T ? *reinterpret_cast<const f16x8 *>(vb + vkey * ldv + (e % VCH) * 8) : f16x8{};
    }
}

// One online-softmax update over NSUB 32-key sub-tiles of scores S^T (element
// i of sub-tile u is key key0 + 32 u + 16 (i / 8) + 8 hl + i % 8; the lane's
// query is shared with lane ^ 32). Scores are scaled by c = scale * log2(e)
// inside the exponent (one fma: exp2(c s - m)), so the running maximum is
// kept on the scaled scale: m is the reference every p and the partial O are
// relative to. It is raised only when some query of the wave sees a scaled
// score more than 8 above it (a wave-uniform branch): until then the
// probabilities are at most 2^8, far inside fp16 and fp32, and the rescale of
// O (and its exp2) is skipped. Keys past T are masked only on the sequence's
// last, partial tile. exp2 is the hardware's v_exp_f32 (about 1 ulp; the
// probabilities are then rounded to fp16).
template <int NSUB>
__device__ __forceinline__ void softmax_step(f32x16 (&s)[NSUB], int key0, int T, float c, int hl, float &m,
                                             float &l, f32x16 *oacc, int dt, f16x8 (&pb)[NSUB][2]) {
    // a key past T never wins the extreme and gets p = 0 (set after the exp2:
    // at c == 0 an infinite score would make it NaN)
    const bool part = key0 + 32 * NSUB > T;
    const float pad = c > 0.0f ? -INFINITY : (c < 0.0f ? INFINITY : 0.0f);
    if (part) {
#pragma unroll
        for (int u = 0; u < NSUB; ++u)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key = key0 + 32 * u + 16 * (i >> 3) + 8 * hl + (i & 7);
                if (key >= T) s[u][i] = pad;
            }
    }
    float tmax = -INFINITY;
    if (c > 0.0f) {
#pragma unroll
        for (int u = 0; u < NSUB; ++u)
#pragma unroll
            for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, s[u][i]);
        tmax *= c;
    } else {
        float tmin = INFINITY;
#pragma unroll
        for (int u = 0; u < NSUB; ++u)
#pragma unroll
            for (int i = 0; i < 16; ++i) tmin = fminf(tmin, s[u][i]);
        tmax = tmin * c;
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));      // finite: the tile's first key is valid
    if (__any(tmax > m + 8.0f)) {
        const float m_new = fmaxf(m, tmax);
        const float alpha = __builtin_amdgcn_exp2f(m - m_new);
        l *= alpha;
        for (int t = 0; t < dt; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) oacc[t][i] *= alpha;
        m = m_new;
    }
    // two copies of the loop under a wave-uniform branch: only the last tile
    // pays for the key test
    float psum = 0.f;
    if (part) {
#pragma unroll
        for (int u = 0; u < NSUB; ++u)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[u][i], c, -m));
                if (key0 + 32 * u + 16 * (i >> 3) + 8 * hl + (i & 7) >= T) p = 0.0f;
                psum += p;
                pb[u][i >> 3][i & 7] = (f16) p;
            }
    } else {
#pragma unroll
        for (int u = 0; u < NSUB; ++u)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[u][i], c, -m));
                psum += p;
                pb[u][i >> 3][i & 7] = (f16) p;
            }
    }
    l += psum;
}

// q and k rows are `ldqk` halves apart, v rows `ldv` (H*D for separate
// tensors; 2*H*D and 3*H*D when q, k come from a [rows, 2, H, D] tensor and v
// from a fused [rows, 3, H, D] projection); out rows are H*D apart.
template <int D, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void attn_fwd(const f16 *__restrict__ q, const f16 *__restrict__ k,
                                                       long long ldqk, const f16 *__restrict__ v, long long ldv,
                                                       f16 *__restrict__ o, int T, int H, float scale_log2e) {
    constexpr int KC = D / 16;   // 16-wide d chunks of q.k
    constexpr int DT = D / 32;   // 32-row tiles of O^T
    constexpr int VCH = D / 8;   // 16-byte chunks per V row
    constexpr int V_STRIDE = v_stride<D>();
    __shared__ __attribute__((aligned(16))) f16 v_all[WAVES][KT * V_STRIDE];
    // the K tile, wave-private, as loaded: 144-byte rows keep the 16 rows one
    // ds_read_b128 phase reads in distinct banks
    constexpr int K_STRIDE = D + 8;
    __shared__ __attribute__((aligned(16))) f16 k_all[WAVES][KT * K_STRIDE];
    // partial outputs, rows padded by 4 floats: 16-byte writes and reads, and the
    // 16 rows of one ds_write_b128 phase fall in distinct 16-byte bank groups
    constexpr int PO_STRIDE = D + 4;
    __shared__ __attribute__((aligned(16))) float part_o[WAVES][QT][PO_STRIDE];
    __shared__ float part_m[WAVES][QT], part_l[WAVES][QT];

    const int bh = blockIdx.y;
    const int b = bh / H, h = bh % H;
    const long long ldo = (long long) H * D;   // output token stride
    const long long row0 = (long long) b * T;   // first row of this image
    const f16 *qb = q + row0 * ldqk + (long long) h * D, *kb = k + row0 * ldqk + (long long) h * D,
              *vb = v + row0 * ldv + (long long) h * D;
    f16 *ob = o + row0 * ldo + (long long) h * D;
    // the wave index through readfirstlane: the compiler then knows every
    // key-tile index derived from it is wave-uniform, so the partial-tile
    // masking below is a scalar branch, not predicated code on every tile
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, hl = lane >> 5,
              c32 = lane & 31;
    const int q0 = blockIdx.x * QT;
    f16 *vt = v_all[wave];
    f16 *ktl = k_all[wave];
    // transpose-read addresses (halves) within the tile: key 8 hl + 4 u + s / 4,
    // d 16 ((lane / 16) % 2) + 4 (s % 4), s = lane % 16; chunk c adds 16 keys, d tile t 32 d
    const int tr_off = (8 * hl + ((lane & 15) >> 2)) * V_STRIDE + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

    // B operand of S^T: query column c32, d = 16 kk + 8 hl .. +8. The 8-wave
    // form (one key tile per wave: the Q load is on its critical path) loads
    // the Q tile like K, 8 lanes per row, and stages it through the wave's K
    // tile (batch 1: 5.8 -> 5.4 us); the 4-wave form, whose waves walk several
    // tiles, loads the operand directly (measured faster there).
    constexpr bool QSTAGE = WAVES == 8;
    f16x8 qraw[QSTAGE ? D / 16 : 1];
    f16x8 qf[KC];
    if constexpr (QSTAGE) {
#pragma unroll
        for (int i = 0; i < D / 16; ++i) {
            const int e = lane + 64 * i;
            qraw[i] = *reinterpret_cast<const f16x8 *>(qb + min(q0 + e / VCH, T - 1) * ldqk + (e % VCH) * 8);
        }
    } else {
        const int qi = min(q0 + c32, T - 1);
#pragma unroll
        for (int kk = 0; kk < KC; ++kk)
            qf[kk] = *reinterpret_cast<const f16x8 *>(qb + qi * ldqk + 16 * kk + 8 * hl);
    }
    const int krow_key = kperm(c32);   // key (within a tile) this lane's K row holds

    f32x16 oacc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) oacc[t] = f32x16{};
    float m = -INFINITY, l = 0.f;

    KvTile<D> cur, nxt;
    int kt = wave * KT;
    if (kt < T) load_tile<D>(kb, ldqk, vb, ldv, T, kt, lane, cur);
    if constexpr (QSTAGE) {
        // the staged Q tile, read back as the operand (the loop's first K write comes after)
#pragma unroll
        for (int i = 0; i < D / 16; ++i) {
            const int e = lane + 64 * i;
            *reinterpret_cast<f16x8 *>(ktl + (e / VCH) * K_STRIDE + (e % VCH) * 8) = qraw[i];
        }
#pragma unroll
        for (int kk = 0; kk < KC; ++kk)
            qf[kk] = *reinterpret_cast<const f16x8 *>(ktl + c32 * K_STRIDE + 16 * kk + 8 * hl);
    }
    for (; kt < T; kt += WAVES * KT) {
        const int kn = kt + WAVES * KT;
        if (kn < T) load_tile<D>(kb, ldqk, vb, ldv, T, kn, lane, nxt);

        // V tile -> wave-private LDS as loaded, [key][d]
#pragma unroll
        for (int i = 0; i < D / 16; ++i) {
            const int e = lane + 64 * i;
            *reinterpret_cast<f16x8 *>(vt + (e / VCH) * V_STRIDE + (e % VCH) * 8) = cur.v[i];
        }

        // K tile -> wave-private LDS as loaded; the S^T operand is key row
        // kperm(c32) of it
#pragma unroll
        for (int i = 0; i < D / 16; ++i) {
            const int e = lane + 64 * i;
            *reinterpret_cast<f16x8 *>(ktl + (e / VCH) * K_STRIDE + (e % VCH) * 8) = cur.k[i];
        }
        f16x8 kf[KC];
#pragma unroll
        for (int kk = 0; kk < KC; ++kk)
            kf[kk] = *reinterpret_cast<const f16x8 *>(ktl + krow_key * K_STRIDE + 16 * kk + 8 * hl);
        f32x16 s = f32x16{};
#pragma unroll
        for (int kk = 0; kk < KC; ++kk) s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[kk], qf[kk], s, 0, 0, 0);

        // element i of this lane is key kt + 16 (i / 8) + 8 hl + i % 8
        f32x16 sv[1] = {s};
        f16x8 pbv[1][2];
        softmax_step<1>(sv, kt, T, scale_log2e, hl, m, l, oacc, DT, pbv);
        const f16x8 pb[2] = {pbv[0][0], pbv[0][1]};

#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                // V^T rows d = 32 t + lane % 32, keys 16 c + 8 hl .. + 8
                const f16 *base = vt + tr_off + 16 * c * V_STRIDE + 32 * t;
                const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) v4i16 *) (base));
                const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) v4i16 *) (base + 4 * V_STRIDE));
                const f16x8 va = __builtin_bit_cast(f16x8, (v8i16){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
                oacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[c], oacc[t], 0, 0, 0);
            }
        cur = nxt;
    }

    // merge the waves: each publishes (m, l, O) for its 32 queries
    l += __shfl_xor(l, 32);
    if (hl == 0) {
        part_m[wave][c32] = m;
        part_l[wave][c32] = l;
    }
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4)
            *reinterpret_cast<f32x4 *>(&part_o[wave][c32][32 * t + i4 * 8 + 4 * hl]) =
                f32x4{oacc[t][4 * i4], oacc[t][4 * i4 + 1], oacc[t][4 * i4 + 2], oacc[t][4 * i4 + 3]};
    __syncthreads();

    // 32 queries x D outputs, 8 consecutive d per thread
    for (int e = threadIdx.x; e < QT * (D / 8); e += 64 * WAVES) {
        const int qq = e / (D / 8), d0 = (e % (D / 8)) * 8;
        const int qi = q0 + qq;
        if (qi >= T) continue;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) mx = fmaxf(mx, part_m[w][qq]);
        float wsum = 0.f, acc[8] = {};
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float a = __builtin_amdgcn_exp2f(part_m[w][qq] - mx);   // 0 for a wave that saw no key
            wsum += a * part_l[w][qq];
            const f32x4 o0 = *reinterpret_cast<const f32x4 *>(&part_o[w][qq][d0]);
            const f32x4 o1 = *reinterpret_cast<const f32x4 *>(&part_o[w][qq][d0 + 4]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[j] += a * o0[j];
                acc[j + 4] += a * o1[j];
            }
        }
        const float inv = 1.0f / wsum;
        f16x8 out;
#pragma unroll
        for (int j = 0; j < 8; ++j) out[j] = (f16) (acc[j] * inv);
        *reinterpret_cast<f16x8 *>(ob + qi * ldo + d0) = out;
    }
}

// ---- many query tiles per workgroup, K and V shared through LDS -------------
//
// attn_fwd gives every wave its own K/V tiles: each (image, head) reads its
// keys and values once per 32-query tile (8 times at T = 256), a workgroup
// owns only 32 queries, and the waves merge their partial results at the end.
// Where the grid is large (many images, or long sequences) this form instead
// gives a workgroup QG x 32 queries of one (image, head): the QG waves of a
// key split walk the same 64-key stages, each stage's K and V loaded once
// (each wave loads 1/QG of it, one stage ahead, into registers) and shared
// through a two-slot LDS ring, one workgroup barrier per stage. With KS key
// splits (QG x KS waves) split k takes stages k, k + KS, ... and the splits'
// (max, sum, O) are merged through LDS at the end, as in attn_fwd; with one
// split each wave normalises and stores its own queries directly. The per-tile
// arithmetic (S^T = K Q^T, the online softmax in exp2, fp16 probabilities,
// O^T = V^T P^T with transpose reads of V) is attn_fwd's; one softmax update
// covers a 64-key stage.
constexpr int KS_KEYS = 64;     // keys per stage

template <int D, int QG, int KS>
__global__ __launch_bounds__(64 * QG * KS) void attn_qg(const f16 *__restrict__ q, const f16 *__restrict__ k,
                                                        long long ldqk, const f16 *__restrict__ v, long long ldv,
                                                        f16 *__restrict__ o, int T, int H, float scale_log2e) {
    constexpr int W = QG * KS;
    constexpr int KC = D / 16, DT = D / 32, VCH = D / 8;
    constexpr int V_STRIDE = v_stride<D>(), K_STRIDE = D + 8;
    constexpr int K_HALVES = KS_KEYS * K_STRIDE, V_HALVES = KS_KEYS * V_STRIDE;
    constexpr int SLOT = K_HALVES + V_HALVES;                  // one stage of one split
    constexpr int PIECES = KS_KEYS * VCH / (64 * QG);          // 16-byte pieces per lane per tensor
    static_assert(KS_KEYS * VCH % (64 * QG) == 0, "the stage splits evenly over the split's waves");
    constexpr int PO_STRIDE = D + 4;
    // two ring slots per split, one with four splits (their LDS would not fit
    // twice; at 256 tokens each split then has one stage anyway)
    constexpr int SLOTS = KS >= 4 ? 1 : 2;
    constexpr int RING_BYTES = KS * SLOTS * SLOT * 2;
    constexpr int MERGE_BYTES = KS > 1 ? W * 32 * PO_STRIDE * 4 : 0;
    constexpr int LDS_BYTES = RING_BYTES > MERGE_BYTES ? RING_BYTES : MERGE_BYTES;
    __shared__ __attribute__((aligned(16))) f16 ring[LDS_BYTES / 2];
    __shared__ float part_m[KS > 1 ? W : 1][32], part_l[KS > 1 ? W : 1][32];

    // A one-dimensional grid of (image, head, query block) tasks, renumbered
    // so that each XCD (the hardware deals workgroup i to XCD i % 8) takes a
    // contiguous run of them: the query blocks of one (image, head) then read
    // its K and V through one L2. A bijection whatever the dealing.
    const int nq = (T + 32 * QG - 1) / (32 * QG);
    const int ntask = gridDim.x, q8 = ntask / 8, r8 = ntask % 8, xcd = blockIdx.x % 8, li = blockIdx.x / 8;
    const int task = (xcd < r8 ? xcd * (q8 + 1) : r8 * (q8 + 1) + (xcd - r8) * q8) + li;
    const int bh = task / nq, qblk = task % nq, b = bh / H, h = bh % H;
    const long long ldo = (long long) H * D, row0 = (long long) b * T;
    const f16 *qb = q + row0 * ldqk + (long long) h * D, *kb = k + row0 * ldqk + (long long) h * D,
              *vb = v + row0 * ldv + (long long) h * D;
    f16 *ob = o + row0 * ldo + (long long) h * D;
    // the wave index through readfirstlane: the compiler then knows every
    // key-tile index derived from it is wave-uniform, so the partial-tile
    // masking below is a scalar branch, not predicated code on every tile
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, hl = lane >> 5,
              c32 = lane & 31;
    const int qg = wave % QG, ks = wave / QG;
    const int q0 = qblk * (32 * QG) + qg * 32;
    const int n_stages = (T + KS_KEYS - 1) / KS_KEYS, iters = (n_stages + KS - 1) / KS;
    const int tr_off = (8 * hl + ((lane & 15) >> 2)) * V_STRIDE + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const int krow_key = kperm(c32);

    // this lane's pieces of a stage: piece e = qg * 64 + lane + 64 QG i is key e / VCH, chunk e % VCH
    f16x8 kr[PIECES], vr[PIECES];
    auto load_stage = [&](int st) {
        const int key0 = st * KS_KEYS;
#pragma unroll
        for (int i = 0; i < PIECES; ++i) {
            const int e = qg * 64 + lane + 64 * QG * i, key = key0 + e / VCH, ch = e % VCH;
            kr[i] = *reinterpret_cast<const f16x8 *>(kb + (long long) min(key, T - 1) * ldqk + ch * 8);
            vr[i] = key < T ? *reinterpret_cast<const f16x8 *>(vb + (long long) key * ldv + ch * 8) : f16x8{};
        }
    };
    auto store_stage = [&](int slot) {
        f16 *kt = ring + (ks * SLOTS + slot) * SLOT, *vt = kt + K_HALVES;
#pragma unroll
        for (int i = 0; i < PIECES; ++i) {
            const int e = qg * 64 + lane + 64 * QG * i, key = e / VCH, ch = e % VCH;
            *reinterpret_cast<f16x8 *>(kt + key * K_STRIDE + ch * 8) = kr[i];
            *reinterpret_cast<f16x8 *>(vt + key * V_STRIDE + ch * 8) = vr[i];
        }
    };

    // the first stage's loads, then this wave's Q^T operand (query c32, d 16 kk + 8 hl ..)
    if (ks < n_stages) load_stage(ks);
    f16x8 qf[KC];
    {
        const int qi = min(q0 + c32, T - 1);
#pragma unroll
        for (int kk = 0; kk < KC; ++kk)
            qf[kk] = *reinterpret_cast<const f16x8 *>(qb + (long long) qi * ldqk + 16 * kk + 8 * hl);
    }
    f32x16 oacc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) oacc[t] = f32x16{};
    float m = -INFINITY, l = 0.f;

    store_stage(0);
    __syncthreads();
    for (int it = 0; it < iters; ++it) {
        const int st = it * KS + ks, slot = SLOTS == 2 ? it & 1 : 0;
        const bool live = st < n_stages;
        if (live && st + KS < n_stages) load_stage(st + KS);   // one stage ahead, into registers
        if (live) {
            const f16 *kt = ring + (ks * SLOTS + slot) * SLOT, *vt = kt + K_HALVES;
            const int key0 = st * KS_KEYS;
            f32x16 s[2];
#pragma unroll
            for (int sub = 0; sub < 2; ++sub) {
                f16x8 kf[KC];
#pragma unroll
                for (int kk = 0; kk < KC; ++kk)
                    kf[kk] = *reinterpret_cast<const f16x8 *>(kt + (32 * sub + krow_key) * K_STRIDE + 16 * kk + 8 * hl);
                s[sub] = f32x16{};
#pragma unroll
                for (int kk = 0; kk < KC; ++kk)
                    s[sub] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[kk], qf[kk], s[sub], 0, 0, 0);
            }
            // element i of sub-tile sub is key key0 + 32 sub + 16 (i / 8) + 8 hl + i % 8
            f16x8 pb[2][2];
            softmax_step<2>(s, key0, T, scale_log2e, hl, m, l, oacc, DT, pb);
#pragma unroll
            for (int sub = 0; sub < 2; ++sub)
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int t = 0; t < DT; ++t) {
                        const f16 *base = vt + tr_off + (32 * sub + 16 * c) * V_STRIDE + 32 * t;
                        const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (__attribute__((address_space(3))) v4i16 *) (base));
                        const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (__attribute__((address_space(3))) v4i16 *) (base + 4 * V_STRIDE));
                        const f16x8 va = __builtin_bit_cast(
                            f16x8, (v8i16){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
                        oacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[sub][c], oacc[t], 0, 0, 0);
                    }
        }
        // the other slot was last read in the previous iteration: every wave is
        // past it once this barrier is, so the next stage can land there (one
        // slot: every wave must be past this stage's reads first)
        if (it + 1 < iters) {
            if constexpr (SLOTS == 1) __syncthreads();
            if (live && st + KS < n_stages) store_stage(SLOTS == 2 ? slot ^ 1 : 0);
            __syncthreads();
        }
    }

    l += __shfl_xor(l, 32);
    if constexpr (KS == 1) {
        // this wave owns its queries over every key: O = O^T / l, 4 consecutive d per store
        const int qi = q0 + c32;
        if (qi < T) {
            const float inv = 1.0f / l;
#pragma unroll
            for (int t = 0; t < DT; ++t)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    f16x4 out;
#pragma unroll
                    for (int e = 0; e < 4; ++e) out[e] = (f16) (oacc[t][4 * i4 + e] * inv);
                    *reinterpret_cast<f16x4 *>(ob + (long long) qi * ldo + 32 * t + 8 * i4 + 4 * hl) = out;
                }
        }
    } else {
        // merge the key splits of each query group through LDS (the ring is done)
        __syncthreads();
        float *po = reinterpret_cast<float *>(ring);      // [W][32][PO_STRIDE]
        if (hl == 0) {
            part_m[wave][c32] = m;
            part_l[wave][c32] = l;
        }
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4)
                *reinterpret_cast<f32x4 *>(po + (wave * 32 + c32) * PO_STRIDE + 32 * t + i4 * 8 + 4 * hl) =
                    f32x4{oacc[t][4 * i4], oacc[t][4 * i4 + 1], oacc[t][4 * i4 + 2], oacc[t][4 * i4 + 3]};
        __syncthreads();
        for (int e = threadIdx.x; e < QG * 32 * (D / 8); e += 64 * W) {
            const int g = e / (32 * (D / 8)), qq = (e / (D / 8)) % 32, d0 = (e % (D / 8)) * 8;
            const int qi = qblk * (32 * QG) + g * 32 + qq;
            if (qi >= T) continue;
            float mx = -INFINITY;
#pragma unroll
            for (int sp = 0; sp < KS; ++sp) mx = fmaxf(mx, part_m[sp * QG + g][qq]);
            float wsum = 0.f, acc[8] = {};
#pragma unroll
            for (int sp = 0; sp < KS; ++sp) {
                const int w = sp * QG + g;
                const float a = __builtin_amdgcn_exp2f(part_m[w][qq] - mx);   // 0 for a split that saw no key
                wsum += a * part_l[w][qq];
                const f32x4 o0 = *reinterpret_cast<const f32x4 *>(po + (w * 32 + qq) * PO_STRIDE + d0);
                const f32x4 o1 = *reinterpret_cast<const f32x4 *>(po + (w * 32 + qq) * PO_STRIDE + d0 + 4);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[j] += a * o0[j];
                    acc[j + 4] += a * o1[j];
                }
            }
            const float inv = 1.0f / wsum;
            f16x8 out;
#pragma unroll
            for (int j = 0; j < 8; ++j) out[j] = (f16) (acc[j] * inv);
            *reinterpret_cast<f16x8 *>(ob + (long long) qi * ldo + d0) = out;
        }
    }
}

// Tuning override for the attention form (0: automatic; else QG * 10 + KS
// for attn_qg, or 1 for attn_fwd), set by hexlib_gpu_attention_override.
std::atomic<int> g_attn_form{0};

// attn_qg with QG query groups and KS key splits; false for a form not built.
bool launch_qg(int qg, int ks, const f16 *Q, const f16 *K, long long ldqk, const f16 *V, long long ldv, f16 *O,
               int T, int H, int D, int batch, float sl2e) {
    const long long tasks = (long long) ((T + 32 * qg - 1) / (32 * qg)) * batch * H;
    if (tasks > 0x7fffffffLL) return false;
    const dim3 grid((unsigned) tasks);
#define HX_QG(D_, QG_, KS_)                                                                             \
    if (D == D_ && qg == QG_ && ks == KS_) {                                                            \
        HX_LAUNCH((attn_qg<D_, QG_, KS_>), grid, dim3(64 * QG_ * KS_), 0, Q, K, ldqk, V, ldv, O, T, H, sl2e); \
        return true;                                                                                    \
    }
    HX_QG(64, 4, 1)
    HX_QG(64, 2, 1)
    HX_QG(64, 2, 2)
    HX_QG(64, 4, 2)
    HX_QG(64, 1, 4)
    HX_QG(32, 4, 1)
    HX_QG(32, 2, 2)
#undef HX_QG
    return false;
}

// The automatic choice: the shared-K/V form wherever its grid still fills the
// chip, else 0 (attn_fwd).
// From a sweep on MI355X (12 heads of 64): 256 tokens at batch 32, 18.6 us
// against 39.0 (the per-wave-tiles kernel); at 784 and 1024 tokens of one
// image the per-wave-tiles kernel is as fast (12.1 us, 14.6 us).
int qg_auto(int T, int H, int batch) {
    const long long heads = (long long) batch * H;
    if (heads * ((T + 127) / 128) >= 2 * CUS) return 41;
    // one image of up to 256 tokens (12 heads: 96 workgroups): four key splits
    // of one 32-query group, each split one stage (4.83 us against 5.07)
    if (T <= 256 && heads * ((T + 31) / 32) <= CUS / 2) return 14;
    // a few images (batch 4: 48 heads): two key splits of two query groups
    // share each stage (5.8 us against 6.5)
    if (T <= 512 && heads * ((T + 63) / 64) >= CUS / 2) return 22;
    return 0;
}

void launch(const hexlib_hf *q, const hexlib_hf *k, long long ldqk, const hexlib_hf *v, long long ldv,
            hexlib_hf *out, int rows, int H, int D, int batch, float scale) {
    const int T = rows / batch;
    const dim3 grid((unsigned) ((T + QT - 1) / QT), (unsigned) (batch * H));
    const float sl2e = scale * 1.4426950408889634f;
    const auto *Q = reinterpret_cast<const f16 *>(q);
    const auto *K = reinterpret_cast<const f16 *>(k);
    const auto *V = reinterpret_cast<const f16 *>(v);
    auto *O = reinterpret_cast<f16 *>(out);
    const int form = g_attn_form.load();
    if (form >= 10) {
        if (launch_qg(form / 10, form % 10, Q, K, ldqk, V, ldv, O, T, H, D, batch, sl2e)) return;
    } else if (form == 0) {
        const int f = qg_auto(T, H, batch);
        if (f && launch_qg(f / 10, f % 10, Q, K, ldqk, V, ldv, O, T, H, D, batch, sl2e)) return;
    }
    // Fewer workgroups than CUs (one 256-token image): 8 waves split each
    // query tile's keys, halving every wave's serial chain; otherwise 4, which
    // keeps two workgroups per CU.
    const bool wide = (long long) grid.x * grid.y < CUS;
    if (D == 64 && wide) HX_LAUNCH((attn_fwd<64, 8>), grid, dim3(64 * 8), 0, Q, K, ldqk, V, ldv, O, T, H, sl2e);
    else if (D == 64) HX_LAUNCH((attn_fwd<64, 4>), grid, dim3(64 * 4), 0, Q, K, ldqk, V, ldv, O, T, H, sl2e);
    else if (wide) HX_LAUNCH((attn_fwd<32, 8>), grid, dim3(64 * 8), 0, Q, K, ldqk, V, ldv, O, T, H, sl2e);
    else HX_LAUNCH((attn_fwd<32, 4>), grid, dim3(64 * 4), 0, Q, K, ldqk, V, ldv, O, T, H, sl2e);
}

bool dims_ok(int rows, int H, int D, int batch) {
    return rows > 0 && H > 0 && batch > 0 && rows % batch == 0 && (D == 32 || D == 64) &&
           (long long) batch * H <= 65535;
}

}  // namespace

extern "C" int hexlib_gpu_attention_override(int form) {
    const bool ok = form == 0 || form == 1 || form == 41 || form == 21 || form == 22 || form == 42 || form == 14;
    if (!ok) return HEXLIB_DSP_ERR_INVAL_PARAMS;
    g_attn_form = form;
    return HEXLIB_DSP_OK;
}

extern "C" void attention_fp16(const hexlib_hf *q, const hexlib_hf *k, const hexlib_hf *v,
                               hexlib_hf *out, int rows, int H, int D, int batch, float scale) {
    if (!q || !k || !v || !out || !dims_ok(rows, H, D, batch)) return;
    if (!hx::aligned(q, 16) || !hx::aligned(k, 16) || !hx::aligned(v, 16) || !hx::aligned(out, 16)) return;
    const long long hd = (long long) H * D;
    launch(q, k, hd, v, hd, out, rows, H, D, batch, scale);
}

extern "C" void attention_qk_v_fp16(const hexlib_hf *qk, const hexlib_hf *qkv, hexlib_hf *out,
                                    int rows, int H, int D, int batch, float scale) {
    if (!qk || !qkv || !out || !dims_ok(rows, H, D, batch)) return;
    if (!hx::aligned(qk, 16) || !hx::aligned(qkv, 16) || !hx::aligned(out, 16)) return;
    const long long hd = (long long) H * D;
    launch(qk, qk + hd, 2 * hd, qkv + 2 * hd, 3 * hd, out, rows, H, D, batch, scale);
}

extern "C" void attention_qkv_fp16(const hexlib_hf *qkv, hexlib_hf *out, int rows, int H, int D, int batch,
                                   float scale) {
    if (!qkv || !out || !dims_ok(rows, H, D, batch)) return;
    if (!hx::aligned(qkv, 16) || !hx::aligned(out, 16)) return;
    const long long hd = (long long) H * D;
    launch(qkv, qkv + hd, 3 * hd, qkv + 2 * hd, 3 * hd, out, rows, H, D, batch, scale);
}
