/* include/hexlib_gpu.h -- the C ABI of libhexlib_gpu.so (MI355X / gfx950).
 *
 * Three layers, each a drop-in for one reference interface:
 *
 *  1. Per-kernel functions with the exact names, argument orders and scalar
 *     types of the reference's kernel_api.h headers. Pointers are DEVICE
 *     pointers; work is enqueued on the library's current HIP stream
 *     (hexlib_gpu_set_stream) and the call returns without waiting. Invalid
 *     dimensions make the call a silent no-op, as in the reference.
 *  2. The entry adapters `int <kernel>_entry(const hexlib_args *)` and the
 *     dispatch table `hexlib_kernel_table[]`, keyed by the reference's wire
 *     KIND_ID (1-12) plus appended ids 13-25. Generated from the host's
 *     RunnerSpec table (hexlib_amd/exec/genentry.py).
 *  3. A session with the reference IDL's lifecycle (open/start/mmap/invoke/
 *     stop/close/hwinfo) that validates a batch blob on the host, resolves
 *     tensors through registered device buffers (no address ever crosses the
 *     wire), and runs every op -- optionally captured once into a hipGraph
 *     and replayed.
 *
 * hexlib_hf is IEEE binary16 storage, bit-compatible with the reference's
 * `typedef __fp16 hexlib_hf`; it is only ever passed by pointer.
 */
#ifndef HEXLIB_GPU_H
#define HEXLIB_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t hexlib_hf;

/* ---- wire constants: hexlib/runtime/skel/hexlib_dsp.h:21-29 ---- */
#define HEXLIB_BATCH_MAGIC   0x424C5848u
#define HEXLIB_BATCH_VERSION 1u
#define HEXLIB_MAX_BUFS      8
#define HEXLIB_MAX_SRC       6
#define HEXLIB_MAX_DST       4
#define HEXLIB_MAX_PARAMS    16
/* The DSP bounds a blob at 512 tensors because its working copies are static
 * (skel_dispatch.c:137-147); the GPU session keeps them on the heap and accepts
 * up to 4096, so batched encoder plans (about 600 tensors at batch 32) fit.
 * The wire layout does not depend on this bound. */
#define HEXLIB_MAX_TENSORS   4096
#define HEXLIB_MAX_MMAPS     32
#define HEXLIB_NO_TENSOR     0xFFFFu

/* Status codes: hexlib/runtime/skel/hexlib_dsp.h:34-54. OK is 1. */
enum hexlib_dsp_status {
    HEXLIB_DSP_OK = 1,
    HEXLIB_DSP_ERR_INTERNAL = 2,
    HEXLIB_DSP_ERR_BAD_MAGIC = 3,
    HEXLIB_DSP_ERR_BAD_VERSION = 4,
    HEXLIB_DSP_ERR_TRUNCATED = 5,
    HEXLIB_DSP_ERR_INVAL_PARAMS = 6,
    HEXLIB_DSP_ERR_UNMAPPED = 7,
    HEXLIB_DSP_ERR_NO_MMAP_SLOT = 8,
    HEXLIB_DSP_ERR_MMAP_FAILED = 9,
    HEXLIB_DSP_ERR_NO_KERNEL = 10,
    HEXLIB_DSP_ERR_VTCM_TOO_SMALL = 11,
    HEXLIB_DSP_ERR_VTCM_RECLAIMED = 12,
    HEXLIB_DSP_ERR_REQUIRES = 13,
    HEXLIB_DSP_ERR_NOT_STARTED = 14,
    HEXLIB_DSP_ERR_CACHE = 15
};

/* Layout ids: hexlib_dsp.h:168-170, plus 3 = q4_0 grouped along K of W^T,
 * 4 = a [K, N] weight stored transposed ([N, K], K contiguous) and 5 = layout
 * 4 with the rows of each rope head pair-interleaved (row 2i of a head holds
 * feature i, row 2i + 1 feature i + D/2). */
#define HEXLIB_LAYOUT_ROW_MAJOR     0u
#define HEXLIB_LAYOUT_TILED_32X32   1u
#define HEXLIB_LAYOUT_Q4_0_REPACKED 2u
#define HEXLIB_LAYOUT_Q4_0_KGROUP   3u
#define HEXLIB_LAYOUT_COL_MAJOR     4u
#define HEXLIB_LAYOUT_COL_MAJOR_ROPE 5u
#define HEXLIB_LAYOUT_Q8_0_KGROUP   6u
#define HEXLIB_LAYOUT_Q8_0_KGROUP_ROPE 7u

/* Dtype ids: hexlib/runtime/wire.py:61. */
#define HEXLIB_DTYPE_FP32  0u
#define HEXLIB_DTYPE_FP16  1u
#define HEXLIB_DTYPE_Q4_0  2u
#define HEXLIB_DTYPE_INT32 3u
#define HEXLIB_DTYPE_Q8_0  4u

/* Wire structs: byte-identical to hexlib_dsp.h:144-197. `base` and `data`
 * are resolver scratch; the host writes 0 and the library never reads them. */
struct hexlib_batch_hdr {
    uint32_t magic, version, total_size, n_bufs, n_tensors, n_ops;
    uint32_t off_bufs, off_tensors, off_ops, flags;
};
struct hexlib_buf_desc {
    uint64_t base;
    uint64_t size;
    uint32_t fd;
    uint32_t flags;
};
struct hexlib_tensor {
    uint32_t bi, offset, nbytes, dtype, layout;
    uint32_t ne[4];
    uint32_t data, pad;
};
struct hexlib_op_desc {
    uint32_t kind;
    uint32_t flags;
    int32_t  params[HEXLIB_MAX_PARAMS];
    uint16_t src[HEXLIB_MAX_SRC];
    uint16_t dst[HEXLIB_MAX_DST];
};
struct hexlib_batch_rsp_hdr {
    uint32_t magic, version, status, n_ops;
    uint64_t cycles_total;   /* GPU nanoseconds (TIMED invokes), else 0 */
    uint32_t arch;           /* 950 */
    uint32_t pad;
};
struct hexlib_op_result {
    uint32_t kind;
    uint32_t status;
    uint64_t cycles;         /* GPU nanoseconds (TIMED invokes), else 0 */
};

/* Kernel entry ABI: hexlib_dsp.h:186-198. `vtcm`/`vtcm_size` are always
 * NULL/0 here: each kernel sizes its own LDS tiles statically. */
typedef struct {
    void       *buf[HEXLIB_MAX_BUFS];
    uint32_t    ne[HEXLIB_MAX_BUFS][4];
    uint32_t    dtype[HEXLIB_MAX_BUFS];
    uint32_t    layout[HEXLIB_MAX_BUFS];
    uint32_t    n_buf;
    uint8_t    *vtcm;
    size_t      vtcm_size;
    const void *params;
    uint32_t    n_threads;
} hexlib_args;

typedef int (*hexlib_kernel_fn)(const hexlib_args *);

struct hexlib_kernel_entry {
    uint32_t         kind;
    const char      *name;
    hexlib_kernel_fn fn;
};

extern const struct hexlib_kernel_entry hexlib_kernel_table[];
extern const uint32_t hexlib_kernel_table_len;

/* ---- 1. per-kernel API (device pointers) ---- */

/* kernels/add_fp16/kernel_api.h:35 -- y = fp16(float(a) + float(b)). */
void add_fp16(const hexlib_hf *a, const hexlib_hf *b, hexlib_hf *y, int n);
/* kernels/scale_fp16/kernel_api.h:37 -- y = fp16(float(x) * factor). */
void scale_fp16(const hexlib_hf *x, hexlib_hf *y, int n, float factor);
/* kernels/cast_f32_f16/kernel_api.h:33 -- y = fp16(x), round to nearest even. */
void cast_f32_f16(const float *x, hexlib_hf *y, int n);
/* kernels/softmax_fp16/kernel_api.h:69 -- row softmax over C, fp32 inside. */
void softmax_fp16(const hexlib_hf *x, hexlib_hf *y, int R, int C);
/* kernels/layernorm_fp16/kernel_api.h:38-39 -- biased variance, fp32 affine. */
void layernorm_fp16(const hexlib_hf *x, const float *w, const float *b,
                    hexlib_hf *y, int R, int C, float eps);
/* kernels/rmsnorm_fp16/kernel_api.h:26-27 -- x * rsqrt(mean(x^2)+eps) * w. */
void rmsnorm_fp16(const hexlib_hf *x, const hexlib_hf *w,
                  hexlib_hf *y, int R, int C, float eps);
/* kernels/rope_2d_fp16/kernel_api.h:120-121 -- split-half rotation, tables [T,D]. */
void rope_2d_fp16(const hexlib_hf *x, const float *costab, const float *sintab,
                  hexlib_hf *y, int T, int H, int D);
/* kernels/transpose_th_fp16/kernel_api.h:38 -- [T,H,D] -> [H,T,D]. */
void transpose_th_fp16(const hexlib_hf *x, hexlib_hf *y, int T, int H, int D);
/* kernels/transpose_hd_fp16/kernel_api.h:67 -- [B,T,D] -> [B,D,T]. */
void transpose_hd_fp16(const hexlib_hf *x, hexlib_hf *y, int B, int T, int D);
/* kernels/patchify_fp32/kernel_api.h:116-118 -- merge-block token order. */
void patchify_fp32(const float *img, float *out, int C, int T, int H, int W,
                   int patch, int merge, int grid_h, int grid_w);
/* kernels/matmul_fp16/kernel_api.h:77-78 -- batched A[b]@B[b], fp32 sum. */
void matmul_fp16(const hexlib_hf *A, const hexlib_hf *B, hexlib_hf *C,
                 int Bn, int M, int K, int N);
/* kernels/matmul_epilogue_fp16/kernel_api.h:188-190 -- act(a @ deq(w) + bias),
 * w = q4_0 [K, N] blocked along N; act 0 none / 1 gelu_tanh / 2 gelu_erf. */
void matmul_epilogue_fp16(const hexlib_hf *a, const unsigned char *w,
                          const float *bias, hexlib_hf *out,
                          int M, int K, int N, int act);

/* Extensions (no kernel_api.h counterpart; each serves one appended KIND_ID
 * or the batch axis of the encoder plan). */
/* [B,T,H,D] -> [B,H,T,D] (KIND 16); B = 1 is transpose_th_fp16. */
void transpose_bth_fp16(const hexlib_hf *x, hexlib_hf *y, int B, int T, int H, int D);
/* patchify over `batch` images stacked as [batch*C, T, H, W] (KIND 6 with
 * params[4] = batch; batch <= 1 is patchify_fp32). */
void patchify_fp32_batched(const float *img, float *out, int BC, int T, int H, int W,
                           int patch, int merge, int grid_h, int grid_w, int batch);
/* act(a @ w + bias), w fp16 [K, N] row-major (KIND 14). bias may be NULL. */
void matmul_epilogue_f16w_fp16(const hexlib_hf *a, const hexlib_hf *w,
                               const float *bias, hexlib_hf *out,
                               int M, int K, int N, int act);
/* act(a @ w + bias), w given transposed: wt fp16 [N, K] (layout col_major of
 * the logical [K, N] weight; KIND 17). The fast fp16 path: both operands are
 * K-contiguous. bias may be NULL. */
void matmul_epilogue_f16wt_fp16(const hexlib_hf *a, const hexlib_hf *wt,
                                const float *bias, hexlib_hf *out,
                                int M, int K, int N, int act);
/* A linear whose output columns [0, 2 * rope_heads * rope_dim) are rotated by
 * rope_2d_fp16's split-half rope in heads of rope_dim (KIND 22): the q and k
 * slots of a fused q/k/v projection. out = act(a @ w + bias) rounded to fp16,
 * then each rope head rotated with fp32 tables cos/sin and rounded again --
 * bit-identical to matmul_epilogue_f16wt_fp16 followed by rope_2d_qk_fp16.
 * wt is W^T [N, K] with the rows of each rope head pair-interleaved (layout
 * 5); bias is in feature order; cos and sin are rope_2d_fp16's [M, rope_dim]
 * tables stored transposed, [rope_dim, M] (layout 4). Requires K % 64 == 0,
 * N % 4 == 0, rope_dim % 4 == 0, 16-byte aligned a and wt, 8-byte aligned
 * out; else a no-op. */
void matmul_epilogue_f16wt_rope_fp16(const hexlib_hf *a, const hexlib_hf *wt, const float *bias,
                                     const float *costab, const float *sintab, hexlib_hf *out,
                                     int M, int K, int N, int act, int rope_heads, int rope_dim);
/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). matmul_epilogue_f16wt_fp16 with the same kernels, tiles
 * and summation order (bit-identical results), but any split-K partials live
 * in a fixed 16 MiB per-GPU device array of the library instead of its
 * grow-only workspace, and nothing is allocated. Returns HEXLIB_DSP_OK;
 * ERR_INVAL_PARAMS for invalid arguments (the other entry's silent no-op);
 * ERR_VTCM_TOO_SMALL, before any launch, when the plan's partials
 * (splits x M x N fp32) exceed the array; ERR_INTERNAL if the array's address
 * cannot be found. Calls that overlap in time on one GPU share the array and
 * race. */
int matmul_epilogue_f16wt_noalloc_fp16(const hexlib_hf *a, const hexlib_hf *wt,
                                       const float *bias, hexlib_hf *out,
                                       int M, int K, int N, int act);
/* fp16(resid + fp16(act(a @ w + bias))), w given transposed as in
 * matmul_epilogue_f16wt_fp16 (KIND 21): a linear followed by the residual
 * add_fp16 that consumes it, each rounded as the reference stores it.
 * resid [M, N] fp16 must not overlap a or wt. bias may be NULL. */
void matmul_epilogue_f16wt_res_fp16(const hexlib_hf *a, const hexlib_hf *wt, const float *bias,
                                    const hexlib_hf *resid, hexlib_hf *out,
                                    int M, int K, int N, int act);
/* act(a @ deq(w) + bias), w = q4_0 blocks of 32 along K of W^T [N, K] --
 * llama.cpp's native Linear layout (KIND 15). bias may be NULL. */
void matmul_epilogue_q4k_fp16(const hexlib_hf *a, const unsigned char *wt,
                              const float *bias, hexlib_hf *out,
                              int M, int K, int N, int act);
/* act(a @ deq(w) + bias), w = q8_0 blocks of 32 along K of W^T [N, K]
 * (34 bytes: fp16 d, 32 int8; hexlib/exec/quant.py:138-220, llama.cpp
 * block_q8_0), each dequantized weight q * d rounded to fp16 (KIND 25). No
 * reference kernel: the reference defines the q8_0 dtype
 * (hexlib/graph/ir.py:15,37-52) and wire id (hexlib/runtime/wire.py:61) but
 * multiplies it only on the CPU. Requires K % 32 == 0 and a 2-byte aligned w;
 * else a no-op. bias may be NULL. */
void matmul_epilogue_q8k_fp16(const hexlib_hf *a, const unsigned char *wt,
                              const float *bias, hexlib_hf *out,
                              int M, int K, int N, int act);
/* Fused full attention (KIND 18): out = softmax(scale * q k^T) v for each of
 * batch images and H heads; q, k, v, out are [rows = batch * T, H, D] fp16
 * (token-major, the layout rope_2d and the linears produce), D = 32 or 64.
 * Replaces the reference's scale -> transpose_hd -> matmul -> softmax ->
 * matmul chain and its transposes (hexlib/models/vit.py:185-193). fp32
 * scores and online softmax; probabilities rounded to fp16 for the P.V
 * product; output rounded once. No-op unless rows % batch == 0 and q, k, v
 * and out are 16-byte aligned. */
void attention_fp16(const hexlib_hf *q, const hexlib_hf *k, const hexlib_hf *v,
                    hexlib_hf *out, int rows, int H, int D, int batch, float scale);
/* rope_2d_fp16 on the q and k parts of a fused projection (KIND 20): qkv is
 * [rows, 3, H, D] fp16 (q, k, v of each token side by side, the output of one
 * [K, 3*H*D] linear); qk is [rows, 2, H, D] = (rope(q), rope(k)), with
 * rope_2d_fp16's arithmetic and fp32 tables cos/sin [rows, D]. */
void rope_2d_qk_fp16(const hexlib_hf *qkv, const float *costab, const float *sintab,
                     hexlib_hf *qk, int rows, int H, int D);
/* attention_fp16 with q and k taken from qk [rows, 2, H, D] (rope_2d_qk_fp16's
 * output) and v from the fused projection qkv [rows, 3, H, D] (KIND 19);
 * out [rows, H, D]. No-op unless rows % batch == 0 and every pointer is
 * 16-byte aligned. */
void attention_qk_v_fp16(const hexlib_hf *qk, const hexlib_hf *qkv, hexlib_hf *out,
                         int rows, int H, int D, int batch, float scale);
/* attention_fp16 with q, k and v all taken from one [rows, 3, H, D] tensor
 * (KIND 23): the output of matmul_epilogue_f16wt_rope_fp16. */
void attention_qkv_fp16(const hexlib_hf *qkv, hexlib_hf *out, int rows, int H, int D, int batch,
                        float scale);
/* layernorm_fp16 over the K features of each row of x [M, K] (fp32 ln_w,
 * ln_b, eps), rounded to fp16, then matmul_epilogue_f16wt_fp16 on the result
 * (KIND 24) -- one launch, bit-identical to the two calls. No reference
 * counterpart: the fusion of kernels/layernorm_fp16/kernel_api.h:38-39 into
 * the linear that consumes it. Requires 512 <= K <= 768, K % 64 == 0,
 * 16-byte aligned x and wt; else a no-op. */
void layernorm_matmul_epilogue_f16wt_fp16(const hexlib_hf *x, const float *ln_w, const float *ln_b,
                                          const hexlib_hf *wt, const float *bias, hexlib_hf *out,
                                          int M, int K, int N, int act, float eps);
/* A LayerNorm (eps) folded into the W^T linear that consumes it, one launch
 * and no normalised activation in memory (KIND 26). x [M, K] is the
 * LayerNorm's raw input; wt [N, K] holds W' = fp16(ln_w[k] * W[k][n])
 * transposed; bias2 holds 2N floats: c2[n] = bias[n] + sum_k ln_b[k] W[k][n],
 * then c1[n] = sum_k W'[k][n]. out = act(rstd (x W' - mean c1) + c2), with
 * each row's mean and one-pass variance taken in fp32 from the x tiles the
 * product reads (the K-across-waves kernel at few rows, the tiled 64x64
 * kernel above a round of its tiles, the large-tile kernel where its 128-row
 * tiles fill the GPU). Within the GEMM tolerance of
 * layernorm_fp16 followed by matmul_epilogue_f16wt_fp16, not bit-identical
 * to them. No reference counterpart: the fusion of
 * kernels/layernorm_fp16/kernel_api.h:38-39 into the linear that consumes
 * it. Requires K % 256 == 0 and 16-byte aligned x and wt; else a no-op. */
void lnfold_matmul_epilogue_f16wt_fp16(const hexlib_hf *x, const hexlib_hf *wt, const float *bias2,
                                       hexlib_hf *out, int M, int K, int N, int act, float eps);
/* The same with the q/k rope of matmul_epilogue_f16wt_rope_fp16 in the
 * epilogue (KIND 27): wt in that entry's pair-interleaved col_major_rope
 * layout, c1 and c2 indexed by output feature as its bias is. Adds that
 * entry's requirements. */
void lnfold_matmul_epilogue_f16wt_rope_fp16(const hexlib_hf *x, const hexlib_hf *wt, const float *bias2,
                                            const float *costab, const float *sintab, hexlib_hf *out,
                                            int M, int K, int N, int act, int rope_heads, int rope_dim,
                                            float eps);

/* The quantized-weight linears with the residual add that consumes them in
 * the epilogue: act(a W + bias) rounded to fp16, then fp16(resid + that) --
 * bit-identical to the plain call followed by add_fp16 (KIND 28: q4_0
 * blocked along N, the matmul_epilogue_fp16 ABI; KIND 29: q8_0 K-grouped
 * W^T, as matmul_epilogue_q8k_fp16; KIND 30: q4_0 K-grouped W^T, as
 * matmul_epilogue_q4k_fp16). resid and out are [M, N]. No reference
 * counterpart: the fusion of kernels/add_fp16/kernel_api.h into the linear
 * before it. Each has its plain form's requirements; else a no-op. */
void matmul_epilogue_res_fp16(const hexlib_hf *a, const unsigned char *w, const float *bias,
                              const hexlib_hf *resid, hexlib_hf *out, int M, int K, int N, int act);
void matmul_epilogue_q8k_res_fp16(const hexlib_hf *a, const unsigned char *wt, const float *bias,
                                  const hexlib_hf *resid, hexlib_hf *out, int M, int K, int N, int act);
void matmul_epilogue_q4k_res_fp16(const hexlib_hf *a, const unsigned char *wt, const float *bias,
                                  const hexlib_hf *resid, hexlib_hf *out, int M, int K, int N, int act);

/* matmul_epilogue_f16wt_rope_fp16 with a q8_0 weight (KIND 31): wt holds
 * the K-grouped q8_0 blocks of W^T whose rows are pair-interleaved within
 * each of the first 2 * rope_heads heads (layout 7, q8_0_kgroup_rope: the
 * col_major_rope row order, then quantized row by row). Requires K % 256 == 0
 * and the rope entry's conditions; else a no-op. No reference counterpart:
 * the fusion of kernels/rope_2d_fp16/kernel_api.h into the q8_0 linear. */
void matmul_epilogue_q8k_rope_fp16(const hexlib_hf *a, const unsigned char *wt, const float *bias,
                                   const float *costab, const float *sintab, hexlib_hf *out, int M, int K,
                                   int N, int act, int rope_heads, int rope_dim);

/* ---- 2. entry adapters (generated) ---- */
int add_fp16_entry(const hexlib_args *a);
int scale_fp16_entry(const hexlib_args *a);
int cast_f32_f16_entry(const hexlib_args *a);
int softmax_fp16_entry(const hexlib_args *a);
int layernorm_fp16_entry(const hexlib_args *a);
int rmsnorm_fp16_entry(const hexlib_args *a);
int rope_2d_fp16_entry(const hexlib_args *a);
int transpose_th_fp16_entry(const hexlib_args *a);
int transpose_hd_fp16_entry(const hexlib_args *a);
int transpose_bth_fp16_entry(const hexlib_args *a);
int patchify_fp32_batched_entry(const hexlib_args *a);
int matmul_fp16_entry(const hexlib_args *a);
int matmul_epilogue_fp16_entry(const hexlib_args *a);
int matmul_epilogue_f16w_fp16_entry(const hexlib_args *a);
int matmul_epilogue_f16wt_fp16_entry(const hexlib_args *a);
int matmul_epilogue_q4k_fp16_entry(const hexlib_args *a);
int matmul_epilogue_f16wt_res_fp16_entry(const hexlib_args *a);
int matmul_epilogue_f16wt_rope_fp16_entry(const hexlib_args *a);
int attention_qkv_fp16_entry(const hexlib_args *a);
int attention_fp16_entry(const hexlib_args *a);
int attention_qk_v_fp16_entry(const hexlib_args *a);
int rope_2d_qk_fp16_entry(const hexlib_args *a);
int layernorm_matmul_epilogue_f16wt_fp16_entry(const hexlib_args *a);
int matmul_epilogue_q8k_fp16_entry(const hexlib_args *a);
int lnfold_matmul_epilogue_f16wt_fp16_entry(const hexlib_args *a);
int lnfold_matmul_epilogue_f16wt_rope_fp16_entry(const hexlib_args *a);
int matmul_epilogue_res_fp16_entry(const hexlib_args *a);
int matmul_epilogue_q8k_res_fp16_entry(const hexlib_args *a);
int matmul_epilogue_q4k_res_fp16_entry(const hexlib_args *a);
int matmul_epilogue_q8k_rope_fp16_entry(const hexlib_args *a);

/* ---- library control ---- */
/* The stream every per-kernel call enqueues on (a hipStream_t; NULL = the
 * default stream). Process-wide. */
void  hexlib_gpu_set_stream(void *stream);
void *hexlib_gpu_get_stream(void);
/* The first HIP error any launch hit since the last call, then cleared
 * (0 = none). The per-kernel API is void, like the reference's; this is how
 * a caller learns that a launch failed. */
int   hexlib_gpu_take_error(void);
const char *hexlib_gpu_error_string(int hip_error);
const char *hexlib_gpu_status_name(int status);
/* GEMM tuning override for every later GEMM launch in the process: tile
 * bm x bn (256x128, 128x128, 64x64, 32x64, 64x32; 0x0 = heuristic), split-K count
 * (0 = heuristic, at most 16) and W^T code path (0 = automatic,
 * 1 = register-staged, 2 = direct-to-LDS, 3 = the small-M register-operand
 * kernel with tile 32x32 or 32x64, 4 = the K-across-waves kernel for
 * K % 256 == 0 (tile 64x64 selects its 64x64 form, 32x24 its 32-row form
 * with 24-column tiles on a plain fp16 W^T, else 32x32), 5 = the
 * large-tile kernel with bm in {128, 256} and bn in {128, 192, 256}, where
 * `splits` is its ring depth instead (0 = 2, at most 3; a form not built falls
 * back to the automatic choice), 7 = the 16-row MFMA kernel for K-grouped
 * q4_0 / q8_0 weights at up to 16 rows (tile 0x0; `splits` its wave count,
 * 4, 8 or 16, 0 = 8); 2 to 5 and 7 apply where their preconditions hold).
 * Returns HEXLIB_DSP_OK or ERR_INVAL_PARAMS. */
int hexlib_gpu_gemm_override(int bm, int bn, int splits, int path);
/* Tuning override (no reference counterpart) for the attention kernels'
 * form, for every later attention launch in the process: 0 = automatic,
 * 1 = the per-wave-tiles kernel (32 queries per workgroup, waves split the
 * keys), QG * 10 + KS = the shared-K/V kernel with QG 32-query groups and KS
 * key splits (41, 21, 22, 42; a form not built for the head width falls
 * back to the per-wave-tiles kernel). Returns HEXLIB_DSP_OK or
 * ERR_INVAL_PARAMS. */
int hexlib_gpu_attention_override(int form);
/* sizeof of each wire struct, in declaration order above (batch_hdr, buf_desc,
 * tensor, op_desc, rsp_hdr, op_result, hexlib_args); returns the count. */
uint32_t hexlib_gpu_struct_sizes(uint32_t *out, uint32_t cap);

/* ---- 3. session: hexlib/runtime/idl/hexlib_iface.idl:28-67 ---- */
typedef struct hexlib_gpu_ctx hexlib_gpu_ctx;

#define HEXLIB_GPU_INVOKE_DRYRUN 0x1u  /* validate + run entries, launch nothing (no HIP call) */
#define HEXLIB_GPU_INVOKE_TIMED  0x2u  /* per-op GPU ns into cycles (eager), or total (graph) */
#define HEXLIB_GPU_INVOKE_GRAPH  0x4u  /* capture the blob into a hipGraph once, replay after */
#define HEXLIB_GPU_INVOKE_NOSYNC 0x8u  /* return once enqueued; caller synchronises */

/* Host-only allocation of an idle session. */
int hexlib_gpu_open(hexlib_gpu_ctx **out);
int hexlib_gpu_close(hexlib_gpu_ctx *ctx);
/* Binds `device`, creates the session stream (default priority). */
int hexlib_gpu_start(hexlib_gpu_ctx *ctx, uint32_t sess_id, int device, uint64_t max_vmem);
int hexlib_gpu_stop(hexlib_gpu_ctx *ctx);
/* Registers device memory [dev_ptr, dev_ptr+size) under handle `fd`; blobs
 * name buffers only by fd (the analogue of fastrpc_mmap + HAP_mmap). */
int hexlib_gpu_mmap(hexlib_gpu_ctx *ctx, uint32_t fd, void *dev_ptr, uint64_t size);
int hexlib_gpu_munmap(hexlib_gpu_ctx *ctx, uint32_t fd);
int hexlib_gpu_hwinfo(hexlib_gpu_ctx *ctx, uint32_t *arch, uint32_t *n_cu,
                      uint32_t *n_threads, uint64_t *lds_per_cu);
/* hexlib_dispatch_batch (hexlib/runtime/skel/skel_dispatch.c:80-302): the
 * response is always self-describing; the return value equals its status. */
int hexlib_gpu_invoke(hexlib_gpu_ctx *ctx, const uint8_t *batch, uint32_t len,
                      uint8_t *rsp, uint32_t rsp_cap, uint32_t *rsp_len, uint32_t flags);
/* The session's stream (a hipStream_t). */
void *hexlib_gpu_session_stream(hexlib_gpu_ctx *ctx);

/* ---- 4. whole-plan files ------------------------------------------------
 * The whole-plan batch (hexlib/exec/wholeplan.py:92-357: arena layout, const
 * image and wire blob) as an on-disk artefact, replayed through
 * hexlib_gpu_invoke with no Python on the host. No reference counterpart: the
 * reference builds the batch in Python for every run
 * (hexlib/tests/test_wholeplan.py:181-183). hexlib_amd/exec/planfile.py
 * writes the files; the format is described in hexlib_amd/csrc/planfile.cpp. */
typedef struct hexlib_plan_info {
    uint32_t version, fd, n_io, n_ops;
    uint64_t arena_bytes, const_bytes, blob_bytes, data_bytes;
} hexlib_plan_info;
typedef struct hexlib_plan_io {
    char name[48];           /* the graph tensor's name, NUL-terminated */
    uint32_t role;           /* 0 = graph input, 1 = graph output */
    uint32_t dtype;          /* wire dtype id (HEXLIB_DTYPE_*) */
    uint64_t offset, nbytes; /* its bytes in the arena */
    uint32_t ne[4];
    uint64_t data_offset;    /* a stored sample input value, or UINT64_MAX */
} hexlib_plan_io;
typedef struct hexlib_gpu_plan hexlib_gpu_plan;
/* Parses and validates a plan file and dry-runs its blob against a mapping
 * of the arena (no HIP call): a status, and the sizes and op count. */
int hexlib_gpu_plan_inspect(const char *path, hexlib_plan_info *info);
/* On a started session: allocates the arena on the session's device, stages
 * the const image and the stored sample inputs, and maps the arena under the
 * blob's fd. The plan owns the arena until hexlib_gpu_plan_free. */
int hexlib_gpu_plan_load(hexlib_gpu_ctx *ctx, const char *path, hexlib_gpu_plan **out);
int hexlib_gpu_plan_info_of(const hexlib_gpu_plan *plan, hexlib_plan_info *info);
int hexlib_gpu_plan_io(const hexlib_gpu_plan *plan, uint32_t i, hexlib_plan_io *io);
/* Host bytes into input i / out of tensor i; nbytes must equal its size. */
int hexlib_gpu_plan_write(hexlib_gpu_plan *plan, uint32_t i, const void *host, uint64_t nbytes);
int hexlib_gpu_plan_read(const hexlib_gpu_plan *plan, uint32_t i, void *host, uint64_t nbytes);
/* hexlib_gpu_invoke of the plan's blob (same flags, same response). */
int hexlib_gpu_plan_run(hexlib_gpu_plan *plan, uint32_t flags, uint8_t *rsp, uint32_t rsp_cap,
                        uint32_t *rsp_len);
int hexlib_gpu_plan_free(hexlib_gpu_plan *plan);

#ifdef __cplusplus
}
#endif

#endif /* HEXLIB_GPU_H */
