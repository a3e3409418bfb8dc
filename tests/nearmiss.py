"""Planted mistakes: plausible WRONG restatements of the hot-path kernels,
each one the reference's own near-miss (`kernels/<k>/nearmiss_*.c`), written
in numpy on the CPU from the mistake each file describes. They exist only to
be rejected: the tests show that each one fails the check the GPU parity test
of that kernel applies -- the `close_f16` bound, or bit-equality where the GPU
test is bit-exact -- on that test's own inputs, so a GPU kernel carrying the
mistake could not pass it. Test infrastructure only; nothing here is ever a
reference for a kernel.
"""
from __future__ import annotations

import numpy as np

from oracle import kernels as K
from oracle.quant import dequantize_q4_0_fp16

H = np.float16
F = np.float32


def matmul_fp16_accumulate(A, B):
    """`kernels/matmul_fp16/nearmiss_fp16_accumulate.c`: the K-reduction's
    running sum is fp16, rounded after every multiply-add."""
    A32, B32 = A.astype(F), B.astype(F)
    acc = np.zeros((A.shape[0], A.shape[1], B.shape[2]), H)
    for k in range(A.shape[2]):
        acc = (acc.astype(F) + A32[:, :, k, None] * B32[:, None, k, :]).astype(H)
    return acc


def _act_ref(x, act):
    x = x.astype(np.float64)
    if act == 0:
        return x
    if act == 1:
        return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))
    from math import erf
    return 0.5 * x * (1.0 + np.vectorize(erf)(x / np.sqrt(2.0)))


def epilogue_fp16_accumulation(a, w_dense, bias, act):
    """`kernels/matmul_epilogue_fp16/nearmiss_fp16_accumulation.c`: the dot
    product's running sum is fp16; bias and activation then follow as in the
    correct kernel. `w_dense` is the [K, N] weight as the kernel multiplies it
    (dequantized and rounded to fp16)."""
    a32, w32 = a.astype(F), w_dense.astype(F)
    acc = np.zeros((a.shape[0], w_dense.shape[1]), H)
    for k in range(a.shape[1]):
        acc = (acc.astype(F) + a32[:, k, None] * w32[None, k, :]).astype(H)
    return _act_ref(acc.astype(np.float64) + bias, act).astype(H)


def epilogue_bias_after_activation(a, w_dense, bias, act):
    """`kernels/matmul_epilogue_fp16/nearmiss_bias_after_activation.c`:
    act(a @ w) + bias instead of act(a @ w + bias)."""
    acc = a.astype(np.float64) @ w_dense.astype(np.float64)
    return (_act_ref(acc, act) + bias).astype(H)


def dequant_scale_off_by_one_block(w_bytes: bytes, K: int, N: int):
    """`kernels/matmul_epilogue_fp16/nearmiss_scale_off_by_one_block.c`: the
    codes of block (k, bb) of the N-blocked q4_0 weight are dequantized with
    the scale of block (k, bb - 1) (block 0 borrows the row's last block's).
    Returns the [K, N] fp16 weight it would multiply with."""
    blk = np.frombuffer(w_bytes, np.uint8).reshape(K, N // 32, 18)
    d = blk[:, :, :2].copy().view(H).astype(F)[:, :, 0]          # [K, N/32]
    d_wrong = np.roll(d, 1, axis=1)
    qs = blk[:, :, 2:]
    codes = np.concatenate([qs & 15, qs >> 4], axis=2).astype(F) - 8.0   # [K, N/32, 32]
    return (codes * d_wrong[:, :, None]).astype(H).reshape(K, N)


def softmax_sum_fp16(x):
    """`kernels/softmax_fp16/nearmiss_sum_fp16.c`: exp of the max-shifted
    scores in fp32, but the denominator summed in fp16, one term at a time."""
    xf = x.astype(F)
    e = np.exp(xf - xf.max(-1, keepdims=True))
    s = np.zeros(x.shape[0], H)
    for c in range(x.shape[1]):
        s = (s.astype(F) + e[:, c]).astype(H)
    return (e / s.astype(F)[:, None]).astype(H)


def softmax_no_max_subtraction(x):
    """`kernels/softmax_fp16/nearmiss_no_max_subtraction.c`: exp(x) / sum,
    with no max subtracted first (overflows to inf, then NaN)."""
    with np.errstate(over="ignore", invalid="ignore"):
        e = np.exp(x.astype(F))
        return (e / e.sum(-1, keepdims=True)).astype(H)


def rmsnorm_no_eps(x, w, eps):
    """`kernels/rmsnorm_fp16/nearmiss_no_eps.c`: eps dropped from the
    denominator."""
    xf = x.astype(F)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = 1.0 / np.sqrt((xf * xf).mean(-1, keepdims=True))
    return (xf * inv * w.astype(F)).astype(H)


def rope_fp16_products(x, cos, sin):
    """`kernels/rope_2d_fp16/nearmiss_fp16_accumulate.c`: each product rounded
    to fp16 before the two are combined."""
    half = x.shape[-1] // 2
    xf = x.astype(F)
    c, s = cos[:, None, :], sin[:, None, :]
    x0, x1 = xf[..., :half], xf[..., half:]
    p0, q0 = (x0 * c[..., :half]).astype(H).astype(F), (x1 * s[..., :half]).astype(H).astype(F)
    p1, q1 = (x1 * c[..., half:]).astype(H).astype(F), (x0 * s[..., half:]).astype(H).astype(F)
    return np.concatenate([p0 - q0, p1 + q1], axis=-1).astype(H)


def rope_table_by_head(x, cos, sin):
    """`kernels/rope_2d_fp16/nearmiss_table_indexed_by_head.c`: the table row
    is the head index instead of the token index."""
    T, Hh, D = x.shape
    out = np.empty_like(x)
    for h in range(Hh):
        out[:, h] = K.rope_2d_fp16(x[:, h:h + 1], np.broadcast_to(cos[h], (T, D)).copy(),
                                   np.broadcast_to(sin[h], (T, D)).copy())[:, 0]
    return out


def patchify_merge_ignored(img, patch, merge, grid_h, grid_w):
    """`kernels/patchify_fp32/nearmiss_merge_ignored.c`: tokens in plain raster
    order (gh * grid_w + gw), the merge blocks never formed."""
    C, T = img.shape[0], img.shape[1]
    rows = []
    for gh in range(grid_h):
        for gw in range(grid_w):
            blk = img[:, :, gh * patch:(gh + 1) * patch, gw * patch:(gw + 1) * patch]
            rows.append(blk.reshape(C * T * patch * patch))
    return np.stack(rows).astype(F)


def dense_q4_nblocked(w_bytes: bytes, K: int, N: int):
    """The [K, N] fp16 weight an N-blocked q4_0 tensor dequantizes to."""
    return dequantize_q4_0_fp16(w_bytes, (K, N))


# ---- structural mistakes: tails, types, lane order, strides ----------------------------
# The reference's kernels work in 128-byte vectors: 64 fp16 lanes, or 32 fp32.
LANES16 = 64
LANES32 = 32


def add_drops_the_tail(a, b, out):
    """`kernels/add_fp16/nearmiss_drops_the_tail.c`: only whole 64-lane
    vectors are written; the last n % 64 outputs keep what `out` held."""
    full = a.size - a.size % LANES16
    y = np.array(out, H, copy=True)
    y[:full] = K.add_fp16(a[:full], b[:full])
    return y


def add_as_integers(a, b):
    """`kernels/add_fp16/nearmiss_integer_add.c`: the two fp16 bit patterns
    added as wrapping 16-bit integers."""
    s = a.view(np.int16).astype(np.int32) + b.view(np.int16).astype(np.int32)
    return (s & 0xFFFF).astype(np.uint16).view(H)


def scale_drops_the_tail(x, factor, out):
    """`kernels/scale_fp16/nearmiss_drops_the_tail.c`: as add's."""
    full = x.size - x.size % LANES16
    y = np.array(out, H, copy=True)
    y[:full] = K.scale_fp16(x[:full], factor)
    return y


def scale_splats_the_number(x, factor):
    """`kernels/scale_fp16/nearmiss_splats_the_numeric_value.c`: the factor
    converted to an integer, whose low 16 bits are then splatted as the fp16
    multiplier (0.125 -> 0 -> +0.0)."""
    f = np.array([int(factor) & 0xFFFF], np.uint16).view(H)[0]
    return (x.astype(F) * F(f)).astype(H)


def _cast_vectors(x, per_vector):
    """Whole 64-output vectors by `per_vector(v)` (the 64 fp16 values of
    output vector v); the tail converted element by element, as every cast
    near-miss does."""
    y = K.cast_f32_f16(x).copy()
    for v in range(x.size // LANES16):
        y[v * LANES16:(v + 1) * LANES16] = per_vector(v)
    return y


def cast_forgets_the_deal(x):
    """`kernels/cast_f32_f16/nearmiss_forgets_the_deal.c`: each output vector
    comes out interleaved -- lane 2j holds element j of its low 32 inputs,
    lane 2j + 1 element j of its high 32 -- because the de-interleave after
    the narrowing is missing."""
    h = K.cast_f32_f16(x)

    def vec(v):
        lo, hi = h[v * 64:v * 64 + 32], h[v * 64 + 32:v * 64 + 64]
        return np.stack([lo, hi], axis=1).reshape(64)
    return _cast_vectors(x, vec)


def cast_one_input_vector_per_output(x):
    """`kernels/cast_f32_f16/nearmiss_reads_one_vector_per_output.c`: output
    vector i narrows input vector i (32 floats) twice, so each of x[32 i ..
    32 i + 31] lands in two adjacent lanes and the second half of x is never
    read."""
    h = K.cast_f32_f16(x)
    return _cast_vectors(x, lambda v: np.repeat(h[v * 32:v * 32 + 32], 2))


def cast_swapped_halves(x):
    """`kernels/cast_f32_f16/nearmiss_swapped_halves.c`: the two 32-lane
    halves of every output vector exchanged."""
    h = K.cast_f32_f16(x)
    return _cast_vectors(x, lambda v: np.concatenate([h[v * 64 + 32:v * 64 + 64], h[v * 64:v * 64 + 32]]))


def layernorm_permuted_affine(x, w, b, eps):
    """`kernels/layernorm_fp16/nearmiss_permuted_affine_lanes.c`: within each
    64-column vector the normalised values stay in place but the weight and
    bias are read in the widening's lane order -- column 2j takes parameter j,
    column 2j + 1 parameter 32 + j -- so w and b meet the wrong columns (the
    mean and variance are still right; the tail columns are unaffected)."""
    C = x.shape[-1]
    perm = np.arange(C)
    for v in range(C // LANES16):
        u = np.arange(64)
        perm[v * 64 + u] = v * 64 + np.where(u % 2 == 0, u // 2, 32 + u // 2)
    return K.layernorm_fp16(x, w[perm], b[perm], eps)


def rmsnorm_mean_not_rms(x, w, eps):
    """`kernels/rmsnorm_fp16/nearmiss_mean_not_rms.c`: normalised by the mean
    of x, not of x squared (NaN where that mean is below -eps)."""
    xf = x.astype(F)
    with np.errstate(invalid="ignore"):
        inv = F(1.0) / np.sqrt(xf.mean(-1, keepdims=True, dtype=F) + F(eps))
        return (xf * inv * w.astype(F)).astype(H)


def _rope_parts(x, cos, sin):
    half = x.shape[-1] // 2
    xf = x.astype(F)
    c, s = cos[:, None, :].astype(F), sin[:, None, :].astype(F)
    return half, xf[..., :half], xf[..., half:], c, s


def rope_negated_term(x, cos, sin):
    """`kernels/rope_2d_fp16/nearmiss_negated_term.c`: the first half's
    x[i + half] * sin term added instead of subtracted."""
    half, x0, x1, c, s = _rope_parts(x, cos, sin)
    y0 = x0 * c[..., :half] + x1 * s[..., :half]
    y1 = x1 * c[..., half:] + x0 * s[..., half:]
    return np.concatenate([y0, y1], axis=-1).astype(H)


def rope_partial_rotation(x, cos, sin, fill):
    """`kernels/rope_2d_fp16/nearmiss_partial_rotation.c`: only the first
    r = D / 2 columns rotated, in pairs r / 2 apart (integer halves; table
    columns 0 .. 2 (r / 2) - 1), columns from r on copied through; an odd r
    leaves column r - 1 unwritten (`fill`)."""
    D = x.shape[-1]
    r = D // 2
    q = r // 2
    y = np.full_like(x, fill)
    y[..., r:] = x[..., r:]
    if q:
        y[..., :2 * q] = K.rope_2d_fp16(x[..., :2 * q], np.ascontiguousarray(cos[:, :2 * q]),
                                        np.ascontiguousarray(sin[:, :2 * q]))
    return y


def rope_swapped_tables(x, cos, sin):
    """`kernels/rope_2d_fp16/nearmiss_swapped_cos_sin.c`: the sin table used
    as cos and the cos table as sin."""
    return K.rope_2d_fp16(x, sin, cos)


def _scatter_rows(x_rows, dst_rows, n_rows, fill):
    """Rows written at computed row indices (later writes win, indices past
    the output skipped): what a kernel with a wrong output stride leaves."""
    y = np.full((n_rows,) + x_rows.shape[1:], fill, x_rows.dtype)
    for src, dst in enumerate(dst_rows):
        if 0 <= dst < n_rows:
            y[dst] = x_rows[src]
    return y


def transpose_th_plain_copy(x):
    """`kernels/transpose_th_fp16/nearmiss_plain_copy.c`: the bytes copied
    unchanged."""
    return x.reshape(x.shape[1], x.shape[0], x.shape[2]).copy()


def transpose_th_swapped_stride(x, fill):
    """`kernels/transpose_th_fp16/nearmiss_swapped_stride.c`: output row
    h * H + t instead of h * T + t (identical when T == H)."""
    T, Hh, D = x.shape
    src = x.reshape(T * Hh, D)
    dst = [h * Hh + t for t in range(T) for h in range(Hh)]
    return _scatter_rows(src, dst, T * Hh, fill).reshape(Hh, T, D)


def transpose_hd_plain_copy(x):
    """`kernels/transpose_hd_fp16/nearmiss_plain_copy.c`."""
    return x.reshape(x.shape[0], x.shape[2], x.shape[1]).copy()


def transpose_hd_swapped_stride(x, fill):
    """`kernels/transpose_hd_fp16/nearmiss_swapped_stride.c`: element
    (b, t, d) written at (b * D + d) * D + t instead of (b * D + d) * T + t."""
    B, T, D = x.shape
    b, t, d = np.meshgrid(np.arange(B), np.arange(T), np.arange(D), indexing="ij")
    i = ((b * D + d) * D + t).ravel()
    keep = i < B * D * T
    y = np.full(B * D * T, fill, x.dtype)
    y[i[keep]] = x.ravel()[keep]
    return y.reshape(B, D, T)


def transpose_hd_batch_last(x):
    """`kernels/transpose_hd_fp16/nearmiss_wrong_batch_stride.c`: y walked
    as (T, D, B), batch last, instead of (B, D, T)."""
    B, T, D = x.shape
    return np.ascontiguousarray(np.transpose(x, (1, 2, 0))).reshape(B, D, T)


def matmul_batch0_a(A, B):
    """`kernels/matmul_fp16/nearmiss_wrong_batch_stride.c`: every batch
    multiplies batch 0's A (its offset built from the row loop's variables);
    B and C are offset correctly."""
    return K.matmul_fp16(np.broadcast_to(A[:1], A.shape).copy(), B)


def patchify_channel_time_swapped(img, patch, merge, grid_h, grid_w, batch=1):
    """`kernels/patchify_fp32/nearmiss_channel_temporal_swap.c`: the source
    plane of (c, t) taken as t * C + c, as if the image were [T, C, H, W]."""
    bc, T, Hh, W = img.shape
    C = bc // batch
    planes = img.reshape(batch, C * T, Hh, W)
    wrong = np.empty_like(planes)
    for c in range(C):
        for t in range(T):
            wrong[:, c * T + t] = planes[:, t * C + c]
    return K.patchify_fp32(wrong.reshape(bc, T, Hh, W), patch, merge, grid_h, grid_w, batch)


def patchify_patch_transposed(img, patch, merge, grid_h, grid_w, batch=1):
    """`kernels/patchify_fp32/nearmiss_patch_interior_swap.c`: feature
    ((c T + t) p + pw) p + ph -- each patch transposed inside its row."""
    good = K.patchify_fp32(img, patch, merge, grid_h, grid_w, batch)
    n = good.shape[0]
    return np.ascontiguousarray(good.reshape(n, -1, patch, patch).transpose(0, 1, 3, 2)).reshape(n, -1)
