"""Planted mistakes: plausible WRONG restatements of the hot-path kernels,
each one the reference's own near-miss (`kernels/<k>/nearmiss_*.c`), written
in numpy on the CPU. They exist only to be rejected: the tests show that each
one fails the same `close_f16` bound the GPU parity tests apply, on the same
inputs, so a GPU kernel carrying that mistake could not pass them. Test
infrastructure only; nothing here is ever a reference for a kernel.
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
