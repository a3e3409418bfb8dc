"""Per-kernel contracts from each `kernels/<k>/kernel_api.h` + `baseline.c`,
vectorised in numpy (test infrastructure only).

Inputs and outputs are numpy arrays in storage dtype (float16 for `hexlib_hf`,
float32 for `float`, uint8 bytes for q4_0). Reductions accumulate in float64
and round once to fp16: the baseline's float32 sequential sum differs from that
by far less than the harness tolerances, and a float64 sum is independent of
any summation order the GPU picks.

| function             | restates                                          | pinned by |
|----------------------|---------------------------------------------------|-----------|
| add_fp16             | kernels/add_fp16/baseline.c:9-15                  | _ref bit-exact |
| scale_fp16           | kernels/scale_fp16/baseline.c:9-13                | _ref bit-exact |
| cast_f32_f16         | kernels/cast_f32_f16/baseline.c:8-12              | _ref bit-exact |
| softmax_fp16         | kernels/softmax_fp16/baseline.c:17-45             | _ref (0.01,1e-3); rows sum to 1 |
| layernorm_fp16       | kernels/layernorm_fp16/baseline.c:11-35           | _ref (0.02,1e-3); mean 0 / var 1 |
| rmsnorm_fp16         | kernels/rmsnorm_fp16/baseline.c:6-19              | _ref (0.02,1e-3); unit RMS |
| rope_2d_fp16         | kernels/rope_2d_fp16/baseline.c:17-40             | _ref bit-exact; identity tables |
| transpose_th_fp16    | kernels/transpose_th_fp16/baseline.c:8-17         | _ref bit-exact; np.transpose |
| transpose_hd_fp16    | kernels/transpose_hd_fp16/baseline.c:8-17         | _ref bit-exact; np.transpose |
| patchify_fp32        | kernels/patchify_fp32/baseline.c:14-55            | _ref bit-exact; golden patches_upstream |
| matmul_fp16          | kernels/matmul_fp16/baseline.c:13-31              | _ref (1e-2,1e-3); float64 brute force |
| matmul_epilogue_fp16 | kernels/matmul_epilogue_fp16/baseline.c:27-97     | _ref (0.01,3e-4) |
| matmul_epilogue_f16w | hexlib/graph/opdefs/fused.py:44-53 with fp16 w    | reduces to matmul_epilogue_fp16 on dequantized weights |
| matmul_q4k           | q4_0 blocks along K of W^T, same numerics as q4_0 | reduces to matmul_epilogue_fp16 via a block transpose |
| matmul_q8k           | q8_0 blocks along K of W^T, weights rounded to fp16 | dequantize_q8_0 pinned by the scalar ggml transcription |
| attention_fp16       | hexlib/models/vit.py:185-193 chain, fused         | equals the composition of the registry references; uniform / one-hot closed forms |
| rope_2d_qk_fp16      | rope_2d_fp16 on the q, k slots of a fused qkv     | rope_2d_fp16 (pinned bit-exact) per slot |
| attention_qk_v_fp16  | attention_fp16 on strided q, k, v                 | attention_fp16 |
| permute_rope_rows    | the col_major_rope weight layout (row order only) | per-head halves land on even / odd rows; v rows untouched |
"""
from __future__ import annotations

import math

import numpy as np

from oracle.quant import dequantize_q4_0_fp16, dequantize_q8_0_fp16

ACT_NONE, ACT_GELU_TANH, ACT_GELU_ERF = 0, 1, 2
_erf = np.vectorize(math.erf, otypes=[np.float64])


def _f32(x):
    return np.asarray(x).astype(np.float32)


def add_fp16(a, b):
    return (_f32(a) + _f32(b)).astype(np.float16)


def scale_fp16(x, factor):
    return (_f32(x) * np.float32(factor)).astype(np.float16)


def cast_f32_f16(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16)


def softmax_fp16(x):
    xf = _f32(x).astype(np.float64)
    e = np.exp(xf - xf.max(axis=-1, keepdims=True))
    return (e / e.sum(axis=-1, keepdims=True)).astype(np.float16)


def layernorm_fp16(x, w, b, eps):
    xf = _f32(x).astype(np.float64)
    mean = xf.mean(axis=-1, keepdims=True)
    var = ((xf - mean) ** 2).mean(axis=-1, keepdims=True)
    inv = 1.0 / np.sqrt(var + np.float64(np.float32(eps)))
    return ((xf - mean) * inv * _f32(w) + _f32(b)).astype(np.float16)


def rmsnorm_fp16(x, w, eps):
    xf = _f32(x).astype(np.float64)
    inv = 1.0 / np.sqrt((xf * xf).mean(axis=-1, keepdims=True) + np.float64(np.float32(eps)))
    return (xf * inv * _f32(w)).astype(np.float16)


def rope_2d_fp16(x, cos, sin):
    """x [T, H, D] fp16; cos/sin [T, D] fp32. float32 products, each rounded,
    then one float32 add -- the same operation order as the baseline."""
    xf = _f32(x)
    half = xf.shape[-1] // 2
    c, s = _f32(cos)[:, None, :], _f32(sin)[:, None, :]
    x0, x1 = xf[..., :half], xf[..., half:]
    y0 = x0 * c[..., :half] - x1 * s[..., :half]
    y1 = x1 * c[..., half:] + x0 * s[..., half:]
    return np.concatenate([y0, y1], axis=-1).astype(np.float16)


def transpose_th_fp16(x):
    return np.ascontiguousarray(np.transpose(x, (1, 0, 2)))


def transpose_hd_fp16(x):
    return np.ascontiguousarray(np.transpose(x, (0, 2, 1)))


def transpose_bth_fp16(x):
    return np.ascontiguousarray(np.transpose(x, (0, 2, 1, 3)))


def patchify_fp32(img, patch, merge, grid_h, grid_w, batch=1):
    """img [batch*C,T,H,W]; out[token][feat] with
    token = ((bh*Bw + bw)*merge + mh)*merge + mw, feat = ((c*T + t)*p + ph)*p + pw."""
    a = np.asarray(img, dtype=np.float32)
    bc, t, h, w = a.shape
    b, c = batch, bc // batch
    a = a.reshape(b, c, t, h, w)
    p, m = patch, merge
    x = a.reshape(b, c, t, grid_h // m, m, p, grid_w // m, m, p)
    x = x.transpose(0, 3, 6, 4, 7, 1, 2, 5, 8)
    return np.ascontiguousarray(x).reshape(b * grid_h * grid_w, c * t * p * p)


def _act(r, act):
    if act == ACT_GELU_TANH:
        return 0.5 * r * (1.0 + np.tanh(0.7978845608028654 * (r + 0.044715 * r ** 3)))
    if act == ACT_GELU_ERF:
        return 0.5 * r * (1.0 + _erf(r / math.sqrt(2.0)))
    return r


def matmul_fp16(A, B):
    """Batched [Bn,M,K] @ [Bn,K,N]; float64 accumulation, one fp16 rounding."""
    return np.matmul(_f32(A).astype(np.float64), _f32(B).astype(np.float64)).astype(np.float16)


def gemm_epilogue(a, w_dense, bias, act):
    """act(a @ w + bias) with an already-dense weight whose values the kernel
    multiplies with; float64 sum, bias before the activation, one rounding."""
    r = _f32(a).astype(np.float64) @ np.asarray(w_dense, dtype=np.float64)
    r = r + _f32(bias).astype(np.float64)
    return _act(r, act).astype(np.float16)


def matmul_epilogue_fp16(a, w_q4, bias, K, N, act):
    """q4_0 weight, logical [K, N], blocks along N; dequantized weight rounded
    to fp16 before the multiply (baseline.c:34-47)."""
    return gemm_epilogue(a, dequantize_q4_0_fp16(w_q4, (K, N)), bias, act)


def matmul_epilogue_f16w(a, w16, bias, act):
    return gemm_epilogue(a, _f32(w16), bias, act)


def matmul_q8k(a, wt_q8, bias, K, N, act):
    """q8_0 blocks along K of the transposed weight: wt_q8 is [N, K] q8_0;
    each dequantized weight rounded to fp16."""
    return gemm_epilogue(a, dequantize_q8_0_fp16(wt_q8, (N, K)).T, bias, act)


def matmul_q4k(a, wt_q4, bias, K, N, act):
    """q4_0 blocks along K of the transposed weight: wt_q4 is [N, K] q4_0."""
    return gemm_epilogue(a, dequantize_q4_0_fp16(wt_q4, (N, K)).T, bias, act)


def close_f16(got, want, rel, abs_tol):
    """`hexlib_close_f16` (include/hexlib/hexlib_harness.h:74-82), elementwise:
    |a-b| <= abs or |a-b| <= rel * max(|a|, |b|). Returns a boolean array."""
    g, w = _f32(got).astype(np.float64), _f32(want).astype(np.float64)
    d = np.abs(g - w)
    return (d <= abs_tol) | (d <= rel * np.maximum(np.abs(g), np.abs(w)))


def attention_fp16(q, k, v, batch, scale):
    """Fused attention over [batch*T, H, D] fp16 q/k/v: float64 inside, one
    rounding to fp16 (the kernel's contract)."""
    from oracle.refs import attention
    (o,) = attention([np.asarray(q, np.float64), np.asarray(k, np.float64), np.asarray(v, np.float64)],
                     {"batch": batch, "scale": scale})
    return o.astype(np.float16)


def rope_2d_qk_fp16(qkv, cos, sin):
    """rope_2d_fp16 on the q and k slots of [rows, 3, H, D] -> [rows, 2, H, D]."""
    qkv = np.asarray(qkv, np.float16)
    return np.stack([rope_2d_fp16(np.ascontiguousarray(qkv[:, j]), cos, sin) for j in (0, 1)], axis=1)


def attention_qk_v_fp16(qk, qkv, batch, scale):
    """attention_fp16 with q, k from qk [rows, 2, H, D] and v from qkv [rows, 3, H, D]."""
    qk, qkv = np.asarray(qk, np.float16), np.asarray(qkv, np.float16)
    return attention_fp16(qk[:, 0], qk[:, 1], qkv[:, 2], batch, scale)


def permute_rope_rows(wt, heads, d):
    """W^T [N, K] with the rows of each of the first 2*heads heads of d
    pair-interleaved (row 2i = feature i, row 2i + 1 = feature i + d/2):
    the col_major_rope layout."""
    wt = np.asarray(wt).copy()
    idx = np.arange(d)
    src = np.where(idx % 2 == 0, idx // 2, idx // 2 + d // 2)
    for h in range(2 * heads):
        wt[h * d:(h + 1) * d] = wt[h * d + src]
    return wt
