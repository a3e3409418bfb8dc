"""The op registry's numpy references, restated (test infrastructure only).

Each function takes `(arrays, attrs)` and returns a tuple of arrays, with the
reference's own precision choices: layernorm, gelu and softmax compute in
float64 and cast back to the first input's dtype; rope computes in float32;
matmul_epilogue adds the bias before the activation and delegates the
activation to the unfused reference.

Pinned by: the committed golden vectors (`tests/golden/qwen35_vision_tiny.npz`,
encoder output within rtol 1e-4 / atol 1e-5 and patchify within 1e-6 of the
upstream model -- reference `hexlib/tests/test_vision_oracle.py:86-150`);
closed forms (softmax rows sum to 1, layernorm zero-mean/unit-variance, rope
with identity tables is the identity, transposes vs np.transpose); and the
reference's compiled `baseline.c` files via `oracle.ref`.
"""
from __future__ import annotations

import math

import numpy as np

_SQRT_2_OVER_PI = math.sqrt(2.0 / math.pi)
# math.erf is scalar; the reference vectorises it the same way
# (`hexlib/graph/opdefs/elementwise.py:22`).
_erf = np.vectorize(math.erf, otypes=[np.float64])


def add(arrays, attrs):  # elementwise.py:40-48
    return ((arrays[0] + arrays[1]).astype(arrays[0].dtype),)


def scale(arrays, attrs):  # elementwise.py:62-67
    return ((arrays[0] * attrs["factor"]).astype(arrays[0].dtype),)


def layernorm(arrays, attrs):  # elementwise.py:82-95
    x = arrays[0].astype(np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    centred = x - mean
    var = np.mean(centred * centred, axis=-1, keepdims=True)
    y = centred / np.sqrt(var + attrs["eps"]) * arrays[1] + arrays[2]
    return (y.astype(arrays[0].dtype),)


def rmsnorm(arrays, attrs):  # kernels/rmsnorm_fp16/baseline.c:6-19, in float64
    x = arrays[0].astype(np.float64)
    ms = np.mean(x * x, axis=-1, keepdims=True)
    y = x / np.sqrt(ms + attrs["eps"]) * arrays[1]
    return (y.astype(arrays[0].dtype),)


def gelu_tanh(arrays, attrs):  # elementwise.py:110-114
    x = arrays[0].astype(np.float64)
    y = 0.5 * x * (1.0 + np.tanh(_SQRT_2_OVER_PI * (x + 0.044715 * x ** 3)))
    return (y.astype(arrays[0].dtype),)


def gelu_erf(arrays, attrs):  # elementwise.py:117-125
    x = arrays[0].astype(np.float64)
    return ((0.5 * x * (1.0 + _erf(x / math.sqrt(2.0)))).astype(arrays[0].dtype),)


def softmax(arrays, attrs):  # elementwise.py:141-146
    axis = attrs["axis"]
    x = arrays[0].astype(np.float64)
    e = np.exp(x - np.max(x, axis=axis, keepdims=True))
    return ((e / np.sum(e, axis=axis, keepdims=True)).astype(arrays[0].dtype),)


def matmul(arrays, attrs):  # structural.py:55-61
    return ((arrays[0] @ arrays[1]).astype(arrays[0].dtype),)


def matmul_epilogue(arrays, attrs):  # fused.py:44-53
    out = (arrays[0] @ arrays[1] + arrays[2]).astype(arrays[0].dtype)
    act = attrs.get("act", "none")
    if act != "none":
        (out,) = REFERENCES[act]((out,), {})
    if len(arrays) == 4:
        # residual folded in (build extension): the linear's result is stored
        # at `round` first, then add (elementwise.py:40-48)
        if attrs.get("round") == "fp16":
            out = out.astype(np.float16).astype(out.dtype)
        out = (arrays[3] + out).astype(out.dtype)
    if len(arrays) == 5:
        # rope folded in (build extension): the linear's result is stored at
        # `round`, then rope_2d (structural.py:240-254) on its first
        # 2 * rope_heads heads of rope_dim -- the q and k slots
        if attrs.get("round") == "fp16":
            out = out.astype(np.float16).astype(out.dtype)
        heads, d = int(attrs["rope_heads"]), int(attrs["rope_dim"])
        rows = out.shape[0]
        qk = out[:, :2 * heads * d].reshape(rows, 2 * heads, d)
        (rot,) = rope_2d((qk, arrays[3], arrays[4]), {})
        out = np.concatenate([rot.reshape(rows, -1), out[:, 2 * heads * d:]], axis=1).astype(out.dtype)
    return (out,)


_NUMPY = {"fp32": np.float32, "fp16": np.float32, "int32": np.int32, "q4_0": np.float32, "q8_0": np.float32}


def cast(arrays, attrs):  # structural.py:81-82 (fp16 is computed as float32)
    return (arrays[0].astype(_NUMPY[attrs["dtype"]]),)


def transpose(arrays, attrs):  # structural.py:98-102
    return (np.transpose(arrays[0], tuple(attrs["perm"])),)


def reshape(arrays, attrs):  # structural.py:118-126
    return (arrays[0].reshape(tuple(attrs["shape"])),)


def patchify(arrays, attrs):  # structural.py:172-207 (+ images stacked on channels)
    batch = int(attrs.get("batch", 1))
    bc, t, h, w = arrays[0].shape
    b, c = batch, bc // batch
    img = arrays[0].reshape(b, c, t, h, w)
    p, m = int(attrs["patch"]), int(attrs["merge"])
    gh, gw = int(attrs["grid_h"]), int(attrs["grid_w"])
    x = img.reshape(b, c, t, gh // m, m, p, gw // m, m, p)
    # token axes (bh, bw, mh, mw), feature axes (c, t, ph, pw)
    x = x.transpose(0, 3, 6, 4, 7, 1, 2, 5, 8)
    return (np.ascontiguousarray(x).reshape(b * gh * gw, c * t * p * p),)


def rope_2d(arrays, attrs):  # structural.py:240-254
    x, cos, sin = arrays
    xf = x.astype(np.float32)
    cosf = cos.astype(np.float32)[:, None, :]
    sinf = sin.astype(np.float32)[:, None, :]
    half = xf.shape[-1] // 2
    rotated = np.concatenate([-xf[..., half:], xf[..., :half]], axis=-1)
    return ((xf * cosf + rotated * sinf).astype(x.dtype),)


def attention(arrays, attrs):
    """Fused attention: the chain it replaces in the encoder
    (`hexlib/models/vit.py:185-193`: scale, transpose_hd, matmul, softmax,
    matmul, with the head transposes around it) computed in float64 with no
    intermediate storage rounding; q, k, v, out are [batch*T, H, D]. The fused-
    projection form takes (qk [batch*T, 2, H, D], qkv [batch*T, 3, H, D]):
    q and k from the first, v from the third slot of the second."""
    if len(arrays) == 2:   # (qk [rows, 2, H, D], qkv [rows, 3, H, D])
        qk, qkv = arrays
        arrays = (qk[:, 0], qk[:, 1], qkv[:, 2])
    elif len(arrays) == 1:  # (qkv [rows, 3, H, D])
        (qkv,) = arrays
        arrays = (qkv[:, 0], qkv[:, 1], qkv[:, 2])
    q, k, v = (np.asarray(a, np.float64) for a in arrays)
    batch = int(attrs.get("batch", 1))
    rows, heads, d = q.shape
    t = rows // batch

    def split(x):  # [B*T, H, D] -> [B, H, T, D]
        return x.reshape(batch, t, heads, d).transpose(0, 2, 1, 3)

    s = split(q) @ split(k).transpose(0, 1, 3, 2) * float(attrs["scale"])
    e = np.exp(s - s.max(axis=-1, keepdims=True))
    o = (e / e.sum(axis=-1, keepdims=True)) @ split(v)
    return (o.transpose(0, 2, 1, 3).reshape(rows, heads, d).astype(arrays[0].dtype),)


def rope_2d_qk(arrays, attrs):
    """rope_2d (structural.py:240-254) on the q and k slots of a fused
    [rows, 3, H, D] projection -> [rows, 2, H, D]."""
    qkv, cos, sin = arrays
    (q,) = rope_2d((qkv[:, 0], cos, sin), {})
    (k,) = rope_2d((qkv[:, 1], cos, sin), {})
    return (np.stack([q, k], axis=1),)


def layernorm_matmul_epilogue(arrays, attrs):
    """layernorm (elementwise.py:82-95) over x's rows, stored at `ln_round`,
    then matmul_epilogue (fused.py:44-53, with this build's rope form) of the
    stored result -- the two ops `fuse_layernorm` replaces."""
    x, g, b = arrays[:3]
    (y,) = layernorm((x, g, b), {"eps": attrs["eps"]})
    if attrs.get("ln_round") == "fp16":
        y = y.astype(np.float16).astype(y.dtype)
    return matmul_epilogue((y,) + tuple(arrays[3:]), attrs)


REFERENCES = {
    "add": add, "scale": scale, "layernorm": layernorm, "rmsnorm": rmsnorm,
    "gelu_tanh": gelu_tanh, "gelu_erf": gelu_erf, "softmax": softmax,
    "matmul": matmul, "matmul_epilogue": matmul_epilogue, "cast": cast,
    "transpose": transpose, "reshape": reshape, "patchify": patchify,
    "rope_2d": rope_2d, "attention": attention, "rope_2d_qk": rope_2d_qk,
    "layernorm_matmul_epilogue": layernorm_matmul_epilogue,
}
