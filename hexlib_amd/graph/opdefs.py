"""Shape/dtype inference for every op kind the encoder graph uses.

The kinds and their shape rules follow the reference registry
(`hexlib/graph/opdefs/elementwise.py:40-156`, `fused.py:16-63`,
`structural.py:38-264`). Two additions, both recorded as build extensions:

* `rmsnorm` -- the reference ships an `rmsnorm_fp16` kernel
  (`kernels/rmsnorm_fp16/kernel_api.h:26-27`) with no op kind; it gets one so
  the graph can select it (`norm="rmsnorm"` in `VitConfig`).
* a leading batch axis: `patchify` takes `batch` images stacked on the
  channel axis, `[batch * C, T, H, W]` (attr `batch`, default 1), and emits
  `[batch * tokens, feat]`; `transpose` accepts any permutation.
"""
from __future__ import annotations

import math

import numpy as np

from hexlib_amd.graph.ir import DTYPES
from hexlib_amd.graph.ops import OpDef, register

ACTIVATIONS = ("none", "gelu_tanh", "gelu_erf")


def _same(inputs, attrs):
    return ((inputs[0].shape, inputs[0].dtype),)


def _add_infer(inputs, attrs):
    shape = tuple(np.broadcast_shapes(inputs[0].shape, inputs[1].shape))
    return ((shape, inputs[0].dtype),)


def _norm_infer(inputs, attrs):
    x = inputs[0]
    for p in inputs[1:]:
        if p.shape != (x.shape[-1],):
            raise ValueError(f"norm parameter {p.name} {p.shape} != ({x.shape[-1]},)")
    return ((x.shape, x.dtype),)


def _matmul_infer(inputs, attrs):
    a, b = inputs[0], inputs[1]
    if len(a.shape) < 2 or len(b.shape) < 2:
        raise ValueError(f"matmul needs rank >= 2, got {a.shape} @ {b.shape}")
    if a.shape[-1] != b.shape[-2]:
        raise ValueError(f"matmul inner dims disagree: {a.shape} @ {b.shape}")
    batch = tuple(np.broadcast_shapes(a.shape[:-2], b.shape[:-2]))
    return ((batch + (a.shape[-2], b.shape[-1]), a.dtype),)


def _matmul_epilogue_infer(inputs, attrs):
    act = attrs.get("act", "none")
    if act not in ACTIVATIONS:
        raise ValueError(f"matmul_epilogue act {act!r} not in {ACTIVATIONS}")
    (out,) = _matmul_infer(inputs[:2], attrs)
    bias = inputs[2]
    if bias.shape != (inputs[1].shape[-1],):
        raise ValueError(f"bias {bias.shape} != ({inputs[1].shape[-1]},)")
    if len(inputs) == 4 and inputs[3].shape != out[0]:     # residual (build extension)
        raise ValueError(f"residual {inputs[3].shape} != output {out[0]}")
    if len(inputs) == 5:                                     # rope tables (build extension)
        heads, d = int(attrs["rope_heads"]), int(attrs["rope_dim"])
        rows = out[0][0]
        if inputs[3].shape != (rows, d) or inputs[4].shape != (rows, d) or 2 * heads * d > out[0][-1]:
            raise ValueError(f"rope tables {inputs[3].shape} for {heads} heads of {d} over {out[0]}")
    return (out,)


def _ln_matmul_infer(inputs, attrs):
    """(x, ln_w, ln_b, w, bias[, cos, sin]): layernorm over x's last axis, then
    matmul_epilogue of the result (a build extension, `fuse_layernorm`)."""
    x, g, b = inputs[:3]
    _norm_infer((x, g, b), attrs)
    return _matmul_epilogue_infer((x,) + tuple(inputs[3:]), attrs)


def _cast_infer(inputs, attrs):
    dtype = attrs["dtype"]
    if dtype not in DTYPES:
        raise ValueError(f"cast to unknown dtype {dtype!r}")
    return ((inputs[0].shape, dtype),)


def _transpose_infer(inputs, attrs):
    perm = tuple(attrs["perm"])
    shape = inputs[0].shape
    if sorted(perm) != list(range(len(shape))):
        raise ValueError(f"perm {perm} is not a permutation of rank {len(shape)}")
    return ((tuple(shape[i] for i in perm), inputs[0].dtype),)


def _reshape_infer(inputs, attrs):
    shape = tuple(attrs["shape"])
    if math.prod(shape) != math.prod(inputs[0].shape):
        raise ValueError(f"reshape {inputs[0].shape} -> {shape} changes element count")
    return ((shape, inputs[0].dtype),)


def _patchify_infer(inputs, attrs):
    img = inputs[0]
    if len(img.shape) != 4:
        raise ValueError(f"patchify wants [C,T,H,W] (or [batch*C,T,H,W]), got {img.shape}")
    batch = int(attrs.get("batch", 1))
    bc, t, h, w = img.shape
    if batch <= 0 or bc % batch:
        raise ValueError(f"patchify: {bc} channels do not split into batch {batch}")
    c = bc // batch
    patch, merge = int(attrs["patch"]), int(attrs["merge"])
    gh, gw = int(attrs["grid_h"]), int(attrs["grid_w"])
    if t != int(attrs["temporal_patch"]):
        raise ValueError(f"image T {t} != temporal_patch {attrs['temporal_patch']}")
    if gh * patch != h or gw * patch != w:
        raise ValueError(f"{h}x{w} does not tile into {gh}x{gw} patches of {patch}")
    if gh % merge or gw % merge:
        raise ValueError(f"grid {gh}x{gw} not divisible by merge {merge}")
    return (((batch * gh * gw, c * t * patch * patch), img.dtype),)


def _rope_infer(inputs, attrs):
    x, cos, sin = inputs
    if len(x.shape) != 3:
        raise ValueError(f"rope_2d wants [tokens, heads, head_dim], got {x.shape}")
    if cos.shape != sin.shape or cos.shape != (x.shape[0], x.shape[2]):
        raise ValueError(f"rope tables {cos.shape}/{sin.shape} vs x {x.shape}")
    if x.shape[2] % 2:
        raise ValueError("rope_2d head_dim must be even")
    return ((x.shape, x.dtype),)


def _attention_infer(inputs, attrs):
    """(q, k, v) each [rows, heads, head_dim]; or (qk [rows, 2, heads,
    head_dim], qkv [rows, 3, heads, head_dim]): q, k from the first, v from
    the third slot of the second. Output [rows, heads, head_dim]."""
    batch = int(attrs.get("batch", 1))
    if len(inputs) == 1:
        (qkv,) = inputs
        if len(qkv.shape) != 4 or qkv.shape[1] != 3:
            raise ValueError(f"attention over one tensor wants [rows, 3, heads, head_dim], got {qkv.shape}")
        out = (qkv.shape[0], qkv.shape[2], qkv.shape[3])
    elif len(inputs) == 2:
        qk, qkv = inputs
        rows, two, heads, d = qk.shape if len(qk.shape) == 4 else (0, 0, 0, 0)
        if two != 2 or qkv.shape != (rows, 3, heads, d):
            raise ValueError(f"attention over qk {qk.shape} and qkv {qkv.shape}")
        out = (rows, heads, d)
    else:
        q, k, v = inputs
        if len(q.shape) != 3 or q.shape != k.shape or q.shape != v.shape:
            raise ValueError(f"attention wants q, k, v of one [rows, heads, head_dim] shape, "
                             f"got {q.shape} {k.shape} {v.shape}")
        out = q.shape
    if batch < 1 or out[0] % batch:
        raise ValueError(f"attention: {out[0]} rows do not split into {batch} images")
    return ((out, inputs[0].dtype),)


def _rope_qk_infer(inputs, attrs):
    qkv, cos, sin = inputs
    if len(qkv.shape) != 4 or qkv.shape[1] != 3:
        raise ValueError(f"rope_2d_qk wants a fused [rows, 3, heads, head_dim] projection, got {qkv.shape}")
    rows, _, heads, d = qkv.shape
    if cos.shape != (rows, d) or sin.shape != (rows, d) or d % 2:
        raise ValueError(f"rope tables {cos.shape}/{sin.shape} vs qkv {qkv.shape}")
    return (((rows, 2, heads, d), qkv.dtype),)


for _kind, _fn in (
    ("add", _add_infer),
    ("scale", _same),
    ("layernorm", _norm_infer),
    ("rmsnorm", _norm_infer),
    ("gelu_tanh", _same),
    ("gelu_erf", _same),
    ("softmax", _same),
    ("matmul", _matmul_infer),
    ("matmul_epilogue", _matmul_epilogue_infer),
    ("cast", _cast_infer),
    ("transpose", _transpose_infer),
    ("reshape", _reshape_infer),
    ("patchify", _patchify_infer),
    ("rope_2d", _rope_infer),
    ("attention", _attention_infer),
    ("rope_2d_qk", _rope_qk_infer),
    ("layernorm_matmul_epilogue", _ln_matmul_infer),
):
    register(OpDef(kind=_kind, infer=_fn))
