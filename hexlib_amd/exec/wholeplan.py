"""A whole encoder plan as ONE batch blob over ONE device arena.

Restates `build_whole_plan_batch` (`hexlib/exec/wholeplan.py:92-357`): every
tensor lives in a single buffer (fd 0) split into regions --

  const  every weight, bias and table, each at its own offset;
  act    activations. By default (`reuse=True`) tensors whose lifetimes do
         not overlap share addresses (lifetimes taken over reshape-unified
         storage owners), which keeps the working set cache-resident and the
         batch-32 arena inside the wire's 32-bit offsets; `reuse=False` gives
         every activation its own offset, the reference's default
         (`alias_activations=False`) and the control case;
  io     the graph input and output.

A reshape emits no op: its output is placed at its input's offset with its own
extents. The variant for each op is chosen on the host (`runner.select`) from
its attrs and input dtypes, and each tensor's bytes take the dtype and layout
the consuming spec declares (the fp32 pos_embed is staged as fp16; a q4_0
weight is quantized here, blocked along N or grouped along K per the chosen
layout; an fp16 weight is stored transposed, `col_major`, by default).
Offsets are 256-byte aligned so every kernel's vector path applies.

The plan order is the fused graph's op order (a valid topological order; with
no aliasing the result does not depend on which one).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Mapping

import numpy as np

from hexlib_amd.exec import wire
from hexlib_amd.exec.runner import KIND_ID, WIRE_RAW, RunnerSpec, select
from hexlib_amd.graph.fuse import LNFOLD_RECIPES, fold_layernorm, fuse, fuse_layernorm, fuse_residual, fuse_rope
from hexlib_amd.graph.ir import Graph
from hexlib_amd.graph.ir import nbytes as ir_nbytes
from hexlib_amd.quant import pack_q4_0_kgrouped, pack_q4_0_nblocked, pack_q8_0_kgrouped

ALIGN = 256
_NP = {"fp32": np.float32, "fp16": np.float16, "int32": np.int32}


class WholePlanError(Exception):
    pass


def align_up(n: int, a: int = ALIGN) -> int:
    return (n + a - 1) // a * a


@dataclass(frozen=True)
class Placement:
    name: str
    offset: int
    nbytes: int
    dtype: str
    layout: str
    ne: tuple[int, int, int, int]
    region: str  # const | act | io | reshape-alias
    shape: tuple[int, ...] = ()


@dataclass
class WholePlanBatch:
    blob: bytes
    payload: bytearray            # initial arena contents (consts + inputs staged)
    placements: dict[str, Placement]
    index: dict[str, int]
    n_ops: int
    arena_bytes: int
    outputs: tuple[str, ...]
    inputs: tuple[str, ...]
    skipped_reshapes: int
    op_names: tuple[str, ...] = field(default=())
    op_specs: tuple[str, ...] = field(default=())
    const_bytes: int = 0
    graph_ops: tuple = field(default=())   # the plan's non-reshape graph ops, in wire order


def stage_col_major_rope(w, heads: int, d: int) -> bytes:
    """A `[K, N]` fp16 weight in the `col_major_rope` layout: stored `[N, K]`
    (W^T), with the rows of each of the first `2 * heads` heads of `d`
    pair-interleaved -- stored row `h*d + 2i` is feature `h*d + i` and row
    `h*d + 2i + 1` is feature `h*d + i + d/2` -- so a GEMM tile holds both
    halves of every rotated pair in adjacent columns."""
    wt = np.ascontiguousarray(np.asarray(w, dtype=np.float16).T)
    i = np.arange(d)
    src = np.where(i % 2 == 0, i // 2, i // 2 + d // 2)
    rows = (np.arange(2 * heads)[:, None] * d + src[None, :]).reshape(-1)
    wt[:2 * heads * d] = wt[rows]
    return wt.tobytes()


def rope_row_order(n: int, heads: int, d: int) -> np.ndarray:
    """The col_major_rope row order of an N-row W^T: within each of the first
    `2 * heads` heads of `d`, stored row 2i is feature i and row 2i + 1 is
    feature i + d/2; rows past them stay in place."""
    i = np.arange(d)
    src = np.where(i % 2 == 0, i // 2, i // 2 + d // 2)
    order = np.arange(n)
    order[:2 * heads * d] = (np.arange(2 * heads)[:, None] * d + src[None, :]).reshape(-1)
    return order


def stage_q8_0_kgroup_rope(w, heads: int, d: int) -> bytes:
    """A `[K, N]` weight in the `q8_0_kgroup_rope` layout: the q8_0 blocks
    along K of W^T in the col_major_rope row order. Rows are quantized one by
    one, so these are the q8_0_kgroup blocks of the same rows, reordered."""
    w = np.asarray(w, dtype=np.float32)
    return pack_q8_0_kgrouped(np.ascontiguousarray(w[:, rope_row_order(w.shape[1], heads, d)]))


def _spec_for(op, graph: Graph, weight_layout: str | None) -> tuple[str, RunnerSpec]:
    """`weight_layout="auto"` stores fp16 weights transposed (col_major: both
    GEMM operands K-contiguous, the fast path) and q4_0 weights in the
    reference's N-blocked layout; any other value is passed to `select`."""
    dtypes = [graph.tensor(n).dtype for n in op.inputs]
    layout = weight_layout
    if weight_layout == "auto":
        layout = "col_major" if op.kind == "matmul_epilogue" and dtypes[1] == "fp16" else None
    name, spec = select(op.kind, dict(op.attrs), dtypes, layout)
    spec.check_requires(dict(op.attrs))
    spec.check_rank([graph.tensor(n).shape for n in op.inputs])
    return name, spec


def _reuse_offsets(g: Graph, acts, reshape_src, owner, wbytes) -> tuple[dict[str, int], int]:
    """Activation offsets that share memory between tensors whose lifetimes do
    not overlap. Lifetimes are computed on storage owners, so a reshape's
    consumers keep its input alive -- the reshape chain is unified BEFORE
    allocation, which is what the reference's slot reuse lacked
    (`hexlib/exec/wholeplan.py:235-252, 369-409`). Largest-first placement at
    the lowest free address, like the reference's VTCM allocator
    (`hexlib/graph/vtcm.py:83-151`); lifetimes are inclusive at both ends."""
    first: dict[str, int] = {}
    last: dict[str, int] = {}
    act_set = set(acts)
    for i, op in enumerate(g.ops):
        for n in op.outputs:
            o = owner(n)
            if o in act_set:
                first.setdefault(o, i)
                last[o] = max(last.get(o, i), i)
        for n in op.inputs:
            o = owner(n)
            if o in act_set:
                last[o] = max(last.get(o, i), i)
    placed: list[tuple[int, int, int, int]] = []   # (offset, end, first, last)
    offsets: dict[str, int] = {}
    for n in sorted(acts, key=lambda n: (-wbytes(n), n)):
        size = align_up(wbytes(n))
        f, l = first.get(n, 0), last.get(n, len(g.ops))
        clash = sorted((o, e) for o, e, f2, l2 in placed if f <= l2 and f2 <= l)
        off = 0
        for o, e in clash:
            if off + size <= o:
                break
            off = max(off, e)
        offsets[n] = off
        placed.append((off, off + size, f, l))
    span = max((e for _, e, _, _ in placed), default=0)
    return offsets, span


def build_whole_plan_batch(graph: Graph, feeds: Mapping[str, Any],
                           weight_layout: str | None = "auto", fuse_first: bool = True,
                           fd: int = 0, reuse: bool = True, residual: bool = False,
                           rope: bool = False, layernorm: bool = False,
                           fold_ln_rows=0) -> WholePlanBatch:
    """`residual=True` also folds each residual add into the linear that
    feeds it (`fuse_residual`: quantized weights in any layout, fp16 weights
    when staged transposed), `rope=True` the q/k rope of a fused q/k/v
    projection into that linear (`fuse_rope`) and `layernorm=True` each
    LayerNorm into the linear it feeds (`fuse_layernorm`, the normalised rows
    recomputed in the linear's prologue), when fp16 weights are staged
    transposed (the only layout with those kernels). `fold_ln_rows` (an int
    > 0: at most that many rows; or a predicate on the row count) folds each
    LayerNorm it admits into the linear it feeds algebraically instead
    (`fold_layernorm`: weight-scaled W' and bias vectors derived here from the
    feeds, row statistics in the GEMM)."""
    g = fuse(graph) if fuse_first else graph
    if rope and weight_layout in ("auto", "col_major"):
        g = fuse_rope(g)
    if residual:
        g = fuse_residual(g, fp16_weights=weight_layout in ("auto", "col_major"))
    derived: dict = {}
    if (callable(fold_ln_rows) or fold_ln_rows > 0) and weight_layout in ("auto", "col_major"):
        g, derived = fold_layernorm(g, max_rows=fold_ln_rows)
    if layernorm and weight_layout in ("auto", "col_major"):
        g = fuse_layernorm(g)
    if derived:
        feeds = dict(feeds)
        for n, (recipe, srcs) in derived.items():
            missing = [s for s in srcs if s not in feeds]
            if missing:
                raise WholePlanError(f"no feed for {missing[0]!r} (needed by derived {n!r})")
            feeds[n] = LNFOLD_RECIPES[recipe](*(feeds[s] for s in srcs))
    tensors = g.tensors
    io = set(g.inputs) | set(g.outputs)
    consts = {n for n, t in tensors.items() if t.const}

    reshape_src: dict[str, str] = {}
    for op in g.ops:
        if op.kind == "reshape":
            reshape_src[op.outputs[0]] = op.inputs[0]
    aliased_io = sorted(n for n in reshape_src if n in io)
    if aliased_io:
        raise WholePlanError(f"graph inputs/outputs produced by reshape: {aliased_io}")

    def owner(name: str) -> str:
        seen = {name}
        while name in reshape_src:
            name = reshape_src[name]
            if name in seen:
                raise WholePlanError(f"reshape cycle at {name!r}")
            seen.add(name)
        return name

    layout_of: dict[str, str] = {}
    dtype_of: dict[str, str] = {}

    def claim(table, name, value, where):
        prev = table.setdefault(name, value)
        if prev != value:
            raise WholePlanError(f"{name!r} is used as {prev!r} and {value!r} ({where})")

    op_specs: dict[int, tuple[str, RunnerSpec]] = {}
    rope_of: dict[str, tuple[int, int]] = {}    # col_major_rope weight -> (heads, head_dim)
    for op in g.ops:
        if op.kind == "reshape":
            continue
        name, spec = _spec_for(op, g, weight_layout)
        op_specs[op.id] = (name, spec)
        for rope_layout in ("col_major_rope", "q8_0_kgroup_rope"):
            if rope_layout in spec.buf_layouts():
                claim(rope_of, op.inputs[spec.buf_layouts().index(rope_layout)],
                      (int(op.attrs["rope_heads"]), int(op.attrs["rope_dim"])), f"op {op.id} rope")
        lays = spec.buf_layouts()
        for i, n in enumerate(op.inputs):
            claim(layout_of, n, lays[i], f"op {op.id} src{i}")
            claim(dtype_of, n, spec.inputs[i], f"op {op.id} src{i}")
        for n in op.outputs:
            claim(layout_of, n, lays[-1], f"op {op.id} dst")
            claim(dtype_of, n, spec.out_dtype, f"op {op.id} dst")

    def wdtype(n):
        return dtype_of.get(n, tensors[n].dtype)

    def wbytes(n):
        return ir_nbytes(tensors[n].shape, wdtype(n))

    placements: dict[str, Placement] = {}

    def place(n, off, region):
        placements[n] = Placement(n, off, wbytes(n), wdtype(n), layout_of.get(n, "row_major"),
                                  wire.pad_ne(tensors[n].shape), region, tensors[n].shape)

    cursor = 0
    for n in sorted(consts):
        place(n, cursor, "const")
        cursor = align_up(cursor + wbytes(n))
    const_end = cursor
    acts = [n for n in tensors if n not in consts and n not in io and n not in reshape_src]
    retyped = [n for n in acts if wdtype(n) != tensors[n].dtype]
    if retyped:
        raise WholePlanError(f"activations staged in another dtype than declared: {retyped[:6]}")
    if reuse:
        offsets, span = _reuse_offsets(g, acts, reshape_src, owner, wbytes)
        for n in sorted(acts):
            place(n, const_end + offsets[n], "act")
        cursor = align_up(const_end + span)
    else:
        for n in sorted(acts):
            place(n, cursor, "act")
            cursor = align_up(cursor + wbytes(n))
    for n in sorted(io):
        place(n, cursor, "io")
        cursor = align_up(cursor + wbytes(n))
    for n in reshape_src:
        base = placements.get(owner(n))
        if base is None:
            raise WholePlanError(f"reshape {n!r} resolves to unplaced {owner(n)!r}")
        if wbytes(n) != base.nbytes:
            raise WholePlanError(f"reshape {n!r} changes the byte count")
        placements[n] = Placement(n, base.offset, base.nbytes, wdtype(n),
                                  layout_of.get(n, "row_major"), wire.pad_ne(tensors[n].shape),
                                  "reshape-alias", tensors[n].shape)
    arena = align_up(max(cursor, ALIGN))

    payload = bytearray(arena)
    for n in sorted(consts) + sorted(g.inputs):
        if n not in feeds:
            raise WholePlanError(f"no feed for {n!r}")
        p = placements[n]
        value = feeds[n]
        if p.dtype in WIRE_RAW:
            if isinstance(value, (bytes, bytearray)):
                data = bytes(value)
            elif p.layout == "q4_0_kgroup":
                data = pack_q4_0_kgrouped(np.asarray(value))
            elif p.layout == "q8_0_kgroup":
                data = pack_q8_0_kgrouped(np.asarray(value))
            elif p.layout == "q8_0_kgroup_rope":
                data = stage_q8_0_kgroup_rope(value, *rope_of[n])
            else:
                data = pack_q4_0_nblocked(np.asarray(value))
        elif p.layout == "col_major_rope":
            data = stage_col_major_rope(value, *rope_of[n])
        elif p.layout == "col_major":
            data = np.ascontiguousarray(np.asarray(value, dtype=_NP[p.dtype]).T).tobytes()
        else:
            data = np.ascontiguousarray(np.asarray(value), dtype=_NP[p.dtype]).tobytes()
        if len(data) != p.nbytes:
            raise WholePlanError(f"feed {n!r} staged {len(data)} bytes, expected {p.nbytes}")
        payload[p.offset:p.offset + p.nbytes] = data

    order = sorted(placements)
    index = {n: i for i, n in enumerate(order)}
    wtensors = [wire.TensorDesc(0, placements[n].offset, placements[n].nbytes,
                                placements[n].dtype, placements[n].layout, placements[n].ne)
                for n in order]
    ops, names, specs, gops = [], [], [], []
    skipped = 0
    for op in g.ops:
        if op.kind == "reshape":
            skipped += 1
            continue
        gops.append(op)
        spec_name, spec = op_specs[op.id]
        shapes = [tensors[n].shape for n in op.inputs]
        ops.append(wire.OpDesc(kind=KIND_ID[spec_name], params=spec.params(shapes, op.attrs),
                               src=tuple(index[n] for n in op.inputs),
                               dst=tuple(index[n] for n in op.outputs)))
        names.append(f"{op.id}:{spec_name}")
        specs.append(spec_name)
    blob = wire.pack_batch([wire.BufDesc(fd=fd, size=arena)], wtensors, ops)
    return WholePlanBatch(blob=blob, payload=payload, placements=placements, index=index,
                          n_ops=len(ops), arena_bytes=arena, outputs=tuple(g.outputs),
                          inputs=tuple(g.inputs), skipped_reshapes=skipped,
                          op_names=tuple(names), op_specs=tuple(specs), const_bytes=const_end,
                          graph_ops=tuple(gops))


def decode(batch: WholePlanBatch, name: str, raw: bytes) -> np.ndarray:
    """Interpret `raw` (the arena bytes of tensor `name`) as float32."""
    p = batch.placements[name]
    arr = np.frombuffer(raw, dtype=_NP[p.dtype], count=int(np.prod(p.shape)))
    return arr.reshape(p.shape).astype(np.float32)
