"""Fusion pass: matmul -> add(const 1-D bias) [-> gelu] becomes matmul_epilogue.

Same rewrite rule as the reference (`hexlib/graph/fuse.py:16-92`): the matmul
output and the add output must each have exactly one consumer and not be a
graph output; the bias must be a const rank-1 tensor on either side of the
add; an activation is folded only if it is gelu_tanh or gelu_erf. Residual
adds (activation + activation) never fuse.
"""
from __future__ import annotations

import math

from hexlib_amd.graph.ir import Graph, Op, Tensor

FUSABLE_ACTS = ("gelu_tanh", "gelu_erf")


class FuseError(ValueError):
    pass


def fuse(graph: Graph) -> Graph:
    problems = graph.problems()
    if problems:
        raise FuseError("graph is structurally invalid:\n" + "\n".join(problems))

    readers: dict[str, list[Op]] = {}
    for op in graph.ops:
        for name in op.inputs:
            readers.setdefault(name, []).append(op)
    outputs = set(graph.outputs)

    def only_reader(name: str, skip: set[int]) -> Op | None:
        if name in outputs:
            return None
        found = [op for op in readers.get(name, ()) if op.id not in skip]
        if len(readers.get(name, ())) != 1 or len(found) != 1:
            return None
        return found[0]

    absorbed: set[int] = set()
    replaced: dict[int, Op] = {}
    dropped: set[str] = set()

    for op in graph.ops:
        if op.kind != "matmul" or op.id in absorbed:
            continue
        mm_out = op.outputs[0]
        add = only_reader(mm_out, absorbed)
        if add is None or add.kind != "add":
            continue
        if len(add.inputs) != 2:
            raise FuseError(f"op {add.id} (add) has {len(add.inputs)} inputs")
        other = [n for n in add.inputs if n != mm_out]
        if len(other) != 1:
            continue
        bias = graph.tensors.get(other[0])
        if bias is None or not bias.const or len(bias.shape) != 1:
            continue
        act, tail = "none", add
        nxt = only_reader(add.outputs[0], absorbed | {add.id})
        if nxt is not None and nxt.kind in FUSABLE_ACTS:
            act, tail = nxt.kind, nxt
        replaced[op.id] = Op(
            id=op.id,
            kind="matmul_epilogue",
            inputs=(op.inputs[0], op.inputs[1], bias.name),
            outputs=tail.outputs,
            attrs={"act": act},
        )
        absorbed.add(add.id)
        dropped.add(mm_out)
        if tail is not add:
            absorbed.add(tail.id)
            dropped.add(add.outputs[0])

    if not replaced:
        return graph
    ops = tuple(replaced.get(op.id, op) for op in graph.ops if op.id not in absorbed)
    tensors = {n: t for n, t in graph.tensors.items() if n not in dropped}
    return Graph(tensors=tensors, ops=ops, inputs=graph.inputs, outputs=graph.outputs)


def fuse_residual(graph: Graph, fp16_weights: bool = True) -> Graph:
    """Fold each residual add into the linear that feeds it (the linear's
    output read only by the add). Quantized weights (q4_0, q8_0) take their
    residual kernels in any layout; fp16 weights only with `fp16_weights`
    (their residual kernel takes the weight transposed)."""
    readers: dict[str, list[Op]] = {}
    for op in graph.ops:
        for name in op.inputs:
            readers.setdefault(name, []).append(op)
    outputs = set(graph.outputs)
    absorbed: set[int] = set()
    replaced: dict[int, Op] = {}
    dropped: set[str] = set()
    for op in graph.ops:
        if op.kind != "matmul_epilogue" or len(op.inputs) != 3 or op.id in absorbed:
            continue
        wdt = graph.tensor(op.inputs[1]).dtype
        if wdt not in ("fp16", "q4_0", "q8_0") or (wdt == "fp16" and not fp16_weights):
            continue
        out = op.outputs[0]
        rd = readers.get(out, [])
        if out in outputs or len(rd) != 1 or rd[0].kind != "add" or rd[0].id in absorbed:
            continue
        add = rd[0]
        other = [n for n in add.inputs if n != out]
        if len(add.inputs) != 2 or len(other) != 1:
            continue
        # the other addend may be an activation of the output's dtype or a
        # stored table of the output's shape (the encoder's fp32 position
        # embedding, staged in the add's fp16 either way)
        res = graph.tensor(other[0])
        if res.shape != graph.tensor(out).shape:
            continue
        if res.dtype != graph.tensor(out).dtype and not (res.const and res.dtype == "fp32"):
            continue
        replaced[op.id] = Op(id=op.id, kind="matmul_epilogue",
                             inputs=op.inputs + (other[0],), outputs=add.outputs,
                             attrs={**dict(op.attrs), "round": graph.tensor(out).dtype})
        absorbed.add(add.id)
        dropped.add(out)
    if not replaced:
        return graph
    ops = tuple(replaced.get(op.id, op) for op in graph.ops if op.id not in absorbed)
    tensors = {n: t for n, t in graph.tensors.items() if n not in dropped}
    return Graph(tensors=tensors, ops=ops, inputs=graph.inputs, outputs=graph.outputs)


def fuse_rope(graph: Graph) -> Graph:
    readers: dict[str, list[Op]] = {}
    producer: dict[str, Op] = {}
    for op in graph.ops:
        for name in op.inputs:
            readers.setdefault(name, []).append(op)
        for name in op.outputs:
            producer[name] = op
    outputs = set(graph.outputs)
    replaced: dict[int, Op] = {}
    absorbed: set[int] = set()
    dropped: set[str] = set()
    for rope in graph.ops:
        if rope.kind != "rope_2d_qk":
            continue
        qkv4, cos, sin = rope.inputs
        qk = rope.outputs[0]
        shp = producer.get(qkv4)
        if shp is None or shp.kind != "reshape" or qk in outputs:
            continue
        mm = producer.get(shp.inputs[0])
        if mm is None or mm.kind != "matmul_epilogue" or len(mm.inputs) != 3:
            continue
        # fp16 weights (staged col_major_rope) and q8_0 ones (K-grouped blocks of
        # the same row order); q4_0 has no rope kernel
        if graph.tensor(mm.inputs[1]).dtype not in ("fp16", "q8_0") or shp.inputs[0] in outputs:
            continue
        if len(readers.get(shp.inputs[0], [])) != 1 or len(readers.get(qk, [])) != 1:
            continue
        attn = readers[qk][0]
        if attn.kind != "attention" or tuple(attn.inputs) != (qk, qkv4):
            continue
        if sorted(op.id for op in readers.get(qkv4, [])) != sorted((rope.id, attn.id)):
            continue
        _, _, heads, d = graph.tensor(qkv4).shape
        replaced[mm.id] = Op(id=mm.id, kind="matmul_epilogue", inputs=tuple(mm.inputs) + (cos, sin),
                             outputs=mm.outputs,
                             attrs={**dict(mm.attrs), "round": graph.tensor(mm.outputs[0]).dtype,
                                    "rope_heads": int(heads), "rope_dim": int(d)})
        replaced[attn.id] = Op(id=attn.id, kind="attention", inputs=(qkv4,), outputs=attn.outputs,
                               attrs=dict(attn.attrs))
        absorbed.add(rope.id)
        dropped.add(qk)
    if not replaced:
        return graph
    ops = tuple(replaced.get(op.id, op) for op in graph.ops if op.id not in absorbed)
    tensors = {n: t for n, t in graph.tensors.items() if n not in dropped}
    return Graph(tensors=tensors, ops=ops, inputs=graph.inputs, outputs=graph.outputs)


def fuse_layernorm(graph: Graph, max_rows: int = 2048) -> Graph:
    readers: dict[str, list[Op]] = {}
    producer: dict[str, Op] = {}
    for op in graph.ops:
        for name in op.inputs:
            readers.setdefault(name, []).append(op)
        for name in op.outputs:
            producer[name] = op
    outputs = set(graph.outputs)
    replaced: dict[int, Op] = {}
    absorbed: set[int] = set()
    dropped: set[str] = set()
    for ln in graph.ops:
        if ln.kind != "layernorm":
            continue
        y = ln.outputs[0]
        users = readers.get(y, [])
        if y in outputs or len(users) != 1:
            continue
        mm = users[0]
        # the plain linear only: with the rope tables the fused op would have seven
        # sources, one more than a wire op carries (hexlib/runtime/wire.py MAX_SRC)
        if mm.kind != "matmul_epilogue" or len(mm.inputs) != 3 or mm.inputs[0] != y:
            continue
        if y in mm.inputs[1:] or graph.tensor(mm.inputs[1]).dtype != "fp16":
            continue
        x = graph.tensor(ln.inputs[0])
        rows, feats = math.prod(x.shape[:-1]), x.shape[-1]
        if len(x.shape) != 2 or not 512 <= feats <= 768 or feats % 64 or rows > max_rows:
            continue
        replaced[mm.id] = Op(id=mm.id, kind="layernorm_matmul_epilogue",
                             inputs=tuple(ln.inputs) + tuple(mm.inputs[1:]), outputs=mm.outputs,
                             attrs={**dict(mm.attrs), "eps": ln.attrs["eps"],
                                    "ln_round": graph.tensor(y).dtype})
        absorbed.add(ln.id)
        dropped.add(y)
    if not replaced:
        return graph
    ops = tuple(replaced.get(op.id, op) for op in graph.ops if op.id not in absorbed)
    tensors = {n: t for n, t in graph.tensors.items() if n not in dropped}
    return Graph(tensors=tensors, ops=ops, inputs=graph.inputs, outputs=graph.outputs)


# ---- LayerNorm folded into the linear it feeds -----------------------------------
#
# LN(x) = (x - mean) rstd * w + b over the last axis, then y = LN(x) W + bias:
#   y = rstd (x W' - mean c1) + c2,  W'[k][n] = fp16(w[k] W[k][n]),
#   c1[n] = sum_k W'[k][n],  c2[n] = bias[n] + sum_k b[k] W[k][n].
# The kernel (lnfold_matmul_epilogue) multiplies the raw x by W' and takes each
# row's mean and rstd from the x tiles it reads, so the LayerNorm needs no
# launch of its own and its fp16 output is never stored. W' and bias2 = [c2|c1]
# are new consts derived from the plan's weights when the plan is staged.

LNFOLD_WEIGHT = "lnfold_weight"   # W' from (W, ln_w)
LNFOLD_BIAS2 = "lnfold_bias2"     # [c2 | c1] from (W, ln_w, ln_b, bias)


def lnfold_weight(w, ln_w):
    """W' = fp16(ln_w[k] * W[k][n]): the exact product rounded once to fp16."""
    import numpy as np
    return (np.asarray(w, dtype=np.float64) * np.asarray(ln_w, dtype=np.float64)[:, None]).astype(np.float16)


def lnfold_bias2(w, ln_w, ln_b, bias):
    """[c2 | c1] as 2N fp32: c2 = bias + ln_b W (float64, rounded once), c1 the
    column sums of the rounded W' (float64, rounded once)."""
    import numpy as np
    w64 = np.asarray(w, dtype=np.float64)
    c1 = lnfold_weight(w, ln_w).astype(np.float64).sum(axis=0)
    c2 = np.asarray(bias, dtype=np.float64) + np.asarray(ln_b, dtype=np.float64) @ w64
    return np.concatenate([c2, c1]).astype(np.float32)


LNFOLD_RECIPES = {LNFOLD_WEIGHT: lnfold_weight, LNFOLD_BIAS2: lnfold_bias2}


def fold_layernorm(graph: Graph, max_rows=256) -> tuple[Graph, dict[str, tuple[str, tuple[str, ...]]]]:
    """Fold each LayerNorm whose only reader is an fp16 linear (plain, or with
    the q/k rope in its epilogue) into that linear: the pair becomes one
    `lnfold_matmul_epilogue` op reading the LayerNorm's input. Applies where
    the kernel's forms do -- K % 256 == 0 -- and at the row counts `max_rows`
    admits: an int (at most that many rows) or a predicate on the row count
    (the caller's choice of where the fold pays); elsewhere the LayerNorm
    stays a launch of its own.

    Returns the new graph and the derived consts it reads, `{name: (recipe,
    source names)}` with the recipe a key of `LNFOLD_RECIPES`; the plan
    builder computes their values from the feeds."""
    readers: dict[str, list[Op]] = {}
    for op in graph.ops:
        for name in op.inputs:
            readers.setdefault(name, []).append(op)
    outputs = set(graph.outputs)
    tensors = dict(graph.tensors)
    replaced: dict[int, Op] = {}
    absorbed: set[int] = set()
    dropped: set[str] = set()
    derived: dict[str, tuple[str, tuple[str, ...]]] = {}
    for ln in graph.ops:
        if ln.kind != "layernorm" or len(ln.inputs) != 3:
            continue
        x_name, lw, lb = ln.inputs
        y = ln.outputs[0]
        users = readers.get(y, [])
        if y in outputs or len(users) != 1:
            continue
        mm = users[0]
        if mm.kind != "matmul_epilogue" or mm.inputs[0] != y or len(mm.inputs) not in (3, 5):
            continue
        rope = len(mm.inputs) == 5
        if rope and "rope_heads" not in mm.attrs:
            continue
        w_name, b_name = mm.inputs[1], mm.inputs[2]
        w, b = graph.tensor(w_name), graph.tensor(b_name)
        x = graph.tensor(x_name)
        if not (w.const and b.const and graph.tensor(lw).const and graph.tensor(lb).const):
            continue
        if w.dtype != "fp16" or len(w.shape) != 2 or len(b.shape) != 1 or len(x.shape) != 2:
            continue
        rows, feats = x.shape
        rows_ok = max_rows(rows) if callable(max_rows) else rows <= max_rows
        if feats % 256 or not rows_ok or w.shape[0] != feats or y in mm.inputs[1:]:
            continue
        n = w.shape[1]
        wf, b2 = f"lnfold{mm.id}.w", f"lnfold{mm.id}.bias2"
        if wf in tensors or b2 in tensors:
            raise FuseError(f"fold_layernorm: names {wf!r} / {b2!r} are taken")
        tensors[wf] = Tensor(wf, "fp16", (feats, n), const=True)
        tensors[b2] = Tensor(b2, "fp32", (2 * n,), const=True)
        derived[wf] = (LNFOLD_WEIGHT, (w_name, lw))
        derived[b2] = (LNFOLD_BIAS2, (w_name, lw, lb, b_name))
        attrs = {k: v for k, v in dict(mm.attrs).items() if k != "round"}
        attrs["eps"] = ln.attrs["eps"]
        replaced[mm.id] = Op(id=mm.id, kind="lnfold_matmul_epilogue",
                             inputs=(x_name, wf, b2) + tuple(mm.inputs[3:]), outputs=mm.outputs,
                             attrs=attrs)
        absorbed.add(ln.id)
        dropped.add(y)
    if not replaced:
        return graph, {}
    ops = tuple(replaced.get(op.id, op) for op in graph.ops if op.id not in absorbed)
    used = {n for op in ops for n in op.inputs + op.outputs} | set(graph.inputs) | set(graph.outputs)
    tensors = {n: t for n, t in tensors.items() if n not in dropped and n in used}
    return Graph(tensors=tensors, ops=ops, inputs=graph.inputs, outputs=graph.outputs), derived
