"""Graph IR: logical tensors, ops and graphs. No layout, no placement.

Mirrors the reference's IR contract (`hexlib/graph/ir.py:15-225`): a tensor is
a name, a storage dtype and a static positive shape; an op reads and writes
tensors by name; a graph is valid only when every read follows a write and
every tensor is written once. Placement in device memory is decided later by
the whole-plan arena builder (`hexlib_amd.exec.wholeplan`), never here.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from types import MappingProxyType
from typing import Any, Mapping

# Storage dtypes a tensor may declare (reference `ir.py:15`).
DTYPES = frozenset({"fp32", "fp16", "int32", "q4_0", "q8_0"})

_ELEM_BYTES = {"fp32": 4, "fp16": 2, "int32": 4}

# Block formats: 32 values per block. q4_0 = fp16 scale + 16 nibble bytes,
# q8_0 = fp16 scale + 32 int8 (reference `ir.py:20-41`, llama.cpp's
# block_q4_0 / block_q8_0).
Q4_0_BLOCK = 32
Q4_0_BLOCK_BYTES = 18
Q8_0_BLOCK = 32
Q8_0_BLOCK_BYTES = 34

_BLOCK = {"q4_0": (Q4_0_BLOCK, Q4_0_BLOCK_BYTES), "q8_0": (Q8_0_BLOCK, Q8_0_BLOCK_BYTES)}


def nbytes(shape: tuple[int, ...], dtype: str) -> int:
    """Bytes a tensor of `shape` occupies in `dtype`.

    Block-quantized dtypes are blocked along the LAST axis, which must be a
    multiple of the block size (reference `ir.py:35-52`).
    """
    if dtype not in DTYPES:
        raise ValueError(f"unknown dtype {dtype!r}; known: {sorted(DTYPES)}")
    count = math.prod(shape) if shape else 1
    if dtype in _BLOCK:
        block, block_bytes = _BLOCK[dtype]
        last = shape[-1] if shape else 0
        if not shape or last % block:
            raise ValueError(
                f"{dtype} tensor {shape}: last dim {last} is not a multiple of "
                f"the {block}-element block"
            )
        return count // block * block_bytes
    return count * _ELEM_BYTES[dtype]


def _valid_attr(value: Any) -> bool:
    if isinstance(value, (bool, int, float, str, type(None))):
        return True
    if isinstance(value, tuple):
        return all(_valid_attr(v) for v in value)
    return False


@dataclass(frozen=True)
class Tensor:
    name: str
    dtype: str
    shape: tuple[int, ...]
    const: bool = False

    def __post_init__(self) -> None:
        if not self.name:
            raise ValueError("a tensor needs a non-empty name")
        if self.dtype not in DTYPES:
            raise ValueError(f"tensor {self.name!r}: unknown dtype {self.dtype!r}")
        if not isinstance(self.shape, tuple):
            raise TypeError(f"tensor {self.name!r}: shape must be a tuple")
        for d in self.shape:
            if isinstance(d, bool) or not isinstance(d, int) or d <= 0:
                raise ValueError(
                    f"tensor {self.name!r}: dim {d!r} is not a positive int; "
                    "shapes are static"
                )

    @property
    def nbytes(self) -> int:
        return nbytes(self.shape, self.dtype)


def _str_tuple(values, what: str) -> tuple[str, ...]:
    out = tuple(values)
    for i, v in enumerate(out):
        if not isinstance(v, str):
            raise TypeError(f"{what}[{i}] must be str, got {type(v).__name__}")
    return out


@dataclass(frozen=True)
class Op:
    id: int
    kind: str
    inputs: tuple[str, ...]
    outputs: tuple[str, ...]
    attrs: Mapping[str, Any] = field(default_factory=dict)

    def __post_init__(self) -> None:
        if not self.kind:
            raise ValueError(f"op {self.id}: empty kind")
        object.__setattr__(self, "inputs", _str_tuple(self.inputs, f"op {self.id} inputs"))
        object.__setattr__(self, "outputs", _str_tuple(self.outputs, f"op {self.id} outputs"))
        for key, value in self.attrs.items():
            if not _valid_attr(value):
                raise TypeError(
                    f"op {self.id}: attr {key!r} is a {type(value).__name__}; attrs "
                    "are scalars or tuples of scalars so plans stay serialisable"
                )
        object.__setattr__(self, "attrs", MappingProxyType(dict(self.attrs)))


@dataclass(frozen=True)
class Graph:
    tensors: Mapping[str, Tensor]
    ops: tuple[Op, ...]
    inputs: tuple[str, ...]
    outputs: tuple[str, ...]

    def __post_init__(self) -> None:
        object.__setattr__(self, "tensors", MappingProxyType(dict(self.tensors)))
        ops = tuple(self.ops)
        for i, op in enumerate(ops):
            if not isinstance(op, Op):
                raise TypeError(f"ops[{i}] must be Op, got {type(op).__name__}")
        object.__setattr__(self, "ops", ops)
        object.__setattr__(self, "inputs", _str_tuple(self.inputs, "inputs"))
        object.__setattr__(self, "outputs", _str_tuple(self.outputs, "outputs"))

    def tensor(self, name: str) -> Tensor:
        try:
            return self.tensors[name]
        except KeyError:
            raise KeyError(f"no tensor named {name!r} in this graph") from None

    def problems(self) -> list[str]:
        """Structural defects as readable strings; empty means valid. Covers
        what the reference validator rejects (`ir.py:175-225`): a graph must
        have ops and outputs, ids must be unique, every name an op or the graph
        touches must be declared, a tensor has exactly one producer (a graph
        input or const counts as one) and every read comes after it.

        Built as two passes: the first records, for every tensor, where its
        value comes from (a source or the position of its producing op) and
        flags second producers; the second checks each read against that
        table, so a read before its producer and a read of a tensor nobody
        produces are told apart."""
        bad: list[str] = []
        declared = self.tensors
        for key, t in declared.items():
            if key != t.name:
                bad.append(f"tensors[{key!r}] holds a tensor called {t.name!r}")
        if not self.ops:
            bad.append("empty graph: no ops to run")
        if not self.outputs:
            bad.append("empty graph: nothing marked as an output")

        SOURCE = -1
        origin: dict[str, int] = {}
        for name in self.inputs:
            if name not in declared:
                bad.append(f"input {name!r}: not in the tensor table")
            origin[name] = SOURCE
        for t in declared.values():
            if t.const:
                origin.setdefault(t.name, SOURCE)
        seen_ids: dict[int, int] = {}
        for pos, op in enumerate(self.ops):
            if op.id in seen_ids:
                bad.append(f"ops[{pos}] and ops[{seen_ids[op.id]}] share id {op.id}")
            seen_ids.setdefault(op.id, pos)
            for name in op.outputs:
                if name not in declared:
                    bad.append(f"{op.kind} #{op.id}: output {name!r} not in the tensor table")
                elif name in origin:
                    first = "a graph input or const" if origin[name] == SOURCE else \
                        f"{self.ops[origin[name]].kind} #{self.ops[origin[name]].id}"
                    bad.append(f"{op.kind} #{op.id}: output {name!r} already produced by {first}")
                else:
                    origin[name] = pos

        for pos, op in enumerate(self.ops):
            for name in op.inputs:
                if name not in declared:
                    bad.append(f"{op.kind} #{op.id}: input {name!r} not in the tensor table")
                elif name not in origin:
                    bad.append(f"{op.kind} #{op.id}: input {name!r} has no producer")
                elif origin[name] >= pos:
                    bad.append(f"{op.kind} #{op.id}: input {name!r} is produced later, by op "
                               f"#{self.ops[origin[name]].id}")
        for name in self.outputs:
            if name not in declared:
                bad.append(f"output {name!r}: not in the tensor table")
            elif name not in origin:
                bad.append(f"output {name!r}: no op produces it")
        return bad
