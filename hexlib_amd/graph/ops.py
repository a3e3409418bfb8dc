"""Op registry: one record per op kind, holding what the host needs to plan it.

The reference keeps `infer`, `working_set` and a numpy `reference` in one
`OpDef` (`hexlib/graph/ops.py:16-40`). Here the record holds only the
planning half (`infer`); the numpy references are the checker's and live in
the test-only `oracle` package, so nothing on the GPU path can reach them.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable


@dataclass(frozen=True)
class OpDef:
    """`infer(inputs: tuple[Tensor], attrs) -> ((shape, dtype), ...)`, one
    pair per output."""

    kind: str
    infer: Callable[..., Any]

    def __post_init__(self) -> None:
        if not self.kind:
            raise ValueError("OpDef needs a kind")
        if not callable(self.infer):
            raise TypeError(f"OpDef {self.kind!r}: infer must be callable")


_DEFS: dict[str, OpDef] = {}


def register(opdef: OpDef) -> None:
    if opdef.kind in _DEFS:
        raise ValueError(f"op kind {opdef.kind!r} registered twice")
    _DEFS[opdef.kind] = opdef


def get(kind: str) -> OpDef:
    try:
        return _DEFS[kind]
    except KeyError:
        raise KeyError(
            f"no OpDef for {kind!r}; registered: {', '.join(sorted(_DEFS))}. "
            "An unregistered op is an error, never a no-op."
        ) from None


def all_kinds() -> tuple[str, ...]:
    return tuple(sorted(_DEFS))
