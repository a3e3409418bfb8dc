"""Oracle executors (test infrastructure only).

`run_fp32` restates the reference eager oracle (`hexlib/graph/eager.py:32-132`):
every dtype is held and computed as float32 (q4_0 as the float32 values it
represents), no storage rounding.

`run_stored` restates the plan executor's numerics (`hexlib/exec/interpreter.py:80-205`
with `hexlib/exec/vtcm.py:90-146`): compute in float32, and every op output
rounded to its declared storage dtype on the way out (`VtcmImage.put` rounds
fp16 slots; `get` widens back to float32). Consts are rounded to their declared
dtype once at load, which is what staging into a slot does. This equals the
reference's `interpreter.run` when every activation has a VTCM slot -- which
its own whole-plan builder requires (`hexlib/exec/wholeplan.py:227-233`
refuses any slot-less activation). Op order is the graph's topological order;
with no aliasing the result does not depend on the plan's step order.
"""
from __future__ import annotations

from typing import Mapping

import numpy as np

from oracle.refs import REFERENCES

_COMPUTE = {"fp32": np.float32, "fp16": np.float32, "int32": np.int32, "q4_0": np.float32,
            "q8_0": np.float32}
_STORE = {"fp32": np.float32, "fp16": np.float16, "int32": np.int32}


def _store(value: np.ndarray, dtype: str) -> np.ndarray:
    if dtype in _STORE:
        return np.asarray(value).astype(_STORE[dtype]).astype(_COMPUTE[dtype])
    return np.asarray(value, dtype=np.float32)


def _run(graph, feeds: Mapping[str, np.ndarray], rounding: bool) -> dict[str, np.ndarray]:
    problems = graph.problems()
    if problems:
        raise ValueError("invalid graph: " + "; ".join(problems))
    env: dict[str, np.ndarray] = {}
    needed = list(graph.inputs) + [t.name for t in graph.tensors.values() if t.const]
    for name in needed:
        if name not in feeds:
            raise KeyError(f"missing feed {name!r}")
        spec = graph.tensor(name)
        arr = np.asarray(feeds[name])
        if tuple(arr.shape) != spec.shape:
            raise ValueError(f"feed {name!r} is {arr.shape}, declared {spec.shape}")
        env[name] = _store(arr, spec.dtype) if rounding else arr.astype(_COMPUTE[spec.dtype])
    for op in graph.ops:
        outs = REFERENCES[op.kind](tuple(env[n] for n in op.inputs), op.attrs)
        if len(outs) != len(op.outputs):
            raise ValueError(f"op {op.id} ({op.kind}) produced {len(outs)} outputs")
        for name, value in zip(op.outputs, outs):
            spec = graph.tensor(name)
            if tuple(np.shape(value)) != spec.shape:
                raise ValueError(f"op {op.id} ({op.kind}) {name!r}: {np.shape(value)} != {spec.shape}")
            env[name] = _store(value, spec.dtype) if rounding else np.asarray(value).astype(_COMPUTE[spec.dtype])
    return {name: env[name] for name in graph.outputs}


def run_fp32(graph, feeds):
    return _run(graph, feeds, rounding=False)


def run_stored(graph, feeds):
    return _run(graph, feeds, rounding=True)
