"""Python side of the GPU session: the drop-in for the reference's DSP backends.

* `GpuSession` wraps `hexlib_gpu_open/start/mmap/invoke/stop/close` (the
  reference IDL lifecycle, `hexlib/runtime/idl/hexlib_iface.idl:28-67`) and
  checks every response the way the reference host does
  (`hexlib/exec/dsp.py:523-549`): batch status, op count, kind echo per op,
  per-op status.
* `GpuPlan` is the whole-plan path (`hexlib/exec/wholeplan.py` +
  `test_wholeplan.py:181`): one device arena, one registered buffer, one blob;
  `run()` replays it, by default as one captured hipGraph launch.
* `GpuBackend.run(kind, arrays, attrs)` is the per-op path
  (`hexlib/exec/dsp.py:382-561`): one op per blob through the same dispatcher
  and generated entries.

Device memory comes from torch (plumbing only); every computation runs in
libhexlib_gpu.so. There is no CPU fallback: without the library or a GPU this
module raises.
"""
from __future__ import annotations

import ctypes
import time
from typing import Any, Mapping, Sequence

import numpy as np

from hexlib_amd import lib as _lib
from hexlib_amd.exec import wire
from hexlib_amd.exec.runner import KIND_ID, WIRE_RAW, select
from hexlib_amd.exec.wholeplan import ALIGN, WholePlanBatch, align_up, decode, stage_col_major_rope
from hexlib_amd.quant import pack_q4_0_kgrouped, pack_q4_0_nblocked, pack_q8_0_kgrouped


class GpuError(RuntimeError):
    pass


def _torch():
    import torch

    if not torch.cuda.is_available():
        raise GpuError("no GPU visible: hexlib_amd's GPU path has no CPU fallback")
    return torch


class GpuSession:
    def __init__(self, device: int = 0, sess_id: int = 0):
        self.lib = _lib.load()
        self.device = device
        h = ctypes.c_void_p()
        rc = self.lib.hexlib_gpu_open(ctypes.byref(h))
        if rc != wire.STATUS["OK"]:
            raise GpuError(f"hexlib_gpu_open: {wire.STATUS_NAME.get(rc, rc)}")
        self.h = h
        rc = self.lib.hexlib_gpu_start(self.h, sess_id, device, 0)
        if rc != wire.STATUS["OK"]:
            self.lib.hexlib_gpu_close(self.h)
            self.h = None
            raise GpuError(f"hexlib_gpu_start: {wire.STATUS_NAME.get(rc, rc)}")
        self._rsp = None

    def close(self) -> None:
        if getattr(self, "h", None):
            self.lib.hexlib_gpu_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def stream(self) -> int:
        return self.lib.hexlib_gpu_session_stream(self.h) or 0

    def mmap(self, fd: int, dev_ptr: int, size: int) -> None:
        rc = self.lib.hexlib_gpu_mmap(self.h, fd, ctypes.c_void_p(dev_ptr), size)
        if rc != wire.STATUS["OK"]:
            raise GpuError(f"hexlib_gpu_mmap(fd={fd}): {wire.STATUS_NAME.get(rc, rc)}")

    def munmap(self, fd: int) -> None:
        self.lib.hexlib_gpu_munmap(self.h, fd)

    def hwinfo(self) -> dict:
        a, n, t, l = (ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64())
        rc = self.lib.hexlib_gpu_hwinfo(self.h, ctypes.byref(a), ctypes.byref(n), ctypes.byref(t),
                                       ctypes.byref(l))
        if rc != wire.STATUS["OK"]:
            raise GpuError(f"hwinfo: {wire.STATUS_NAME.get(rc, rc)}")
        return {"arch": a.value, "n_cu": n.value, "n_threads": t.value, "lds_per_cu": l.value}

    def invoke_raw(self, blob: bytes, flags: int = 0, n_ops_hint: int | None = None) -> wire.BatchResponse:
        n_ops = n_ops_hint if n_ops_hint is not None else _blob_n_ops(blob)
        cap = wire.RSP_HDR_SIZE + wire.RESULT_SIZE * max(n_ops, 0)
        if self._rsp is None or len(self._rsp) < cap:
            self._rsp = ctypes.create_string_buffer(cap)
        out_len = ctypes.c_uint32()
        self.lib.hexlib_gpu_invoke(self.h, blob, len(blob), self._rsp, cap, ctypes.byref(out_len), flags)
        return wire.unpack_response(self._rsp.raw[:out_len.value])

    def invoke(self, blob: bytes, kinds: Sequence[int], flags: int = 0) -> wire.BatchResponse:
        rsp = self.invoke_raw(blob, flags, len(kinds))
        if rsp.status != wire.STATUS["OK"]:
            bad = next((i for i, r in enumerate(rsp.results) if not r.ok), None)
            raise GpuError(f"invoke status {wire.STATUS_NAME.get(rsp.status, rsp.status)}"
                           + (f" at op {bad} (kind {rsp.results[bad].kind})" if bad is not None else ""))
        if rsp.n_ops != len(kinds):
            raise GpuError(f"blob carried {len(kinds)} ops, response reports {rsp.n_ops}")
        for i, (r, k) in enumerate(zip(rsp.results, kinds)):
            if r.kind != k:
                raise GpuError(f"op {i}: asked kind {k}, response answers kind {r.kind}")
            if not r.ok:
                raise GpuError(f"op {i}: status {wire.STATUS_NAME.get(r.status, r.status)}")
        return rsp


def _blob_n_ops(blob: bytes) -> int:
    if len(blob) < wire.HDR_SIZE:
        return 0
    return int.from_bytes(blob[20:24], "little")


def blob_kinds(blob: bytes) -> list[int]:
    import struct

    hdr = struct.unpack_from(wire._HDR, blob)
    n_ops, off_ops = hdr[5], hdr[8]
    return [struct.unpack_from("<I", blob, off_ops + i * wire.OP_SIZE)[0] for i in range(n_ops)]


class GpuPlan:
    """A whole plan resident on the GPU: arena allocated and staged once."""

    def __init__(self, batch: WholePlanBatch, session: GpuSession | None = None, fd: int = 0):
        torch = _torch()
        self.torch = torch
        self.batch = batch
        self.session = session or GpuSession()
        self._own_session = session is None
        self.arena = torch.empty(batch.arena_bytes, dtype=torch.uint8, device=f"cuda:{self.session.device}")
        host = torch.frombuffer(bytearray(batch.payload), dtype=torch.uint8)
        self.arena.copy_(host)
        torch.cuda.synchronize()
        self.session.mmap(fd, self.arena.data_ptr(), batch.arena_bytes)
        self.kinds = blob_kinds(batch.blob)

    def close(self):
        self.session.munmap(0)
        if self._own_session:
            self.session.close()

    def set_input(self, name: str, value: np.ndarray) -> None:
        p = self.batch.placements[name]
        data = np.ascontiguousarray(value, dtype=np.float16 if p.dtype == "fp16" else np.float32)
        t = self.torch.from_numpy(data.view(np.uint8).reshape(-1).copy())
        self.arena[p.offset:p.offset + p.nbytes].copy_(t)
        self.torch.cuda.synchronize()

    def run(self, graph: bool = True, timed: bool = False, sync: bool = True) -> wire.BatchResponse:
        flags = (_lib.INVOKE_GRAPH if graph else 0) | (_lib.INVOKE_TIMED if timed else 0)
        if not sync:
            flags |= _lib.INVOKE_NOSYNC
        return self.session.invoke(self.batch.blob, self.kinds, flags)

    def read(self, name: str) -> np.ndarray:
        p = self.batch.placements[name]
        raw = self.arena[p.offset:p.offset + p.nbytes].cpu().numpy().tobytes()
        return decode(self.batch, name, raw)

    def outputs(self) -> dict[str, np.ndarray]:
        return {n: self.read(n) for n in self.batch.outputs}


class GpuBackend:
    """One op per blob through the dispatcher -- the per-op drop-in for the
    reference's `DspSimBackend.run` (`hexlib/exec/dsp.py:382-561`)."""

    def __init__(self, session: GpuSession | None = None):
        self.torch = _torch()
        self.session = session or GpuSession()
        self._buf = None
        self._fd = 7

    def run(self, kind: str, arrays: Sequence[Any], attrs: Mapping[str, Any],
            out_shape: tuple[int, ...], weight_layout: str | None = None,
            in_dtypes: Sequence[str] | None = None):
        name, spec = select(kind, attrs, in_dtypes, weight_layout)
        spec.check_requires(attrs)
        spec.check_rank([a[1] if isinstance(a, tuple) else np.shape(a) for a in arrays])
        if len(arrays) != len(spec.inputs):
            raise GpuError(f"{kind} takes {len(spec.inputs)} inputs, got {len(arrays)}")
        lays = spec.buf_layouts()
        payload = bytearray()
        tensors, shapes = [], []
        for i, (a, dt) in enumerate(zip(arrays, spec.inputs)):
            if dt in WIRE_RAW:
                if isinstance(a, tuple):          # (bytes, logical shape)
                    data, shape = a
                else:
                    arr = np.asarray(a, dtype=np.float32)
                    shape = arr.shape
                    data = (pack_q8_0_kgrouped(arr) if lays[i] == "q8_0_kgroup" else
                            pack_q4_0_kgrouped(arr) if lays[i] == "q4_0_kgroup" else pack_q4_0_nblocked(arr))
            else:
                arr = np.ascontiguousarray(a, dtype=np.float16 if dt == "fp16" else np.float32)
                shape = arr.shape
                if lays[i] == "col_major_rope":
                    data = stage_col_major_rope(arr, int(attrs["rope_heads"]), int(attrs["rope_dim"]))
                else:
                    data = (np.ascontiguousarray(arr.T) if lays[i] == "col_major" else arr).tobytes()
            off = len(payload)
            tensors.append(wire.TensorDesc(0, off, len(data), dt, lays[i], wire.pad_ne(shape)))
            shapes.append(tuple(shape))
            payload += data
            payload += b"\0" * (align_up(len(payload), ALIGN) - len(payload))
        odt = np.float16 if spec.out_dtype == "fp16" else np.float32
        out_bytes = int(np.prod(out_shape)) * np.dtype(odt).itemsize
        out_off = len(payload)
        tensors.append(wire.TensorDesc(0, out_off, out_bytes, spec.out_dtype, lays[-1],
                                       wire.pad_ne(out_shape)))
        payload += b"\0" * out_bytes
        size = align_up(len(payload), ALIGN)
        payload += b"\0" * (size - len(payload))
        torch = self.torch
        buf = torch.from_numpy(np.frombuffer(bytes(payload), dtype=np.uint8).copy()).to(
            f"cuda:{self.session.device}")
        torch.cuda.synchronize()
        self.session.mmap(self._fd, buf.data_ptr(), size)
        try:
            ops = [wire.OpDesc(KIND_ID[name], spec.params(shapes, attrs),
                               tuple(range(len(arrays))), (len(arrays),))]
            blob = wire.pack_batch([wire.BufDesc(self._fd, size)], tensors, ops)
            t0 = time.perf_counter()
            rsp = self.session.invoke(blob, [KIND_ID[name]], _lib.INVOKE_TIMED)
            _ = time.perf_counter() - t0
            raw = buf[out_off:out_off + out_bytes].cpu().numpy().tobytes()
        finally:
            self.session.munmap(self._fd)
        return np.frombuffer(raw, dtype=odt).reshape(out_shape), rsp


class _Meta:
    """Shape/dtype stand-in handed to an OpDef's infer."""

    def __init__(self, shape, dtype, name="input"):
        self.shape = tuple(shape)
        self.dtype = dtype
        self.name = name


def interpreter_backends(gpu: GpuBackend, kinds=None) -> dict:
    """One plan-executor backend per op kind that has a GPU kernel -- the
    drop-in for the reference's `interpreter_backends(sim, kinds)`
    (`hexlib/exec/dsp.py:656-715`): `{kind: backend(arrays, attrs) -> (out,)}`.

    As there, the variant is resolved per call from the op's attrs (`select`),
    an op no variant accepts is refused, and a dense weight whose spec declares
    q4_0 is quantized on the way in -- the kernel then multiplies with the 4-bit
    weight, so an accuracy comparison must be made against the dequantized
    bytes, not the fp32 original. The output shape comes from the op's infer.
    """
    from hexlib_amd.exec.runner import SPECS
    from hexlib_amd.graph import ops as graph_ops

    available = sorted({spec.kind for spec in SPECS.values()} - {"reshape"})
    wanted = available if kinds is None else [k for k in kinds if k in available]

    def make(kind: str):
        def backend(arrays, attrs):
            metas = [_Meta(np.shape(a), "fp32") for a in arrays]
            ((out_shape, _),) = graph_ops.get(kind).infer(metas, dict(attrs))
            out, _ = gpu.run(kind, list(arrays), dict(attrs), tuple(out_shape))
            return (out,)

        return backend

    return {kind: make(kind) for kind in wanted}
