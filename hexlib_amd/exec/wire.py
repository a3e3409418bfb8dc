"""The batch blob and response format (byte-identical to the reference's).

Restates `hexlib/runtime/wire.py:23-234` and `hexlib/runtime/skel/hexlib_dsp.h:18-210`:
header, buffer descriptors, tensor descriptors and op descriptors, all
little-endian, with NO address field on the wire (the GPU side resolves each
buffer through its own registration table, exactly as the DSP resolves fds).
Status codes are shared with the C side; OK is 1 so a zeroed response never
reads as success. The C structs in `include/hexlib_gpu.h` are the same layout
and `tests/test_wire.py` binds the two through the library's size probe.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

BATCH_MAGIC = 0x424C5848  # 'HXLB'
BATCH_VERSION = 1

MAX_BUFS = 8
MAX_SRC = 6
MAX_DST = 4
MAX_PARAMS = 16
# 512 on the DSP (static working copies); the GPU session accepts 4096.
MAX_TENSORS = 4096

STATUS = {
    "OK": 1, "ERR_INTERNAL": 2, "ERR_BAD_MAGIC": 3, "ERR_BAD_VERSION": 4,
    "ERR_TRUNCATED": 5, "ERR_INVAL_PARAMS": 6, "ERR_UNMAPPED": 7,
    "ERR_NO_MMAP_SLOT": 8, "ERR_MMAP_FAILED": 9, "ERR_NO_KERNEL": 10,
    "ERR_VTCM_TOO_SMALL": 11, "ERR_VTCM_RECLAIMED": 12, "ERR_REQUIRES": 13,
    "ERR_NOT_STARTED": 14, "ERR_CACHE": 15,
}
STATUS_NAME = {v: k for k, v in STATUS.items()}

# Wire ids. The first three layouts are the reference's; appended:
# `q4_0_kgroup` (q4_0 blocks along K of W^T), `col_major` (a [K, N] weight
# stored as W^T [N, K]) and `col_major_rope` (col_major with the rows of each
# rope head pair-interleaved: row 2i = feature i, row 2i + 1 = feature i + D/2)
# and `q8_0_kgroup` (q8_0 blocks along K of W^T), `q8_0_kgroup_rope`
# (q8_0_kgroup of the col_major_rope row order).
DTYPE_ID = {"fp32": 0, "fp16": 1, "q4_0": 2, "int32": 3, "q8_0": 4}
LAYOUT_ID = {"row_major": 0, "tiled_32x32": 1, "q4_0_repacked": 2, "q4_0_kgroup": 3,
             "col_major": 4, "col_major_rope": 5, "q8_0_kgroup": 6, "q8_0_kgroup_rope": 7}

_HDR = "<10I"
_BUF = "<QQII"
_TENSOR = "<11I"
_OP = f"<II{MAX_PARAMS}i{MAX_SRC}H{MAX_DST}H"
_RSP_HDR = "<IIIIQII"
_RESULT = "<IIQ"

HDR_SIZE = struct.calcsize(_HDR)
BUF_SIZE = struct.calcsize(_BUF)
TENSOR_SIZE = struct.calcsize(_TENSOR)
OP_SIZE = struct.calcsize(_OP)
RSP_HDR_SIZE = struct.calcsize(_RSP_HDR)
RESULT_SIZE = struct.calcsize(_RESULT)

NO_TENSOR = 0xFFFF


class WireError(Exception):
    pass


@dataclass(frozen=True)
class BufDesc:
    fd: int
    size: int
    flags: int = 0


@dataclass(frozen=True)
class TensorDesc:
    bi: int
    offset: int
    nbytes: int
    dtype: str
    layout: str
    ne: tuple[int, int, int, int]


@dataclass(frozen=True)
class OpDesc:
    kind: int
    params: tuple[int, ...] = ()
    src: tuple[int, ...] = ()
    dst: tuple[int, ...] = ()
    flags: int = 0


@dataclass(frozen=True)
class OpResult:
    kind: int
    status: int
    cycles: int

    @property
    def ok(self) -> bool:
        return self.status == STATUS["OK"]


@dataclass(frozen=True)
class BatchResponse:
    status: int
    n_ops: int
    cycles_total: int
    arch: int
    results: tuple[OpResult, ...] = field(default=())

    @property
    def ok(self) -> bool:
        return self.status == STATUS["OK"] and all(r.ok for r in self.results)


def pad_ne(shape) -> tuple[int, int, int, int]:
    if len(shape) > 4:
        raise WireError(f"shape {tuple(shape)} has more than 4 dims")
    return tuple(int(s) for s in shape) + (1,) * (4 - len(shape))  # type: ignore[return-value]


def pack_batch(bufs, tensors, ops) -> bytes:
    """Serialise a batch, refusing malformed input on the host first
    (reference `wire.py:135-208`)."""
    if len(bufs) > MAX_BUFS:
        raise WireError(f"{len(bufs)} buffers > MAX_BUFS {MAX_BUFS}")
    if len(tensors) > MAX_TENSORS:
        raise WireError(f"{len(tensors)} tensors > MAX_TENSORS {MAX_TENSORS}")
    for i, t in enumerate(tensors):
        if not 0 <= t.bi < len(bufs):
            raise WireError(f"tensor {i} names buffer {t.bi} of {len(bufs)}")
        if t.offset + t.nbytes > bufs[t.bi].size:
            raise WireError(f"tensor {i} ends at {t.offset + t.nbytes} > buffer size {bufs[t.bi].size}")
        if t.dtype not in DTYPE_ID:
            raise WireError(f"tensor {i}: unknown dtype {t.dtype!r}")
        if t.layout not in LAYOUT_ID:
            raise WireError(f"tensor {i}: unknown layout {t.layout!r}")
    for i, op in enumerate(ops):
        if len(op.params) > MAX_PARAMS:
            raise WireError(f"op {i}: {len(op.params)} params > {MAX_PARAMS}")
        if len(op.src) > MAX_SRC or len(op.dst) > MAX_DST:
            raise WireError(f"op {i}: too many sources or destinations")
        if len(op.src) + len(op.dst) > MAX_BUFS:
            raise WireError(f"op {i}: {len(op.src)} + {len(op.dst)} buffers > MAX_BUFS {MAX_BUFS}")
        for j in tuple(op.src) + tuple(op.dst):
            if not 0 <= j < len(tensors):
                raise WireError(f"op {i} names tensor {j}, out of range")
    off_bufs = HDR_SIZE
    off_tensors = off_bufs + BUF_SIZE * len(bufs)
    off_ops = off_tensors + TENSOR_SIZE * len(tensors)
    total = off_ops + OP_SIZE * len(ops)
    out = bytearray(struct.pack(_HDR, BATCH_MAGIC, BATCH_VERSION, total, len(bufs),
                                len(tensors), len(ops), off_bufs, off_tensors, off_ops, 0))
    for b in bufs:
        out += struct.pack(_BUF, 0, b.size, b.fd, b.flags)
    for t in tensors:
        out += struct.pack(_TENSOR, t.bi, t.offset, t.nbytes, DTYPE_ID[t.dtype],
                           LAYOUT_ID[t.layout], *t.ne, 0, 0)
    for op in ops:
        params = tuple(op.params) + (0,) * (MAX_PARAMS - len(op.params))
        src = tuple(op.src) + (NO_TENSOR,) * (MAX_SRC - len(op.src))
        dst = tuple(op.dst) + (NO_TENSOR,) * (MAX_DST - len(op.dst))
        out += struct.pack(_OP, op.kind, op.flags, *params, *src, *dst)
    if len(out) != total:
        raise WireError("internal: blob length disagrees with its header")
    return bytes(out)


def unpack_response(raw: bytes) -> BatchResponse:
    if len(raw) < RSP_HDR_SIZE:
        raise WireError(f"response truncated: {len(raw)} < {RSP_HDR_SIZE}")
    magic, version, status, n_ops, cycles, arch, _ = struct.unpack_from(_RSP_HDR, raw)
    if magic != BATCH_MAGIC:
        raise WireError(f"response magic 0x{magic:08x} != 0x{BATCH_MAGIC:08x}")
    if version != BATCH_VERSION:
        raise WireError(f"response version {version} != {BATCH_VERSION}")
    if status not in STATUS_NAME:
        raise WireError(f"response status {status} is unknown")
    need = RSP_HDR_SIZE + RESULT_SIZE * n_ops
    if len(raw) < need:
        raise WireError(f"response claims {n_ops} results ({need} bytes), has {len(raw)}")
    results = tuple(OpResult(*struct.unpack_from(_RESULT, raw, RSP_HDR_SIZE + i * RESULT_SIZE))
                    for i in range(n_ops))
    return BatchResponse(status, n_ops, cycles, arch, results)


def float_param(value: float) -> int:
    """A float attr crosses as its IEEE-754 bits in an int32 slot
    (reference `hexlib/exec/dsp.py:286-305`)."""
    return struct.unpack("<i", struct.pack("<f", float(value)))[0]
