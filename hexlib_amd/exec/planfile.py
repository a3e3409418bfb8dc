"""Whole-plan files: a `WholePlanBatch` written to disk and replayed by the C
library (`hexlib_gpu_plan_load` / `hexlib_gpu_plan_run`) or the
`hxplan_replay` program with no Python on the host.

The reference builds the whole-plan batch in Python on every run
(`hexlib/exec/wholeplan.py:92-357`; `hexlib/tests/test_wholeplan.py:181-183`
hands blob and arena image to the simulator). Here the batch is an artefact.
Layout (little-endian, sections back to back; `hexlib_amd/csrc/planfile.cpp`
is the reader):

    header  64 B   b"HXPLAN1\\0", u32 version 1, u32 fd, u64 arena_bytes,
                   u64 const_bytes, u64 blob_bytes, u32 n_io, u32 0,
                   u64 data_bytes, u64 0
    io      n_io x 96 B: name[48], u32 role (0 input, 1 output), u32 wire
                   dtype id, u64 arena offset, u64 nbytes, u32 ne[4],
                   u64 data offset (a stored sample input) or 2**64 - 1
    blob    the wire batch (`wire.pack_batch`)
    const   arena[0, const_bytes): the staged constants (weights, tables)
    data    stored sample inputs

Reshapes were already unified with their sources before allocation by
`build_whole_plan_batch`, so the blob names no reshape op and every alias
shares its source's bytes.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

from hexlib_amd.exec import wire
from hexlib_amd.exec.wholeplan import WholePlanBatch

MAGIC = b"HXPLAN1\0"
VERSION = 1
NO_DATA = (1 << 64) - 1
_HDR = "<8sIIQQQIIQQ"
_IO = "<48sIIQQ4IQ"
assert struct.calcsize(_HDR) == 64 and struct.calcsize(_IO) == 96


class PlanFileError(ValueError):
    pass


@dataclass(frozen=True)
class PlanIO:
    name: str
    role: int
    dtype: str
    offset: int
    nbytes: int
    ne: tuple[int, int, int, int]
    data: bytes | None


@dataclass(frozen=True)
class PlanFile:
    fd: int
    arena_bytes: int
    blob: bytes
    const_image: bytes
    io: tuple[PlanIO, ...]


def to_bytes(batch: WholePlanBatch, fd: int = 0, with_inputs: bool = True) -> bytes:
    """The file's bytes. `with_inputs` stores the batch's staged inputs as
    sample values, so the file replays to a known output on its own."""
    dtype_ids = wire.DTYPE_ID
    entries, data = [], bytearray()
    for role, names in ((0, batch.inputs), (1, batch.outputs)):
        for name in names:
            p = batch.placements[name]
            if len(name.encode()) >= 48:
                raise PlanFileError(f"tensor name {name!r} is longer than 47 bytes")
            doff = NO_DATA
            if role == 0 and with_inputs:
                doff = len(data)
                data += bytes(batch.payload[p.offset:p.offset + p.nbytes])
            entries.append(struct.pack(_IO, name.encode(), role, dtype_ids[p.dtype], p.offset, p.nbytes,
                                       *p.ne, doff))
    const = bytes(batch.payload[:batch.const_bytes])
    head = struct.pack(_HDR, MAGIC, VERSION, fd, batch.arena_bytes, len(const), len(batch.blob),
                       len(entries), 0, len(data), 0)
    return head + b"".join(entries) + batch.blob + const + bytes(data)


def save(batch: WholePlanBatch, path: str, fd: int = 0, with_inputs: bool = True) -> int:
    raw = to_bytes(batch, fd, with_inputs)
    with open(path, "wb") as f:
        f.write(raw)
    return len(raw)


def parse(raw: bytes) -> PlanFile:
    if len(raw) < 64:
        raise PlanFileError("shorter than the header")
    magic, version, fd, arena, cbytes, bbytes, n_io, _, dbytes, _ = struct.unpack_from(_HDR, raw, 0)
    if magic != MAGIC:
        raise PlanFileError("bad magic")
    if version != VERSION:
        raise PlanFileError(f"version {version}")
    if 64 + 96 * n_io + bbytes + cbytes + dbytes != len(raw):
        raise PlanFileError("section sizes do not add up to the file size")
    pos = 64 + 96 * n_io
    blob = raw[pos:pos + bbytes]
    const = raw[pos + bbytes:pos + bbytes + cbytes]
    data = raw[pos + bbytes + cbytes:]
    ids = {v: k for k, v in wire.DTYPE_ID.items()}
    io = []
    for i in range(n_io):
        name, role, dt, off, nb, n0, n1, n2, n3, doff = struct.unpack_from(_IO, raw, 64 + 96 * i)
        io.append(PlanIO(name.rstrip(b"\0").decode(), role, ids[dt], off, nb, (n0, n1, n2, n3),
                         None if doff == NO_DATA else data[doff:doff + nb]))
    return PlanFile(fd, arena, blob, const, tuple(io))


def load(path: str) -> PlanFile:
    with open(path, "rb") as f:
        return parse(f.read())
