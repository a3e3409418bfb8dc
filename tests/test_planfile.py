"""Whole-plan files on the CPU: the writer's format, the C library's parser
and dry-run validation (`hexlib_gpu_plan_inspect`, no HIP call), refusal of
malformed files, and the committed artefact being current."""
import ctypes
import os
import struct

import numpy as np
import pytest

from hexlib_amd import encoder as E
from hexlib_amd import lib as L
from hexlib_amd.exec import planfile, wire
from hexlib_amd.exec.wholeplan import build_whole_plan_batch
from tests.golden import make_tiny_plan as G

OK = wire.STATUS["OK"]


@pytest.fixture(scope="module")
def tiny():
    return G.build()


def inspect(path):
    info = L.PlanInfo()
    return L.load().hexlib_gpu_plan_inspect(str(path).encode(), ctypes.byref(info)), info


def test_round_trip(tiny, tmp_path):
    g, feeds, wb = tiny
    path = tmp_path / "p.hxplan"
    planfile.save(wb, str(path))
    pf = planfile.load(str(path))
    assert pf.blob == wb.blob and pf.arena_bytes == wb.arena_bytes
    assert pf.const_image == bytes(wb.payload[:wb.const_bytes])
    (inp,), (out,) = [e for e in pf.io if e.role == 0], [e for e in pf.io if e.role == 1]
    p = wb.placements["image"]
    assert (inp.name, inp.offset, inp.nbytes, inp.dtype) == ("image", p.offset, p.nbytes, "fp32")
    assert inp.data == bytes(wb.payload[p.offset:p.offset + p.nbytes])
    assert out.name == g.outputs[0] and out.data is None and out.dtype == "fp16"
    assert out.offset == wb.placements[out.name].offset


def test_the_library_parses_and_dry_runs_it(tiny, tmp_path):
    _, _, wb = tiny
    path = tmp_path / "p.hxplan"
    planfile.save(wb, str(path))
    rc, info = inspect(path)
    assert rc == OK
    assert (info.version, info.n_io, info.n_ops, info.arena_bytes, info.const_bytes, info.blob_bytes) == (
        1, 2, wb.n_ops, wb.arena_bytes, wb.const_bytes, len(wb.blob))


def _corrupt(raw, off, fmt, value):
    b = bytearray(raw)
    struct.pack_into(fmt, b, off, value)
    return bytes(b)


@pytest.mark.parametrize("how,want", [
    ("magic", "ERR_BAD_MAGIC"), ("version", "ERR_BAD_VERSION"), ("truncated", "ERR_TRUNCATED"),
    ("const_past_arena", "ERR_INVAL_PARAMS"), ("io_past_arena", "ERR_INVAL_PARAMS"),
    ("input_data_past_section", "ERR_INVAL_PARAMS"), ("unknown_kind", "ERR_NO_KERNEL"),
    ("arena_too_small_for_blob", "ERR_INVAL_PARAMS")])
def test_malformed_files_are_refused(tiny, tmp_path, how, want):
    _, _, wb = tiny
    raw = planfile.to_bytes(wb)
    n_io = struct.unpack_from("<I", raw, 40)[0]
    blob_at = 64 + 96 * n_io
    if how == "magic":
        raw = raw[:3] + b"Y" + raw[4:]
    elif how == "version":
        raw = _corrupt(raw, 8, "<I", 2)
    elif how == "truncated":
        raw = raw[:-1]
    elif how == "const_past_arena":
        raw = _corrupt(raw, 24, "<Q", wb.arena_bytes + 1)
    elif how == "io_past_arena":
        raw = _corrupt(raw, 64 + 56, "<Q", wb.arena_bytes - 4)
    elif how == "input_data_past_section":
        raw = _corrupt(raw, 64 + 88, "<Q", 1 << 20)
    elif how == "unknown_kind":
        hdr = struct.unpack_from(wire._HDR, raw, blob_at)
        n_buf, n_t = hdr[3], hdr[4]
        op0 = blob_at + wire.HDR_SIZE + n_buf * wire.BUF_SIZE + n_t * wire.TENSOR_SIZE
        raw = _corrupt(raw, op0, "<I", 99)
    elif how == "arena_too_small_for_blob":
        raw = _corrupt(raw, 16, "<Q", wb.const_bytes)
    path = tmp_path / "bad.hxplan"
    path.write_bytes(raw)
    rc, _ = inspect(path)
    assert rc == wire.STATUS[want], (how, rc)


def test_committed_artefact_is_current(tiny):
    """tests/golden/tiny_encoder.hxplan is what the current builder writes for
    the cfg-1 encoder, and tiny_encoder_out.npy the oracle's output for it
    (regenerate both with tests/golden/make_tiny_plan.py)."""
    g, feeds, wb = tiny
    with open(G.PLAN, "rb") as f:
        assert f.read() == planfile.to_bytes(wb)
    np.testing.assert_array_equal(np.load(G.EXPECTED, allow_pickle=False), G.expected(g, feeds))
    rc, info = inspect(G.PLAN)
    assert rc == OK and info.n_ops == wb.n_ops


def test_names_longer_than_the_field_are_refused():
    from dataclasses import replace
    cfg = E.TINY_ENCODER
    g = E.build_vision_encoder(cfg)
    wb = build_whole_plan_batch(g, E.synthetic_feeds(g, cfg))
    long = "x" * 48
    wb2 = replace(wb, inputs=(long,), placements={**wb.placements, long: wb.placements["image"]})
    with pytest.raises(planfile.PlanFileError):
        planfile.to_bytes(wb2)
