"""Whole-plan files on the GPU: the committed cfg-1 artefact and the cfg-4
product plan replayed by the C program `hxplan_replay` (no Python in the
replaying process) and through the plan API, against the Python session
running the same batch (bit-identical: same blob, same kernels) and the
oracle's output."""
import ctypes
import json
import os
import subprocess
import sys

import numpy as np
import pytest

from hexlib_amd import build as B
from hexlib_amd import encoder as E
from hexlib_amd import lib as L
from hexlib_amd.exec import planfile, wire
from hexlib_amd.exec.gpu import GpuPlan, GpuSession
from tests.golden import make_tiny_plan as G

pytestmark = pytest.mark.gpu
OK = wire.STATUS["OK"]


@pytest.fixture(scope="module")
def session(torch_gpu):
    s = GpuSession()
    yield s
    s.close()


def replay(plan_path, outdir, *extra):
    print(f"[hxplan_replay] {plan_path}", flush=True)
    proc = subprocess.run([B.REPLAY_PATH, str(plan_path), str(outdir), "--reps", "5", *extra],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stderr
    return json.loads(proc.stdout.strip().splitlines()[-1])


def _python_run(session, wb):
    plan = GpuPlan(wb, session)
    try:
        rsp = plan.run(graph=True)
        assert rsp.ok
        return {n: plan.read(n) for n in wb.outputs}
    finally:
        plan.close()


def test_replay_the_committed_artefact(session, tmp_path):
    g, feeds, wb = G.build()
    info = replay(G.PLAN, tmp_path)
    assert info["ops"] == wb.n_ops
    name = g.outputs[0]
    got = np.fromfile(tmp_path / f"{name}.bin", dtype=np.float16).reshape(g.tensor(name).shape)
    want_py = _python_run(session, wb)[name].astype(np.float16)
    np.testing.assert_array_equal(got.view(np.uint16), want_py.view(np.uint16))
    err = np.abs(got.astype(np.float32) - np.load(G.EXPECTED, allow_pickle=False).astype(np.float32)).max()
    print(f"[cfg-1 artefact] {info['gpu_ns_per_run'] / 1e3:.1f} us per replay; max abs vs oracle {err:.3e}",
          flush=True)
    assert err <= 2e-2


def test_product_plan_replays_bit_identically(session, tmp_path):
    """The bench's cfg-4 product plan (fused q/k/v with rope, fused attention,
    residual epilogues) from a file, with the sample image and with another
    image given on the command line."""
    from dataclasses import replace
    from hexlib_amd.exec.wholeplan import build_whole_plan_batch
    cfg = replace(E.QWEN35_VISION_FP16, attention="fused_qkv_rope")
    g = E.build_vision_encoder(cfg)
    feeds = E.synthetic_feeds(g, cfg, seed=2)
    wb = build_whole_plan_batch(g, feeds, residual=True, rope=True)
    path = tmp_path / "cfg4.hxplan"
    planfile.save(wb, str(path))
    info = replay(path, tmp_path)
    name = g.outputs[0]
    got = np.fromfile(tmp_path / f"{name}.bin", dtype=np.float16)
    want = _python_run(session, wb)[name].astype(np.float16).reshape(-1)
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))
    print(f"[cfg-4 plan file] {info['ops']} ops, {info['gpu_ns_per_run'] / 1e3:.1f} us per replay", flush=True)
    img = np.random.default_rng(5).random(g.tensor("image").shape, dtype=np.float32)
    img.tofile(tmp_path / "img.bin")
    os.makedirs(tmp_path / "o2")
    replay(path, tmp_path / "o2", "--input", f"image={tmp_path / 'img.bin'}")
    got2 = np.fromfile(tmp_path / "o2" / f"{name}.bin", dtype=np.float16)
    plan = GpuPlan(wb, session)
    try:
        plan.set_input("image", img)
        assert plan.run(graph=True).ok
        want2 = plan.read(name).astype(np.float16).reshape(-1)
    finally:
        plan.close()
    np.testing.assert_array_equal(got2.view(np.uint16), want2.view(np.uint16))
    assert not np.array_equal(got2, got)


def test_plan_api_through_ctypes(session):
    """hexlib_gpu_plan_load / io / write / run / read on the committed
    artefact, and their refusals."""
    lib = L.load()
    ctx = ctypes.c_void_p()
    assert lib.hexlib_gpu_open(ctypes.byref(ctx)) == OK
    assert lib.hexlib_gpu_start(ctx, 0, 0, 0) == OK
    plan = ctypes.c_void_p()
    try:
        assert lib.hexlib_gpu_plan_load(ctx, G.PLAN.encode(), ctypes.byref(plan)) == OK
        info = L.PlanInfo()
        assert lib.hexlib_gpu_plan_info_of(plan, ctypes.byref(info)) == OK
        ios = []
        for i in range(info.n_io):
            e = L.PlanIO()
            assert lib.hexlib_gpu_plan_io(plan, i, ctypes.byref(e)) == OK
            ios.append(e)
        assert lib.hexlib_gpu_plan_io(plan, info.n_io, ctypes.byref(L.PlanIO())) == wire.STATUS["ERR_INVAL_PARAMS"]
        i_in = next(i for i, e in enumerate(ios) if e.role == 0)
        i_out = next(i for i, e in enumerate(ios) if e.role == 1)
        buf = (ctypes.c_uint8 * ios[i_out].nbytes)()
        # an output is not writable, and sizes must match
        assert lib.hexlib_gpu_plan_write(plan, i_out, buf, ios[i_out].nbytes) == wire.STATUS["ERR_INVAL_PARAMS"]
        assert lib.hexlib_gpu_plan_read(plan, i_out, buf, ios[i_out].nbytes - 2) == wire.STATUS["ERR_INVAL_PARAMS"]
        cap = 64 + 16 * (info.n_ops + 1)
        rsp, n = ctypes.create_string_buffer(cap), ctypes.c_uint32()
        assert lib.hexlib_gpu_plan_run(plan, L.INVOKE_GRAPH, rsp, cap, ctypes.byref(n)) == OK
        assert wire.unpack_response(rsp.raw[:n.value]).n_ops == info.n_ops
        assert lib.hexlib_gpu_plan_read(plan, i_out, buf, ios[i_out].nbytes) == OK
        got = np.frombuffer(bytes(buf), np.float16).astype(np.float32)
        want = np.load(G.EXPECTED, allow_pickle=False).astype(np.float32).reshape(-1)
        assert np.abs(got - want).max() <= 2e-2
        img = np.zeros(ios[i_in].nbytes // 4, np.float32)
        assert lib.hexlib_gpu_plan_write(plan, i_in, img.ctypes.data_as(ctypes.c_void_p), img.nbytes) == OK
        assert lib.hexlib_gpu_plan_run(plan, L.INVOKE_GRAPH, rsp, cap, ctypes.byref(n)) == OK
        assert lib.hexlib_gpu_plan_read(plan, i_out, buf, ios[i_out].nbytes) == OK
        assert not np.array_equal(np.frombuffer(bytes(buf), np.float16).astype(np.float32), got)
    finally:
        if plan:
            assert lib.hexlib_gpu_plan_free(plan) == OK
        lib.hexlib_gpu_close(ctx)
