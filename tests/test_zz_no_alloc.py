"""The no-allocation GEMM entry point (`matmul_epilogue_f16wt_noalloc_fp16`):
the same kernels as `matmul_epilogue_f16wt_fp16`, with any split-K partials in
the library's fixed per-GPU device array instead of its grow-only workspace.
Called through the C ABI twice in a row -- the second call smaller, at shapes
whose plan splits K, so the array really carries the partials -- and each
output must equal the allocating entry point's bit for bit (same tile, same
split, same summation order). A shape whose partials exceed the array is
refused with ERR_VTCM_TOO_SMALL and writes nothing."""
import ctypes

import numpy as np
import pytest

from hexlib_amd.exec import wire
from oracle import kernels as K
from tests.gpu_util import Dev, h16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(torch_gpu):
    d = Dev(torch_gpu)
    d.lib.matmul_epilogue_f16wt_noalloc_fp16.restype = ctypes.c_int
    return d


def _operands(r, M, Kd, N):
    a = h16(r.standard_normal((M, Kd)))
    wt = h16(r.standard_normal((N, Kd)) * 0.02)
    bias = (r.standard_normal(N) * 0.02).astype(np.float32)
    return a, wt, bias


def test_noalloc_matches_the_allocating_entry_on_two_calls(dev):
    r = np.random.default_rng(11)
    # K = 4160 (65 slices of 64, K % 256 != 0): these shapes take the tiled
    # kernel with K split 8 ways (64 x 64 tiles), 8 MiB and 2 MiB of partials
    for M, Kd, N, act in ((512, 4160, 512, 1), (256, 4160, 256, 0)):
        a, wt, bias = _operands(r, M, Kd, N)
        da, dw, db = dev.up(a), dev.up(wt), dev.up(bias)
        want_d = dev.empty((M, N), np.float16)
        got_d = dev.empty((M, N), np.float16)
        dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(want_d), M, Kd, N, act)
        rc = dev.lib.matmul_epilogue_f16wt_noalloc_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(got_d),
                                                        M, Kd, N, act)
        dev.check()
        assert rc == wire.STATUS["OK"], rc
        got, want = dev.down(got_d), dev.down(want_d)
        print(f"[noalloc {M}x{Kd}x{N} act {act}] bit-identical: {np.array_equal(got.view(np.uint16), want.view(np.uint16))}",
              flush=True)
        np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))
        ref = K.matmul_epilogue_f16w(a, wt.T.copy(), bias, act)
        assert K.close_f16(got, ref, 0.01, 3e-4).all()


def test_noalloc_refuses_partials_beyond_its_array(dev):
    """1024 x 8256 x 512 plans 128 x 128 tiles with K split 15 ways: 31.5 MB of
    partials, past the 16 MiB array. Refused before any launch: the poisoned
    output stays untouched."""
    r = np.random.default_rng(12)
    M, Kd, N = 1024, 8256, 512
    a, wt, bias = _operands(r, M, Kd, N)
    da, dw, db = dev.up(a), dev.up(wt), dev.up(bias)
    out = dev.empty((M, N), np.float16)
    rc = dev.lib.matmul_epilogue_f16wt_noalloc_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(out),
                                                    M, Kd, N, 0)
    dev.check()
    assert rc == wire.STATUS["ERR_VTCM_TOO_SMALL"]
    assert (dev.down(out) == np.float16(12345.0)).all()
    bad = dev.lib.matmul_epilogue_f16wt_noalloc_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(out),
                                                     M, Kd, N, 7)
    assert bad == wire.STATUS["ERR_INVAL_PARAMS"]
