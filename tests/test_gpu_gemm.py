"""GEMM parity on the GPU through the C ABI: matmul_fp16 (batched attention
shapes and the harness shape), matmul_epilogue_fp16 (q4_0 blocked along N, the
reference ABI), matmul_epilogue_f16w_fp16 (BASELINE cfg 3 sweep) and
matmul_epilogue_q4k_fp16 (cfg 5 shapes), each against the oracle with the
reference harness tolerance (rel 1e-2; abs 1e-3 for matmul, 3e-4 for the
epilogue, `kernels/matmul_fp16/harness.c:145`,
`kernels/matmul_epilogue_fp16/harness.c:259-260`)."""
import numpy as np
import pytest

from hexlib_amd.quant import pack_q4_0_kgrouped, pack_q4_0_nblocked
from oracle import kernels as K
from oracle.quant import dequantize_q4_0_fp16
from tests.gpu_util import Dev, h16, report

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(torch_gpu):
    return Dev(torch_gpu)


def rng(s):
    return np.random.default_rng(s)


@pytest.mark.parametrize("dims", [(12, 256, 64, 256), (12, 256, 256, 64), (3, 40, 128, 200),
                                  (2, 17, 33, 45), (1, 256, 768, 2304), (12, 784, 64, 784),
                                  (1, 1, 64, 8)])
def test_matmul(dev, dims):
    Bn, M, Kd, N = dims
    A = h16(rng(1).standard_normal((Bn, M, Kd)))
    B = h16(rng(2).standard_normal((Bn, Kd, N)) * 0.1)
    dA, dB, dC = dev.up(A), dev.up(B), dev.empty((Bn, M, N), np.float16)
    dev.lib.matmul_fp16(dev.ptr(dA), dev.ptr(dB), dev.ptr(dC), Bn, M, Kd, N)
    dev.check()
    got, want = dev.down(dC), K.matmul_fp16(A, B)
    report(f"matmul {dims}", got, want)
    assert K.close_f16(got, want, 1e-2, 1e-3).all()


def test_matmul_misaligned_operands(dev):
    A = h16(rng(3).standard_normal((2, 24, 40)))
    B = h16(rng(4).standard_normal((2, 40, 24)))
    dA, dB, dC = dev.up(A, 2), dev.up(B, 6), dev.empty((2, 24, 24), np.float16, 2)
    dev.lib.matmul_fp16(dev.ptr(dA), dev.ptr(dB), dev.ptr(dC), 2, 24, 40, 24)
    dev.check()
    assert K.close_f16(dev.down(dC), K.matmul_fp16(A, B), 1e-2, 1e-3).all()


def _q4_inputs(M, Kd, N, seed):
    r = rng(seed)
    a = h16(r.standard_normal((M, Kd)))
    w = (r.standard_normal((Kd, N)) * r.uniform(0.005, 0.02)).astype(np.float32)
    bias = (0.05 * r.standard_normal(N)).astype(np.float32)
    return a, w, bias


@pytest.mark.parametrize("M,Kd,N,act", [(20, 128, 160, 1), (256, 768, 768, 0), (64, 3072, 1024, 2),
                                        (3, 96, 64, 2), (256, 1536, 768, 0), (1, 896, 4864, 0),
                                        (16, 4864, 896, 0), (256, 2048, 2048, 0)])
def test_matmul_epilogue_q4_nblocked(dev, M, Kd, N, act):
    a, w, bias = _q4_inputs(M, Kd, N, 5)
    wq = pack_q4_0_nblocked(w)
    da, dw, db, do = dev.up(a), dev.up(np.frombuffer(wq, np.uint8)), dev.up(bias), dev.empty((M, N), np.float16)
    dev.lib.matmul_epilogue_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(do), M, Kd, N, act)
    dev.check()
    got, want = dev.down(do), K.matmul_epilogue_fp16(a, wq, bias, Kd, N, act)
    report(f"q4n {M}x{Kd}x{N} act{act}", got, want)
    assert K.close_f16(got, want, 0.01, 3e-4).all()


@pytest.mark.parametrize("M,Kd,N,act", [(256, 768, 2304, 0), (256, 768, 768, 1), (256, 768, 3072, 1),
                                        (70, 512, 128, 2), (1, 256, 64, 0), (300, 1024, 192, 0),
                                        (256, 3072, 768, 0), (64, 3072, 1024, 2)])
def test_q4_nblocked_kw_path(dev, M, Kd, N, act):
    """The reference-ABI q4_0 weight (blocks along N) on the K-across-waves
    kernel's [K][N] forms (override path 4 with tile 64x64 and with the
    32-column tile, and the automatic route at these shapes) is bit-identical
    to the same kernel's fp16 [K][N] form on the dequantized weight, and within the epilogue tolerance of the oracle and of
    the register-staged kernel (path 1)."""
    a, w, bias = _q4_inputs(M, Kd, N, 17)
    wq = pack_q4_0_nblocked(w)
    wd = h16(dequantize_q4_0_fp16(wq, (Kd, N)))
    da, dw, db, dwd = dev.up(a), dev.up(np.frombuffer(wq, np.uint8)), dev.up(bias), dev.up(wd)
    outs = []
    for ov, dense in (((64, 64, 0, 4), False), ((0, 0, 0, 0), False), ((0, 0, 1, 1), False), ((64, 64, 0, 4), True),
                      ((0, 0, 0, 4), False), ((0, 0, 0, 4), True)):
        do = dev.empty((M, N), np.float16)
        assert dev.lib.hexlib_gpu_gemm_override(*ov) == 1
        try:
            if dense:
                dev.lib.matmul_epilogue_f16w_fp16(dev.ptr(da), dev.ptr(dwd), dev.ptr(db), dev.ptr(do), M, Kd, N, act)
            else:
                dev.lib.matmul_epilogue_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(do), M, Kd, N, act)
            dev.check()
        finally:
            dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
        outs.append(dev.down(do))
    np.testing.assert_array_equal(outs[0].view(np.uint16), outs[3].view(np.uint16))
    np.testing.assert_array_equal(outs[1].view(np.uint16), outs[3].view(np.uint16))
    # the 32-column form: the same sums in the same order as the 64-column one
    np.testing.assert_array_equal(outs[4].view(np.uint16), outs[5].view(np.uint16))
    np.testing.assert_array_equal(outs[4].view(np.uint16), outs[3].view(np.uint16))
    want = K.matmul_epilogue_fp16(a, wq, bias, Kd, N, act)
    assert K.close_f16(outs[0], want, 0.01, 3e-4).all()
    assert K.close_f16(outs[2], want, 0.01, 3e-4).all()


@pytest.mark.parametrize("M,Kd,N", [(1, 896, 4864), (16, 896, 4864), (256, 896, 4864),
                                    (1, 4864, 896), (16, 4864, 896), (256, 4864, 896),
                                    (1, 2048, 2048), (16, 2048, 2048), (256, 2048, 2048)])
def test_matmul_q4k_cfg5(dev, M, Kd, N):
    """BASELINE cfg 5: nibbles uniform, fp16 scales U(0.005, 0.02), zero point 8,
    activations N(0,1), no bias, no activation."""
    r = rng(6)
    n_blocks = N * Kd // 32
    blocks = np.empty((n_blocks, 18), np.uint8)
    blocks[:, :2] = r.uniform(0.005, 0.02, n_blocks).astype(np.float16).view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = r.integers(0, 256, (n_blocks, 16), dtype=np.uint8)
    wq = blocks.tobytes()
    a = h16(r.standard_normal((M, Kd)))
    bias = np.zeros(N, np.float32)
    da, dw, db, do = dev.up(a), dev.up(blocks), dev.up(bias), dev.empty((M, N), np.float16)
    dev.lib.matmul_epilogue_q4k_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(do), M, Kd, N, 0)
    dev.check()
    got, want = dev.down(do), K.matmul_q4k(a, wq, bias, Kd, N, 0)
    report(f"q4k {M}x{Kd}x{N}", got, want)
    assert K.close_f16(got, want, 0.01, 3e-4).all()


def test_q4k_and_nblocked_agree_on_the_same_weight(dev):
    a, w, bias = _q4_inputs(64, 256, 128, 7)
    outs = []
    for fn, wq in (("matmul_epilogue_q4k_fp16", pack_q4_0_kgrouped(w)),
                   ("matmul_epilogue_fp16", pack_q4_0_nblocked(w))):
        da, dw, db, do = dev.up(a), dev.up(np.frombuffer(wq, np.uint8)), dev.up(bias), dev.empty((64, 128), np.float16)
        getattr(dev.lib, fn)(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(do), 64, 256, 128, 1)
        dev.check()
        outs.append(dev.down(do))
    # Both quantize the same weight along different axes: each must track the
    # unquantized product closely; they differ from each other only by format error.
    dense = K.gemm_epilogue(a, w.astype(np.float16).astype(np.float32), bias, 1).astype(np.float64)
    for o in outs:
        assert np.corrcoef(o.astype(np.float64).ravel(), dense.ravel())[0, 1] > 0.98


@pytest.mark.parametrize("M,Kd,N,act,scale", [(256, 768, 2304, 1, 0.02), (256, 768, 768, 0, 0.02),
                                              (256, 768, 3072, 1, 0.02), (256, 3072, 768, 0, 0.02),
                                              (256, 768, 768, 1, 1.0), (64, 3072, 3072, 2, 1.0),
                                              (8192, 768, 768, 1, 1.0), (17, 40, 24, 2, 1.0)])
def test_matmul_epilogue_f16w(dev, M, Kd, N, act, scale):
    """BASELINE cfg 3 (A/B ~ N(0, 0.02), bias + GELU) plus unit-scale cases
    where the absolute tolerance cannot hide a wrong product."""
    r = rng(8)
    a = h16(r.standard_normal((M, Kd)) * scale)
    w = h16(r.standard_normal((Kd, N)) * (0.02 if scale < 1 else 1.0 / np.sqrt(Kd)))
    bias = (0.02 * r.standard_normal(N)).astype(np.float32)
    da, dw, db, do = dev.up(a), dev.up(w), dev.up(bias), dev.empty((M, N), np.float16)
    dev.lib.matmul_epilogue_f16w_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(do), M, Kd, N, act)
    dev.check()
    got, want = dev.down(do), K.matmul_epilogue_f16w(a, w, bias, act)
    report(f"f16w {M}x{Kd}x{N} act{act}", got, want)
    assert K.close_f16(got, want, 1e-2, 1e-3).all()


@pytest.mark.parametrize("M,Kd,N,act", [(256, 768, 768, 0), (256, 3072, 768, 0), (256, 768, 3072, 1),
                                        (8192, 768, 768, 1), (8192, 3072, 768, 0), (8192, 768, 3072, 1),
                                        (64, 3072, 3072, 2), (784, 768, 768, 0), (17, 40, 24, 2),
                                        (1, 896, 4864, 0), (300, 200, 136, 1)])
def test_matmul_epilogue_f16wt(dev, M, Kd, N, act):
    """fp16 weight stored transposed (W^T [N, K]): the encoder's default GEMM."""
    r = rng(9)
    a = h16(r.standard_normal((M, Kd)))
    w = h16(r.standard_normal((Kd, N)) / np.sqrt(Kd))
    bias = (0.02 * r.standard_normal(N)).astype(np.float32)
    da, dw, db, do = dev.up(a), dev.up(np.ascontiguousarray(w.T)), dev.up(bias), dev.empty((M, N), np.float16)
    dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(do), M, Kd, N, act)
    dev.check()
    got, want = dev.down(do), K.matmul_epilogue_f16w(a, w, bias, act)
    report(f"f16wt {M}x{Kd}x{N} act{act}", got, want)
    assert K.close_f16(got, want, 1e-2, 1e-3).all()


@pytest.mark.parametrize("fn", ["matmul_epilogue_f16wt_fp16", "matmul_epilogue_f16w_fp16"])
def test_split_k_is_deterministic(dev, fn):
    """M = 256 with K = 3072 runs split-K; the fixed-order reduction must give
    identical bits on every run."""
    r = rng(10)
    M, Kd, N = 256, 3072, 768
    a = h16(r.standard_normal((M, Kd)))
    w = h16(r.standard_normal((Kd, N)) / np.sqrt(Kd))
    wdev = np.ascontiguousarray(w.T) if fn.endswith("wt_fp16") else w
    bias = np.zeros(N, np.float32)
    da, dw, db = dev.up(a), dev.up(wdev), dev.up(bias)
    outs = []
    for _ in range(3):
        do = dev.empty((M, N), np.float16)
        getattr(dev.lib, fn)(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(do), M, Kd, N, 0)
        dev.check()
        outs.append(dev.down(do))
    for o in outs[1:]:
        np.testing.assert_array_equal(o.view(np.uint16), outs[0].view(np.uint16))
    assert K.close_f16(outs[0], K.matmul_epilogue_f16w(a, w, bias, 0), 1e-2, 1e-3).all()


@pytest.mark.parametrize("M,Kd,N", [(256, 768, 768), (300, 320, 138), (33, 1024, 70), (8, 4096, 256)])
@pytest.mark.parametrize("tile", [(64, 64), (128, 128), (256, 128), (32, 64), (64, 32)])
@pytest.mark.parametrize("splits", [2, 5, 16])
@pytest.mark.parametrize("path", [1, 2])
def test_forced_tiles_and_splits(dev, M, Kd, N, tile, splits, path):
    """Every tile, split-K factor and W^T code path, forced through the tuning
    override, on ragged shapes (M and N not multiples of the tile, N % 4 != 0):
    in-kernel split-K reduction against the oracle, and bit-identical on a
    second call (the per-tile arrival counters must be back at zero)."""
    r = rng(11)
    a = h16(r.standard_normal((M, Kd)))
    w = h16(r.standard_normal((Kd, N)) / np.sqrt(Kd))
    bias = (0.02 * r.standard_normal(N)).astype(np.float32)
    da, dw, db = dev.up(a), dev.up(np.ascontiguousarray(w.T)), dev.up(bias)
    assert dev.lib.hexlib_gpu_gemm_override(tile[0], tile[1], splits, path) == 1
    try:
        outs = []
        for act in (1, 1):
            do = dev.empty((M, N), np.float16)
            dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(do), M, Kd, N, act)
            dev.check()
            outs.append(dev.down(do))
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    want = K.matmul_epilogue_f16w(a, w, bias, 1)
    assert K.close_f16(outs[0], want, 1e-2, 1e-3).all()
    np.testing.assert_array_equal(outs[1].view(np.uint16), outs[0].view(np.uint16))


@pytest.mark.parametrize("splits", [3, 8])
def test_forced_split_batched_matmul(dev, splits):
    """Split-K on the batched matmul: counters are per (batch, tile)."""
    r = rng(12)
    Bn, M, Kd, N = 5, 70, 512, 90
    a = h16(r.standard_normal((Bn, M, Kd)))
    b = h16(r.standard_normal((Bn, Kd, N)) / np.sqrt(Kd))
    da, dbm, do = dev.up(a), dev.up(b), dev.empty((Bn, M, N), np.float16)
    assert dev.lib.hexlib_gpu_gemm_override(64, 64, splits, 0) == 1
    try:
        dev.lib.matmul_fp16(dev.ptr(da), dev.ptr(dbm), dev.ptr(do), Bn, M, Kd, N)
        dev.check()
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    assert K.close_f16(dev.down(do), K.matmul_fp16(a, b), 1e-2, 1e-3).all()


def test_override_rejects_bad_values(dev):
    for args in [(32, 32, 0, 0), (64, 64, 17, 0), (64, 64, -1, 0), (64, 64, 0, 6), (256, 256, 0, 0),
                 (32, 128, 0, 3), (128, 32, 0, 3), (64, 64, 0, 5), (256, 256, 4, 5), (192, 256, 0, 5),
                 (64, 64, 0, 7), (0, 0, 2, 7), (0, 0, 12, 7), (0, 0, 0, 6), (0, 0, 0, 8),
                 (32, 24, 0, 3), (32, 24, 0, 5)]:
        assert dev.lib.hexlib_gpu_gemm_override(*args) != 1
    assert dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0) == 1


@pytest.mark.parametrize("M,Kd,N,act", [(256, 768, 768, 0), (256, 3072, 768, 0), (8192, 3072, 768, 0),
                                        (300, 320, 136, 1), (17, 64, 40, 2), (256, 768, 3072, 1)])
def test_matmul_epilogue_f16wt_res(dev, M, Kd, N, act):
    """KIND 21: the linear then the residual add in one epilogue. Bit-identical
    to this library's own matmul_epilogue_f16wt followed by add_fp16 (same
    tile plan, same accumulation order), including split-K shapes; and
    within the harness tolerance of the oracle."""
    r = rng(13)
    a = h16(r.standard_normal((M, Kd)))
    w = h16(r.standard_normal((Kd, N)) / np.sqrt(Kd))
    bias = (0.02 * r.standard_normal(N)).astype(np.float32)
    res = h16(r.standard_normal((M, N)))
    da, dw, db, dr = dev.up(a), dev.up(np.ascontiguousarray(w.T)), dev.up(bias), dev.up(res)
    d1, d2 = dev.empty((M, N), np.float16), dev.empty((M, N), np.float16)
    dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(d1), M, Kd, N, act)
    dev.lib.matmul_epilogue_f16wt_res_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(dr), dev.ptr(d2),
                                           M, Kd, N, act)
    dev.check()
    lin, got = dev.down(d1), dev.down(d2)
    # the add is exact given the linear; the linear meets the GEMM tolerance
    # (a tolerance on the sum would be meaningless where r + lin cancels)
    np.testing.assert_array_equal(got.view(np.uint16), K.add_fp16(res, lin).view(np.uint16))
    assert K.close_f16(lin, K.matmul_epilogue_f16w(a, w, bias, act), 1e-2, 1e-3).all()


@pytest.mark.parametrize("tile,splits,path", [((64, 64), 4, 2), ((128, 128), 3, 1), ((64, 64), 1, 1)])
def test_residual_epilogue_every_path(dev, tile, splits, path):
    """Residual epilogue through each code path the override can force:
    direct-to-LDS and register-staged kernels, direct and split-K (reduce
    kernel) epilogues, ragged M and N."""
    r = rng(14)
    M, Kd, N = 200, 1024, 200
    a = h16(r.standard_normal((M, Kd)))
    w = h16(r.standard_normal((Kd, N)) / np.sqrt(Kd))
    bias = (0.02 * r.standard_normal(N)).astype(np.float32)
    res = h16(r.standard_normal((M, N)))
    da, dw, db, dr = dev.up(a), dev.up(np.ascontiguousarray(w.T)), dev.up(bias), dev.up(res)
    d1, d2 = dev.empty((M, N), np.float16), dev.empty((M, N), np.float16)
    assert dev.lib.hexlib_gpu_gemm_override(tile[0], tile[1], splits, path) == 1
    try:
        dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(d1), M, Kd, N, 0)
        dev.lib.matmul_epilogue_f16wt_res_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(dr),
                                               dev.ptr(d2), M, Kd, N, 0)
        dev.check()
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    np.testing.assert_array_equal(dev.down(d2).view(np.uint16), K.add_fp16(res, dev.down(d1)).view(np.uint16))


@pytest.mark.parametrize("M,Kd,N", [(256, 768, 768), (256, 3072, 768), (256, 768, 2304), (64, 3072, 1024),
                                    (300, 320, 136), (1, 896, 4864), (33, 64, 40), (512, 256, 96)])
@pytest.mark.parametrize("bm,bn", [(32, 32), (32, 64), (64, 32), (64, 64)])
@pytest.mark.parametrize("residual", [False, True])
def test_skinny_small_m_path(dev, M, Kd, N, bm, bn, residual):
    """The small-M register-operand kernel (path 3), both tile widths, ragged
    M and N, K from one to 48 slices, with and without the residual epilogue:
    against the oracle, and bit-identical on a repeat call."""
    r = rng(15)
    a = h16(r.standard_normal((M, Kd)))
    w = h16(r.standard_normal((Kd, N)) / np.sqrt(Kd))
    bias = (0.02 * r.standard_normal(N)).astype(np.float32)
    res = h16(r.standard_normal((M, N)))
    da, dw, db, dr = dev.up(a), dev.up(np.ascontiguousarray(w.T)), dev.up(bias), dev.up(res)
    outs = []
    assert dev.lib.hexlib_gpu_gemm_override(bm, bn, 0, 3) == 1
    try:
        for _ in range(2):
            do = dev.empty((M, N), np.float16)
            if residual:
                dev.lib.matmul_epilogue_f16wt_res_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(dr),
                                                       dev.ptr(do), M, Kd, N, 1)
            else:
                dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(do), M, Kd, N, 1)
            dev.check()
            outs.append(dev.down(do))
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    np.testing.assert_array_equal(outs[1].view(np.uint16), outs[0].view(np.uint16))
    lin = K.matmul_epilogue_f16w(a, w, bias, 1)
    if residual:
        # the add is exact on the fp16 linear; compare the linear part through it
        got_lin = (outs[0].astype(np.float32) - res.astype(np.float32))
        assert np.abs(got_lin - lin.astype(np.float32)).max() <= 2e-2
    else:
        assert K.close_f16(outs[0], lin, 1e-2, 1e-3).all()


def _rope_tables(r, M, d):
    ang = r.random((M, d // 2)) * 6.0
    return (np.concatenate([np.cos(ang)] * 2, axis=1).astype(np.float32),
            np.concatenate([np.sin(ang)] * 2, axis=1).astype(np.float32))


@pytest.mark.parametrize("M,Kd,heads,d,extra,tile,splits", [
    (256, 768, 12, 64, 768, None, 1), (1024, 768, 12, 64, 768, None, 1), (65, 128, 2, 32, 64, None, 1),
    (200, 256, 3, 16, 0, None, 1), (256, 768, 12, 64, 768, (64, 64), 1), (256, 768, 12, 64, 768, (128, 128), 1),
    (300, 512, 4, 64, 256, (256, 128), 1), (130, 256, 2, 64, 128, (32, 64), 1), (130, 256, 2, 64, 128, (64, 32), 1),
    (256, 768, 12, 64, 768, (64, 64), 2), (200, 1024, 3, 16, 32, (64, 64), 3), (300, 512, 4, 64, 256, (128, 128), 4),
    (256, 768, 12, 64, 768, None, 0)])
def test_matmul_epilogue_f16wt_rope(dev, M, Kd, heads, d, extra, tile, splits):
    """KIND 22: the fused q/k/v linear with rope_2d on its first 2 * heads
    heads in the epilogue, its weight in the pair-interleaved col_major_rope
    layout: in the tiled kernel's epilogue (one split) or in the split-K
    reduce. Bit-identical to this library's direct-to-LDS matmul_epilogue_f16wt
    with the same tile and split count followed by rope_2d on those heads; and
    the linear part within the harness tolerance of the oracle. splits 0 is
    the heuristic plan (the encoder's shape: tiles too few to fill the chip, so
    it splits K)."""
    r = rng(21)
    N = 2 * heads * d + extra
    a = h16(r.standard_normal((M, Kd)))
    w = h16(r.standard_normal((Kd, N)) / np.sqrt(Kd))
    bias = (0.05 * r.standard_normal(N)).astype(np.float32)
    cos, sin = _rope_tables(r, M, d)
    da, db = dev.up(a), dev.up(bias)
    dc, ds = dev.up(np.ascontiguousarray(cos.T)), dev.up(np.ascontiguousarray(sin.T))   # [d, M]
    dw = dev.up(np.ascontiguousarray(w.T))
    dwr = dev.up(K.permute_rope_rows(w.T, heads, d))
    d1, d2 = dev.empty((M, N), np.float16), dev.empty((M, N), np.float16)
    bm, bn = tile or (0, 0)
    assert dev.lib.hexlib_gpu_gemm_override(bm, bn, splits, 2) == 1
    try:
        dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(d1), M, Kd, N, 0)
        dev.lib.matmul_epilogue_f16wt_rope_fp16(dev.ptr(da), dev.ptr(dwr), dev.ptr(db), dev.ptr(dc), dev.ptr(ds),
                                                dev.ptr(d2), M, Kd, N, 0, heads, d)
        dev.check()
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    lin, got = dev.down(d1), dev.down(d2)
    qk = lin[:, :2 * heads * d].reshape(M, 2 * heads, d)
    want = lin.copy()
    want[:, :2 * heads * d] = K.rope_2d_fp16(qk, cos, sin).reshape(M, -1)
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))
    assert K.close_f16(lin, K.matmul_epilogue_f16w(a, w, bias, 0), 1e-2, 1e-3).all()


def test_matmul_epilogue_f16wt_rope_invalid_is_a_silent_no_op(dev):
    """Shapes the rope epilogue has no form for leave the output untouched."""
    M, Kd, heads, d = 64, 128, 2, 32
    N = 3 * heads * d
    z = np.zeros((M, Kd), np.float16)
    da, dw = dev.up(z), dev.up(np.zeros((N, Kd), np.float16))
    db, dc = dev.up(np.zeros(N, np.float32)), dev.up(np.zeros((d, M), np.float32))
    out = dev.up(np.full((M, N), 7, np.float16))
    for kk, hh, dd in ((96, heads, d), (Kd, heads, 30), (Kd, 4, d)):
        dev.lib.matmul_epilogue_f16wt_rope_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(dc), dev.ptr(dc),
                                                dev.ptr(out), M, kk, N, 0, hh, dd)
    dev.check()
    assert (dev.down(out) == 7).all()


def _ln_inputs(r, M, Kd):
    x = h16(r.standard_normal((M, Kd)) * 2.0 + 0.5)
    g = (1.0 + 0.1 * r.standard_normal(Kd)).astype(np.float32)
    b = (0.1 * r.standard_normal(Kd)).astype(np.float32)
    return x, g, b


@pytest.mark.parametrize("M,Kd,N,act", [(256, 768, 3072, 1), (256, 768, 2304, 0), (65, 512, 200, 2),
                                        (784, 768, 3072, 1), (130, 640, 96, 0), (1, 768, 64, 1)])
def test_layernorm_matmul_epilogue(dev, M, Kd, N, act):
    """KIND 24: layernorm_fp16 over K, then the W^T linear, in one launch with
    the normalised row block resident in LDS. Bit-identical to layernorm_fp16
    followed by matmul_epilogue_f16wt_fp16 on the same (64x64, one split)
    tile; the LayerNorm within its harness tolerance of the oracle."""
    r = rng(31)
    x, g, b = _ln_inputs(r, M, Kd)
    w = h16(r.standard_normal((Kd, N)) / np.sqrt(Kd))
    bias = (0.05 * r.standard_normal(N)).astype(np.float32)
    dx, dg, db_, dw, dbias = dev.up(x), dev.up(g), dev.up(b), dev.up(np.ascontiguousarray(w.T)), dev.up(bias)
    dy = dev.empty((M, Kd), np.float16)
    d1, d2 = dev.empty((M, N), np.float16), dev.empty((M, N), np.float16)
    assert dev.lib.hexlib_gpu_gemm_override(64, 64, 1, 2) == 1
    try:
        dev.lib.layernorm_fp16(dev.ptr(dx), dev.ptr(dg), dev.ptr(db_), dev.ptr(dy), M, Kd, 1e-6)
        dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(dy), dev.ptr(dw), dev.ptr(dbias), dev.ptr(d1), M, Kd, N, act)
        dev.check()
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    dev.lib.layernorm_matmul_epilogue_f16wt_fp16(dev.ptr(dx), dev.ptr(dg), dev.ptr(db_), dev.ptr(dw), dev.ptr(dbias),
                                                 dev.ptr(d2), M, Kd, N, act, 1e-6)
    dev.check()
    np.testing.assert_array_equal(dev.down(d2).view(np.uint16), dev.down(d1).view(np.uint16))
    y = dev.down(dy)
    assert K.close_f16(y, K.layernorm_fp16(x, g, b, 1e-6), 0.02, 1e-3).all()
    assert K.close_f16(dev.down(d1), K.matmul_epilogue_f16w(y, w, bias, act), 1e-2, 1e-3).all()


def test_layernorm_matmul_epilogue_invalid_is_a_silent_no_op(dev):
    """Feature counts the resident row block does not hold leave the output
    untouched."""
    M, N = 64, 64
    out = dev.up(np.full((M, N), 7, np.float16))
    for Kd in (448, 832, 600):
        x = dev.up(np.zeros((M, Kd), np.float16))
        g, b = dev.up(np.ones(Kd, np.float32)), dev.up(np.zeros(Kd, np.float32))
        w, bias = dev.up(np.zeros((N, Kd), np.float16)), dev.up(np.zeros(N, np.float32))
        dev.lib.layernorm_matmul_epilogue_f16wt_fp16(dev.ptr(x), dev.ptr(g), dev.ptr(b), dev.ptr(w), dev.ptr(bias),
                                                     dev.ptr(out), M, Kd, N, 0, 1e-6)
    dev.check()
    assert (dev.down(out) == 7).all()


@pytest.mark.parametrize("M,Kd,N,act", [(1, 896, 4864, 0), (16, 896, 4864, 0), (256, 896, 4864, 0),
                                        (256, 4864, 896, 0), (256, 2048, 2048, 0), (256, 768, 3072, 1),
                                        (70, 96, 40, 2), (300, 768, 2304, 0)])
def test_matmul_q8k(dev, M, Kd, N, act):
    """KIND 25: q8_0 blocks along K of W^T -- random int8 codes (including
    -128) and fp16 scales U(0.005, 0.02) as in cfg 5's q4_0 recipe -- against
    the oracle's dequantize-to-fp16 product, harness tolerance (0.01, 3e-4)."""
    r = rng(9)
    n_blocks = N * Kd // 32
    blocks = np.empty((n_blocks, 34), np.uint8)
    blocks[:, :2] = r.uniform(0.005, 0.02, n_blocks).astype(np.float16).view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = r.integers(0, 256, (n_blocks, 32), dtype=np.uint8)
    wq = blocks.tobytes()
    a = h16(r.standard_normal((M, Kd)))
    bias = (0.02 * r.standard_normal(N)).astype(np.float32)
    da, dw, db, do = dev.up(a), dev.up(blocks), dev.up(bias), dev.empty((M, N), np.float16)
    dev.lib.matmul_epilogue_q8k_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(do), M, Kd, N, act)
    dev.check()
    got, want = dev.down(do), K.matmul_q8k(a, wq, bias, Kd, N, act)
    report(f"q8k {M}x{Kd}x{N}", got, want)
    assert K.close_f16(got, want, 0.01, 3e-4).all()


@pytest.mark.parametrize("M", [64, 2])
def test_q8k_is_the_f16_gemm_on_its_dequantized_weight(dev, M):
    """A q8_0 weight with d = 1 in every block and integer codes dequantizes
    to those integers exactly; with activations on a quarter grid every
    partial sum is exact in fp32, so the kernel's output is the exact product
    rounded once to fp16 (M = 2: the one-wave-per-column kernel)."""
    from hexlib_amd.quant import quantize_q8_0
    r = rng(10)
    Kd, N = 256, 96
    w = r.integers(-127, 128, (Kd, N)).astype(np.float32)
    w[::32, :] = 127.0                               # amax 127 in every block along K -> d = 1
    wq = quantize_q8_0(np.ascontiguousarray(w.T))
    a = h16(r.integers(-2, 3, (M, Kd)).astype(np.float32) / 4)
    bias = np.zeros(N, np.float32)
    da, dw, db, do = dev.up(a), dev.up(np.frombuffer(wq, np.uint8)), dev.up(bias), dev.empty((M, N), np.float16)
    dev.lib.matmul_epilogue_q8k_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(do), M, Kd, N, 0)
    dev.check()
    exact = (a.astype(np.float64) @ w.astype(np.float64)).astype(np.float16)
    np.testing.assert_array_equal(dev.down(do), exact)


KW_TILES = {32: (0, 0), 64: (64, 64), 24: (32, 24)}


@pytest.mark.parametrize("tile", [32, 64, 24])
@pytest.mark.parametrize("M,Kd,N,act,resid", [(256, 3072, 768, 0, True), (256, 3072, 768, 1, False),
                                              (64, 3072, 3072, 1, False), (64, 3072, 1024, 0, False),
                                              (70, 2048, 40, 2, True), (1, 4096, 64, 0, False),
                                              (300, 256, 136, 0, True), (33, 512, 100, 1, False),
                                              (40, 256, 77, 1, True), (256, 768, 760, 0, True)])
def test_kw_long_k_path(dev, tile, M, Kd, N, act, resid):
    """The K-across-waves kernels (32x32, 64x64 and 32x24 tiles, forced with
    path 4; automatic where their workgroups fit one round): ragged M and N
    (N = 77: no vector stores; 760 and 100: a 32x24 grid's last tile 16 and 4
    columns wide), every activation, with and without the residual epilogue.
    Within the GEMM tolerance of the oracle; the residual form bit-identical to
    the plain form followed by add_fp16."""
    r = rng(15)
    a = h16(r.standard_normal((M, Kd)))
    w = h16(r.standard_normal((Kd, N)) / np.sqrt(Kd))
    bias = (0.02 * r.standard_normal(N)).astype(np.float32)
    res = h16(r.standard_normal((M, N)))
    da, dw, db, dr = dev.up(a), dev.up(np.ascontiguousarray(w.T)), dev.up(bias), dev.up(res)
    d1, d2 = dev.empty((M, N), np.float16), dev.empty((M, N), np.float16)
    assert dev.lib.hexlib_gpu_gemm_override(*KW_TILES[tile], 0, 4) == 1
    try:
        dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(d1), M, Kd, N, act)
        if resid:
            dev.lib.matmul_epilogue_f16wt_res_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(dr), dev.ptr(d2),
                                                   M, Kd, N, act)
        dev.check()
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    lin = dev.down(d1)
    report(f"kw{tile} {M}x{Kd}x{N}", lin, K.matmul_epilogue_f16w(a, w, bias, act))
    assert K.close_f16(lin, K.matmul_epilogue_f16w(a, w, bias, act), 1e-2, 1e-3).all()
    if resid:
        np.testing.assert_array_equal(dev.down(d2).view(np.uint16), K.add_fp16(res, lin).view(np.uint16))


@pytest.mark.parametrize("M,Kd,heads,d,extra", [(256, 768, 12, 64, 768), (200, 512, 3, 16, 32), (70, 256, 2, 64, 128)])
def test_kw64_rope_epilogue(dev, M, Kd, heads, d, extra):
    """The 64x64 K-across-waves kernel with the rope epilogue (the encoder's
    q/k/v linear at batch 1) is bit-identical to the same kernel's plain
    output followed by rope_2d on the q and k heads."""
    r = rng(22)
    N = 2 * heads * d + extra
    a = h16(r.standard_normal((M, Kd)))
    w = h16(r.standard_normal((Kd, N)) / np.sqrt(Kd))
    bias = (0.05 * r.standard_normal(N)).astype(np.float32)
    cos, sin = _rope_tables(r, M, d)
    da, db = dev.up(a), dev.up(bias)
    dc, ds = dev.up(np.ascontiguousarray(cos.T)), dev.up(np.ascontiguousarray(sin.T))
    dw, dwr = dev.up(np.ascontiguousarray(w.T)), dev.up(K.permute_rope_rows(w.T, heads, d))
    d1, d2 = dev.empty((M, N), np.float16), dev.empty((M, N), np.float16)
    assert dev.lib.hexlib_gpu_gemm_override(64, 64, 0, 4) == 1
    try:
        dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(d1), M, Kd, N, 0)
        dev.lib.matmul_epilogue_f16wt_rope_fp16(dev.ptr(da), dev.ptr(dwr), dev.ptr(db), dev.ptr(dc), dev.ptr(ds),
                                                dev.ptr(d2), M, Kd, N, 0, heads, d)
        dev.check()
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    lin, got = dev.down(d1), dev.down(d2)
    want = lin.copy()
    want[:, :2 * heads * d] = K.rope_2d_fp16(lin[:, :2 * heads * d].reshape(M, 2 * heads, d), cos, sin).reshape(M, -1)
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))
    assert K.close_f16(lin, K.matmul_epilogue_f16w(a, w, bias, 0), 1e-2, 1e-3).all()


BIG_FORMS = [(256, 256, 2), (256, 192, 2), (128, 256, 2), (128, 256, 3), (128, 192, 2), (128, 192, 3),
             (256, 128, 2), (256, 128, 3), (128, 128, 2), (128, 128, 3)]


@pytest.mark.parametrize("form", BIG_FORMS)
@pytest.mark.parametrize("M,Kd,N,act,resid", [(300, 256, 136, 1, True), (520, 1024, 392, 2, False),
                                              (1100, 768, 776, 0, True), (64, 64, 8, 1, False)])
def test_big_tile_path(dev, form, M, Kd, N, act, resid):
    """The large-tile kernel (path 5), every built tile and ring depth: ragged M
    and N (N % 8 == 0, down to one 8-column group), K from one slice, every
    activation, with and without the residual epilogue. Bit-identical to the
    direct-to-LDS 64x64 kernel without split-K (the same per-output MFMA
    accumulation order), within the GEMM tolerance of the oracle, and the
    residual form bit-identical to the plain form followed by add_fp16."""
    bm, bn, stages = form
    r = rng(16)
    a = h16(r.standard_normal((M, Kd)))
    w = h16(r.standard_normal((Kd, N)) / np.sqrt(Kd))
    bias = (0.02 * r.standard_normal(N)).astype(np.float32)
    res = h16(r.standard_normal((M, N)))
    da, dw, db, dr = dev.up(a), dev.up(np.ascontiguousarray(w.T)), dev.up(bias), dev.up(res)
    d0, d1, d2 = (dev.empty((M, N), np.float16) for _ in range(3))
    assert dev.lib.hexlib_gpu_gemm_override(64, 64, 1, 2) == 1
    try:
        dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(d0), M, Kd, N, act)
        assert dev.lib.hexlib_gpu_gemm_override(bm, bn, stages, 5) == 1
        dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(d1), M, Kd, N, act)
        if resid:
            dev.lib.matmul_epilogue_f16wt_res_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(dr), dev.ptr(d2),
                                                   M, Kd, N, act)
        dev.check()
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    lin = dev.down(d1)
    np.testing.assert_array_equal(lin.view(np.uint16), dev.down(d0).view(np.uint16))
    assert K.close_f16(lin, K.matmul_epilogue_f16w(a, w, bias, act), 1e-2, 1e-3).all()
    if resid:
        np.testing.assert_array_equal(dev.down(d2).view(np.uint16), K.add_fp16(res, lin).view(np.uint16))


@pytest.mark.parametrize("form", [(128, 128, 2), (128, 192, 2), None])
@pytest.mark.parametrize("M,Kd,heads,d,extra,act", [(1100, 768, 12, 64, 768, 0), (300, 256, 3, 16, 64, 1),
                                                    (520, 512, 4, 32, 128, 2), (2048, 768, 12, 64, 768, 0),
                                                    (1102, 768, 4, 64, 128, 1), (2048, 256, 2, 64, 0, 2)])
def test_big_tile_rope_epilogue(dev, form, M, Kd, heads, d, extra, act):
    """The large-tile kernel's rope epilogue (forced with path 5, or the
    automatic choice where the grid fills a round: form None) is bit-identical
    to the same kernel's plain output followed by rope_2d on the q and k
    heads; ragged M, head widths 16 to 64, every activation. Its 128 x 128
    and 128 x 192 forms take rope_d 64 (each thread gathering its own table
    values); narrower heads take the other rope epilogues."""
    r = rng(23)
    N = 2 * heads * d + extra
    a = h16(r.standard_normal((M, Kd)))
    w = h16(r.standard_normal((Kd, N)) / np.sqrt(Kd))
    bias = (0.05 * r.standard_normal(N)).astype(np.float32)
    cos, sin = _rope_tables(r, M, d)
    da, db = dev.up(a), dev.up(bias)
    dc, ds = dev.up(np.ascontiguousarray(cos.T)), dev.up(np.ascontiguousarray(sin.T))
    dw, dwr = dev.up(np.ascontiguousarray(w.T)), dev.up(K.permute_rope_rows(w.T, heads, d))
    d1, d2 = dev.empty((M, N), np.float16), dev.empty((M, N), np.float16)
    if form:
        assert dev.lib.hexlib_gpu_gemm_override(form[0], form[1], form[2], 5) == 1
    try:
        dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(d1), M, Kd, N, act)
        dev.lib.matmul_epilogue_f16wt_rope_fp16(dev.ptr(da), dev.ptr(dwr), dev.ptr(db), dev.ptr(dc), dev.ptr(ds),
                                                dev.ptr(d2), M, Kd, N, act, heads, d)
        dev.check()
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    lin, got = dev.down(d1), dev.down(d2)
    want = lin.copy()
    want[:, :2 * heads * d] = K.rope_2d_fp16(lin[:, :2 * heads * d].reshape(M, 2 * heads, d), cos, sin).reshape(M, -1)
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))
    assert K.close_f16(lin, K.matmul_epilogue_f16w(a, w, bias, act), 1e-2, 1e-3).all()


@pytest.mark.parametrize("tile,splits", [((64, 64), 1), ((128, 128), 1), ((256, 128), 1), ((32, 64), 1),
                                         ((64, 64), 3), ((128, 128), 2)])
@pytest.mark.parametrize("M,Kd,N,act", [(256, 768, 2304, 1), (300, 512, 192, 0), (70, 256, 64, 2)])
def test_kn_weight_direct_path(dev, tile, splits, M, Kd, N, act):
    """matmul_epilogue_f16w ([K][N] weight, N % 64 == 0) on the direct-to-LDS
    ring with transpose reads of the weight: bit-identical to the W^T kernel
    with the same tile and split count (the same per-output MFMA order), and
    within the harness tolerance of the oracle."""
    r = rng(24)
    a = h16(r.standard_normal((M, Kd)))
    w = h16(r.standard_normal((Kd, N)) / np.sqrt(Kd))
    bias = (0.02 * r.standard_normal(N)).astype(np.float32)
    da, dw, dwt, db = dev.up(a), dev.up(w), dev.up(np.ascontiguousarray(w.T)), dev.up(bias)
    d1, d2 = dev.empty((M, N), np.float16), dev.empty((M, N), np.float16)
    assert dev.lib.hexlib_gpu_gemm_override(tile[0], tile[1], splits, 2) == 1
    try:
        dev.lib.matmul_epilogue_f16w_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(d1), M, Kd, N, act)
        dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(da), dev.ptr(dwt), dev.ptr(db), dev.ptr(d2), M, Kd, N, act)
        dev.check()
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    got = dev.down(d1)
    np.testing.assert_array_equal(got.view(np.uint16), dev.down(d2).view(np.uint16))
    assert K.close_f16(got, K.matmul_epilogue_f16w(a, w, bias, act), 1e-2, 1e-3).all()


@pytest.mark.parametrize("dims", [(12, 256, 64, 256), (12, 256, 256, 64), (3, 128, 512, 128)])
def test_batched_matmul_kn_direct_matches_register_path(dev, dims):
    """The batched matmul_fp16 on the direct-to-LDS [K][N] path equals the
    register-staged kernel (path 1) within the harness tolerance, and both
    meet the oracle."""
    Bn, M, Kd, N = dims
    r = rng(25)
    a = h16(r.standard_normal((Bn, M, Kd)))
    b = h16(r.standard_normal((Bn, Kd, N)) / np.sqrt(Kd))
    da, dbm = dev.up(a), dev.up(b)
    outs = []
    for path in (0, 1):
        do = dev.empty((Bn, M, N), np.float16)
        assert dev.lib.hexlib_gpu_gemm_override(0, 0, 0, path) == 1
        try:
            dev.lib.matmul_fp16(dev.ptr(da), dev.ptr(dbm), dev.ptr(do), Bn, M, Kd, N)
            dev.check()
        finally:
            dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
        outs.append(dev.down(do))
    want = K.matmul_fp16(a, b)
    for o in outs:
        assert K.close_f16(o, want, 1e-2, 1e-3).all()


@pytest.mark.parametrize("tile", [64, 32])
@pytest.mark.parametrize("M,Kd,N,act", [(256, 768, 2304, 1), (256, 768, 768, 0), (200, 512, 192, 2), (256, 3072, 768, 0),
                                        (33, 512, 96, 1), (64, 3072, 1024, 2)])
def test_kn_weight_kw_path(dev, tile, M, Kd, N, act):
    """matmul_epilogue_f16w on the K-across-waves kernel's [K][N] forms (path 4;
    K % 256 == 0): tile 64x64 (N % 64 == 0; else another path) and the
    32-column tile (N % 32 == 0), each bit-identical to the W^T form of the
    same tile, and within the harness tolerance of the oracle."""
    r = rng(26)
    a = h16(r.standard_normal((M, Kd)))
    w = h16(r.standard_normal((Kd, N)) / np.sqrt(Kd))
    bias = (0.02 * r.standard_normal(N)).astype(np.float32)
    da, dw, dwt, db = dev.up(a), dev.up(w), dev.up(np.ascontiguousarray(w.T)), dev.up(bias)
    d1, d2 = dev.empty((M, N), np.float16), dev.empty((M, N), np.float16)
    assert dev.lib.hexlib_gpu_gemm_override(tile if tile == 64 else 0, tile if tile == 64 else 0, 0, 4) == 1
    try:
        dev.lib.matmul_epilogue_f16w_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(d1), M, Kd, N, act)
        dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(da), dev.ptr(dwt), dev.ptr(db), dev.ptr(d2), M, Kd, N, act)
        dev.check()
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    got = dev.down(d1)
    if tile == 32 or N % 64 == 0:
        np.testing.assert_array_equal(got.view(np.uint16), dev.down(d2).view(np.uint16))
    assert K.close_f16(got, K.matmul_epilogue_f16w(a, w, bias, act), 1e-2, 1e-3).all()


@pytest.mark.parametrize("tile", [32, 64])
@pytest.mark.parametrize("M,Kd,N,act", [(256, 768, 2304, 1), (256, 3072, 768, 0), (64, 3072, 1024, 2),
                                        (70, 512, 100, 1), (1, 256, 64, 0)])
def test_q8k_kw_path(dev, tile, M, Kd, N, act):
    """The q8_0 weight on the K-across-waves kernel (path 4; K % 256 == 0):
    bit-identical to the same kernel on the fp16 W^T it dequantizes to
    (fp16(d * q), as oracle.quant.dequantize_q8_0_fp16 rounds it), and within
    the harness tolerance of the register-staged q8_0 kernel (path 1) and the
    oracle. Random int8 codes including -128, ragged M and N."""
    from oracle.quant import dequantize_q8_0_fp16
    r = rng(27)
    n_blocks = N * Kd // 32
    blocks = np.empty((n_blocks, 34), np.uint8)
    blocks[:, :2] = r.uniform(0.005, 0.02, n_blocks).astype(np.float16).view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = r.integers(0, 256, (n_blocks, 32), dtype=np.uint8)
    wq = blocks.tobytes()
    wt16 = h16(dequantize_q8_0_fp16(wq, (N, Kd)))
    a = h16(r.standard_normal((M, Kd)))
    bias = (0.02 * r.standard_normal(N)).astype(np.float32)
    da, dq, dwt, db = dev.up(a), dev.up(blocks), dev.up(np.ascontiguousarray(wt16)), dev.up(bias)
    d1, d2, d3 = (dev.empty((M, N), np.float16) for _ in range(3))
    bm = 64 if tile == 64 else 0
    try:
        assert dev.lib.hexlib_gpu_gemm_override(bm, bm, 0, 4) == 1
        dev.lib.matmul_epilogue_q8k_fp16(dev.ptr(da), dev.ptr(dq), dev.ptr(db), dev.ptr(d1), M, Kd, N, act)
        dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(da), dev.ptr(dwt), dev.ptr(db), dev.ptr(d2), M, Kd, N, act)
        assert dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 1) == 1
        dev.lib.matmul_epilogue_q8k_fp16(dev.ptr(da), dev.ptr(dq), dev.ptr(db), dev.ptr(d3), M, Kd, N, act)
        dev.check()
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    got = dev.down(d1)
    np.testing.assert_array_equal(got.view(np.uint16), dev.down(d2).view(np.uint16))
    assert K.close_f16(got, dev.down(d3), 0.01, 3e-4).all()
    assert K.close_f16(got, K.matmul_q8k(a, wq, bias, Kd, N, act), 0.01, 3e-4).all()


@pytest.mark.parametrize("qb", [4, 8])
@pytest.mark.parametrize("M,Kd,N,act", [(1, 896, 4864, 0), (1, 4864, 896, 0), (1, 2048, 2048, 1), (3, 1024, 100, 2),
                                        (4, 4864, 896, 1), (2, 96, 5, 0), (2, 768, 3072, 1)])
def test_gemv_quantized_path(dev, qb, M, Kd, N, act):
    """q4_0 (K-grouped) and q8_0 weights at up to 2 rows (4 with K >= 896)
    take the one-wave-per-column kernel on the automatic route (BASELINE cfg
    5's shapes at M = 1, K % 256 != 0, ragged N): within the harness tolerance
    of the oracle and of the register-staged kernel (path 1)."""
    r = rng(29 + qb)
    blk = 18 if qb == 4 else 34
    n_blocks = N * Kd // 32
    blocks = np.empty((n_blocks, blk), np.uint8)
    blocks[:, :2] = r.uniform(0.005, 0.02, n_blocks).astype(np.float16).view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = r.integers(0, 256, (n_blocks, blk - 2), dtype=np.uint8)
    wq = blocks.tobytes()
    a = h16(r.standard_normal((M, Kd)))
    bias = (0.02 * r.standard_normal(N)).astype(np.float32)
    da, dq, db = dev.up(a), dev.up(blocks), dev.up(bias)
    d1, d2 = (dev.empty((M, N), np.float16) for _ in range(2))
    fn = dev.lib.matmul_epilogue_q4k_fp16 if qb == 4 else dev.lib.matmul_epilogue_q8k_fp16
    try:
        fn(dev.ptr(da), dev.ptr(dq), dev.ptr(db), dev.ptr(d1), M, Kd, N, act)
        assert dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 1) == 1
        fn(dev.ptr(da), dev.ptr(dq), dev.ptr(db), dev.ptr(d2), M, Kd, N, act)
        dev.check()
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    got = dev.down(d1)
    want = K.matmul_q4k(a, wq, bias, Kd, N, act) if qb == 4 else K.matmul_q8k(a, wq, bias, Kd, N, act)
    assert K.close_f16(got, want, 0.01, 3e-4).all()
    assert K.close_f16(got, dev.down(d2), 0.01, 3e-4).all()


@pytest.mark.parametrize("qb", [4, 8])
@pytest.mark.parametrize("M,Kd,N,act", [(16, 896, 4864, 0), (16, 4864, 896, 0), (16, 2048, 2048, 1),
                                        (1, 2048, 2048, 0), (5, 1024, 100, 2), (11, 96, 40, 0), (16, 32, 17, 1)])
def test_q16_mfma_quantized_path(dev, qb, M, Kd, N, act):
    """q4_0 (K-grouped) and q8_0 weights at up to 16 rows on the 16x16x32 MFMA
    kernel (override path 7): BASELINE cfg 5's shapes at M = 16, ragged M and
    N, a one-block K: within the harness tolerance of the oracle and of the
    register-staged kernel (path 1)."""
    r = rng(47 + qb)
    blk = 18 if qb == 4 else 34
    n_blocks = N * Kd // 32
    blocks = np.empty((n_blocks, blk), np.uint8)
    blocks[:, :2] = r.uniform(0.005, 0.02, n_blocks).astype(np.float16).view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = r.integers(0, 256, (n_blocks, blk - 2), dtype=np.uint8)
    wq = blocks.tobytes()
    a = h16(r.standard_normal((M, Kd)))
    bias = (0.02 * r.standard_normal(N)).astype(np.float32)
    da, dq, db = dev.up(a), dev.up(blocks), dev.up(bias)
    fn = dev.lib.matmul_epilogue_q4k_fp16 if qb == 4 else dev.lib.matmul_epilogue_q8k_fp16
    outs = {}
    try:
        for nw, path in ((4, 7), (8, 7), (16, 7), (0, 1)):   # wave counts of the 16-row kernel; register-staged
            d = dev.empty((M, N), np.float16)
            assert dev.lib.hexlib_gpu_gemm_override(0, 0, nw, path) == 1
            fn(dev.ptr(da), dev.ptr(dq), dev.ptr(db), dev.ptr(d), M, Kd, N, act)
            dev.check()
            outs[nw] = dev.down(d)
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    want = K.matmul_q4k(a, wq, bias, Kd, N, act) if qb == 4 else K.matmul_q8k(a, wq, bias, Kd, N, act)
    for nw in (4, 8, 16):
        report(f"q16x{nw} q{qb} {M}x{Kd}x{N}", outs[nw], want)
        assert K.close_f16(outs[nw], want, 0.01, 3e-4).all()
        assert K.close_f16(outs[nw], outs[0], 0.01, 3e-4).all()


@pytest.mark.parametrize("tile", [32, 64])
@pytest.mark.parametrize("M,Kd,N,act", [(16, 4864, 896, 0), (1, 2048, 2048, 0), (256, 768, 2304, 1), (70, 512, 100, 2)])
def test_q4k_kw_path(dev, tile, M, Kd, N, act):
    """K-grouped q4_0 weights on the K-across-waves kernel (forced with path 4,
    whatever K; automatic up to K = 3072; BASELINE cfg 5's 4864 x 896 and
    2048 x 2048 at M 1 and 16): bit-identical
    to the same kernel on the fp16 W^T they dequantize to (fp16(d * (q - 8))),
    and within the harness tolerance of the register-staged q4 kernel and the
    oracle."""
    from oracle.quant import dequantize_q4_0_fp16
    r = rng(28)
    n_blocks = N * Kd // 32
    blocks = np.empty((n_blocks, 18), np.uint8)
    blocks[:, :2] = r.uniform(0.005, 0.02, n_blocks).astype(np.float16).view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = r.integers(0, 256, (n_blocks, 16), dtype=np.uint8)
    wq = blocks.tobytes()
    wt16 = h16(dequantize_q4_0_fp16(wq, (N, Kd)))
    a = h16(r.standard_normal((M, Kd)))
    bias = (0.02 * r.standard_normal(N)).astype(np.float32)
    da, dq, dwt, db = dev.up(a), dev.up(blocks), dev.up(np.ascontiguousarray(wt16)), dev.up(bias)
    d1, d2, d3 = (dev.empty((M, N), np.float16) for _ in range(3))
    bm = 64 if tile == 64 else 0
    try:
        assert dev.lib.hexlib_gpu_gemm_override(bm, bm, 0, 4) == 1
        dev.lib.matmul_epilogue_q4k_fp16(dev.ptr(da), dev.ptr(dq), dev.ptr(db), dev.ptr(d1), M, Kd, N, act)
        dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(da), dev.ptr(dwt), dev.ptr(db), dev.ptr(d2), M, Kd, N, act)
        assert dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 1) == 1
        dev.lib.matmul_epilogue_q4k_fp16(dev.ptr(da), dev.ptr(dq), dev.ptr(db), dev.ptr(d3), M, Kd, N, act)
        dev.check()
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    got = dev.down(d1)
    np.testing.assert_array_equal(got.view(np.uint16), dev.down(d2).view(np.uint16))
    assert K.close_f16(got, dev.down(d3), 0.01, 3e-4).all()
    assert K.close_f16(got, K.matmul_q4k(a, wq, bias, Kd, N, act), 0.01, 3e-4).all()


# ---- the reference harnesses' adversarial cells --------------------------------------

def test_matmul_harness_adversarial_element(dev):
    """`kernels/matmul_fp16/harness.c`'s shape (3, 40, 128, 200) and its
    element C[1][5][7]: one dominant product plus 127 one-ulp followers. The
    kernel is within the matmul bound of the oracle there (2.1240234375 in
    fp32, one rounding); the fp16-accumulating near-miss (2.0) is not, so this
    test would reject a kernel that carried it."""
    from tests import harness_data as HD, nearmiss as NM
    A, B, (b, m, n) = HD.matmul_adversarial()
    dA, dB, dC = dev.up(A), dev.up(B), dev.empty((3, 40, 200), np.float16)
    dev.lib.matmul_fp16(dev.ptr(dA), dev.ptr(dB), dev.ptr(dC), 3, 40, 128, 200)
    dev.check()
    got, want = dev.down(dC), K.matmul_fp16(A, B)
    report("matmul harness", got, want)
    assert K.close_f16(got, want, 1e-2, 1e-3).all()
    assert abs(float(got[b, m, n]) - 2.1240234375) <= 1e-3
    assert not K.close_f16(got, NM.matmul_fp16_accumulate(A, B), 1e-2, 1e-3).all()


def test_epilogue_harness_cell1(dev):
    """`kernels/matmul_epilogue_fp16/harness.c` cell 1 on the reference-ABI
    q4_0 GEMM: out[0, 0] = 1 + 63 * 2^-12 (1.015625 once rounded); the
    fp16-running-sum near-miss gives 1.0 and fails the epilogue bound."""
    from tests import harness_data as HD, nearmiss as NM
    a, w, bias, M, Kd, N, act = HD.epilogue_cell1()
    da, db = dev.up(a), dev.up(bias)
    dw = dev.up(np.frombuffer(w, np.uint8))
    dout = dev.empty((M, N), np.float16)
    dev.lib.matmul_epilogue_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(dout), M, Kd, N, act)
    dev.check()
    got = dev.down(dout)
    assert K.close_f16(got, K.matmul_epilogue_fp16(a, w, bias, Kd, N, act), 0.01, 3e-4).all()
    assert float(got[0, 0]) == 1.015625
    bad = NM.epilogue_fp16_accumulation(a, NM.dense_q4_nblocked(w, Kd, N), bias, act)
    assert not K.close_f16(got, bad, 0.01, 3e-4).all()


@pytest.mark.parametrize("path", [0, 1, 2, 3, 4])
def test_f16wt_harness_cell1_every_path(dev, path):
    """Cell 1 on the fp16-weight W^T linear at K = 768, through every small-M
    code path (automatic, register-staged, direct-to-LDS, small-M register
    operands, K across waves): each within the epilogue bound of the oracle,
    and none as close to the fp16-running-sum near-miss (1.0 at [0, 0], where
    the value is 1.1872...)."""
    from tests import harness_data as HD, nearmiss as NM
    a, w, bias, act = HD.epilogue_cell1_f16()
    M, Kd = a.shape
    N = w.shape[1]
    da, dw, db = dev.up(a), dev.up(np.ascontiguousarray(w.T)), dev.up(bias)
    dout = dev.empty((M, N), np.float16)
    assert dev.lib.hexlib_gpu_gemm_override(0, 0, 0, path) == 1
    try:
        dev.lib.matmul_epilogue_f16wt_fp16(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(dout), M, Kd, N, act)
        dev.check()
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    got = dev.down(dout)
    assert K.close_f16(got, K.matmul_epilogue_f16w(a, w, bias, act), 0.01, 3e-4).all()
    assert abs(float(got[0, 0]) - 1.1872558) < 1e-3
    assert not K.close_f16(got, NM.epilogue_fp16_accumulation(a, w, bias, act), 0.01, 3e-4).all()


@pytest.mark.parametrize("fmt", ["q4n", "q8k", "q4k"])
@pytest.mark.parametrize("M,Kd,N,act", [(256, 768, 768, 1), (256, 3072, 768, 0), (16, 896, 4864, 0),
                                        (16, 4864, 896, 2), (1, 768, 256, 1), (4, 896, 4864, 0),
                                        (70, 512, 96, 1), (300, 1024, 160, 2)])
def test_quantized_residual_epilogue(dev, fmt, M, Kd, N, act):
    """KIND 28-30: the quantized linears with the residual add in the
    epilogue are bit-identical to the plain call followed by add_fp16, on
    every route the shape takes (one wave per column at M <= 4, the 16-row
    MFMA form and its split-K reduce at M = 16, the K-across-waves and
    register-staged kernels above)."""
    from hexlib_amd.quant import pack_q8_0_kgrouped
    r = rng(61)
    a = h16(r.standard_normal((M, Kd)))
    w = (r.standard_normal((Kd, N)) * 0.02).astype(np.float32)
    bias = (0.05 * r.standard_normal(N)).astype(np.float32)
    res = h16(r.standard_normal((M, N)))
    packed = {"q4n": pack_q4_0_nblocked, "q8k": pack_q8_0_kgrouped, "q4k": pack_q4_0_kgrouped}[fmt](w)
    plain = {"q4n": dev.lib.matmul_epilogue_fp16, "q8k": dev.lib.matmul_epilogue_q8k_fp16,
             "q4k": dev.lib.matmul_epilogue_q4k_fp16}[fmt]
    fused = {"q4n": dev.lib.matmul_epilogue_res_fp16, "q8k": dev.lib.matmul_epilogue_q8k_res_fp16,
             "q4k": dev.lib.matmul_epilogue_q4k_res_fp16}[fmt]
    da, dw, db, dr = dev.up(a), dev.up(np.frombuffer(packed, np.uint8)), dev.up(bias), dev.up(res)
    d1, d2 = dev.empty((M, N), np.float16), dev.empty((M, N), np.float16)
    plain(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(d1), M, Kd, N, act)
    fused(dev.ptr(da), dev.ptr(dw), dev.ptr(db), dev.ptr(dr), dev.ptr(d2), M, Kd, N, act)
    dev.check()
    np.testing.assert_array_equal(dev.down(d2).view(np.uint16), K.add_fp16(res, dev.down(d1)).view(np.uint16))


@pytest.mark.parametrize("M,Kd,heads,d,extra", [(256, 768, 12, 64, 768), (70, 512, 2, 64, 128), (200, 256, 3, 16, 32)])
def test_q8k_rope_epilogue(dev, M, Kd, heads, d, extra):
    """KIND 31: the q8_0 weight in the q8_0_kgroup_rope layout (W^T rows in the
    col_major_rope order, quantized row by row) on the K-across-waves kernel
    with the rope epilogue is bit-identical to the fp16 rope linear (the same
    64x64 K-across-waves tile) on the weight it dequantizes to."""
    from hexlib_amd.exec.wholeplan import rope_row_order, stage_q8_0_kgroup_rope
    from oracle.quant import dequantize_q8_0_fp16
    r = rng(62)
    N = 2 * heads * d + extra
    a = h16(r.standard_normal((M, Kd)))
    w = (r.standard_normal((Kd, N)) * 0.02).astype(np.float32)
    bias = (0.05 * r.standard_normal(N)).astype(np.float32)
    cos, sin = _rope_tables(r, M, d)
    wq = stage_q8_0_kgroup_rope(w, heads, d)
    # the fp16 W^T it dequantizes to, already in the col_major_rope row order
    wt16 = h16(dequantize_q8_0_fp16(wq, (N, Kd)))
    da, db, dq, dw16 = dev.up(a), dev.up(bias), dev.up(np.frombuffer(wq, np.uint8)), dev.up(np.ascontiguousarray(wt16))
    dc, ds = dev.up(np.ascontiguousarray(cos.T)), dev.up(np.ascontiguousarray(sin.T))
    d1, d2 = dev.empty((M, N), np.float16), dev.empty((M, N), np.float16)
    assert dev.lib.hexlib_gpu_gemm_override(64, 64, 0, 4) == 1
    try:
        dev.lib.matmul_epilogue_f16wt_rope_fp16(dev.ptr(da), dev.ptr(dw16), dev.ptr(db), dev.ptr(dc), dev.ptr(ds),
                                                dev.ptr(d1), M, Kd, N, 0, heads, d)
        dev.check()
    finally:
        dev.lib.hexlib_gpu_gemm_override(0, 0, 0, 0)
    dev.lib.matmul_epilogue_q8k_rope_fp16(dev.ptr(da), dev.ptr(dq), dev.ptr(db), dev.ptr(dc), dev.ptr(ds),
                                          dev.ptr(d2), M, Kd, N, 0, heads, d)
    dev.check()
    np.testing.assert_array_equal(dev.down(d2).view(np.uint16), dev.down(d1).view(np.uint16))
    # and the rows really are the original weight's, reordered
    from hexlib_amd.quant import pack_q8_0_kgrouped
    w16_orig = h16(dequantize_q8_0_fp16(pack_q8_0_kgrouped(w), (N, Kd)))
    np.testing.assert_array_equal(wt16, w16_orig[rope_row_order(N, heads, d)])
