"""Per-kernel parity on the GPU, through the C ABI (libhexlib_gpu.so).

Each kernel runs at BASELINE's cfg-2 encoder shapes and at the reference
harness shapes (with their tails and odd widths, misaligned bases forcing the
scalar paths), with outputs poisoned first. Movement ops and single-rounding
elementwise ops must be BIT-EXACT against the oracle; reductions must meet the
reference harness tolerance (hexlib_close_f16(rel, abs), `kernels/*/harness.c`)
and BASELINE's ceiling (<= 2e-3 max abs for norms and softmax).
"""
import numpy as np
import pytest

from hexlib_amd import encoder as E
from oracle import kernels as K
from tests.gpu_util import Dev, h16, report

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(torch_gpu):
    return Dev(torch_gpu)


def rng(s):
    return np.random.default_rng(s)


def exact(got, want):
    np.testing.assert_array_equal(np.asarray(got).view(np.uint8), np.asarray(want).view(np.uint8))


# ---- elementwise -----------------------------------------------------------------

@pytest.mark.parametrize("n,off", [(4100, 0), (196608, 0), (7, 0), (12345, 2)])
def test_add(dev, n, off):
    a, b = h16(rng(1).standard_normal(n) * 4), h16(rng(2).standard_normal(n) * 4)
    da, db, dy = dev.up(a, off), dev.up(b, off), dev.empty(n, np.float16, off)
    dev.lib.add_fp16(dev.ptr(da), dev.ptr(db), dev.ptr(dy), n)
    dev.check()
    exact(dev.down(dy), K.add_fp16(a, b))


@pytest.mark.parametrize("n,factor,off", [(4100, 0.125, 0), (196608, 0.125, 0), (4100, 0.3, 0), (999, 0.7, 6)])
def test_scale(dev, n, factor, off):
    x = h16(rng(3).standard_normal(n) * 8)
    dx, dy = dev.up(x, off), dev.empty(n, np.float16, off)
    dev.lib.scale_fp16(dev.ptr(dx), dev.ptr(dy), n, factor)
    dev.check()
    exact(dev.down(dy), K.scale_fp16(x, factor))


@pytest.mark.parametrize("n,off", [(4160, 0), (4133, 0), (196608, 0), (1001, 4)])
def test_cast(dev, n, off):
    x = (rng(4).standard_normal(n) * 3000).astype(np.float32)
    x[:6] = [65504.0, 65520.0, 1e-8, -6.1e-5, np.inf, -0.0]
    dx, dy = dev.up(x, off), dev.empty(n, np.float16, off)
    dev.lib.cast_f32_f16(dev.ptr(dx), dev.ptr(dy), n)
    dev.check()
    with np.errstate(over="ignore"):
        exact(dev.down(dy), K.cast_f32_f16(x))


# ---- row reductions ----------------------------------------------------------------

@pytest.mark.parametrize("R,C,scale,off", [(3072, 256, 0.125, 0), (6, 256, 1.0, 0), (9408, 784, 0.125, 0),
                                           (5, 100, 3.0, 0), (7, 130, 2.0, 2), (3, 5000, 1.0, 0),
                                           (2, 1, 1.0, 0)])
def test_softmax(dev, R, C, scale, off):
    x = h16(rng(5).standard_normal((R, C)) * scale)
    x[0] = 0.0
    if C > 5:
        x[min(1, R - 1), 5] = 11.0
    dx, dy = dev.up(x, off), dev.empty((R, C), np.float16, off)
    dev.lib.softmax_fp16(dev.ptr(dx), dev.ptr(dy), R, C)
    dev.check()
    got, want = dev.down(dy), K.softmax_fp16(x)
    assert report(f"softmax {R}x{C}", got, want) <= 2e-3
    assert K.close_f16(got, want, 0.01, 1e-3).all()


@pytest.mark.parametrize("R,C,rel,atol,off", [(256, 768, 0.02, 1e-3, 0), (4, 64, 0.004, 1e-4, 0),
                                              (4, 768, 0.02, 1e-3, 0), (3, 100, 0.02, 1e-3, 2),
                                              (2, 6000, 0.02, 1e-3, 0), (784, 768, 0.02, 1e-3, 0)])
def test_layernorm(dev, R, C, rel, atol, off):
    x = h16(rng(6).standard_normal((R, C)) * 2 + 3)
    w = (1 + 0.1 * rng(7).standard_normal(C)).astype(np.float32)
    b = (0.1 * rng(8).standard_normal(C)).astype(np.float32)
    dx, dw, db, dy = dev.up(x, off), dev.up(w), dev.up(b), dev.empty((R, C), np.float16, off)
    dev.lib.layernorm_fp16(dev.ptr(dx), dev.ptr(dw), dev.ptr(db), dev.ptr(dy), R, C, 1e-6)
    dev.check()
    got, want = dev.down(dy), K.layernorm_fp16(x, w, b, 1e-6)
    assert report(f"layernorm {R}x{C}", got, want) <= 2e-3
    assert K.close_f16(got, want, rel, atol).all()


@pytest.mark.parametrize("R,C,eps,off", [(256, 768, 1e-6, 0), (8, 128, 1e-5, 0), (16, 64, 1e-6, 0),
                                         (3, 70, 1e-6, 2), (2, 5000, 1e-6, 0)])
def test_rmsnorm(dev, R, C, eps, off):
    x = h16(rng(9).standard_normal((R, C)))
    x[min(2, R - 1)] = 1e-3
    w = h16(1 + 0.1 * rng(10).standard_normal(C))
    dx, dw, dy = dev.up(x, off), dev.up(w), dev.empty((R, C), np.float16, off)
    dev.lib.rmsnorm_fp16(dev.ptr(dx), dev.ptr(dw), dev.ptr(dy), R, C, eps)
    dev.check()
    got, want = dev.down(dy), K.rmsnorm_fp16(x, w, eps)
    assert report(f"rmsnorm {R}x{C}", got, want) <= 2e-3
    assert K.close_f16(got, want, 0.02, 1e-3).all()


# ---- rope ----------------------------------------------------------------------------

def _encoder_rope_tables():
    return E.rope_tables(E.QWEN35_VISION_FP16)


@pytest.mark.parametrize("T,H,D,tables,off", [(256, 12, 64, "encoder", 0), (6, 3, 64, "random", 0),
                                              (5, 2, 10, "random", 0), (7, 3, 64, "random", 2)])
def test_rope(dev, T, H, D, tables, off):
    x = h16(rng(11).standard_normal((T, H, D)))
    if tables == "encoder":
        cos, sin = _encoder_rope_tables()
    else:
        ang = rng(12).standard_normal((T, D))
        cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    dx, dc, ds, dy = dev.up(x, off), dev.up(cos), dev.up(sin), dev.empty((T, H, D), np.float16, off)
    dev.lib.rope_2d_fp16(dev.ptr(dx), dev.ptr(dc), dev.ptr(ds), dev.ptr(dy), T, H, D)
    dev.check()
    # products and the sum rounded separately in fp32: identical to the oracle
    exact(dev.down(dy), K.rope_2d_fp16(x, cos, sin))


# ---- movement -------------------------------------------------------------------------

@pytest.mark.parametrize("shape,off", [((256, 12, 64), 0), ((8, 3, 64), 0), ((8, 3, 40), 0),
                                       ((5, 7, 3), 0), ((12, 256, 64), 2)])
def test_transpose_th(dev, shape, off):
    x = h16(rng(13).standard_normal(shape))
    dx, dy = dev.up(x, off), dev.empty((shape[1], shape[0], shape[2]), np.float16, off)
    dev.lib.transpose_th_fp16(dev.ptr(dx), dev.ptr(dy), *shape)
    dev.check()
    exact(dev.down(dy), K.transpose_th_fp16(x))


@pytest.mark.parametrize("shape", [(2, 256, 12, 64), (3, 5, 4, 6)])
def test_transpose_bth(dev, shape):
    x = h16(rng(14).standard_normal(shape))
    B, T, H, D = shape
    dx, dy = dev.up(x), dev.empty((B, H, T, D), np.float16)
    dev.lib.transpose_bth_fp16(dev.ptr(dx), dev.ptr(dy), *shape)
    dev.check()
    exact(dev.down(dy), K.transpose_bth_fp16(x))


@pytest.mark.parametrize("shape,off", [((12, 256, 64), 0), ((5, 64, 7), 0), ((5, 40, 7), 0),
                                       ((3, 100, 70), 0), ((12, 784, 64), 0), ((2, 128, 64), 2)])
def test_transpose_hd(dev, shape, off):
    x = h16(rng(15).standard_normal(shape))
    B, T, D = shape
    dx, dy = dev.up(x, off), dev.empty((B, D, T), np.float16, off)
    dev.lib.transpose_hd_fp16(dev.ptr(dx), dev.ptr(dy), B, T, D)
    dev.check()
    exact(dev.down(dy), K.transpose_hd_fp16(x))


@pytest.mark.parametrize("geom,batch", [((3, 1, 256, 256, 16, 2, 16, 16), 1), ((3, 2, 256, 256, 16, 2, 16, 16), 1),
                                        ((2, 3, 12, 12, 3, 2, 4, 4), 1), ((3, 1, 64, 64, 16, 2, 4, 4), 2),
                                        ((3, 1, 448, 448, 16, 2, 28, 28), 1)])
def test_patchify(dev, geom, batch):
    C, T, H, W, p, m, gh, gw = geom
    img = rng(16).random((batch * C, T, H, W), dtype=np.float32)
    out_shape = (batch * gh * gw, C * T * p * p)
    di, do = dev.up(img), dev.empty(out_shape, np.float32)
    if batch == 1:
        dev.lib.patchify_fp32(dev.ptr(di), dev.ptr(do), C, T, H, W, p, m, gh, gw)
    else:
        dev.lib.patchify_fp32_batched(dev.ptr(di), dev.ptr(do), batch * C, T, H, W, p, m, gh, gw, batch)
    dev.check()
    exact(dev.down(do), K.patchify_fp32(img, p, m, gh, gw, batch))


def test_invalid_dims_are_silent_no_ops(dev):
    # Buffers are large enough that even a call which did run would stay in bounds.
    x = h16(np.ones(4096))
    dx, dy = dev.up(x), dev.empty(4096, np.float16)
    dev.lib.scale_fp16(dev.ptr(dx), dev.ptr(dy), -5, 2.0)
    dev.lib.patchify_fp32(dev.ptr(dx), dev.ptr(dy), 3, 1, 10, 10, 3, 2, 4, 4)   # 4*3 != 10
    dev.check()
    assert (dev.down(dy) == np.float16(12345.0)).all()


# ---- the reference harnesses' adversarial rows ----------------------------------------

def test_softmax_harness_rows(dev):
    """`kernels/softmax_fp16/harness.c` rows 0 (a 90.0: exp overflows without
    the max subtracted) and 1 (one 20.0 and 255 followers at 13.5: an fp16
    running sum loses 8% of the denominator): within (0.01, 1e-3) of the
    oracle, and the two near-misses are not."""
    from tests import harness_data as HD, nearmiss as NM
    x = HD.softmax_rows()
    dx, dy = dev.up(x), dev.empty(x.shape, np.float16)
    dev.lib.softmax_fp16(dev.ptr(dx), dev.ptr(dy), 6, 256)
    dev.check()
    got = dev.down(dy)
    assert K.close_f16(got, K.softmax_fp16(x), 0.01, 1e-3).all()
    assert not K.close_f16(got[1:2], NM.softmax_sum_fp16(x)[1:2], 0.01, 1e-3).all()
    with np.errstate(invalid="ignore"):
        assert not K.close_f16(got, NM.softmax_no_max_subtraction(x), 0.01, 1e-3).all()


def test_rmsnorm_harness_eps_row(dev):
    """`kernels/rmsnorm_fp16/harness.c` row 0 (values of 1e-4, where eps
    dominates the mean square): within (0.02, 1e-3), and the no-eps
    near-miss is not."""
    from tests import harness_data as HD, nearmiss as NM
    x, w, eps = HD.rmsnorm_rows()
    dx, dw, dy = dev.up(x), dev.up(w), dev.empty(x.shape, np.float16)
    dev.lib.rmsnorm_fp16(dev.ptr(dx), dev.ptr(dw), dev.ptr(dy), x.shape[0], x.shape[1], eps)
    dev.check()
    got = dev.down(dy)
    assert K.close_f16(got, K.rmsnorm_fp16(x, w, eps), 0.02, 1e-3).all()
    assert not K.close_f16(got[:1], NM.rmsnorm_no_eps(x, w, eps)[:1], 0.02, 1e-3).all()


def test_rope_harness_near_cancellation(dev):
    """`kernels/rope_2d_fp16/harness.c`'s crafted last token: two products of
    about 500 that cancel to -0.1 and 0.1. Bit-exact with the oracle; the
    fp16-products and table-by-head near-misses are outside (0.02, 1e-3)."""
    from tests import harness_data as HD, nearmiss as NM
    x, cos, sin = HD.rope_near_cancellation()
    T, Hh, D = x.shape
    dx, dc, ds, dy = dev.up(x), dev.up(cos), dev.up(sin), dev.empty(x.shape, np.float16)
    dev.lib.rope_2d_fp16(dev.ptr(dx), dev.ptr(dc), dev.ptr(ds), dev.ptr(dy), T, Hh, D)
    dev.check()
    got = dev.down(dy)
    exact(got, K.rope_2d_fp16(x, cos, sin))
    assert not K.close_f16(got[-1:], NM.rope_fp16_products(x, cos, sin)[-1:], 0.02, 1e-3).all()
    assert not K.close_f16(got, NM.rope_table_by_head(x, cos, sin), 0.02, 1e-3).all()
