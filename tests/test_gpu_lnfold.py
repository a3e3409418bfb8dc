"""The LayerNorm folded into the linear it feeds (KIND 26 / 27) on the GPU,
through the C ABI.

`lnfold_matmul_epilogue_f16wt*` multiplies the LayerNorm's raw input by the
weight-scaled W' and applies rstd (acc - mean c1) + c2 in the epilogue, with
each row's mean and rstd taken from the x tiles the product reads. Two checks
per case:
- against a float64 model of that same formula (`lnfold_model`): tight, so a
  wrong row statistic, a c1/c2 mix-up or a dropped term fails at once;
- against the exact product (the LayerNorm and the linear in float64, no
  intermediate rounding), beside the oracle's layernorm_fp16 then
  matmul_epilogue_f16w (the reference's two kernels,
  `kernels/layernorm_fp16/baseline.c`, `kernels/matmul_epilogue_fp16/baseline.c`):
  the fold must be as accurate as that two-kernel path. The two paths round
  different intermediates -- the reference the normalised row, the fold the
  scaled weight -- so they differ from each other by about twice either's
  error (up to ~4e-3 at unit-scale outputs), while each sits the same rms
  distance from the exact result.
"""
import numpy as np
import pytest

from hexlib_amd.graph.fuse import lnfold_bias2, lnfold_weight
from oracle import kernels as K
from tests.gpu_util import Dev, h16, report

pytestmark = pytest.mark.gpu

EPS = 1e-6


@pytest.fixture(scope="module")
def dev(torch_gpu):
    return Dev(torch_gpu)


def _gelu_tanh(v):
    return 0.5 * v * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (v + 0.044715 * v ** 3)))


def _act(v, act):
    if act == 1:
        return _gelu_tanh(v)
    if act == 2:
        from scipy.special import erf
        return 0.5 * v * (1.0 + erf(v / np.sqrt(2.0)))
    return v


def lnfold_model(x, w, g, b, bias, act, eps=EPS):
    """float64 restatement of the folded kernel's arithmetic before its one
    rounding to fp16: rstd (x W' - mean c1) + c2, then the activation."""
    wf = lnfold_weight(w, g).astype(np.float64)
    b2 = lnfold_bias2(w, g, b, bias).astype(np.float64)
    n = w.shape[1]
    c2, c1 = b2[:n], b2[n:]
    xf = x.astype(np.float64)
    mean = xf.mean(axis=1, keepdims=True)
    var = np.maximum((xf * xf).mean(axis=1, keepdims=True) - mean * mean, 0.0)
    inv = 1.0 / np.sqrt(var + np.float32(eps))
    return _act(inv * (xf @ wf - mean * c1[None, :]) + c2[None, :], act)


def exact_linear(x, g, b, w, bias, act, eps=EPS):
    """LayerNorm then the linear and the activation in float64, no rounding."""
    xf = x.astype(np.float64)
    m = xf.mean(axis=1, keepdims=True)
    v = ((xf - m) ** 2).mean(axis=1, keepdims=True)
    y = (xf - m) / np.sqrt(v + np.float32(eps)) * g + b
    return _act(y @ w.astype(np.float64) + bias, act)


def assert_as_accurate(name, got, ref, exact):
    """`got` (the fold) is as close to `exact` as `ref` (the reference's
    two-kernel path) is: rms within 10%, worst element within 1.5x."""
    eg = np.abs(got.astype(np.float64) - exact)
    er = np.abs(ref.astype(np.float64) - exact)
    rg, rr = np.sqrt((eg ** 2).mean()), np.sqrt((er ** 2).mean())
    print(f"[{name}] vs exact: fold rms {rg:.3e} max {eg.max():.3e}; layernorm + linear rms {rr:.3e} "
          f"max {er.max():.3e}", flush=True)
    assert rg <= 1.1 * rr + 1e-7
    assert eg.max() <= 1.5 * er.max() + 1e-6


def _inputs(seed, M, Kd, N, offset=0.5, scale=2.0):
    r = np.random.default_rng(seed)
    x = h16(r.standard_normal((M, Kd)) * scale + offset)
    g = (1.0 + 0.1 * r.standard_normal(Kd)).astype(np.float32)
    b = (0.1 * r.standard_normal(Kd)).astype(np.float32)
    w = h16(r.standard_normal((Kd, N)) / np.sqrt(Kd))
    bias = (0.05 * r.standard_normal(N)).astype(np.float32)
    return x, g, b, w, bias


@pytest.mark.parametrize("M,Kd,N,act", [(256, 768, 3072, 1), (256, 768, 2304, 0), (200, 512, 200, 2),
                                        (65, 256, 64, 1), (1, 768, 96, 0), (784, 768, 3072, 1),
                                        (256, 1024, 136, 0),
                                        # the tiled 64x64 form (more 64x64 tiles than CUs; ragged N)
                                        (1000, 256, 1100, 2),
                                        # the large-tile form: 128 x 192 tiles (ragged M), 128 x 128
                                        (4160, 768, 1536, 1), (8192, 768, 3072, 1), (8192, 512, 512, 0)])
def test_lnfold_linear(dev, M, Kd, N, act):
    """KIND 26 on the K-across-waves form (its 64x64 tiles within a round of
    CUs), the tiled 64x64 form (784 rows: 448x448) and the large-tile form
    (128-row tiles filling a round of CUs)."""
    x, g, b, w, bias = _inputs(41, M, Kd, N)
    wt = np.ascontiguousarray(lnfold_weight(w, g).T)
    b2 = lnfold_bias2(w, g, b, bias)
    dx, dw, db = dev.up(x), dev.up(wt), dev.up(b2)
    do = dev.empty((M, N), np.float16)
    dev.lib.lnfold_matmul_epilogue_f16wt_fp16(dev.ptr(dx), dev.ptr(dw), dev.ptr(db), dev.ptr(do), M, Kd, N, act,
                                              EPS)
    dev.check()
    got = dev.down(do)
    model = lnfold_model(x, w, g, b, bias, act)
    report(f"lnfold {M}x{Kd}x{N} act {act} vs model", got, model.astype(np.float16))
    assert K.close_f16(got, model, 2e-3, 2e-4).all()
    want = K.matmul_epilogue_f16w(K.layernorm_fp16(x, g, b, EPS), w, bias, act)
    assert_as_accurate(f"lnfold {M}x{Kd}x{N} act {act}", got, want, exact_linear(x, g, b, w, bias, act))


@pytest.mark.parametrize("offset,scale", [(8.0, 1.0), (-3.0, 0.25), (0.0, 30.0)])
def test_lnfold_row_statistics(dev, offset, scale):
    """Rows far from zero mean, narrow rows and wide rows: with the one-pass
    fp32 variance the fold stays as accurate as the two-pass LayerNorm path."""
    M, Kd, N = 128, 768, 256
    x, g, b, w, bias = _inputs(43, M, Kd, N, offset=offset, scale=scale)
    dx, dw = dev.up(x), dev.up(np.ascontiguousarray(lnfold_weight(w, g).T))
    db, do = dev.up(lnfold_bias2(w, g, b, bias)), dev.empty((M, N), np.float16)
    dev.lib.lnfold_matmul_epilogue_f16wt_fp16(dev.ptr(dx), dev.ptr(dw), dev.ptr(db), dev.ptr(do), M, Kd, N, 0, EPS)
    dev.check()
    got = dev.down(do)
    assert K.close_f16(got, lnfold_model(x, w, g, b, bias, 0), 2e-3, 2e-4).all()
    want = K.matmul_epilogue_f16w(K.layernorm_fp16(x, g, b, EPS), w, bias, 0)
    assert_as_accurate(f"lnfold stats offset {offset} scale {scale}", got, want, exact_linear(x, g, b, w, bias, 0))


def _rope_tables(r, M, d):
    ang = r.random((M, d // 2)) * 6.0
    return (np.concatenate([np.cos(ang)] * 2, axis=1).astype(np.float32),
            np.concatenate([np.sin(ang)] * 2, axis=1).astype(np.float32))


@pytest.mark.parametrize("M,Kd,heads,d,extra", [(256, 768, 12, 64, 768), (70, 256, 2, 64, 128),
                                                (200, 512, 3, 16, 32),
                                                # the tiled 64x64 rope form
                                                (784, 768, 12, 64, 768), (1000, 256, 8, 16, 1088),
                                                # the large-tile rope forms: 128 x 192, 128 x 128
                                                (8192, 768, 12, 64, 768), (8192, 256, 3, 64, 128)])
def test_lnfold_rope_linear(dev, M, Kd, heads, d, extra):
    """KIND 27: the folded LayerNorm with the q/k rope in the epilogue (the
    encoder's q/k/v linear): against the model (its v columns tight, its q/k
    columns through rope_2d) and as accurate as layernorm + linear + rope_2d
    against the exact product."""
    N = 2 * heads * d + extra
    x, g, b, w, bias = _inputs(47, M, Kd, N)
    r = np.random.default_rng(48)
    cos, sin = _rope_tables(r, M, d)
    wt = K.permute_rope_rows(lnfold_weight(w, g).T, heads, d)
    dx, dw, db = dev.up(x), dev.up(wt), dev.up(lnfold_bias2(w, g, b, bias))
    dc, ds = dev.up(np.ascontiguousarray(cos.T)), dev.up(np.ascontiguousarray(sin.T))
    do = dev.empty((M, N), np.float16)
    dev.lib.lnfold_matmul_epilogue_f16wt_rope_fp16(dev.ptr(dx), dev.ptr(dw), dev.ptr(db), dev.ptr(dc), dev.ptr(ds),
                                                   dev.ptr(do), M, Kd, N, 0, heads, d, EPS)
    dev.check()
    got = dev.down(do)
    rq = 2 * heads * d

    def roped(lin):
        out = lin.astype(np.float16).copy()
        out[:, :rq] = K.rope_2d_fp16(out[:, :rq].reshape(M, 2 * heads, d), cos, sin).reshape(M, -1)
        return out

    def roped64(lin):
        out = lin.copy()
        q = out[:, :rq].reshape(M, 2 * heads, d)
        h = d // 2
        c, s_ = cos[:, None, :].astype(np.float64), sin[:, None, :].astype(np.float64)
        rot = np.concatenate([-q[..., h:], q[..., :h]], axis=-1)
        out[:, :rq] = (q * c + rot * s_).reshape(M, -1)
        return out

    lin = lnfold_model(x, w, g, b, bias, 0)
    # v columns: the model's one rounding; q/k columns: rotated after that
    # rounding, so a one-ulp difference in a rotated pair's inputs moves a
    # near-cancelling output by up to an ulp of the inputs (4e-3 at |x| < 8)
    assert K.close_f16(got[:, rq:], lin[:, rq:], 2e-3, 2e-4).all()
    assert np.abs(lin[:, :rq]).max() < 8.0
    assert K.close_f16(got[:, :rq], roped(lin)[:, :rq], 4e-3, 4e-3).all()
    want = roped(K.matmul_epilogue_f16w(K.layernorm_fp16(x, g, b, EPS), w, bias, 0))
    assert_as_accurate(f"lnfold rope {M}x{Kd}x{N}", got, want, roped64(exact_linear(x, g, b, w, bias, 0)))


def test_lnfold_invalid_is_a_silent_no_op(dev):
    """K not a multiple of 256 and a misaligned x leave the output untouched,
    as every kernel_api.h entry does on invalid dimensions."""
    M, N = 64, 64
    out = dev.up(np.full((M, N), 7, np.float16))
    for Kd, off in ((128, 0), (384, 0), (256, 2)):
        x = dev.up(np.zeros((M, Kd), np.float16), off)
        w, b2 = dev.up(np.zeros((N, Kd), np.float16)), dev.up(np.zeros(2 * N, np.float32))
        dev.lib.lnfold_matmul_epilogue_f16wt_fp16(dev.ptr(x), dev.ptr(w), dev.ptr(b2), dev.ptr(out), M, Kd, N, 0,
                                                  EPS)
    dev.check()
    assert (dev.down(out) == 7).all()
