"""Fused attention (KIND 18, `attention_fp16`) on the GPU through the C ABI,
against the float64 oracle (`oracle.kernels.attention_fp16`): encoder shapes
(256 and 784 tokens, 12 heads of 64), ragged token counts that leave partial
query and key tiles, head_dim 32, several images per call, and the closed
forms. Tolerance: the matmul harness's (rel 1e-2, abs 1e-3,
`kernels/matmul_fp16/harness.c:145`); the kernel rounds the probabilities to
fp16 once before the P.V product, as the unfused chain rounds them."""
import numpy as np
import pytest

from oracle import kernels as K
from tests.gpu_util import Dev, h16, report

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(torch_gpu):
    return Dev(torch_gpu)


def run(dev, q, k, v, B, scale):
    rows, H, D = q.shape
    dq, dk, dv = dev.up(q), dev.up(k), dev.up(v)
    do = dev.empty((rows, H, D), np.float16)
    dev.lib.attention_fp16(dev.ptr(dq), dev.ptr(dk), dev.ptr(dv), dev.ptr(do), rows, H, D, B, scale)
    dev.check()
    return dev.down(do)


@pytest.mark.parametrize("B,T,H,D", [(1, 256, 12, 64), (1, 784, 12, 64), (1, 17, 3, 32), (2, 33, 2, 64),
                                     (1, 1, 1, 64), (3, 64, 4, 32), (1, 96, 2, 64), (4, 256, 2, 64)])
def test_attention(dev, B, T, H, D):
    r = np.random.default_rng(60 + T)
    q, k, v = (h16(r.standard_normal((B * T, H, D))) for _ in range(3))
    got = run(dev, q, k, v, B, D ** -0.5)
    want = K.attention_fp16(q, k, v, B, D ** -0.5)
    report(f"attention B{B} T{T} H{H} D{D}", got, want)
    assert K.close_f16(got, want, 1e-2, 1e-3).all()


def test_attention_sharp_scores(dev):
    """Large logits (scale 1, |q.k| up to ~60): the running max must keep
    exp2 in range; compared with the oracle."""
    r = np.random.default_rng(70)
    q, k, v = (h16(r.standard_normal((256, 4, 64)) * 1.0) for _ in range(3))
    got = run(dev, q, k, v, 1, 1.0)
    want = K.attention_fp16(q, k, v, 1, 1.0)
    report("attention sharp", got, want)
    assert np.isfinite(got.astype(np.float32)).all()
    assert K.close_f16(got, want, 1e-2, 1e-3).all()


def test_attention_uniform_is_mean_of_v(dev):
    r = np.random.default_rng(71)
    T, H, D = 100, 3, 64
    q = h16(np.zeros((T, H, D)))
    k, v = (h16(r.standard_normal((T, H, D))) for _ in range(2))
    got = run(dev, q, k, v, 1, 0.125)
    want = np.broadcast_to(v.astype(np.float64).mean(axis=0), got.shape)
    assert np.abs(got.astype(np.float64) - want).max() <= 2e-3


def test_attention_invalid_is_a_silent_no_op(dev):
    x = h16(np.ones((64, 2, 48)))
    dx = dev.up(x)
    do = dev.empty((64, 2, 48), np.float16)
    dev.lib.attention_fp16(dev.ptr(dx), dev.ptr(dx), dev.ptr(dx), dev.ptr(do), 64, 2, 48, 1, 0.1)   # D=48
    dev.lib.attention_fp16(dev.ptr(dx), dev.ptr(dx), dev.ptr(dx), dev.ptr(do), 63, 2, 32, 2, 0.1)   # 63 % 2
    dev.check()
    assert (dev.down(do) == np.float16(12345.0)).all()


def _tables(r, rows, T, H, D, B):
    from dataclasses import replace
    from hexlib_amd import encoder as E
    grid = int(round(np.sqrt(T)))
    if grid * grid == T:
        cfg = replace(E.QWEN35_VISION_FP16, image_size=16 * grid, hidden_size=H * D, num_heads=H, batch=B)
        return E.rope_tables(cfg)
    ang = r.random((rows, D // 2)) * 6.0
    return (np.concatenate([np.cos(ang)] * 2, axis=1).astype(np.float32),
            np.concatenate([np.sin(ang)] * 2, axis=1).astype(np.float32))


@pytest.mark.parametrize("B,T,H,D", [(1, 256, 12, 64), (1, 784, 12, 64), (2, 33, 2, 64), (3, 17, 2, 32)])
def test_rope_2d_qk_and_attention_qk_v(dev, B, T, H, D):
    """KIND 20 then KIND 19: rope_2d on the q and k slots of one fused
    [rows, 3, H, D] projection (bit-exact against rope_2d_fp16, itself pinned
    bit-exact against the reference baseline), then attention with q, k from
    its output and v from the projection."""
    r = np.random.default_rng(80 + T)
    rows = B * T
    qkv = h16(r.standard_normal((rows, 3, H, D)))
    cos, sin = _tables(r, rows, T, H, D, B)
    dqkv, dc, ds = dev.up(qkv), dev.up(cos), dev.up(sin)
    dqk = dev.empty((rows, 2, H, D), np.float16)
    dev.lib.rope_2d_qk_fp16(dev.ptr(dqkv), dev.ptr(dc), dev.ptr(ds), dev.ptr(dqk), rows, H, D)
    dev.check()
    qk = dev.down(dqk)
    np.testing.assert_array_equal(qk.view(np.uint16), K.rope_2d_qk_fp16(qkv, cos, sin).view(np.uint16))
    do = dev.empty((rows, H, D), np.float16)
    dev.lib.attention_qk_v_fp16(dev.ptr(dqk), dev.ptr(dqkv), dev.ptr(do), rows, H, D, B, D ** -0.5)
    dev.check()
    got = dev.down(do)
    want = K.attention_qk_v_fp16(qk, qkv, B, D ** -0.5)
    report(f"attention_qk_v B{B} T{T} H{H} D{D}", got, want)
    assert K.close_f16(got, want, 1e-2, 1e-3).all()


@pytest.mark.parametrize("B,T,H,D", [(1, 256, 12, 64), (1, 784, 12, 64), (2, 33, 2, 64), (3, 17, 2, 32),
                                     (32, 256, 12, 64)])
def test_attention_qkv(dev, B, T, H, D):
    """KIND 23: q, k, v all read from one [rows, 3, H, D] tensor -- the output
    of the q/k/v linear with rope in its epilogue. Bit-identical to KIND 19 fed
    the same q, k slots as a separate [rows, 2, H, D] tensor (same kernel,
    other strides), and within tolerance of the oracle."""
    r = np.random.default_rng(90 + T)
    rows = B * T
    qkv = h16(r.standard_normal((rows, 3, H, D)))
    qk = np.ascontiguousarray(qkv[:, :2])
    dqkv, dqk = dev.up(qkv), dev.up(qk)
    o1, o2 = dev.empty((rows, H, D), np.float16), dev.empty((rows, H, D), np.float16)
    dev.lib.attention_qkv_fp16(dev.ptr(dqkv), dev.ptr(o1), rows, H, D, B, D ** -0.5)
    dev.lib.attention_qk_v_fp16(dev.ptr(dqk), dev.ptr(dqkv), dev.ptr(o2), rows, H, D, B, D ** -0.5)
    dev.check()
    got = dev.down(o1)
    np.testing.assert_array_equal(got.view(np.uint16), dev.down(o2).view(np.uint16))
    want = K.attention_fp16(qkv[:, 0], qkv[:, 1], qkv[:, 2], B, D ** -0.5)
    report(f"attention_qkv B{B} T{T} H{H} D{D}", got, want)
    assert K.close_f16(got, want, 1e-2, 1e-3).all()


@pytest.mark.parametrize("form", [41, 21, 22, 42, 14, 1])
@pytest.mark.parametrize("B,T,H,D", [(4, 256, 2, 64), (1, 784, 2, 64), (2, 100, 3, 64), (3, 33, 2, 32),
                                     (1, 1, 1, 64), (2, 130, 2, 32)])
def test_attention_forms(dev, form, B, T, H, D):
    """Every attention form, forced through the override: the shared-K/V
    kernel with QG query groups and KS key splits (form QG * 10 + KS; the
    D = 32 build has 41 and 22, other forms fall back; 14 has one ring slot
    per split, so 784 tokens reuse it stage after stage), and the
    per-wave-tiles kernel (1). Ragged T leaves partial query groups, partial
    64-key stages and key splits with no stage at all; each against the
    float64 oracle."""
    r = np.random.default_rng(100 + T + form)
    q, k, v = (h16(r.standard_normal((B * T, H, D))) for _ in range(3))
    assert dev.lib.hexlib_gpu_attention_override(form) == 1
    try:
        got = run(dev, q, k, v, B, D ** -0.5)
    finally:
        dev.lib.hexlib_gpu_attention_override(0)
    want = K.attention_fp16(q, k, v, B, D ** -0.5)
    report(f"attention form {form} B{B} T{T} H{H} D{D}", got, want)
    assert K.close_f16(got, want, 1e-2, 1e-3).all()


def test_attention_override_rejects_unknown_forms(dev):
    for form in (2, 3, 11, 12, 44, -1):
        assert dev.lib.hexlib_gpu_attention_override(form) != 1
    assert dev.lib.hexlib_gpu_attention_override(0) == 1
