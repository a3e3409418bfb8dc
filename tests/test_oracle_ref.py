"""Pin the numpy kernel oracle (`oracle.kernels`) before trusting it.

Three independent checks per kernel:
1. against the reference's OWN scalar baselines (`kernels/*/baseline.c`,
   compiled unmodified into `oracle/_ref/libhexlib_ref.so`), at the harness
   shapes including their tails, with the harness tolerance -- bit-exact where
   the contract is a single rounding or a copy;
2. closed forms / invariants (softmax rows sum to 1, layernorm output has
   mean 0 and variance 1, rope with identity tables is the identity, the
   transposes are numpy permutations);
3. planted mistakes, restating the reference's near-miss files: each must
   FAIL the same comparison, so the comparison has teeth.
"""
import os

import numpy as np
import pytest

from oracle import kernels as K
from oracle import quant as Q
from oracle import ref as R

needs_ref = pytest.mark.skipif(
    not R.available() and not os.path.isdir("/root/reference"),
    reason="oracle/_ref not built and the reference tree is absent")


@pytest.fixture(scope="module", autouse=True)
def _ref_built():
    if not R.available() and os.path.isdir("/root/reference"):
        import subprocess
        subprocess.run(["make", "-s", "-C", os.path.dirname(R.__file__)], check=True)


def rng(seed=0):
    return np.random.default_rng(seed)


def h(x):
    return np.asarray(x, dtype=np.float16)


def close(got, want, rel, abs_tol):
    return bool(K.close_f16(got, want, rel, abs_tol).all())


# ---- 1. oracle vs the reference's compiled baselines --------------------------

@needs_ref
@pytest.mark.parametrize("n", [4100, 64, 7, 196608])
def test_add_bit_exact(n):
    a, b = h(rng(1).standard_normal(n) * 4), h(rng(2).standard_normal(n) * 4)
    np.testing.assert_array_equal(K.add_fp16(a, b).view(np.uint16), R.add_fp16(a, b).view(np.uint16))


@needs_ref
@pytest.mark.parametrize("factor", [0.125, 0.3])
def test_scale_bit_exact(factor):
    x = h(rng(3).standard_normal(4100) * 8)
    np.testing.assert_array_equal(K.scale_fp16(x, factor).view(np.uint16),
                                  R.scale_fp16(x, factor).view(np.uint16))


@needs_ref
@pytest.mark.parametrize("n", [4160, 4133])
def test_cast_bit_exact(n):
    x = (rng(4).standard_normal(n) * 1000).astype(np.float32)
    x[:4] = [65504.0, 65520.0, 1e-8, -6.1e-5]   # max, overflow-to-inf, underflow, subnormal
    np.testing.assert_array_equal(K.cast_f32_f16(x).view(np.uint16), R.cast_f32_f16(x).view(np.uint16))


@needs_ref
@pytest.mark.parametrize("R_,C", [(6, 256), (3, 784), (4, 100)])
def test_softmax_vs_baseline(R_, C):
    x = h(rng(5).standard_normal((R_, C)) * 3)
    x[0, :] = 0.0          # uniform row
    x[1, 5] = 11.0         # one dominant logit
    assert close(K.softmax_fp16(x), R.softmax_fp16(x), 0.01, 1e-3)


@needs_ref
@pytest.mark.parametrize("R_,C,rel,atol", [(4, 768, 0.02, 1e-3), (4, 64, 0.004, 1e-4)])
def test_layernorm_vs_baseline(R_, C, rel, atol):
    x = h(rng(6).standard_normal((R_, C)) + 30.0)   # large mean: two-pass matters
    w = (1 + 0.1 * rng(7).standard_normal(C)).astype(np.float32)
    b = (0.1 * rng(8).standard_normal(C)).astype(np.float32)
    assert close(K.layernorm_fp16(x, w, b, 1e-6), R.layernorm_fp16(x, w, b, 1e-6), rel, atol)


@needs_ref
def test_rmsnorm_vs_baseline():
    x = h(rng(9).standard_normal((8, 128)))
    x[3] = 1e-3                                   # eps-dominated row
    w = h(1 + 0.1 * rng(10).standard_normal(128))
    for eps in (1e-5, 1e-6):
        assert close(K.rmsnorm_fp16(x, w, eps), R.rmsnorm_fp16(x, w, eps), 0.02, 1e-3)


@needs_ref
@pytest.mark.parametrize("T,H,D", [(6, 3, 64), (5, 2, 10)])
def test_rope_bit_exact(T, H, D):
    x = h(rng(11).standard_normal((T, H, D)))
    ang = rng(12).standard_normal((T, D))
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    np.testing.assert_array_equal(K.rope_2d_fp16(x, cos, sin).view(np.uint16),
                                  R.rope_2d_fp16(x, cos, sin).view(np.uint16))


@needs_ref
@pytest.mark.parametrize("shape", [(8, 3, 64), (8, 3, 40)])
def test_transpose_th_exact(shape):
    x = h(rng(13).standard_normal(shape))
    np.testing.assert_array_equal(K.transpose_th_fp16(x), R.transpose_th_fp16(x))


@needs_ref
@pytest.mark.parametrize("shape", [(5, 64, 7), (5, 40, 7), (12, 256, 64)])
def test_transpose_hd_exact(shape):
    x = h(rng(14).standard_normal(shape))
    np.testing.assert_array_equal(K.transpose_hd_fp16(x), R.transpose_hd_fp16(x))


@needs_ref
@pytest.mark.parametrize("geom", [(3, 2, 256, 256, 16, 2, 16, 16), (2, 3, 12, 12, 3, 2, 4, 4),
                                  (3, 1, 256, 256, 16, 2, 16, 16)])
def test_patchify_exact(geom):
    C, T, H, W, p, m, gh, gw = geom
    img = rng(15).random((C, T, H, W), dtype=np.float32)
    np.testing.assert_array_equal(K.patchify_fp32(img, p, m, gh, gw), R.patchify_fp32(img, p, m, gh, gw))


@needs_ref
@pytest.mark.parametrize("dims", [(3, 40, 128, 200), (2, 16, 64, 32)])
def test_matmul_vs_baseline(dims):
    Bn, M, Kd, N = dims
    A, B = h(rng(16).standard_normal((Bn, M, Kd))), h(rng(17).standard_normal((Bn, Kd, N)))
    assert close(K.matmul_fp16(A, B), R.matmul_fp16(A, B), 1e-2, 1e-3)


@needs_ref
@pytest.mark.parametrize("M,Kd,N,act", [(4, 64, 32, 0), (20, 128, 160, 1), (3, 96, 64, 2)])
def test_matmul_epilogue_q4_vs_baseline(M, Kd, N, act):
    from hexlib_amd.quant import quantize_q4_0
    a = h(rng(18).standard_normal((M, Kd)))
    w = quantize_q4_0(rng(19).standard_normal((Kd, N)).astype(np.float32) * 0.1)
    bias = (0.5 * rng(20).standard_normal(N)).astype(np.float32)
    assert close(K.matmul_epilogue_fp16(a, w, bias, Kd, N, act),
                 R.matmul_epilogue_fp16(a, w, bias, Kd, N, act), 0.01, 3e-4)


# ---- 2. closed forms ------------------------------------------------------------

def test_softmax_rows_sum_to_one():
    y = K.softmax_fp16(h(rng(21).standard_normal((12, 256)))).astype(np.float64)
    np.testing.assert_allclose(y.sum(-1), 1.0, atol=256 * 2 ** -11)


def test_layernorm_standardises():
    x = h(rng(22).standard_normal((16, 768)) * 5 + 3)
    y = K.layernorm_fp16(x, np.ones(768, np.float32), np.zeros(768, np.float32), 1e-6).astype(np.float64)
    np.testing.assert_allclose(y.mean(-1), 0, atol=2e-3)
    np.testing.assert_allclose(y.var(-1), 1, atol=5e-3)


def test_rmsnorm_unit_rms():
    y = K.rmsnorm_fp16(h(rng(23).standard_normal((16, 768)) * 7), h(np.ones(768)), 1e-6).astype(np.float64)
    np.testing.assert_allclose(np.sqrt((y * y).mean(-1)), 1, atol=2e-3)


def test_rope_identity_tables_are_identity():
    x = h(rng(24).standard_normal((6, 3, 64)))
    y = K.rope_2d_fp16(x, np.ones((6, 64), np.float32), np.zeros((6, 64), np.float32))
    np.testing.assert_array_equal(y, x)


def test_rope_quarter_turn_rotates_halves():
    x = h(rng(25).standard_normal((2, 1, 8)))
    y = K.rope_2d_fp16(x, np.zeros((2, 8), np.float32), np.ones((2, 8), np.float32))
    np.testing.assert_array_equal(y[..., :4], -x[..., 4:])
    np.testing.assert_array_equal(y[..., 4:], x[..., :4])


def test_matmul_brute_force_tiny():
    A, B = h(rng(26).standard_normal((1, 3, 5))), h(rng(27).standard_normal((1, 5, 2)))
    want = np.zeros((3, 2))
    for i in range(3):
        for j in range(2):
            want[i, j] = sum(float(A[0, i, k]) * float(B[0, k, j]) for k in range(5))
    np.testing.assert_array_equal(K.matmul_fp16(A, B)[0], h(want))


def test_patchify_merge_order_by_hand():
    # 1 channel, 4x4 image, patch 1, merge 2: tokens walk 2x2 blocks.
    img = np.arange(16, dtype=np.float32).reshape(1, 1, 4, 4)
    out = K.patchify_fp32(img, 1, 2, 4, 4)[:, 0]
    np.testing.assert_array_equal(out, [0, 1, 4, 5, 2, 3, 6, 7, 8, 9, 12, 13, 10, 11, 14, 15])


def test_q4k_reduces_to_nblocked_on_the_transposed_weight():
    from hexlib_amd.quant import pack_q4_0_kgrouped, quantize_q4_0
    w = rng(28).standard_normal((64, 32)).astype(np.float32)
    a = h(rng(29).standard_normal((3, 64)))
    bias = np.zeros(32, np.float32)
    got = K.matmul_q4k(a, pack_q4_0_kgrouped(w), bias, 64, 32, 0)
    dq = Q.dequantize_q4_0_fp16(quantize_q4_0(w.T.copy()), (32, 64)).T
    np.testing.assert_array_equal(got, K.gemm_epilogue(a, dq, bias, 0))


# ---- 3. planted mistakes must fail --------------------------------------------------

@needs_ref
def test_nearmiss_unbiased_variance_fails():
    x = h(rng(30).standard_normal((4, 64)))
    w, b = np.ones(64, np.float32), np.zeros(64, np.float32)
    xf = x.astype(np.float64)
    mean = xf.mean(-1, keepdims=True)
    bad = ((xf - mean) / np.sqrt(xf.var(-1, ddof=1, keepdims=True) + 1e-6)).astype(np.float16)
    assert not close(bad, R.layernorm_fp16(x, w, b, 1e-6), 0.004, 1e-4)


@needs_ref
def test_nearmiss_softmax_wrong_axis_fails():
    x = h(rng(31).standard_normal((6, 256)))
    xf = x.astype(np.float64)
    bad = (np.exp(xf - xf.max(0)) / np.exp(xf - xf.max(0)).sum(0)).astype(np.float16)
    assert not close(bad, R.softmax_fp16(x), 0.01, 1e-3)


@needs_ref
def test_nearmiss_rope_adjacent_pairing_fails():
    x = h(rng(32).standard_normal((6, 3, 64)))
    ang = rng(33).standard_normal((6, 64))
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    xf = x.astype(np.float32)
    rot = np.empty_like(xf)
    rot[..., 0::2], rot[..., 1::2] = -xf[..., 1::2], xf[..., 0::2]
    bad = (xf * cos[:, None] + rot * sin[:, None]).astype(np.float16)
    assert not close(bad, R.rope_2d_fp16(x, cos, sin), 0.02, 1e-3)


@needs_ref
def test_nearmiss_matmul_transposed_operand_fails():
    A, B = h(rng(34).standard_normal((1, 16, 16))), h(rng(35).standard_normal((1, 16, 16)))
    bad = K.matmul_fp16(A, np.swapaxes(B, 1, 2))
    assert not close(bad, R.matmul_fp16(A, B), 1e-2, 1e-3)


@needs_ref
def test_nearmiss_q4_swapped_nibbles_fails():
    from hexlib_amd.quant import quantize_q4_0
    a = h(rng(36).standard_normal((4, 64)))
    w = bytearray(quantize_q4_0(rng(37).standard_normal((64, 32)).astype(np.float32)))
    good = R.matmul_epilogue_fp16(a, bytes(w), np.zeros(32, np.float32), 64, 32, 0)
    for blk in range(len(w) // 18):
        for j in range(16):
            v = w[blk * 18 + 2 + j]
            w[blk * 18 + 2 + j] = ((v & 0xF) << 4) | (v >> 4)
    bad = K.matmul_epilogue_fp16(a, bytes(w), np.zeros(32, np.float32), 64, 32, 0)
    assert not close(bad, good, 0.01, 3e-4)


@needs_ref
def test_nearmiss_gelu_swap_fails():
    from hexlib_amd.quant import quantize_q4_0
    a = h(rng(38).standard_normal((8, 64)) * 2)
    w = quantize_q4_0(rng(39).standard_normal((64, 64)).astype(np.float32) * 0.3)
    bias = np.full(64, -2.7, np.float32)
    good = R.matmul_epilogue_fp16(a, w, bias, 64, 64, 2)
    bad = K.matmul_epilogue_fp16(a, w, bias, 64, 64, 1)
    assert not close(bad, good, 0.01, 3e-4)


# ---- extensions: batch axis ------------------------------------------------------

@needs_ref
def test_transpose_bth_is_per_image_transpose_th():
    """[B,T,H,D] -> [B,H,T,D] is the reference transpose_th on each image."""
    x = h(rng(40).standard_normal((3, 8, 5, 16)))
    got = K.transpose_bth_fp16(x)
    for b in range(3):
        np.testing.assert_array_equal(got[b], R.transpose_th_fp16(x[b]))


@needs_ref
def test_batched_patchify_is_per_image_patchify():
    """A batch stacked on channels ([B*C,T,H,W]) patchifies to the per-image
    reference outputs stacked along tokens."""
    B, C, T, H, W, p, m, gh, gw = 3, 3, 1, 64, 64, 16, 2, 4, 4
    img = rng(41).random((B * C, T, H, W), dtype=np.float32)
    got = K.patchify_fp32(img, p, m, gh, gw, batch=B)
    want = np.concatenate([R.patchify_fp32(img[b * C:(b + 1) * C], p, m, gh, gw) for b in range(B)])
    np.testing.assert_array_equal(got, want)


# ---- fused attention (extension) ---------------------------------------------------

def _attn_inputs(B, T, H, D, seed):
    r = rng(seed)
    return [r.standard_normal((B * T, H, D)).astype(np.float32) for _ in range(3)]


@pytest.mark.parametrize("B,T,H,D", [(1, 16, 2, 32), (2, 9, 3, 64)])
def test_attention_is_the_chain_of_registry_references(B, T, H, D):
    """The fused op equals the reference chain it replaces (vit.py:185-193),
    composed from the pinned registry references: per image, [T,H,D] ->
    transpose(1,0,2) -> scale -> matmul with transpose(0,2,1) of k -> softmax
    -> matmul with v -> transpose(1,0,2)."""
    from oracle.refs import REFERENCES as RF
    q, k, v = _attn_inputs(B, T, H, D, 50)
    scale = D ** -0.5
    (got,) = RF["attention"]([q, k, v], {"scale": scale, "batch": B})
    for b in range(B):
        sl = slice(b * T, (b + 1) * T)
        qt, kt, vt = (RF["transpose"]([x[sl]], {"perm": (1, 0, 2)})[0] for x in (q, k, v))
        qs = RF["scale"]([qt], {"factor": scale})[0]
        ktt = RF["transpose"]([kt], {"perm": (0, 2, 1)})[0]
        p = RF["softmax"]([RF["matmul"]([qs, ktt], {})[0]], {"axis": -1})[0]
        ctx = RF["matmul"]([p, vt], {})[0]
        want = RF["transpose"]([ctx], {"perm": (1, 0, 2)})[0]
        np.testing.assert_allclose(got[sl], want, rtol=1e-4, atol=1e-5)


def test_attention_closed_forms():
    """q = 0: uniform weights, the output is each head's mean of v over keys.
    A key whose score dominates: the output is that key's v row."""
    from oracle.refs import attention
    _, k, v = _attn_inputs(1, 12, 2, 32, 51)
    q = np.zeros_like(k)
    (o,) = attention([q, k, v], {"scale": 0.125, "batch": 1})
    np.testing.assert_allclose(o, np.broadcast_to(v.mean(axis=0), o.shape), rtol=1e-6, atol=1e-7)
    q = np.broadcast_to(k[5] * 50.0, k.shape).copy()      # key 5 aligns with every query
    k2 = k.copy()
    k2[5] *= 4.0
    (o,) = attention([q, k2, v], {"scale": 1.0, "batch": 1})
    np.testing.assert_allclose(o, np.broadcast_to(v[5], o.shape), rtol=1e-5, atol=1e-5)


def test_nearmiss_attention_without_scale_fails():
    from oracle.refs import attention
    q, k, v = _attn_inputs(1, 16, 2, 32, 52)
    (good,) = attention([q, k, v], {"scale": 32 ** -0.5, "batch": 1})
    (bad,) = attention([q, k, v], {"scale": 1.0, "batch": 1})
    assert not close(bad.astype(np.float16), good.astype(np.float16), 1e-2, 1e-3)
