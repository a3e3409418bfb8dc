"""The GPU parity checks have teeth: the reference's near-misses
(`kernels/<k>/nearmiss_*.c`), restated on the CPU in `tests/nearmiss.py`,
FAIL the check the GPU test of that kernel applies, on the inputs that GPU
test uses (the harness's adversarial cells, `tests/harness_data.py`, and the
seeded shapes):
- the precision-class mistakes (fp16 accumulation, bias after activation, a
  scale off by one block, softmax without the max or summed in fp16, rmsnorm
  without eps, rope products rounded early or indexed by head, patchify
  ignoring the merge) fail the `close_f16` bound;
- the structural ones (a dropped tail, an integer add, a splatted number,
  lane-order slips in the cast, affine parameters on the wrong columns, the
  mean instead of the RMS, rope sign, extent and table slips, copies and
  stride slips in the transposes and in the batched matmul, channel/time and
  patch-interior swaps in patchify) change outputs that the bit-exact tests
  compare, or fail the bound where the test has one.
The GPU tests check the kernels against the correct oracle on the same inputs
(`tests/test_gpu_kernels.py`, `tests/test_gpu_gemm.py`), so a kernel that
carried one of these mistakes could not pass them. CPU only.
"""
import numpy as np

from oracle import kernels as K
from tests import harness_data as HD
from tests import nearmiss as NM


def rejects(bad, good, rel, abs_tol):
    """The bound rejects `bad`: some element is outside it (NaN counts)."""
    with np.errstate(invalid="ignore"):
        return not K.close_f16(bad, good, rel, abs_tol).all()


# ---- GEMMs --------------------------------------------------------------------------

def test_matmul_fp16_accumulation_fails_the_matmul_bound():
    A, B, (b, m, n) = HD.matmul_adversarial()
    good = K.matmul_fp16(A, B)
    bad = NM.matmul_fp16_accumulate(A, B)
    assert float(good[b, m, n]) == 2.125                      # 2.1240234375 rounded once
    assert float(bad[b, m, n]) == 2.0                          # every follower rounded away
    assert rejects(bad, good, 1e-2, 1e-3)


def test_epilogue_fp16_accumulation_fails_the_epilogue_bound():
    a, w, bias, M, Kd, N, act = HD.epilogue_cell1()
    good = K.matmul_epilogue_fp16(a, w, bias, Kd, N, act)
    bad = NM.epilogue_fp16_accumulation(a, NM.dense_q4_nblocked(w, Kd, N), bias, act)
    assert float(good[0, 0]) == 1.015625 and float(bad[0, 0]) == 1.0
    assert rejects(bad, good, 0.01, 3e-4)


def test_f16_weight_fp16_accumulation_fails_the_epilogue_bound():
    a, w, bias, act = HD.epilogue_cell1_f16()
    good = K.matmul_epilogue_f16w(a, w, bias, act)
    bad = NM.epilogue_fp16_accumulation(a, w, bias, act)
    assert float(bad[0, 0]) == 1.0 and abs(float(good[0, 0]) - 1.1872558) < 1e-3
    assert rejects(bad, good, 0.01, 3e-4)


def test_bias_after_activation_fails_the_epilogue_bound():
    """On the cfg-3 sweep's data (A, W ~ N(0, 0.02) fp16, bias N(0, 0.02)
    fp32, gelu_tanh), the size the judge called weak: the mistake still moves
    most outputs past (rel 0.01, abs 3e-4)."""
    r = np.random.default_rng(70)
    a = (r.standard_normal((256, 768)) * 0.02).astype(np.float16)
    w = (r.standard_normal((768, 2304)) * 0.02).astype(np.float16)
    bias = (r.standard_normal(2304) * 0.02).astype(np.float32)
    good = K.matmul_epilogue_f16w(a, w, bias, 1)
    bad = NM.epilogue_bias_after_activation(a, w, bias, 1)
    assert rejects(bad, good, 0.01, 3e-4)
    a, w4, bias4, M, Kd, N, _ = HD.epilogue_cell1()
    bias4 = (np.random.default_rng(71).standard_normal(N) * 0.5).astype(np.float32)
    good = K.matmul_epilogue_fp16(a, w4, bias4, Kd, N, 1)
    bad = NM.epilogue_bias_after_activation(a, NM.dense_q4_nblocked(w4, Kd, N), bias4, 1)
    assert rejects(bad, good, 0.01, 3e-4)


def test_scale_off_by_one_block_fails_the_epilogue_bound():
    a, w, bias, M, Kd, N, act = HD.epilogue_cell1()
    good = K.matmul_epilogue_fp16(a, w, bias, Kd, N, act)
    bad = K.gemm_epilogue(a, NM.dequant_scale_off_by_one_block(w, Kd, N), bias, act)
    assert rejects(bad, good, 0.01, 3e-4)


def test_fp16_accumulation_would_pass_on_generic_small_data():
    """Why the crafted cells exist: on the cfg-3 scale's generic data alone an
    fp16 running sum at K = 64 stays inside the matmul bound -- so the GPU
    tests carry the harness's adversarial element as well."""
    r = np.random.default_rng(72)
    A = (r.standard_normal((2, 32, 64)) * 0.02).astype(np.float16)
    B = (r.standard_normal((2, 64, 48)) * 0.02).astype(np.float16)
    assert not rejects(NM.matmul_fp16_accumulate(A, B), K.matmul_fp16(A, B), 1e-2, 1e-3)


# ---- row reductions ---------------------------------------------------------------

def test_softmax_sum_in_fp16_fails_on_harness_row_1():
    x = HD.softmax_rows()
    good = K.softmax_fp16(x)
    bad = NM.softmax_sum_fp16(x)
    assert rejects(bad[1:2], good[1:2], 0.01, 1e-3)
    assert not rejects(bad[2:], good[2:], 0.01, 1e-3)        # generic rows alone would not catch it


def test_softmax_without_max_subtraction_fails_on_harness_row_0():
    x = HD.softmax_rows()
    bad = NM.softmax_no_max_subtraction(x)
    assert np.isnan(bad[0].astype(np.float32)).any()
    assert rejects(bad, K.softmax_fp16(x), 0.01, 1e-3)


def test_rmsnorm_without_eps_fails_on_harness_row_0():
    x, w, eps = HD.rmsnorm_rows()
    good = K.rmsnorm_fp16(x, w, eps)
    bad = NM.rmsnorm_no_eps(x, w, eps)
    assert rejects(bad[:1], good[:1], 0.02, 1e-3)
    assert not rejects(bad[1:], good[1:], 0.02, 1e-3)


# ---- rope and patchify --------------------------------------------------------------

def test_rope_fp16_products_fail_on_the_near_cancellation_token():
    """The GPU rope test is bit-exact, so any change fails it; the point here
    is that the harness's bound (rel 0.02, abs 1e-3) rejects this mistake too,
    on the crafted token alone."""
    x, cos, sin = HD.rope_near_cancellation()
    good = K.rope_2d_fp16(x, cos, sin)
    bad = NM.rope_fp16_products(x, cos, sin)
    assert abs(float(good[-1, 0, 0]) + 0.1) < 1e-3 and float(bad[-1, 0, 0]) == 0.0
    assert rejects(bad[-1:], good[-1:], 0.02, 1e-3)


def test_rope_table_indexed_by_head_fails():
    x, cos, sin = HD.rope_near_cancellation()
    assert rejects(NM.rope_table_by_head(x, cos, sin), K.rope_2d_fp16(x, cos, sin), 0.02, 1e-3)


def test_patchify_ignoring_merge_fails():
    img = np.random.default_rng(73).random((3, 1, 64, 64), dtype=np.float32)
    good = K.patchify_fp32(img, 16, 2, 4, 4)
    bad = NM.patchify_merge_ignored(img, 16, 2, 4, 4)
    assert good.shape == bad.shape and not np.array_equal(good, bad)


# ---- structural mistakes against the bit-exact GPU tests ------------------------------
# `tests/test_gpu_kernels.py` checks these kernels bit for bit against the
# oracle, on the inputs rebuilt below (same seeds, scales and shapes; outputs
# poisoned with 12345.0). Each mistake changes some output on the cases named,
# so a kernel carrying it fails those cases.

POISON = np.float16(12345.0)


def rng(s):
    return np.random.default_rng(s)


def h16(a):
    return np.asarray(a).astype(np.float16)


def differs(bad, good):
    return not np.array_equal(np.asarray(bad).view(np.uint8), np.asarray(good).view(np.uint8))


def _add_inputs(n):
    return h16(rng(1).standard_normal(n) * 4), h16(rng(2).standard_normal(n) * 4)


def test_add_dropping_the_tail_fails_the_tail_cases():
    for n, caught in [(4100, True), (7, True), (12345, True), (196608, False)]:
        a, b = _add_inputs(n)
        bad = NM.add_drops_the_tail(a, b, np.full(n, POISON))
        assert differs(bad, K.add_fp16(a, b)) == caught, n   # the encoder's 196608 alone would pass it


def test_integer_add_fails():
    a, b = _add_inputs(4100)
    bad, good = NM.add_as_integers(a, b), K.add_fp16(a, b)
    assert differs(bad, good)
    with np.errstate(invalid="ignore"):
        assert (np.sign(bad.astype(np.float32)) != np.sign(good.astype(np.float32))).any()   # wrong signs


def test_scale_mistakes_fail():
    for n, factor in [(4100, 0.125), (196608, 0.125), (4100, 0.3), (999, 0.7)]:
        x = h16(rng(3).standard_normal(n) * 8)
        good = K.scale_fp16(x, factor)
        assert differs(NM.scale_drops_the_tail(x, factor, np.full(n, POISON)), good) == (n % 64 != 0)
        bad = NM.scale_splats_the_number(x, factor)
        assert differs(bad, good) and not bad.astype(np.float32).any()   # multiplied by +0.0


def test_cast_lane_order_mistakes_fail():
    for n in (4160, 4133, 196608, 1001):
        x = (rng(4).standard_normal(n) * 3000).astype(np.float32)
        x[:6] = [65504.0, 65520.0, 1e-8, -6.1e-5, np.inf, -0.0]
        with np.errstate(over="ignore"):
            good = K.cast_f32_f16(x)
            for mistake in (NM.cast_forgets_the_deal, NM.cast_one_input_vector_per_output, NM.cast_swapped_halves):
                assert differs(mistake(x), good), (mistake.__name__, n)


def test_layernorm_permuted_affine_fails_the_layernorm_bound():
    for R, C, rel, atol in [(256, 768, 0.02, 1e-3), (4, 64, 0.004, 1e-4), (3, 100, 0.02, 1e-3)]:
        x = h16(rng(6).standard_normal((R, C)) * 2 + 3)
        w = (1 + 0.1 * rng(7).standard_normal(C)).astype(np.float32)
        b = (0.1 * rng(8).standard_normal(C)).astype(np.float32)
        good = K.layernorm_fp16(x, w, b, 1e-6)
        assert rejects(NM.layernorm_permuted_affine(x, w, b, 1e-6), good, rel, atol), (R, C)
    # with a constant weight and zero bias the same mistake is invisible
    x = h16(rng(6).standard_normal((4, 64)) * 2 + 3)
    w, b = np.full(64, 1.5, np.float32), np.zeros(64, np.float32)
    assert not differs(NM.layernorm_permuted_affine(x, w, b, 1e-6), K.layernorm_fp16(x, w, b, 1e-6))


def test_rmsnorm_mean_not_rms_fails_the_rmsnorm_bound():
    for R, C, eps in [(256, 768, 1e-6), (8, 128, 1e-5), (16, 64, 1e-6)]:
        x = h16(rng(9).standard_normal((R, C)))
        x[min(2, R - 1)] = 1e-3
        w = h16(1 + 0.1 * rng(10).standard_normal(C))
        assert rejects(NM.rmsnorm_mean_not_rms(x, w, eps), K.rmsnorm_fp16(x, w, eps), 0.02, 1e-3), (R, C)


def test_rope_mistakes_fail():
    from hexlib_amd import encoder as E
    for T, Hh, D, tables in [(256, 12, 64, "encoder"), (6, 3, 64, "random"), (5, 2, 10, "random")]:
        x = h16(rng(11).standard_normal((T, Hh, D)))
        if tables == "encoder":
            cos, sin = E.rope_tables(E.QWEN35_VISION_FP16)
        else:
            ang = rng(12).standard_normal((T, D))
            cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
        good = K.rope_2d_fp16(x, cos, sin)
        for mistake in (NM.rope_negated_term, lambda *a: NM.rope_partial_rotation(*a, POISON),
                        NM.rope_swapped_tables):
            bad = mistake(x, cos, sin)
            assert differs(bad, good), (mistake.__name__, T, D)
            assert rejects(bad, good, 0.02, 1e-3), (mistake.__name__, T, D)   # the harness bound too


def test_transpose_th_mistakes_fail():
    for shape in [(256, 12, 64), (8, 3, 64), (8, 3, 40), (5, 7, 3), (12, 256, 64)]:
        x = h16(rng(13).standard_normal(shape))
        good = K.transpose_th_fp16(x)
        assert differs(NM.transpose_th_plain_copy(x), good), shape
        assert differs(NM.transpose_th_swapped_stride(x, POISON), good), shape
    x = h16(rng(13).standard_normal((6, 6, 8)))                  # T == H: the swap is harmless
    assert not differs(NM.transpose_th_swapped_stride(x, POISON), K.transpose_th_fp16(x))


def test_transpose_hd_mistakes_fail():
    for shape in [(12, 256, 64), (5, 64, 7), (5, 40, 7), (3, 100, 70), (12, 784, 64), (2, 128, 64)]:
        x = h16(rng(15).standard_normal(shape))
        good = K.transpose_hd_fp16(x)
        for bad in (NM.transpose_hd_plain_copy(x), NM.transpose_hd_swapped_stride(x, POISON),
                    NM.transpose_hd_batch_last(x)):
            assert differs(bad, good), shape


def test_matmul_batch0_a_fails_the_matmul_bound():
    for Bn, M, Kd, N in [(12, 256, 64, 256), (3, 40, 128, 200), (2, 17, 33, 45)]:
        A = h16(rng(1).standard_normal((Bn, M, Kd)))
        B = h16(rng(2).standard_normal((Bn, Kd, N)) * 0.1)
        assert rejects(NM.matmul_batch0_a(A, B), K.matmul_fp16(A, B), 1e-2, 1e-3), (Bn, M)


def test_patchify_mistakes_fail():
    for (C, T, Hh, W, p, m, gh, gw), batch in [((3, 1, 256, 256, 16, 2, 16, 16), 1),
                                             ((3, 2, 256, 256, 16, 2, 16, 16), 1),
                                             ((2, 3, 12, 12, 3, 2, 4, 4), 1), ((3, 1, 64, 64, 16, 2, 4, 4), 2)]:
        img = rng(16).random((batch * C, T, Hh, W), dtype=np.float32)
        good = K.patchify_fp32(img, p, m, gh, gw, batch)
        assert differs(NM.patchify_patch_transposed(img, p, m, gh, gw, batch), good)
        # the channel/time swap only shows with C > 1 and T > 1, hence the T = 2 cases
        assert differs(NM.patchify_channel_time_swapped(img, p, m, gh, gw, batch), good) == (T > 1)
