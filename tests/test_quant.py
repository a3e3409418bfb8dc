"""q4_0 and q8_0 packing: the product's vectorised quantizers against the
oracle's scalar transcriptions, plus known answers restated from the
reference's tests (`hexlib/tests/test_quant_q4_0.py`, `test_quant_q8_0.py`):
q4_0 nibble pairing j / j+16, signed scale, truncation (not banker's rounding)
at .5, the all-zero block; q8_0 positive scale, no bias, int8 element order,
half-away-from-zero rounding, saturation."""
import numpy as np

from hexlib_amd.quant import pack_q4_0_kgrouped, pack_q4_0_nblocked, q4_0_nbytes, quantize_q4_0
from oracle import quant as Q


def test_vectorised_equals_scalar_transcription():
    rng = np.random.default_rng(0)
    for shape in [(32,), (4, 64), (3, 96)]:
        x = (rng.standard_normal(shape) * rng.uniform(0.01, 5)).astype(np.float32)
        assert quantize_q4_0(x) == Q.quantize_q4_0_scalar(x)


def test_all_zero_block():
    b = quantize_q4_0(np.zeros(32, np.float32))
    # d = 0 / -8 = -0.0 (sign bit set), every code 8 -> value 0
    assert b == bytes([0x00, 0x80]) + bytes([0x88] * 16)
    assert b == Q.quantize_q4_0_scalar(np.zeros(32, np.float32))
    np.testing.assert_array_equal(Q.dequantize_q4_0(b, (32,)), 0)


def test_scale_is_signed_max_over_minus_8():
    x = np.linspace(-1, 4, 32).astype(np.float32)     # extreme element is +4
    b = quantize_q4_0(x)
    assert Q.block_scale(b, 0) == np.float16(-0.5)
    assert b[2] & 0x0F == 10                              # element 0 = -1 -> -1/-0.5 + 8.5 -> 10
    assert b[2 + 15] >> 4 == 0                            # element 31 = +4 -> q = 0


def test_nibble_pairing_is_j_with_j_plus_16():
    x = np.zeros(32, np.float32)
    x[0], x[16] = -8.0, 3.0     # signed max -8 -> d = 1
    b = quantize_q4_0(x)
    assert (b[2] & 0xF, b[2] >> 4) == (0, 11)          # byte 0 holds elements 0 and 16
    assert all(v == 0x88 for v in b[3:])
    v = Q.dequantize_q4_0(b, (32,))
    assert v[0] == -8.0 and v[16] == 3.0 and np.count_nonzero(v) == 2
    # the clamp is one-sided: +8 against d = 1 would need code 16 -> 15 (value 7)
    x[16] = 8.0
    assert Q.dequantize_q4_0(quantize_q4_0(x), (32,))[16] == 7.0


def test_truncation_not_round_half_even():
    # x/d + 8.5 = 10.0 exactly -> trunc 10; banker's rounding of 1.5 would give 2 (=10 too),
    # so use 2.5 -> +8.5 = 11.0 exactly -> 11, where round-half-even(2.5) = 2 -> 10.
    x = np.zeros(32, np.float32)
    x[0] = -8.0                    # d = 1
    x[1] = 2.5
    b = quantize_q4_0(x)
    assert b[3] & 0xF == 11


def test_round_trip_error_bounded():
    """Per block: an element rounds to the nearest of the 16 levels (q - 8) * d,
    so its error is at most d / 2, except where x / d >= 7.5 clips the code at
    15 (the opposite extreme of a block holding both signs), where it is at
    most d. d is the block's stored fp16 scale; the slack covers the fp32
    product x * (1 / d)."""
    rng = np.random.default_rng(1)
    x = rng.standard_normal((16, 64)).astype(np.float32)
    x[0, :32] = np.linspace(-1.0, 1.0, 32)           # both extremes in one block: a clipped code
    b = quantize_q4_0(x)
    y = Q.dequantize_q4_0(b, x.shape)
    signed_d = (np.frombuffer(b, np.uint8).reshape(-1, 18)[:, :2].copy().view(np.float16)
                .astype(np.float64).reshape(-1, 1))            # [blocks, 1]
    d = np.abs(signed_d)
    xb = x.reshape(-1, 32).astype(np.float64)
    err = np.abs(xb - y.reshape(-1, 32))
    clipped = np.trunc(xb / signed_d + 8.5) > 15
    assert clipped.sum() >= 1 and clipped.mean() < 0.01
    slack = d * 1e-6
    assert (err[~clipped] <= np.broadcast_to(0.5 * d + slack, err.shape)[~clipped]).all()
    assert (err[clipped] <= np.broadcast_to(d + slack, err.shape)[clipped]).all()


def test_layouts_and_sizes():
    w = np.random.default_rng(2).standard_normal((64, 96)).astype(np.float32)
    assert len(pack_q4_0_nblocked(w)) == q4_0_nbytes(64, 96)
    assert len(pack_q4_0_kgrouped(w)) == q4_0_nbytes(64, 96)
    np.testing.assert_array_equal(Q.dequantize_q4_0(pack_q4_0_kgrouped(w), (96, 64)),
                                  Q.dequantize_q4_0(quantize_q4_0(w.T.copy()), (96, 64)))


# ---- q8_0 (hexlib/exec/quant.py:138-220; reference tests test_quant_q8_0.py) ----

def _q8_blocks(raw):
    b = np.frombuffer(raw, np.uint8).reshape(-1, 34)
    return b[:, :2].copy().view(np.float16).reshape(-1), b[:, 2:].copy().view(np.int8)


def test_q8_0_matches_the_scalar_ggml_transcription():
    from hexlib_amd.quant import quantize_q8_0
    from oracle.quant import quantize_q8_0_scalar
    r = np.random.default_rng(11)
    for x in (r.standard_normal((8, 64)).astype(np.float32),
              (r.standard_normal((4, 96)) * 1e-3).astype(np.float32),
              r.standard_normal((2, 32)).astype(np.float16).astype(np.float32)):
        assert quantize_q8_0(x) == quantize_q8_0_scalar(x)


def test_q8_0_scale_is_positive_and_has_no_bias():
    """d = amax / 127 > 0 whichever sign the extreme has (q4_0's signed trick
    would negate the block); q is a plain signed byte per element."""
    from hexlib_amd.quant import quantize_q8_0
    for sign in (1.0, -1.0):
        blk = np.linspace(-0.5, 0.5, 32).astype(np.float32)
        blk[7] = sign * 2.0
        d, q = _q8_blocks(quantize_q8_0(blk))
        assert d[0] > 0 and abs(float(d[0]) - 2.0 / 127) < 1e-3
        assert q[0, 7] == int(sign * 127)
        assert q[0, 16] == int(np.sign(blk[16]) * np.floor(abs(blk[16] / np.float32(d[0])) + 0.5))


def test_q8_0_rounds_half_away_from_zero():
    """roundf, not banker's rounding: with d = 1 exactly (amax 127), 2.5 -> 3
    and -2.5 -> -3 (np.round would give 2 and -2)."""
    from hexlib_amd.quant import quantize_q8_0
    blk = np.zeros(32, np.float32)
    blk[0], blk[1], blk[2], blk[3], blk[4] = 127.0, 2.5, -2.5, 0.5, -1.5
    d, q = _q8_blocks(quantize_q8_0(blk))
    assert float(d[0]) == 1.0
    assert list(q[0, :5]) == [127, 3, -3, 1, -2]


def test_q8_0_saturates_after_the_fp16_narrowing_of_d():
    """amax / 127 narrowed DOWN to fp16 makes |x / d| above 127 for the
    extreme element -- enough to round to 128 where d is an fp16 subnormal
    (tiny blocks): it must clip to 127, not wrap to -128."""
    from hexlib_amd.quant import quantize_q8_0
    from oracle.quant import quantize_q8_0_scalar
    found = False
    for amax in np.geomspace(1e-8, 10.0, 4000).astype(np.float32):
        d16 = np.float16(amax / np.float32(127.0))
        if 0 < np.float32(d16) < amax / np.float32(127.0) and amax / np.float32(d16) >= np.float32(127.5):
            blk = np.zeros(32, np.float32)
            blk[3] = amax
            _, q = _q8_blocks(quantize_q8_0(blk))
            assert q[0, 3] == 127
            assert quantize_q8_0(blk) == quantize_q8_0_scalar(blk)
            found = True
            break
    assert found


def test_q8_0_zero_block_and_round_trip():
    from hexlib_amd.quant import quantize_q8_0
    from oracle.quant import dequantize_q8_0
    d, q = _q8_blocks(quantize_q8_0(np.zeros((1, 32), np.float32)))
    assert float(d[0]) == 0.0 and not q.any()
    r = np.random.default_rng(12)
    x = r.standard_normal((16, 128)).astype(np.float32)
    y = dequantize_q8_0(quantize_q8_0(x), x.shape)
    amax = np.abs(x.reshape(-1, 32)).max(axis=1, keepdims=True)
    # |error| <= d / 2 per element, d ~ amax / 127 (plus fp16 narrowing of d)
    assert (np.abs((y - x).reshape(-1, 32)) <= amax / 127 * 0.51 + 1e-7).all()
    assert len(quantize_q8_0(x)) == 16 * 128 // 32 * 34
