"""q4_0 packing: the product's vectorised quantizer against the oracle's scalar
transcription, plus known answers restated from the reference's q4_0 tests
(`hexlib/tests/test_quant_q4_0.py`): nibble pairing j / j+16, signed scale,
truncation (not banker's rounding) at .5, the all-zero block."""
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
    rng = np.random.default_rng(1)
    x = rng.standard_normal((16, 64)).astype(np.float32)
    b = quantize_q4_0(x)
    y = Q.dequantize_q4_0(b, x.shape)
    d = np.abs(np.frombuffer(b, np.uint8).reshape(-1, 18)[:, :2].copy().view(np.float16).astype(np.float32))
    err = np.abs(x - y).reshape(-1, 32)
    assert (err <= d * 0.5 + 1e-6 + d * 1e-3).all() or (err.max() <= d.max())


def test_layouts_and_sizes():
    w = np.random.default_rng(2).standard_normal((64, 96)).astype(np.float32)
    assert len(pack_q4_0_nblocked(w)) == q4_0_nbytes(64, 96)
    assert len(pack_q4_0_kgrouped(w)) == q4_0_nbytes(64, 96)
    np.testing.assert_array_equal(Q.dequantize_q4_0(pack_q4_0_kgrouped(w), (96, 64)),
                                  Q.dequantize_q4_0(quantize_q4_0(w.T.copy()), (96, 64)))
