"""The reference harnesses' adversarial inputs, restated as data.

Each reference `kernels/<k>/harness.c` plants a few crafted values where a
quiet, precision-class mistake (an fp16 running sum, a dropped eps, ...) turns
into an error far outside the kernel's tolerance, while generic data would let
it through. These builders restate those values (the construction each
harness's header describes) on top of seeded generic data, so the GPU tests
and the planted-mistake tests (`tests/nearmiss.py`) run on the same inputs.
Test infrastructure only.
"""
from __future__ import annotations

import numpy as np

from hexlib_amd.quant import BLOCK_BYTES

H = np.float16


def matmul_adversarial(seed: int = 60):
    """`kernels/matmul_fp16/harness.c:39-81,122-127`: shape (Bn, M, K, N) =
    (3, 40, 128, 200), and the element C[1][5][7] made of one dominant product
    (A[1][5][0] = 2, B[1][0][7] = 1) plus 127 followers of exactly one fp16
    ulp at that magnitude (A[1][5][k] = 2^-10, B[1][k][7] = 1): 2.1240234375
    summed in fp32, 2.0 summed in fp16. Returns (A, B, (b, m, n))."""
    r = np.random.default_rng(seed)
    A = r.standard_normal((3, 40, 128)).astype(H)
    B = (r.standard_normal((3, 128, 200)) * 0.1).astype(H)
    A[1, 5, 0] = 2.0
    A[1, 5, 1:] = 2.0 ** -10
    B[1, :, 7] = 1.0
    return A, B, (1, 5, 7)


def q4_block(d: float, codes) -> bytes:
    """One 18-byte q4_0 block with an exact fp16 scale and 32 exact codes
    (element j: nibble j & 15 of byte 2 + (j & 15), low for j < 16)."""
    c = np.asarray(codes, np.uint8)
    out = bytearray(np.float16(d).tobytes())
    out += bytes(int(c[j]) | (int(c[j + 16]) << 4) for j in range(16))
    return bytes(out)


def epilogue_cell1(seed: int = 61):
    """`kernels/matmul_epilogue_fp16/harness.c:27-79,143-180` cell 1 (test 1:
    M = 8, K = 64, N = 128, no activation): a[0, :] = 1; column 0's
    dequantized weight is exactly 1.0 at k = 0 (scale 1, code 9) and exactly
    2^-12 at every other k (scale 2^-12, code 9), so out[0, 0] is
    1 + 63 * 2^-12 = 1.015380859375 -- 1.015625 rounded once, 1.0 with an fp16
    running sum (-1.5%). Every other block holds seeded codes under a seeded
    scale. The weight is q4_0 blocked along N (`kernel_api.h:68-109`): row k
    holds N / 32 blocks. Returns (a, w_bytes, bias, M, K, N, act)."""
    M, K, N = 8, 64, 128
    r = np.random.default_rng(seed)
    a = r.standard_normal((M, K)).astype(H)
    a[0] = 1.0
    blocks = []
    for k in range(K):
        for nb in range(N // 32):
            codes = r.integers(0, 16, 32)
            d = r.uniform(0.005, 0.02)
            if nb == 0:
                codes[0] = 9
                d = 1.0 if k == 0 else 2.0 ** -12
            blocks.append(q4_block(d, codes))
    w = b"".join(blocks)
    assert len(w) == K * N // 32 * BLOCK_BYTES
    bias = np.zeros(N, np.float32)
    return a, w, bias, M, K, N, 0


def epilogue_cell1_f16(seed: int = 62):
    """Cell 1 for the fp16-weight linears (`matmul_epilogue_f16wt_fp16`,
    W^T [N, K]): a[0, :] = 1, column 0's weights 1.0 at k = 0 and 2^-12
    elsewhere, at the encoder's K = 768 (the running sum then stays at 1.0
    where the true value is 1 + 767 * 2^-12 = 1.187255859375). Returns
    (a, w [K, N], bias, act)."""
    M, K, N = 64, 768, 128
    r = np.random.default_rng(seed)
    a = r.standard_normal((M, K)).astype(H)
    w = (r.standard_normal((K, N)) * 0.02).astype(H)
    a[0] = 1.0
    w[:, 0] = 2.0 ** -12
    w[0, 0] = 1.0
    bias = (r.standard_normal(N) * 0.02).astype(np.float32)
    bias[0] = 0.0
    return a, w, bias, 0


def softmax_rows(seed: int = 63):
    """`kernels/softmax_fp16/harness.c:16-84`, R = 6, C = 256: row 0 holds a
    90.0 (exp overflows fp32 without the max subtracted); row 1 is one 20.0
    and 255 followers at 13.5 (each probability about 0.0015: an fp16
    running sum of them loses 8% of the denominator); rows 2-5 seeded."""
    r = np.random.default_rng(seed)
    x = r.standard_normal((6, 256)).astype(np.float32)
    x[0] = 0.1 * ((np.arange(256) % 13) - 6)
    x[0, 0] = 90.0
    x[1] = 13.5
    x[1, 0] = 20.0
    return x.astype(H)


def rmsnorm_rows(seed: int = 64):
    """`kernels/rmsnorm_fp16/harness.c:6-7,27-28`: row 0 is near-degenerate
    (1e-4 * ((c % 5) - 2)), so eps dominates its mean square; the other rows
    seeded. R = 4, C = 768, eps 1e-6, gain 0.5 + 0.01 (c % 17)."""
    r = np.random.default_rng(seed)
    C = 768
    x = r.standard_normal((4, C)).astype(np.float32)
    x[0] = 1e-4 * ((np.arange(C) % 5) - 2)
    w = (0.5 + 0.01 * (np.arange(C) % 17)).astype(H)
    return x.astype(H), w, 1e-6


def rope_near_cancellation(seed: int = 65):
    """`kernels/rope_2d_fp16/harness.c:20-60`: T = 6, H = 3, D = 64 (all
    different), tables whose halves differ, and on the last token a
    near-cancellation at pair i = 0 for every head: x[i] = x[i + 32] = 1000,
    cos[i] = 0.5, sin[i] = 0.5001, cos[i + 32] = 0.5, sin[i + 32] = -0.4999,
    so y[i] = 500 - 500.1 = -0.1 and y[i + 32] = 0.1, lost entirely when the
    products are rounded to fp16 before they are combined."""
    r = np.random.default_rng(seed)
    T, Hh, D = 6, 3, 64
    x = r.standard_normal((T, Hh, D)).astype(np.float32)
    ang = r.uniform(-3, 3, (T, D))
    cos, sin = np.cos(ang).astype(np.float32), np.sin(1.3 * ang).astype(np.float32)
    x[T - 1, :, 0] = 1000.0
    x[T - 1, :, D // 2] = 1000.0
    cos[T - 1, 0], sin[T - 1, 0] = 0.5, 0.5001
    cos[T - 1, D // 2], sin[T - 1, D // 2] = 0.5, -0.4999
    return x.astype(H), cos, sin
