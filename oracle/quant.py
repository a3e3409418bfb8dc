"""q4_0 and q8_0 oracle (test infrastructure only).

`quantize_q4_0_scalar` is a per-block scalar transcription of llama.cpp's
`quantize_row_q4_0_ref` as the reference documents it
(`hexlib/exec/quant.py:12-47`): d = (signed max-magnitude element) / -8,
stored as fp16 and used at fp16 precision; q = min(15, trunc(x / d + 8.5));
low nibble of byte j = element j, high nibble = element j + 16. It is slow by
design and used on small inputs to pin the product's vectorised quantizer.

`dequantize_q4_0` is the inverse, v = (q - 8) * d in float32
(`hexlib/exec/quant.py:114-135`). `dequantize_q4_0_fp16` additionally rounds
each dequantized value to fp16, which is the weight the reference kernel
multiplies with (`kernels/matmul_epilogue_fp16/baseline.c:34-47`).

`quantize_q8_0_scalar` is a per-block scalar transcription of llama.cpp's
`quantize_row_q8_0_ref` as the reference documents it (`hexlib/exec/quant.py:138-171`):
amax = max |x|; d = amax / 127 stored as fp16 and used at fp16 precision;
id = 1 / d (0 when d is 0); q = roundf(x * id), half away from zero, saturated
to int8; byte j = element j. `dequantize_q8_0` is v = q * d in float32
(`hexlib/exec/quant.py:210-220`); `dequantize_q8_0_fp16` rounds each value to
fp16, the weight the GPU kernel multiplies with (the q4_0 kernel's convention,
`kernels/matmul_epilogue_fp16/baseline.c:34-47`; the reference has no q8_0
kernel).

Pinned by: the reference's q4_0 and q8_0 tests' known answers restated in
`tests/test_quant.py` (nibble order, signed / positive scale, truncation /
half-away rounding, int8 element order and saturation, all-zero block) and
round-trip error bounds.
"""
from __future__ import annotations

import math
import struct

import numpy as np

QK = 32
BLOCK_BYTES = 18


def _f16(x: float) -> float:
    return float(np.float32(np.float16(np.float32(x))))


def quantize_q4_0_scalar(x: np.ndarray) -> bytes:
    a = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    if a.size % QK:
        raise ValueError("q4_0 needs a multiple of 32 elements along the blocked axis")
    out = bytearray()
    for b in range(a.size // QK):
        blk = [float(v) for v in a[b * QK:(b + 1) * QK]]
        amax, mx = 0.0, 0.0
        for v in blk:
            if abs(v) > amax:
                amax, mx = abs(v), v
        d = float(np.float32(np.float32(mx) / np.float32(-8.0)))
        d16 = _f16(d)
        inv = float(np.float32(1.0) / np.float32(d16)) if d16 != 0.0 else 0.0
        q = []
        for v in blk:
            t = float(np.float32(np.float32(v) * np.float32(inv)) + np.float32(8.5))
            q.append(min(15, max(0, int(math.trunc(t)))))
        out += np.float16(d16).tobytes()
        out += bytes((q[j] & 0xF) | ((q[j + 16] & 0xF) << 4) for j in range(16))
    return bytes(out)


def dequantize_q4_0(data: bytes, shape: tuple[int, ...]) -> np.ndarray:
    n = int(np.prod(shape))
    if len(data) != n // QK * BLOCK_BYTES:
        raise ValueError(f"{len(data)} bytes is not a q4_0 tensor of shape {shape}")
    raw = np.frombuffer(data, dtype=np.uint8).reshape(-1, BLOCK_BYTES)
    d = raw[:, :2].copy().view(np.float16).astype(np.float32)
    qs = raw[:, 2:]
    q = np.concatenate([qs & 0x0F, qs >> 4], axis=1).astype(np.int32) - 8
    return (q.astype(np.float32) * d).reshape(shape)


def dequantize_q4_0_fp16(data: bytes, shape: tuple[int, ...]) -> np.ndarray:
    return dequantize_q4_0(data, shape).astype(np.float16).astype(np.float32)


def block_scale(data: bytes, block: int) -> float:
    return struct.unpack_from("<e", data, block * BLOCK_BYTES)[0]


Q8_BLOCK_BYTES = 34


def quantize_q8_0_scalar(x: np.ndarray) -> bytes:
    a = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    if a.size % QK:
        raise ValueError("q8_0 needs a multiple of 32 elements along the blocked axis")
    out = bytearray()
    for b in range(a.size // QK):
        blk = [np.float32(v) for v in a[b * QK:(b + 1) * QK]]
        amax = np.float32(0.0)
        for v in blk:
            amax = max(amax, np.float32(abs(v)))
        d16 = _f16(float(np.float32(amax / np.float32(127.0))))
        inv = np.float32(1.0) / np.float32(d16) if d16 != 0.0 else np.float32(0.0)
        q = []
        for v in blk:
            t = float(np.float32(v * inv))
            r = math.floor(abs(t) + 0.5)          # roundf: half away from zero
            r = r if t >= 0 else -r
            q.append(min(127, max(-128, int(r))))
        out += np.float16(d16).tobytes()
        out += bytes((v + 256) % 256 for v in q)
    return bytes(out)


def dequantize_q8_0(data: bytes, shape: tuple[int, ...]) -> np.ndarray:
    n = int(np.prod(shape))
    if len(data) != n // QK * Q8_BLOCK_BYTES:
        raise ValueError(f"{len(data)} bytes is not a q8_0 tensor of shape {shape}")
    raw = np.frombuffer(data, dtype=np.uint8).reshape(-1, Q8_BLOCK_BYTES)
    d = raw[:, :2].copy().view(np.float16).astype(np.float32)
    q = raw[:, 2:].copy().view(np.int8).astype(np.float32)
    return (q * d).reshape(shape)


def dequantize_q8_0_fp16(data: bytes, shape: tuple[int, ...]) -> np.ndarray:
    return dequantize_q8_0(data, shape).astype(np.float16).astype(np.float32)
