"""q4_0 and q8_0 weight packing for staging (host side, vectorised).

Same block format and arithmetic as the reference quantizer
(`hexlib/exec/quant.py:62-111`, llama.cpp `block_q4_0`): 32 values per block,
blocks along the LAST axis; d = (signed element of largest magnitude) / -8,
stored fp16 and used at fp16 precision; q = clip(trunc(x / d + 8.5), 0, 15);
byte j holds element j in its low nibble and element j + 16 in its high nibble.

Two weight layouts are produced from a logical `[K, N]` weight:
* `pack_q4_0_nblocked` -- the reference kernel ABI: blocks along N, row k of
  the weight is `N/32` contiguous blocks (`kernels/matmul_epilogue_fp16/kernel_api.h:68-109`).
* `pack_q4_0_kgrouped` -- groups of 32 along K: the transposed weight `[N, K]`
  quantized along its last axis, i.e. llama.cpp's native `W^T[N][K/32]`.

q8_0 (`hexlib/exec/quant.py:138-220`, llama.cpp `block_q8_0`): 32 values per
block, 34 bytes: an fp16 scale d = max|x| / 127 (positive), then 32 int8
q = roundf(x / d) (half away from zero), saturated to [-128, 127], in element
order. `pack_q8_0_kgrouped` stores the transposed weight `W^T[N][K/32]`, the
GPU kernel's layout.
"""
from __future__ import annotations

import numpy as np

QK = 32
BLOCK_BYTES = 18


def quantize_q4_0(x: np.ndarray) -> bytes:
    a = np.ascontiguousarray(x, dtype=np.float32)
    if a.ndim == 0 or a.shape[-1] % QK:
        raise ValueError(f"q4_0 needs a last axis that is a multiple of {QK}; got {a.shape}")
    blocks = a.reshape(-1, QK)
    n = blocks.shape[0]
    pick = np.abs(blocks).argmax(axis=1)
    signed_max = blocks[np.arange(n), pick]
    d16 = (signed_max / np.float32(-8.0)).astype(np.float32).astype(np.float16)
    d = d16.astype(np.float32)
    inv = np.zeros_like(d)
    np.divide(np.float32(1.0), d, out=inv, where=d != 0)
    q = np.trunc(blocks * inv[:, None] + np.float32(8.5)).astype(np.int32)
    q = np.clip(q, 0, 15).astype(np.uint8)
    out = np.empty((n, BLOCK_BYTES), np.uint8)
    out[:, :2] = d16.view(np.uint8).reshape(n, 2)
    out[:, 2:] = q[:, :16] | (q[:, 16:] << 4)
    return out.tobytes()


def pack_q4_0_nblocked(w_kn: np.ndarray) -> bytes:
    return quantize_q4_0(w_kn)


def pack_q4_0_kgrouped(w_kn: np.ndarray) -> bytes:
    return quantize_q4_0(np.ascontiguousarray(np.asarray(w_kn, dtype=np.float32).T))


def q4_0_nbytes(k: int, n: int) -> int:
    return k * n // QK * BLOCK_BYTES


Q8_BLOCK_BYTES = 34


def quantize_q8_0(x: np.ndarray) -> bytes:
    a = np.ascontiguousarray(x, dtype=np.float32)
    if a.ndim == 0 or a.shape[-1] % QK:
        raise ValueError(f"q8_0 needs a last axis that is a multiple of {QK}; got {a.shape}")
    blocks = a.reshape(-1, QK)
    n = blocks.shape[0]
    d16 = (np.abs(blocks).max(axis=1) / np.float32(127.0)).astype(np.float32).astype(np.float16)
    d = d16.astype(np.float32)
    inv = np.zeros_like(d)
    np.divide(np.float32(1.0), d, out=inv, where=d != 0)
    scaled = blocks * inv[:, None]
    q = np.clip(np.sign(scaled) * np.floor(np.abs(scaled) + np.float32(0.5)), -128, 127).astype(np.int8)
    out = np.empty((n, Q8_BLOCK_BYTES), np.uint8)
    out[:, :2] = d16.view(np.uint8).reshape(n, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.tobytes()


def pack_q8_0_kgrouped(w_kn: np.ndarray) -> bytes:
    return quantize_q8_0(np.ascontiguousarray(np.asarray(w_kn, dtype=np.float32).T))


def q8_0_nbytes(k: int, n: int) -> int:
    return k * n // QK * Q8_BLOCK_BYTES
