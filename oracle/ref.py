"""ctypes access to the reference's compiled scalar baselines (test
infrastructure only).

`oracle/_ref/libhexlib_ref.so` is built by `oracle/Makefile` from
`/root/reference/kernels/*/baseline.c` exactly as written (no copy of the
sources lives in this repository). Each wrapper allocates the output, calls
`<kernel>_baseline` with host pointers, and returns numpy arrays; fp16 buffers
cross as uint16 bit patterns, which is what `__fp16` storage is.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_ref", "libhexlib_ref.so")

_lib = None


def available() -> bool:
    return os.path.isfile(LIB_PATH)


def lib():
    global _lib
    if _lib is None:
        if not available():
            raise FileNotFoundError(f"{LIB_PATH} is not built (make -C oracle)")
        _lib = ctypes.CDLL(LIB_PATH)
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _h(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float16)


def _f(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def add_fp16(a, b):
    a, b = _h(a), _h(b)
    y = np.empty_like(a)
    lib().add_fp16_baseline(_p(a), _p(b), _p(y), ctypes.c_int(a.size))
    return y


def scale_fp16(x, factor):
    x = _h(x)
    y = np.empty_like(x)
    lib().scale_fp16_baseline(_p(x), _p(y), ctypes.c_int(x.size), ctypes.c_float(factor))
    return y


def cast_f32_f16(x):
    x = _f(x)
    y = np.empty(x.shape, np.float16)
    lib().cast_f32_f16_baseline(_p(x), _p(y), ctypes.c_int(x.size))
    return y


def softmax_fp16(x):
    x = _h(x)
    y = np.empty_like(x)
    C = x.shape[-1]
    lib().softmax_fp16_baseline(_p(x), _p(y), ctypes.c_int(x.size // C), ctypes.c_int(C))
    return y


def layernorm_fp16(x, w, b, eps):
    x, w, b = _h(x), _f(w), _f(b)
    y = np.empty_like(x)
    C = x.shape[-1]
    lib().layernorm_fp16_baseline(_p(x), _p(w), _p(b), _p(y), ctypes.c_int(x.size // C),
                                  ctypes.c_int(C), ctypes.c_float(eps))
    return y


def rmsnorm_fp16(x, w, eps):
    x, w = _h(x), _h(w)
    y = np.empty_like(x)
    C = x.shape[-1]
    lib().rmsnorm_fp16_baseline(_p(x), _p(w), _p(y), ctypes.c_int(x.size // C),
                                ctypes.c_int(C), ctypes.c_float(eps))
    return y


def rope_2d_fp16(x, cos, sin):
    x, cos, sin = _h(x), _f(cos), _f(sin)
    y = np.empty_like(x)
    T, H, D = x.shape
    lib().rope_2d_fp16_baseline(_p(x), _p(cos), _p(sin), _p(y), ctypes.c_int(T),
                                ctypes.c_int(H), ctypes.c_int(D))
    return y


def transpose_th_fp16(x):
    x = _h(x)
    T, H, D = x.shape
    y = np.empty((H, T, D), np.float16)
    lib().transpose_th_fp16_baseline(_p(x), _p(y), ctypes.c_int(T), ctypes.c_int(H), ctypes.c_int(D))
    return y


def transpose_hd_fp16(x):
    x = _h(x)
    B, T, D = x.shape
    y = np.empty((B, D, T), np.float16)
    lib().transpose_hd_fp16_baseline(_p(x), _p(y), ctypes.c_int(B), ctypes.c_int(T), ctypes.c_int(D))
    return y


def patchify_fp32(img, patch, merge, grid_h, grid_w):
    img = _f(img)
    C, T, H, W = img.shape
    out = np.empty((grid_h * grid_w, C * T * patch * patch), np.float32)
    lib().patchify_fp32_baseline(_p(img), _p(out), *[ctypes.c_int(v) for v in
                                 (C, T, H, W, patch, merge, grid_h, grid_w)])
    return out


def matmul_fp16(A, B):
    A, B = _h(A), _h(B)
    Bn, M, K = A.shape
    N = B.shape[-1]
    C = np.empty((Bn, M, N), np.float16)
    lib().matmul_fp16_baseline(_p(A), _p(B), _p(C), *[ctypes.c_int(v) for v in (Bn, M, K, N)])
    return C


def matmul_epilogue_fp16(a, w_q4: bytes, bias, K, N, act):
    a, bias = _h(a), _f(bias)
    M = a.shape[0]
    w = np.frombuffer(w_q4, dtype=np.uint8).copy()
    out = np.empty((M, N), np.float16)
    lib().matmul_epilogue_fp16_baseline(_p(a), _p(w), _p(bias), _p(out),
                                        *[ctypes.c_int(v) for v in (M, K, N, act)])
    return out
