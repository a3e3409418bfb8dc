"""ctypes binding of libhexlib_gpu.so -- the only way Python reaches the GPU path.

Loading fails loudly (ImportError naming the missing file) when the library
has not been built; there is no fallback implementation of any kernel.
"""
from __future__ import annotations

import ctypes
import os
import re

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libhexlib_gpu.so")
HEADER = os.path.join(os.path.dirname(PKG), "include", "hexlib_gpu.h")

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64

# name -> (restype, argtypes)
SIGNATURES = {
    "add_fp16": (None, [_P, _P, _P, _I]),
    "scale_fp16": (None, [_P, _P, _I, _F]),
    "cast_f32_f16": (None, [_P, _P, _I]),
    "softmax_fp16": (None, [_P, _P, _I, _I]),
    "layernorm_fp16": (None, [_P, _P, _P, _P, _I, _I, _F]),
    "rmsnorm_fp16": (None, [_P, _P, _P, _I, _I, _F]),
    "rope_2d_fp16": (None, [_P, _P, _P, _P, _I, _I, _I]),
    "transpose_th_fp16": (None, [_P, _P, _I, _I, _I]),
    "transpose_hd_fp16": (None, [_P, _P, _I, _I, _I]),
    "transpose_bth_fp16": (None, [_P, _P, _I, _I, _I, _I]),
    "patchify_fp32": (None, [_P, _P] + [_I] * 8),
    "patchify_fp32_batched": (None, [_P, _P] + [_I] * 9),
    "matmul_fp16": (None, [_P, _P, _P, _I, _I, _I, _I]),
    "matmul_epilogue_fp16": (None, [_P, _P, _P, _P, _I, _I, _I, _I]),
    "matmul_epilogue_f16w_fp16": (None, [_P, _P, _P, _P, _I, _I, _I, _I]),
    "matmul_epilogue_q4k_fp16": (None, [_P, _P, _P, _P, _I, _I, _I, _I]),
    "matmul_epilogue_q8k_fp16": (None, [_P, _P, _P, _P, _I, _I, _I, _I]),
    "matmul_epilogue_f16wt_fp16": (None, [_P, _P, _P, _P, _I, _I, _I, _I]),
    "matmul_epilogue_f16wt_res_fp16": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I]),
    "matmul_epilogue_res_fp16": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I]),
    "matmul_epilogue_q8k_res_fp16": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I]),
    "matmul_epilogue_q4k_res_fp16": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I]),
    "matmul_epilogue_q8k_rope_fp16": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I]),
    "matmul_epilogue_f16wt_rope_fp16": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I]),
    "attention_qkv_fp16": (None, [_P, _P, _I, _I, _I, _I, _F]),
    "layernorm_matmul_epilogue_f16wt_fp16": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F]),
    "lnfold_matmul_epilogue_f16wt_fp16": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _F]),
    "lnfold_matmul_epilogue_f16wt_rope_fp16": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F]),
    "attention_fp16": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _F]),
    "attention_qk_v_fp16": (None, [_P, _P, _P, _I, _I, _I, _I, _F]),
    "rope_2d_qk_fp16": (None, [_P, _P, _P, _P, _I, _I, _I]),
    "hexlib_gpu_gemm_override": (_I, [_I, _I, _I, _I]),
    "hexlib_gpu_attention_override": (_I, [_I]),
    "matmul_epilogue_f16wt_noalloc_fp16": (_I, [_P, _P, _P, _P, _I, _I, _I, _I]),
    "hexlib_gpu_set_stream": (None, [_P]),
    "hexlib_gpu_get_stream": (_P, []),
    "hexlib_gpu_take_error": (_I, []),
    "hexlib_gpu_error_string": (ctypes.c_char_p, [_I]),
    "hexlib_gpu_status_name": (ctypes.c_char_p, [_I]),
    "hexlib_gpu_struct_sizes": (_U32, [ctypes.POINTER(_U32), _U32]),
    "hexlib_gpu_open": (_I, [ctypes.POINTER(_P)]),
    "hexlib_gpu_close": (_I, [_P]),
    "hexlib_gpu_start": (_I, [_P, _U32, _I, _U64]),
    "hexlib_gpu_stop": (_I, [_P]),
    "hexlib_gpu_mmap": (_I, [_P, _U32, _P, _U64]),
    "hexlib_gpu_munmap": (_I, [_P, _U32]),
    "hexlib_gpu_hwinfo": (_I, [_P, ctypes.POINTER(_U32), ctypes.POINTER(_U32),
                               ctypes.POINTER(_U32), ctypes.POINTER(_U64)]),
    "hexlib_gpu_invoke": (_I, [_P, ctypes.c_char_p, _U32, _P, _U32, ctypes.POINTER(_U32), _U32]),
    "hexlib_gpu_session_stream": (_P, [_P]),
    "hexlib_gpu_plan_inspect": (_I, [ctypes.c_char_p, _P]),
    "hexlib_gpu_plan_load": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(_P)]),
    "hexlib_gpu_plan_info_of": (_I, [_P, _P]),
    "hexlib_gpu_plan_io": (_I, [_P, _U32, _P]),
    "hexlib_gpu_plan_write": (_I, [_P, _U32, _P, _U64]),
    "hexlib_gpu_plan_read": (_I, [_P, _U32, _P, _U64]),
    "hexlib_gpu_plan_run": (_I, [_P, _U32, _P, _U32, ctypes.POINTER(_U32)]),
    "hexlib_gpu_plan_free": (_I, [_P]),
}


class PlanInfo(ctypes.Structure):
    """hexlib_plan_info (include/hexlib_gpu.h)."""
    _fields_ = [("version", _U32), ("fd", _U32), ("n_io", _U32), ("n_ops", _U32),
                ("arena_bytes", _U64), ("const_bytes", _U64), ("blob_bytes", _U64), ("data_bytes", _U64)]


class PlanIO(ctypes.Structure):
    """hexlib_plan_io (include/hexlib_gpu.h)."""
    _fields_ = [("name", ctypes.c_char * 48), ("role", _U32), ("dtype", _U32), ("offset", _U64),
                ("nbytes", _U64), ("ne", _U32 * 4), ("data_offset", _U64)]

INVOKE_DRYRUN = 0x1
INVOKE_TIMED = 0x2
INVOKE_GRAPH = 0x4
INVOKE_NOSYNC = 0x8

_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.isfile(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run `python -m hexlib_amd.build` (or "
            "__graft_entry__.build()). hexlib_amd has no CPU fallback.")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def header_functions(path: str = HEADER) -> list[str]:
    """Every function name declared in include/hexlib_gpu.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^(?:const\s+)?(?:void|int|uint32_t|char)\s*\**\s*(\w+)\s*\(",
                       text, flags=re.M)
    return sorted(set(names))


def header_objects(path: str = HEADER) -> list[str]:
    text = open(path).read()
    return re.findall(r"^extern\s+const\s+[\w\s]+?\b(\w+)(?:\[\])?;", text, flags=re.M)


def check_error(lib=None) -> None:
    lib = lib or load()
    err = lib.hexlib_gpu_take_error()
    if err:
        raise RuntimeError(f"HIP launch failed: {lib.hexlib_gpu_error_string(err).decode()}")
