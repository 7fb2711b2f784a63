"""ctypes binding of libmoat_int4.so (the gfx950 kernels).

Follows the reference's FFI pattern (``antigravity-engine/src/native_bridge.py:95-160``:
explicit argtypes/restypes; a nonzero status becomes a Python exception),
with device pointers from torch tensors and torch's current HIP stream.

There is no fallback: a missing library or a missing GPU raises.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmoat_int4.so")

MOAT_OK = 0
MOAT_ERR_INVALID = -2
MOAT_ERR_HIP = -3
MOAT_ERR_WORKSPACE = -4
MOAT_ERR_TOO_LARGE = -5
WS_HANDOFF_TIMEOUT = 1

DTYPE_F32, DTYPE_F16, DTYPE_I8, DTYPE_F64, DTYPE_I64 = 0, 1, 2, 3, 4
SCALE_F32, SCALE_F16 = 0, 1
GEMM_AUTO, GEMM_DOT2, GEMM_MFMA = 0, 1, 2
FINISH_AUTO, FINISH_DEVICE_ATOMICS, FINISH_FENCES, FINISH_SECOND_KERNEL = 0, 1, 2, 3
FRONT_AUTO, FRONT_LDS, FRONT_DIRECT, FRONT_LDS_DMA, FRONT_RECORDS = 0, 1, 2, 3, 4


class GemmOptions(ctypes.Structure):
    """``moat_int4_gemm_options``: zero fields mean automatic."""
    _fields_ = [("algo", ctypes.c_int32), ("splits", ctypes.c_int32),
                ("batch", ctypes.c_int32), ("finish", ctypes.c_int32), ("front", ctypes.c_int32),
                ("group", ctypes.c_int32),
                ("waves", ctypes.c_int32)]

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64

# name -> (restype, argtypes); every symbol declared in include/moat_int4.h
SIGNATURES = {
    "moat_int4_version": (_I32, []),
    "moat_int4_status_string": (ctypes.c_char_p, [_I32]),
    "moat_int4_dequant": (_I32, [_P, _I64, _P, _P]),
    "moat_int4_gemm_workspace_size": (_I64, [_I32, _I32, _I32]),
    "moat_int4_gemm": (_I32, [_P, _P, _P, _I32, _I32, _I32, _P, _I64, _P]),
    "moat_int4_gemm_noalloc": (_I32, [_P, _P, _P, _I32, _I32, _I32, _P]),
    "moat_int4_gemm_ex_workspace_size": (_I64, [_I32, _I32, _I32, ctypes.POINTER(GemmOptions)]),
    "moat_int4_gemm_ex": (_I32, [_P, _P, _P, _I32, _I32, _I32, ctypes.POINTER(GemmOptions), _P, _I64, _P]),
    "moat_int4_records_to_tiles": (_I32, [_P, _I32, _I32, _P, _P]),
    "moat_int4_gemm_tiles": (_I32, [_P, _P, _P, _I32, _I32, _I32, ctypes.POINTER(GemmOptions), _P, _I64, _P]),
    "moat_int4_workspace_clear": (_I32, [_P, _I64, _P]),
    "moat_dense_gemm_workspace_size": (_I64, [_I32, _I32, _I32, _I32]),
    "moat_dense_gemm": (_I32, [_P, _P, _P, _I32, _I32, _I32, _I32, _P, _I64, _P]),
    "moat_int4_records_to_strips": (_I32, [_P, _I32, _I32, _P, _P]),
    "moat_int4_strips_to_records": (_I32, [_P, _I32, _I32, _P, _P]),
    "moat_int4_i8_div_to_f16": (_I32, [_P, _I64, ctypes.c_float, _P, _P]),
    "moat_int4_swiglu_f32": (_I32, [_P, _I32, _I32, _I64, _P, _P]),
    "moat_int4_gemm_strips_swiglu": (_I32, [_P, _P, _P, _I32, _I32, _I32, _P, _P]),
    "moat_int4_interleave_strips": (_I32, [_P, _P, _I32, _I32, _P, _P]),
    "moat_int4_gemm_strips_workspace_size": (_I64, [_I32, _I32, _I32, ctypes.POINTER(GemmOptions)]),
    "moat_int4_gemm_strips": (_I32, [_P, _P, _P, _I32, _I32, _I32, ctypes.POINTER(GemmOptions), _P, _I64, _P]),
    "moat_int4_workspace_status": (_I32, [_P, _I64, ctypes.POINTER(_I32), _P]),
    "moat_int4_stream_read": (_I32, [_P, _I64, _I32, _P, _P]),
    "moat_int4_gemm_multi_workspace_size": (_I64, [_I32, _I32, _I32, _I32]),
    "moat_int4_gemm_multi": (_I32, [_P, _P, _P, _I32, _I32, _I32, _I32, _P, _I64, _P]),
    "moat_int4_gemm_swiglu_workspace_size": (_I64, [_I32, _I32, _I32]),
    "moat_int4_gemm_swiglu": (_I32, [_P, _P, _P, _P, _I32, _I32, _I32, _P, _I64, _P]),
    "moat_int4_quantize": (_I32, [_P, _I32, _I64, _I32, _I32, _P, _P, _P]),
    "moat_int4_pack_superblocks": (_I32, [_P, _P, _I64, _P, _P]),
    "moat_int4_quantize_pack": (_I32, [_P, _I32, _I64, _I32, _P, _P]),
    "moat_int4_pack_nibbles": (_I32, [_P, _I64, _P, _P]),
    "moat_int4_unpack_nibbles": (_I32, [_P, _I64, _P, _P]),
    "moat_int4_group_dequant": (_I32, [_P, _I32, _P, _I32, _I64, _I32, _I32, _P, _P, _P]),
    "moat_int4_lut_gather": (_I32, [_P, _I64, _I32, _P, _I64, _I32, _P, _P]),
    "moat_int4_any_negative": (_I32, [_P, _I64, _P, _P]),
    "moat_int4_to_f16": (_I32, [_P, _I32, _I64, _P, _P]),
    "moat_sample_workspace_size": (_I64, [_I32, _I32]),
    "moat_lut_softmax_workspace_size": (_I64, [_I32, _I32]),
    "moat_lut_softmax": (_I32, [_P, _I32, _I32, _I32, _P, _I32, ctypes.c_float, _P, _P, _I64, _P]),
    "moat_sample_tokens": (_I32, [_P, _I32, _I32, _I32, ctypes.c_double, _I32, ctypes.c_uint64, _P, _I32,
                                  ctypes.c_float, _P, _P, _P, _I64, _P]),
    "moat_lut_lookup": (_I32, [_P, _I64, _P, _I32, ctypes.c_float, _P, _P]),
}

_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the library once.  torch is imported first so that the library
    binds to the same HIP runtime as torch's tensors and streams."""
    global _lib
    if _lib is not None:
        return _lib
    import torch  # noqa: F401  (loads torch's libamdhip64 before ours)

    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with `python -m moat_amd.build_lib` "
            "(moat_amd has no CPU fallback)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    if status == MOAT_OK:
        return
    msg = load().moat_int4_status_string(status).decode()
    if status in (MOAT_ERR_INVALID, MOAT_ERR_WORKSPACE, MOAT_ERR_TOO_LARGE):
        raise ValueError(f"{what}: {msg} (status {status})")
    raise RuntimeError(f"{what}: {msg} (status {status})")
