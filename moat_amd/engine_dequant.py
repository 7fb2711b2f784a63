"""Drop-in for the reference's ``antigravity-engine/src/dequant.py`` (surface B), on MI355X.

Same names, arguments, defaults, return types (including the list of
per-superblock dicts) and exceptions as ``antigravity-engine/src/dequant.py:22-252``;
the arithmetic runs in the gfx950 kernels of libmoat_int4.so.  numpy in ->
numpy out; torch GPU tensors in -> GPU tensors out.
"""

from __future__ import annotations

from typing import Tuple

import numpy as np
import torch

from . import _device as D
from . import _lib
from .dequant import _float_dtype_code

__all__ = [
    "quantize_weights_int4",
    "quantize_fp16_to_int4",
    "repack_to_superblocks",
    "unpack_superblock",
    "build_dequant_lut",
    "lut_dequantize",
    "arithmetic_dequantize",
]


def quantize_weights_int4(weights_fp16, group_size: int = 32) -> Tuple[np.ndarray, np.ndarray]:
    """1-D INT4 group quantization with the scale rounded to fp16 before the
    division (``antigravity-engine/src/dequant.py:22-60``).  ValueError for a
    non-1-D input or a length that is not a multiple of ``group_size``."""
    if len(weights_fp16.shape) != 1:
        raise ValueError(f"Expected 1D array, got shape {tuple(weights_fp16.shape)}")
    n = int(weights_fp16.shape[0])
    if n % group_size != 0:
        raise ValueError(f"Weight length {n} is not divisible by group_size={group_size}")
    want_t = D.is_tensor(weights_fp16)
    w, code = _float_dtype_code(D.to_device(weights_fp16))
    q = torch.empty(n, dtype=torch.int8, device=w.device)
    s = torch.empty(n // group_size, dtype=torch.float16, device=w.device)
    _lib.check(_lib.load().moat_int4_quantize(D.ptr(w), code, n, group_size, _lib.SCALE_F16,
                                              D.ptr(q), D.ptr(s), D.stream()), "quantize_weights_int4")
    return D.out_like(q, want_t), D.out_like(s, want_t)


quantize_fp16_to_int4 = quantize_weights_int4


def _codes_int8(q) -> torch.Tensor:
    """q as int8 codes whose (value + 8) & 15 equals the reference's
    ``(q.astype(int16) + 8).astype(uint8) & 15`` (wrap-around is mod 16 safe)."""
    t = D.to_device(q)
    if t.is_floating_point():
        t = t.to(torch.int16)
    return t.to(torch.int8).reshape(-1).contiguous()


def repack_to_superblocks(q_weights, scales, group_size: int = 32, groups_per_superblock: int = 8) -> list:
    """Per-superblock records ``{'scales', 'packed_nibbles', 'raw_int4'}``
    (``antigravity-engine/src/dequant.py:69-132``): nibble pairs with the even
    element in the low nibble, values stored as q+8.  ValueError unless the
    length is a multiple of ``group_size * groups_per_superblock``."""
    per_sb = group_size * groups_per_superblock
    n = int(q_weights.shape[0]) if len(q_weights.shape) else 0
    if n % per_sb != 0:
        raise ValueError(f"Weight length {n} not divisible by super-block size {per_sb}")
    want_t = D.is_tensor(q_weights)
    n_sb = n // per_sb
    codes = _codes_int8(q_weights)
    packed = torch.empty(n // 2, dtype=torch.uint8, device=codes.device)
    _lib.check(_lib.load().moat_int4_pack_nibbles(D.ptr(codes), n, D.ptr(packed), D.stream()),
               "repack_to_superblocks")
    packed = packed.reshape(n_sb, per_sb // 2)
    if not want_t:
        packed = D.to_host(packed)
    out = []
    for i in range(n_sb):
        out.append({
            "scales": scales[i * groups_per_superblock:(i + 1) * groups_per_superblock].copy()
            if not D.is_tensor(scales) else scales[i * groups_per_superblock:(i + 1) * groups_per_superblock].clone(),
            "packed_nibbles": packed[i].copy() if not want_t else packed[i].clone(),
            "raw_int4": q_weights[i * per_sb:(i + 1) * per_sb].copy() if not want_t
            else q_weights[i * per_sb:(i + 1) * per_sb].clone(),
        })
    return out


def unpack_superblock(superblock: dict, group_size: int = 32):
    """Nibble pairs back to int8 values in [-8, 7], even element from the low
    nibble (``antigravity-engine/src/dequant.py:135-156``)."""
    packed = superblock["packed_nibbles"]
    want_t = D.is_tensor(packed)
    t = D.to_device(packed)
    if t.dtype != torch.uint8:
        t = t.to(torch.int64).bitwise_and(0xFF).to(torch.uint8) if not t.is_floating_point() else t.to(torch.uint8)
    t = t.reshape(-1).contiguous()
    out = torch.empty(2 * t.numel(), dtype=torch.int8, device=t.device)
    _lib.check(_lib.load().moat_int4_unpack_nibbles(D.ptr(t), t.numel(), D.ptr(out), D.stream()),
               "unpack_superblock")
    return D.out_like(out, want_t)


def _scales_device(scales, count: int) -> Tuple[torch.Tensor, int]:
    s = D.to_device(scales).reshape(-1)[:count]
    if s.dtype == torch.float16:
        return s.contiguous(), _lib.DTYPE_F16
    if s.dtype == torch.float32:
        return s.contiguous(), _lib.DTYPE_F32
    return s.to(torch.float64).contiguous(), _lib.DTYPE_F64


def _q_device(q) -> Tuple[torch.Tensor, int]:
    t = D.to_device(q).reshape(-1)
    if t.dtype == torch.int8:
        return t, _lib.DTYPE_I8
    if t.dtype == torch.bool:
        return t.to(torch.int8), _lib.DTYPE_I8
    if t.is_floating_point():
        return t.to(torch.float32).contiguous(), _lib.DTYPE_F32
    return t.to(torch.int64).contiguous(), _lib.DTYPE_I64


def _group_dequant(q_weights, scales, group_size: int, table_mode: int):
    if len(q_weights.shape) != 1:
        raise ValueError(f"Expected 1D quantized weights, got shape {tuple(q_weights.shape)}")
    want_t = D.is_tensor(q_weights)
    n = int(q_weights.shape[0])
    n_groups = n // group_size
    if len(scales) < n_groups:
        raise IndexError(f"index {len(scales)} is out of bounds for axis 0 with size {len(scales)}")
    dev = D.require_gpu()
    out = torch.zeros(n, dtype=torch.float16, device=dev)
    if n_groups == 0:
        return D.out_like(out, want_t)
    if table_mode:
        t = D.to_device(q_weights).reshape(-1)
        if t.dtype == torch.int8:
            q, qcode = t, _lib.DTYPE_I8
        else:  # the reference indexes with q.astype(int16) + 8
            q, qcode = t.to(torch.int16).to(torch.int64).contiguous(), _lib.DTYPE_I64
    else:
        q, qcode = _q_device(q_weights)
    s, scode = _scales_device(scales, n_groups)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    _lib.check(_lib.load().moat_int4_group_dequant(D.ptr(q), qcode, D.ptr(s), scode, n_groups, group_size,
                                                   table_mode, D.ptr(out), D.ptr(flag), D.stream()),
               "lut_dequantize" if table_mode else "arithmetic_dequantize")
    if table_mode and int(flag.item()):
        raise IndexError("index out of bounds for axis 0 with size 16")
    return D.out_like(out, want_t)


def build_dequant_lut(scale) -> np.ndarray:
    """``LUT[k + 8] = fp16(k * scale)`` for k in [-8, 7], the product in float32
    (``antigravity-engine/src/dequant.py:163-180``)."""
    q = np.arange(-8, 8, dtype=np.int8)
    return _group_dequant(q, np.array([float(scale)], dtype=np.float64), 16, 0)


def lut_dequantize(q_weights, scales, group_size: int = 32):
    """Per-group 16-entry table lookup ``lut_g[q + 8]``
    (``antigravity-engine/src/dequant.py:183-220``); elements past the last
    whole group stay 0."""
    return _group_dequant(q_weights, scales, group_size, 1)


def arithmetic_dequantize(q_weights, scales, group_size: int = 32):
    """``fp16(f32(q) * scale_g)`` per group (``antigravity-engine/src/dequant.py:223-252``);
    elements past the last whole group stay 0."""
    return _group_dequant(q_weights, scales, group_size, 0)
