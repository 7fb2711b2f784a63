"""Drop-in for the reference's ``src/dequant.py`` (surface A), on MI355X.

Same names, arguments, defaults, return types and exceptions as
``src/dequant.py:9-187``; the arithmetic runs in the gfx950 kernels of
libmoat_int4.so.  Every function accepts numpy arrays (returns numpy, like
the reference) or torch tensors on the GPU (returns GPU tensors, enqueued on
torch's current stream).

Additions the reference lacks:

* :func:`pack_superblocks_bytes` -- the writer of the 144-byte records that
  :func:`unpack_superblock_weights` reads;
* :func:`quantize_to_superblocks` -- quantize + write in one kernel;
* :func:`batched_int4_matmul` -- ``Y = X @ deq(W)`` for N parallel traces,
  the call shape of ``antigravity-engine/src/batch_generator.py:282-291``
  with superblock weights (the reference's fused kernel for it,
  ``antigravity-engine/src/shaders/batched_gemm.metal:116-169``, has no caller).
"""

from __future__ import annotations

import ctypes
from typing import Dict, Tuple, Union

import numpy as np
import torch

from . import _device as D
from . import _lib

GROUP_SIZE = 32
SUPERBLOCK_ELEMS = 256
SUPERBLOCK_BYTES = 144
MAX_BATCH_PER_CALL = 32

__all__ = [
    "ensure_aligned_array",
    "quantize_fp16_to_int4",
    "repack_weights_to_superblock",
    "lut_dequantize_fp16",
    "unpack_superblock_weights",
    "calculate_memory_footprint",
    "pack_superblocks_bytes",
    "quantize_to_superblocks",
    "batched_int4_matmul",
]


def _float_dtype_code(t: torch.Tensor) -> Tuple[torch.Tensor, int]:
    if t.dtype == torch.float32:
        return t, _lib.DTYPE_F32
    if t.dtype == torch.float16:
        return t, _lib.DTYPE_F16
    if t.dtype == torch.float64:
        return t, _lib.DTYPE_F64
    return t.to(torch.float32), _lib.DTYPE_F32  # integer/bool/bfloat16 values: exact or RNE like numpy


# --------------------------------------------------------------------------
# host-memory helper (src/dequant.py:9-23)
# --------------------------------------------------------------------------

def ensure_aligned_array(arr: np.ndarray, alignment: int = 128) -> np.ndarray:
    """C-contiguous view or copy of ``arr`` whose data pointer is a multiple of
    ``alignment`` bytes (``src/dequant.py:9-23``).  Host memory layout only."""
    contig = np.ascontiguousarray(arr)
    if contig.ctypes.data % alignment == 0:
        return contig
    raw = np.empty(contig.nbytes + alignment, dtype=np.uint8)
    start = -raw.ctypes.data % alignment
    view = raw[start:start + contig.nbytes].view(contig.dtype).reshape(contig.shape)
    view[...] = contig
    return view


# --------------------------------------------------------------------------
# quantize (src/dequant.py:26-55)
# --------------------------------------------------------------------------

def quantize_fp16_to_int4(weights_fp16, group_size: int = 32):
    """Symmetric INT4 quantization in groups of ``group_size`` along the C-order
    flat index (``src/dequant.py:26-55``): scale ``alpha/7`` in float32 (1 for an
    all-zero group), ``q = clip(round_half_even(w/scale), -8, 7)`` as int8 in the
    input's shape, scales returned as fp16.  AssertionError when the size is not
    a multiple of ``group_size``."""
    want_t = D.is_tensor(weights_fp16)
    shape = tuple(weights_fp16.shape)
    n = int(np.prod(shape, dtype=np.int64))
    assert n % group_size == 0, (
        f"Weight array length ({n}) must be a multiple of group_size ({group_size})."
    )
    w, code = _float_dtype_code(D.to_device(weights_fp16))
    q = torch.empty(n, dtype=torch.int8, device=w.device)
    s = torch.empty(n // group_size, dtype=torch.float16, device=w.device)
    _lib.check(_lib.load().moat_int4_quantize(D.ptr(w), code, n, group_size, _lib.SCALE_F32,
                                              D.ptr(q), D.ptr(s), D.stream()), "quantize_fp16_to_int4")
    return D.out_like(q.view(shape), want_t), D.out_like(s, want_t)


# --------------------------------------------------------------------------
# one-byte-per-weight superblock view (src/dequant.py:58-76)
# --------------------------------------------------------------------------

def repack_weights_to_superblock(weights_int4, group_size: int = 32):
    """Reshape int weights to ``(S, 8, group_size)`` int8, 128-byte aligned
    (``src/dequant.py:58-76``).  AssertionError unless the length is a multiple
    of 256.  A layout operation: no arithmetic is involved."""
    if D.is_tensor(weights_int4):
        flat = weights_int4.reshape(-1)
        assert flat.numel() % 256 == 0, "Weight array length must be a multiple of 256."
        out = flat.reshape(flat.numel() // 256, 8, group_size).to(torch.int8).contiguous()
        return D.aligned(out, 128)
    flat = np.asarray(weights_int4).flatten()
    assert len(flat) % 256 == 0, "Weight array length must be a multiple of 256."
    rep = flat.reshape(len(flat) // 256, 8, group_size).astype(np.int8)
    return ensure_aligned_array(rep, alignment=128)


# --------------------------------------------------------------------------
# table gather (src/dequant.py:79-112)
# --------------------------------------------------------------------------

def _lut_to_f16(lut) -> torch.Tensor:
    t = D.to_device(lut)
    if t.dtype == torch.float16:
        return t
    if t.dtype not in (torch.float32, torch.float64):
        t = t.to(torch.float64)  # integer tables: exact
    code = _lib.DTYPE_F64 if t.dtype == torch.float64 else _lib.DTYPE_F32
    out = torch.empty(t.shape, dtype=torch.float16, device=t.device)
    _lib.check(_lib.load().moat_int4_to_f16(D.ptr(t), code, t.numel(), D.ptr(out), D.stream()),
               "lut_dequantize_fp16 (table to fp16)")
    return out


def _index_mode(q: torch.Tensor, host_dtype) -> Tuple[torch.Tensor, int]:
    """Index rule of src/dequant.py:87-95: int8 -> q+8; other signed ints ->
    q+8 only if any value is negative; everything else -> q as int32."""
    lib = _lib.load()
    kind = np.dtype(host_dtype).kind if host_dtype is not None else None
    if q.dtype == torch.int8:
        return q.to(torch.int64), 0
    if q.dtype in (torch.int16, torch.int32, torch.int64) and kind != "u":
        q64 = q.to(torch.int64).contiguous()
        if q64.numel() == 0:
            raise ValueError("zero-size array to reduction operation minimum which has no identity")
        flag = torch.zeros(1, dtype=torch.int32, device=q64.device)
        _lib.check(lib.moat_int4_any_negative(D.ptr(q64), q64.numel(), D.ptr(flag), D.stream()),
                   "lut_dequantize_fp16 (sign test)")
        return q64, (1 if int(flag.item()) else 2)
    if q.is_floating_point():
        return q.trunc().to(torch.int64), 2  # astype(int32) truncates toward zero
    return q.to(torch.int64), 2


def lut_dequantize_fp16(q_weights, lut):
    """Clipped gather ``lut[clip(idx, 0, L-1)]`` with the index rule and the
    1-D / 2-D / 3-D table layouts of ``src/dequant.py:79-112``; fp16 out in
    q's shape."""
    want_t = D.is_tensor(q_weights)
    lut_shape = tuple(lut.shape)
    if len(lut_shape) not in (1, 2, 3):
        raise ValueError(f"Unsupported LUT shape {lut_shape}. Must be 1D, 2D, or 3D.")
    q_shape = tuple(q_weights.shape)
    host_dtype = None if want_t else np.asarray(q_weights).dtype
    lut16 = _lut_to_f16(lut)
    lut_len = lut_shape[-1]
    rows = 1 if len(lut_shape) == 1 else int(np.prod(lut_shape[:-1]))
    n = int(np.prod(q_shape, dtype=np.int64))
    if n % rows != 0:
        raise ValueError(f"cannot reshape array of size {n} into shape ({rows},newaxis)")
    q64, mode = _index_mode(D.to_device(q_weights), host_dtype)
    out = torch.empty(n, dtype=torch.float16, device=q64.device)
    per_row_rows = rows if len(lut_shape) > 1 else 1
    _lib.check(_lib.load().moat_int4_lut_gather(D.ptr(q64), n, mode, D.ptr(lut16), per_row_rows, lut_len,
                                                D.ptr(out), D.stream()), "lut_dequantize_fp16")
    return D.out_like(out.view(q_shape), want_t)


# --------------------------------------------------------------------------
# the 144-byte decoder (src/dequant.py:116-147)
# --------------------------------------------------------------------------

def _blob_to_device(superblock_bytes, num_superblocks: int) -> torch.Tensor:
    if D.is_tensor(superblock_bytes):
        t = superblock_bytes
        if t.element_size() != 1:
            raise TypeError("superblock stream must be a byte tensor (uint8/int8)")
        if t.numel() != num_superblocks * SUPERBLOCK_BYTES:
            raise ValueError(f"cannot reshape array of size {t.numel()} into shape ({num_superblocks},144)")
        return D.aligned(D.to_device(t).view(torch.uint8).reshape(-1), 16)
    arr = np.asarray(superblock_bytes)
    if arr.dtype.itemsize != 1:
        raise TypeError("superblock stream must be a byte array (uint8/int8)")
    arr = arr.reshape(num_superblocks, SUPERBLOCK_BYTES)  # ValueError on a size mismatch, like the reference
    return D.to_device(arr.view(np.uint8).reshape(-1))


def unpack_superblock_weights(superblock_bytes, num_superblocks: int):
    """Decode ``num_superblocks`` 144-byte records (8 fp16 scales + 128 nibble
    bytes, low nibble = even element) to ``num_superblocks*256`` fp16 values,
    ``fp16((nibble - 8) * scale)`` (``src/dequant.py:116-147``)."""
    want_t = D.is_tensor(superblock_bytes)
    blob = _blob_to_device(superblock_bytes, num_superblocks)
    out = torch.empty(num_superblocks * SUPERBLOCK_ELEMS, dtype=torch.float16, device=blob.device)
    _lib.check(_lib.load().moat_int4_dequant(D.ptr(blob), num_superblocks, D.ptr(out), D.stream()),
               "unpack_superblock_weights")
    return D.out_like(out, want_t)


# --------------------------------------------------------------------------
# footprint (src/dequant.py:150-187)
# --------------------------------------------------------------------------

def calculate_memory_footprint(num_params: int, group_size: int = 32, bits: int = 4) -> Dict[str, Union[int, float, bool]]:
    """Bytes of ``num_params`` weights at ``bits`` bits plus one fp16 scale per
    group, against the reference's 4.5 GB budget (``src/dequant.py:150-187``)."""
    weight_bytes = num_params * (bits / 8.0)
    scale_bytes = (num_params // group_size) * 2.0
    total = weight_bytes + scale_bytes
    limit_gb = 4.5
    total_gb = total / (1024 ** 3)
    return {
        "num_params": num_params,
        "weight_bytes": weight_bytes,
        "scale_bytes": scale_bytes,
        "total_bytes": total,
        "total_mb": total / (1024 ** 2),
        "total_gb": total_gb,
        "ram_limit_gb": limit_gb,
        "fits_in_ram": total_gb <= limit_gb,
        "bytes_per_param_effective": total / num_params,
    }


# --------------------------------------------------------------------------
# additions: writer, fused quantize+write, batched projection
# --------------------------------------------------------------------------

def pack_superblocks_bytes(q_weights, scales):
    """Write the 144-byte records: ``uint8[S, 144]`` from int q (C-order flat
    index = element index; each value stored as ``(q + 8) & 15``) and one fp16
    scale per 32 elements.  Inverse of :func:`unpack_superblock_weights`."""
    want_t = D.is_tensor(q_weights)
    n = int(np.prod(tuple(q_weights.shape), dtype=np.int64))
    if n % SUPERBLOCK_ELEMS != 0:
        raise ValueError(f"element count {n} is not a multiple of {SUPERBLOCK_ELEMS}")
    n_sb = n // SUPERBLOCK_ELEMS
    if int(np.prod(tuple(scales.shape), dtype=np.int64)) != n_sb * 8:
        raise ValueError(f"expected {n_sb * 8} scales, got {int(np.prod(tuple(scales.shape)))}")
    q = D.to_device(q_weights)
    if q.is_floating_point():
        q = q.to(torch.int16)
    q = q.to(torch.int8).reshape(-1)
    s = D.to_device(scales)
    s = (s if s.dtype == torch.float16 else _lut_to_f16(s)).reshape(-1)
    blob = torch.empty((n_sb, SUPERBLOCK_BYTES), dtype=torch.uint8, device=q.device)
    _lib.check(_lib.load().moat_int4_pack_superblocks(D.ptr(q), D.ptr(s), n_sb, D.ptr(blob), D.stream()),
               "pack_superblocks_bytes")
    return D.out_like(blob, want_t)


def quantize_to_superblocks(weights, scale_rule: str = "f32"):
    """Quantize (group 32) and write the 144-byte records in one kernel.
    ``scale_rule='f32'`` divides by the float32 scale (this module's
    quantizer), ``'f16'`` by the fp16-rounded one (the engine module's)."""
    want_t = D.is_tensor(weights)
    n = int(np.prod(tuple(weights.shape), dtype=np.int64))
    if n % SUPERBLOCK_ELEMS != 0:
        raise ValueError(f"element count {n} is not a multiple of {SUPERBLOCK_ELEMS}")
    if scale_rule not in ("f32", "f16"):
        raise ValueError("scale_rule must be 'f32' or 'f16'")
    w, code = _float_dtype_code(D.to_device(weights))
    blob = torch.empty((n // SUPERBLOCK_ELEMS, SUPERBLOCK_BYTES), dtype=torch.uint8, device=w.device)
    mode = _lib.SCALE_F32 if scale_rule == "f32" else _lib.SCALE_F16
    _lib.check(_lib.load().moat_int4_quantize_pack(D.ptr(w), code, n, mode, D.ptr(blob), D.stream()),
               "quantize_to_superblocks")
    return D.out_like(blob, want_t)


def _gemm_into(x: torch.Tensor, blob: torch.Tensor, y: torch.Tensor, K: int, M: int,
               algo: int = _lib.GEMM_AUTO, splits: int = 0, batch: int = 0, finish: int = 0, front: int = 0,
               group: int = 0, waves: int = 0, tile_order: bool = False, strip_order: bool = False) -> None:
    lib = _lib.load()
    n = x.shape[0]
    opt = _lib.GemmOptions(algo, splits, batch, finish, front, group, waves)
    if strip_order:
        ws_bytes = lib.moat_int4_gemm_strips_workspace_size(n, K, M, ctypes.byref(opt))
        if ws_bytes < 0:
            raise ValueError(f"strip order needs K >= 2048, K % 32 == 0 and M % 32 == 0 (got K={K}, M={M}, N={n})")
        ws = D.workspaces.get(ws_bytes)
        _lib.check(lib.moat_int4_gemm_strips(D.ptr(x), D.ptr(blob), D.ptr(y), n, K, M, ctypes.byref(opt), D.ptr(ws),
                                             ws_bytes, D.stream()), "batched_int4_matmul")
        return
    ws_bytes = lib.moat_int4_gemm_ex_workspace_size(n, K, M, ctypes.byref(opt))
    if ws_bytes < 0:
        raise ValueError(f"unsupported GEMM configuration N={n} K={K} M={M} algo={algo} splits={splits} "
                         f"batch={batch} finish={finish} front={front} group={group} waves={waves}")
    ws = D.workspaces.get(ws_bytes)
    fn = lib.moat_int4_gemm_tiles if tile_order else lib.moat_int4_gemm_ex
    _lib.check(fn(D.ptr(x), D.ptr(blob), D.ptr(y), n, K, M, ctypes.byref(opt), D.ptr(ws), ws_bytes, D.stream()),
               "batched_int4_matmul")


def records_to_tiles(superblocks, K: int, M: int) -> torch.Tensor:
    """The 144-byte records of a row-major K x M stream (``M % 256 == 0``) in
    tile order: the K rows of each 256-column tile contiguous, tiles in
    column order (row r of tile j at record ``j * K + r``).  A GPU uint8
    tensor; :func:`batched_int4_matmul` reads it with ``tile_order=True``,
    with the same result bits and a faster weight stream.  (A storage order
    with no counterpart in the reference, whose stream is the row order.)"""
    K, M = int(K), int(M)
    if K < 1 or M < 256 or M % 256 != 0:
        raise ValueError(f"tile order needs M % 256 == 0 (got K={K}, M={M})")
    n_sb = K * M // SUPERBLOCK_ELEMS
    blob = _blob_to_device(superblocks, n_sb)
    tiles = torch.empty(n_sb * SUPERBLOCK_BYTES, dtype=torch.uint8, device=blob.device)
    _lib.check(_lib.load().moat_int4_records_to_tiles(D.ptr(blob), K, M, D.ptr(tiles), D.stream()),
               "records_to_tiles")
    return tiles


def records_to_strips(superblocks, K: int, M: int) -> torch.Tensor:
    """The quantized weights of a row-major K x M stream (``K % 8 == 0``,
    ``M % 32 == 0``) in strip order: strip g = columns 32g..32g+31, strips in
    column order, and inside a strip one 144-byte record per 8 rows (their 8
    scales of the strip's group, then the 16 payload bytes of each column
    pair for rows 0 2 1 3 4 6 5 7).  A GPU uint8 tensor, read by
    :func:`batched_int4_matmul` with ``strip_order=True`` (``K >= 2048``):
    every workgroup streams one contiguous range of it.  (A storage order
    with no counterpart in the reference, whose stream is the row order; the
    q values and scales are unchanged.)"""
    K, M = int(K), int(M)
    if K < 8 or K % 8 != 0 or M < 32 or M % 32 != 0:
        raise ValueError(f"strip order needs K % 8 == 0 and M % 32 == 0 (got K={K}, M={M})")
    n_sb = K * M // SUPERBLOCK_ELEMS
    blob = _blob_to_device(superblocks, n_sb)
    strips = torch.empty(n_sb * SUPERBLOCK_BYTES, dtype=torch.uint8, device=blob.device)
    _lib.check(_lib.load().moat_int4_records_to_strips(D.ptr(blob), K, M, D.ptr(strips), D.stream()),
               "records_to_strips")
    return strips


def strips_to_records(strips, K: int, M: int) -> torch.Tensor:
    """Row-order records (``uint8[K*M/256, 144]`` on the GPU) from a strip-order
    stream: the inverse of :func:`records_to_strips`."""
    K, M = int(K), int(M)
    if K < 8 or K % 8 != 0 or M < 32 or M % 32 != 0:
        raise ValueError(f"strip order needs K % 8 == 0 and M % 32 == 0 (got K={K}, M={M})")
    n_sb = K * M // SUPERBLOCK_ELEMS
    blob = _blob_to_device(strips, n_sb)
    out = torch.empty((n_sb, SUPERBLOCK_BYTES), dtype=torch.uint8, device=blob.device)
    _lib.check(_lib.load().moat_int4_strips_to_records(D.ptr(blob), K, M, D.ptr(out), D.stream()),
               "strips_to_records")
    return out


def to_f16(t) -> torch.Tensor:
    """A GPU fp16 tensor of the same shape: fp16 as is; fp32 and fp64 rounded
    once, nearest-even (numpy's ``astype(float16)``; a device float64 ->
    float32 -> float16 chain would round twice); bf16 through float32 (exact);
    integers and bools through float64 (exact below 2^53)."""
    t = D.to_device(t)
    if t.dtype == torch.float16:
        return t
    if t.dtype not in (torch.float32, torch.float64):
        t = t.to(torch.float32 if t.dtype == torch.bfloat16 else torch.float64)
    t = t.contiguous()
    code = _lib.DTYPE_F64 if t.dtype == torch.float64 else _lib.DTYPE_F32
    out = torch.empty(t.shape, dtype=torch.float16, device=t.device)
    _lib.check(_lib.load().moat_int4_to_f16(D.ptr(t), code, t.numel(), D.ptr(out), D.stream()), "to_f16")
    return out


def i8_div_to_f16(q, divisor: float) -> torch.Tensor:
    """``fp16(f32(q) / divisor)`` for int8 ``q``: numpy's float16 division of
    ``q.astype(float16) / divisor`` (one float32 division, then one rounding
    to float16), on the GPU."""
    t = D.to_device(q)
    if t.dtype != torch.int8:
        raise ValueError("i8_div_to_f16 takes int8 values")
    t = t.contiguous()
    out = torch.empty(t.shape, dtype=torch.float16, device=t.device)
    _lib.check(_lib.load().moat_int4_i8_div_to_f16(D.ptr(t), t.numel(), float(divisor), D.ptr(out), D.stream()),
               "i8_div_to_f16")
    return out


def _fused_inputs(x, K: int, M: int, blobs):
    K, M = int(K), int(M)
    if K < 1 or K % 32 != 0 or M < 128 or M % 128 != 0:
        raise ValueError(f"fused projections need K % 32 == 0 and M % 128 == 0 (got K={K}, M={M}); "
                         "use batched_int4_matmul per matrix")
    xs = D.to_device(x)
    if xs.dim() == 1:
        xs = xs.reshape(1, -1)
    if xs.dim() != 2 or xs.shape[1] != K:
        raise ValueError(f"x must be (N, {K}), got {tuple(xs.shape)}")
    if xs.dtype != torch.float16:
        xs = xs.to(torch.float16)
    xs = D.aligned(xs.contiguous(), 16)
    n_sb = K * M // SUPERBLOCK_ELEMS
    return xs, [_blob_to_device(b, n_sb) for b in blobs]


def batched_int4_matmul_multi(x, superblocks_list, K: int, M: int):
    """``[f32(X) @ f32(deq(W_i)) for W_i in superblocks_list]``: 1 to 4
    matrices of one shape (K x M) that share the activations X, in one launch
    per 32 rows of X (``moat_int4_gemm_multi``); each result equals
    :func:`batched_int4_matmul` on that matrix (to float32 summation order).
    ValueError unless ``K % 32 == 0`` and ``M % 128 == 0``."""
    want_t = D.is_tensor(x)
    blobs_in = list(superblocks_list)
    if not 1 <= len(blobs_in) <= 4:
        raise ValueError(f"1 to 4 matrices, got {len(blobs_in)}")
    xs, blobs = _fused_inputs(x, K, M, blobs_in)
    N = xs.shape[0]
    ys = [torch.empty((N, M), dtype=torch.float32, device=xs.device) for _ in blobs]
    for r0 in range(0, N, MAX_BATCH_PER_CALL):
        r1 = min(N, r0 + MAX_BATCH_PER_CALL)
        _multi_into(xs[r0:r1], blobs, [y[r0:r1] for y in ys], int(K), int(M))
    if want_t:
        return ys
    res = [D.to_host(y) for y in ys]
    D.workspaces.check("batched_int4_matmul_multi")
    return res


def _multi_into(x: torch.Tensor, blobs, ys, K: int, M: int) -> None:
    """One ``moat_int4_gemm_multi`` launch: x (n <= 32, K) fp16 16-byte
    aligned, device record streams, (n, M) fp32 outputs."""
    lib = _lib.load()
    n, count = x.shape[0], len(blobs)
    ws_bytes = lib.moat_int4_gemm_multi_workspace_size(count, n, K, M)
    if ws_bytes < 0:
        raise ValueError(f"unsupported fused configuration count={count} N={n} K={K} M={M}")
    ws = D.workspaces.get(ws_bytes)
    sb_ptrs = (ctypes.c_void_p * count)(*[D.ptr(b) for b in blobs])
    y_ptrs = (ctypes.c_void_p * count)(*[D.ptr(y) for y in ys])
    _lib.check(lib.moat_int4_gemm_multi(D.ptr(x), sb_ptrs, y_ptrs, count, n, K, M, D.ptr(ws), ws_bytes, D.stream()),
               "batched_int4_matmul_multi")


def int4_swiglu(x, gate_superblocks, up_superblocks, K: int, M: int):
    """``h = fp16(silu(g) * u)`` with ``g = f32(X) @ f32(deq(W_gate))``,
    ``u = f32(X) @ f32(deq(W_up))`` and ``silu(g) = g / (1 + exp(-g))`` in
    fp32 (antigravity-engine/src/shaders/transformer_ops.metal:216-232 on the
    two projections of transformer_engine.mm:694-713), in one launch per 32
    rows of X (``moat_int4_gemm_swiglu``); fp16 (N, M) out, the down
    projection's input.  ValueError unless ``K % 32 == 0`` and
    ``M % 128 == 0``."""
    want_t = D.is_tensor(x)
    xs, (gb, ub) = _fused_inputs(x, K, M, [gate_superblocks, up_superblocks])
    N = xs.shape[0]
    h = torch.empty((N, M), dtype=torch.float16, device=xs.device)
    for r0 in range(0, N, MAX_BATCH_PER_CALL):
        r1 = min(N, r0 + MAX_BATCH_PER_CALL)
        _swiglu_into(xs[r0:r1], gb, ub, h[r0:r1], int(K), int(M))
    if want_t:
        return h
    res = D.to_host(h)
    D.workspaces.check("int4_swiglu")
    return res


def interleave_strips(gate_strips, up_strips, K: int, M: int) -> torch.Tensor:
    """The strip-order streams of two K x M matrices (:func:`records_to_strips`)
    interleaved strip by strip: gate strip c, then up strip c.  A GPU uint8
    tensor of both matrices' bytes, the weights of :func:`int4_swiglu_strips`.
    (A load-time layout with no counterpart in the reference.)"""
    K, M = int(K), int(M)
    if K < 8 or K % 8 != 0 or M < 32 or M % 32 != 0:
        raise ValueError(f"strip order needs K % 8 == 0 and M % 32 == 0 (got K={K}, M={M})")
    n_sb = K * M // SUPERBLOCK_ELEMS
    g = _blob_to_device(gate_strips, n_sb)
    u = _blob_to_device(up_strips, n_sb)
    out = torch.empty(2 * n_sb * SUPERBLOCK_BYTES, dtype=torch.uint8, device=g.device)
    _lib.check(_lib.load().moat_int4_interleave_strips(D.ptr(g), D.ptr(u), K, M, D.ptr(out), D.stream()),
               "interleave_strips")
    return out


def int4_swiglu_strips(x, gate_up_strips, K: int, M: int, splits: int = 0):
    """:func:`int4_swiglu` over strip order in one launch per 32 rows of X
    (``moat_int4_gemm_strips_swiglu``): ``gate_up_strips`` from
    :func:`interleave_strips`; every workgroup computes whole gate/up strip
    pairs and writes h for their 32 columns.  fp16 (N, M) out.  ValueError
    unless ``K >= 2048``, ``K % 32 == 0`` and ``M % 32 == 0``; ``splits`` =
    workgroups (0 automatic)."""
    want_t = D.is_tensor(x)
    K, M = int(K), int(M)
    if K < 2048 or K % 32 != 0 or M < 32 or M % 32 != 0:
        raise ValueError(f"strip order needs K >= 2048, K % 32 == 0 and M % 32 == 0 (got K={K}, M={M})")
    xs = D.to_device(x)
    if xs.dim() == 1:
        xs = xs.reshape(1, -1)
    if xs.dim() != 2 or xs.shape[1] != K:
        raise ValueError(f"x must be (N, {K}), got {tuple(xs.shape)}")
    if xs.dtype != torch.float16:
        xs = xs.to(torch.float16)
    xs = D.aligned(xs.contiguous(), 16)
    blob = _blob_to_device(gate_up_strips, 2 * K * M // SUPERBLOCK_ELEMS)
    N = xs.shape[0]
    h = torch.empty((N, M), dtype=torch.float16, device=xs.device)
    lib = _lib.load()
    opt = _lib.GemmOptions(0, int(splits), 0, 0, 0, 0, 0)
    for r0 in range(0, N, MAX_BATCH_PER_CALL):
        rows = min(MAX_BATCH_PER_CALL, N - r0)
        _lib.check(lib.moat_int4_gemm_strips_swiglu(D.ptr(xs[r0:r0 + rows]), D.ptr(blob), D.ptr(h[r0:r0 + rows]), rows,
                                                    K, M, ctypes.byref(opt), D.stream()), "int4_swiglu_strips")
    return h if want_t else D.to_host(h)


def _swiglu_into(x: torch.Tensor, gate: torch.Tensor, up: torch.Tensor, h: torch.Tensor, K: int, M: int) -> None:
    """One ``moat_int4_gemm_swiglu`` launch: x (n <= 32, K) fp16 16-byte
    aligned, device record streams, (n, M) fp16 output."""
    lib = _lib.load()
    n = x.shape[0]
    ws_bytes = lib.moat_int4_gemm_swiglu_workspace_size(n, K, M)
    if ws_bytes < 0:
        raise ValueError(f"unsupported fused configuration N={n} K={K} M={M}")
    ws = D.workspaces.get(ws_bytes)
    _lib.check(lib.moat_int4_gemm_swiglu(D.ptr(x), D.ptr(gate), D.ptr(up), D.ptr(h), n, K, M, D.ptr(ws), ws_bytes,
                                         D.stream()), "int4_swiglu")


def batched_int4_matmul(x, superblocks, K: int, M: int, out=None, *, algo: int = _lib.GEMM_AUTO,
                        splits: int = 0, batch: int = 0, finish: int = 0, front: int = 0, group: int = 0,
                        waves: int = 0, tile_order: bool = False, strip_order: bool = False):
    """``Y[N, M] = f32(X[N, K]) @ f32(deq(W)[K, M])`` with W the 144-byte stream
    of a row-major K x M matrix; fp32 out.  Equal (to float32 summation order)
    to decoding with :func:`unpack_superblock_weights` and a float32 matmul.
    ValueError unless ``M % 32 == 0`` and ``K*M % 256 == 0``.  N above 32 is
    processed in slices of 32 rows.  ``algo``/``splits``/``batch``/``finish``/
    ``front``/``group``/``waves`` override the launch choices of
    ``moat_int4_gemm_options`` (0 = automatic).  ``tile_order``: the stream is
    in the tile order of :func:`records_to_tiles` (``M % 256 == 0``,
    ``K % 32 == 0``); ``strip_order``: in the strip order of
    :func:`records_to_strips` (``K >= 2048``, ``K % 32 == 0``; ``splits`` =
    workgroups, ``batch`` = ring depth)."""
    want_t = D.is_tensor(x)
    K, M = int(K), int(M)
    if K < 1 or M < 32 or M % 32 != 0 or (K * M) % SUPERBLOCK_ELEMS != 0:
        raise ValueError(f"need M % 32 == 0 and K*M % 256 == 0 (got K={K}, M={M})")
    xs = D.to_device(x)
    if xs.dim() == 1:
        xs = xs.reshape(1, -1)
    if xs.dim() != 2 or xs.shape[1] != K:
        raise ValueError(f"x must be (N, {K}), got {tuple(xs.shape)}")
    if xs.dtype != torch.float16:
        xs = xs.to(torch.float16)
    xs = D.aligned(xs.contiguous(), 16)
    n_sb = K * M // SUPERBLOCK_ELEMS
    blob = _blob_to_device(superblocks, n_sb)
    N = xs.shape[0]
    if out is not None and D.is_tensor(out):
        y = out
        if y.shape != (N, M) or y.dtype != torch.float32 or not y.is_contiguous() or y.device != xs.device:
            raise ValueError("out must be a contiguous float32 (N, M) tensor on the GPU")
    else:
        y = torch.empty((N, M), dtype=torch.float32, device=xs.device)
    for r0 in range(0, N, MAX_BATCH_PER_CALL):
        r1 = min(N, r0 + MAX_BATCH_PER_CALL)
        _gemm_into(xs[r0:r1], blob, y[r0:r1], K, M, algo, splits, batch, finish, front, group, waves, tile_order,
                   strip_order)
    if out is not None and not D.is_tensor(out):
        np.copyto(out, D.to_host(y))
        D.workspaces.check("batched_int4_matmul")
        return out
    if not want_t:  # the host copy waits for the call anyway
        res = D.to_host(y)
        D.workspaces.check("batched_int4_matmul")
        return res
    return y


def check_gemm_workspace() -> None:
    """Raise RuntimeError if an in-kernel hand-off of a GEMM on the current
    stream ran out of time since the last check (those results, and those
    of every later call on the stream's workspace, are NaN); the workspace is
    cleared first.  Synchronises the stream.  Calls with numpy outputs check
    by themselves."""
    D.workspaces.check("GEMM")
