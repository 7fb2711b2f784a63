"""Dense fp16 decode product on the GPU: ``fp16(f32(X) @ f32(W))``.

The reference's dense path (``antigravity-engine/src/transformer_engine.mm:463-500``
``dispatchGEMM``) picks ``batched_gemm_simdgroup``
(``antigravity-engine/src/shaders/batched_gemm.metal:74-109``, 8 x 8 tiles,
half sums, N a multiple of 8) or, for one row, ``gemv_kernel``
(``antigravity-engine/src/shaders/transformer_ops.metal:270-286``, fp32 sums,
half result).  :func:`dense_gemm` is one ``moat_dense_gemm`` launch per 32
rows for every N: fp32 sums, each output rounded to fp16 once -- the
GEMV's arithmetic, and that of the reference's CPU product
(``antigravity-engine/tests/test_batched_speed.py:31-42``).
"""

from __future__ import annotations

import numpy as np
import torch

from . import _device as D
from . import _lib


def _f16_rows(a, name: str) -> torch.Tensor:
    t = D.to_device(a)
    if t.dtype != torch.float16:
        raise ValueError(f"{name} must be float16 (got {t.dtype})")
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D (got shape {tuple(t.shape)})")
    return D.aligned(t.contiguous(), 16)


def dense_gemm(x, w, out=None, *, splits: int = 0):
    """``Y[N, M] = fp16(f32(X[N, K]) @ f32(W[K, M]))``: X and W float16,
    row-major; the sums in float32.  ValueError unless ``K % 8 == 0`` and
    ``M % 8 == 0`` (``K, M >= 8``, ``N >= 1``).  Row r of Y does not depend
    on the other rows (it equals the one-row call on ``X[r]``).  Numpy inputs
    give a numpy result; ``out`` (float16, N x M) receives it when given.
    ``splits``: workgroups a 64-column block's rows are split over (0:
    automatic)."""
    want_t = D.is_tensor(x) or D.is_tensor(w)
    xs, ws_ = _f16_rows(x, "x"), _f16_rows(w, "w")
    N, K = xs.shape
    K2, M = ws_.shape
    if K2 != K:
        raise ValueError(f"x is {N} x {K} but w is {K2} x {M}")
    if N < 1 or K < 8 or K % 8 != 0 or M < 8 or M % 8 != 0:
        raise ValueError(f"need N >= 1, K % 8 == 0 and M % 8 == 0 (got N={N}, K={K}, M={M})")
    if splits < 0:
        raise ValueError(f"splits must be >= 0 (got {splits})")
    lib = _lib.load()
    ws_bytes = lib.moat_dense_gemm_workspace_size(N, K, M, int(splits))
    if ws_bytes < 0:
        raise ValueError(f"unsupported dense product N={N} K={K} M={M} splits={splits}")
    work = D.dense_workspaces.get(ws_bytes)
    if out is not None and D.is_tensor(out):
        if out.dtype != torch.float16 or tuple(out.shape) != (N, M) or not out.is_contiguous():
            raise ValueError(f"out must be a contiguous float16 tensor of shape {(N, M)}")
        if out.device != xs.device:
            raise ValueError(f"out must be on {xs.device} (got {out.device})")
        y = out
    else:
        y = torch.empty((N, M), dtype=torch.float16, device=xs.device)
    _lib.check(lib.moat_dense_gemm(D.ptr(xs), D.ptr(ws_), D.ptr(y), N, K, M, int(splits), D.ptr(work), ws_bytes,
                                   D.stream()), "dense_gemm")
    if out is not None and not D.is_tensor(out):
        np.copyto(out, D.to_host(y))
        return out
    return y if want_t else D.to_host(y)


def dense_gemv(x, w):
    """The one-row product ``y[M] = fp16(f32(x[K]) @ f32(W[K, M]))``
    (``gemv_kernel``, ``transformer_ops.metal:270-286``): :func:`dense_gemm`
    on a 1 x K row."""
    t = D.is_tensor(x)
    xr = x.reshape(1, -1)
    y = dense_gemm(xr, w)
    return y.reshape(-1) if t or D.is_tensor(y) else np.asarray(y).reshape(-1)
