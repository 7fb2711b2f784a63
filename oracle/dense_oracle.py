"""CPU restatement of the reference's dense fp16 products (test infrastructure
only: imported by tests, the smoke check and the bench's CPU baseline, never
by ``moat_amd``).

* :func:`gemv_ref` -- ``gemv_kernel``
  (``antigravity-engine/src/shaders/transformer_ops.metal:270-286``): per
  column, ``sum += (float)x[k] * (float)B[k * N + col]`` for k = 0 .. K-1 in
  order, in float32, then ``(half)sum``.  Vectorised over columns, the same
  float32 operations in the same order, so bit for bit.
* :func:`dense_gemm_ref` -- the reference's CPU product
  (``antigravity-engine/tests/test_batched_speed.py:31-42``,
  ``(X.astype(f32) @ W.astype(f32)).astype(W.dtype)``): BLAS float32 sums,
  then fp16.
* :func:`dense_exact` -- the exact product (float64; exact for the integer
  inputs the tests use), rounded to fp16.

Pinned by the reference's known answers (``antigravity-engine/tests/
test_metal_kernels.cpp:94-131``: ones(8 x 16) @ 0.5 * ones(16 x 16) = 8.0;
``antigravity-engine/src/metal_runner.cpp:84-98``: X = 1, W = -0.5 gives
-0.5 * K) and by integer products, where every path is exact and a
transposed operand or a dropped row shows.
"""

from __future__ import annotations

import numpy as np


def dense_gemm_ref(x, w) -> np.ndarray:
    """``fp16(f32(X) @ f32(W))`` (``test_batched_speed.py:39-42``)."""
    x32 = np.asarray(x).astype(np.float32)
    w32 = np.asarray(w).astype(np.float32)
    return (x32 @ w32).astype(np.float16)


def gemv_ref(x_row, w) -> np.ndarray:
    """``gemv_kernel``: float32 sums in k order, one fp16 result per column."""
    x32 = np.asarray(x_row).astype(np.float32).reshape(-1)
    w32 = np.asarray(w).astype(np.float32)
    acc = np.zeros(w32.shape[1], dtype=np.float32)
    for k in range(x32.shape[0]):
        acc = (acc + x32[k] * w32[k]).astype(np.float32)  # f16 x f16 is exact in f32
    return acc.astype(np.float16)


def dense_exact(x, w) -> np.ndarray:
    """``fp16(X @ W)`` with the sums in float64."""
    return (np.asarray(x).astype(np.float64) @ np.asarray(w).astype(np.float64)).astype(np.float16)


def fp16_ulp(v) -> np.ndarray:
    """The spacing of fp16 values at |v| (2^-24 below the normal range)."""
    a = np.abs(np.asarray(v, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return np.maximum(2.0 ** (e - 10), 2.0 ** -24)


def dense_tolerance(x, w) -> np.ndarray:
    """Per-output bound for an fp16 result of float32 sums in any order:
    one fp16 ulp of the exact value (the rounding may fall on either side
    when the float32 sum lies near a half-way point) plus K float32
    roundings of the absolute products."""
    x64 = np.abs(np.asarray(x).astype(np.float64))
    w64 = np.abs(np.asarray(w).astype(np.float64))
    exact = np.asarray(x).astype(np.float64) @ np.asarray(w).astype(np.float64)
    k = x64.shape[-1]
    return fp16_ulp(exact) + k * 2.0 ** -24 * (x64 @ w64)
