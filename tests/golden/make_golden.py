"""Writes the golden fixtures of this directory (run from the repository root:
``python tests/golden/make_golden.py``).

Every expected value is computed here from the format and from IEEE-754
rounding written out by hand (``tests/ieee_exact.py``: binary16 from Python's
``struct`` packer, binary32 from exact rationals) -- not from the oracle and
not from the reference's code:

* quantization of each group of 32 float32 weights with exact rationals
  (alpha = max|w|, s = f32(alpha / 7), q = clip(round_half_even(f32(w / s)),
  -8, 7), scale stored as binary16), the float32-scale rule of
  ``src/dequant.py:26-55``;
* the 144-byte records built with Python integers from the layout of
  ``src/dequant.py:116-147`` / ``batched_gemm.metal:16-35`` (8 little-endian
  binary16 scales, then 128 bytes holding element 2j in the low nibble and
  2j+1 in the high nibble, stored as q + 8; superblock i covers flat elements
  256i .. 256i+255 of the row-major K x M matrix);
* dequantized weights as binary16 bits of (q * s), one rounding of an exact
  product;
* Y = X @ W summed exactly (rationals) and rounded once to float64.

Inputs come from ``numpy.random.default_rng`` with fixed seeds.  The cases
cover a record-aligned width (M % 256 == 0), rows that start half-way into a
record (M % 256 == 128) with N above 16, and a shape the record-stream kernel
does not take (K % 32 != 0, M % 128 != 0).
"""

from __future__ import annotations

import os
import sys
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))  # tests/ for ieee_exact

from ieee_exact import f16_bits, f16_value, quantize_group_exact  # noqa: E402

CASES = [
    # name, K, M, N, weight seed, activation seed
    ("aligned_k64_m256_n3", 64, 256, 3, 11, 21),
    ("shifted_k96_m384_n17", 96, 384, 17, 12, 22),
    ("ragged_k40_m96_n5", 40, 96, 5, 13, 23),
]


def make_case(K: int, M: int, N: int, wseed: int, xseed: int) -> dict:
    w = (np.random.default_rng(wseed).standard_normal((K, M), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    flat = [float(v) for v in w.reshape(-1)]
    n = len(flat)
    assert n % 256 == 0
    q = [0] * n
    scale_bits = []
    for g in range(n // 32):
        qs, sb = quantize_group_exact(flat[32 * g:32 * g + 32], fp16_scale_first=False)
        q[32 * g:32 * g + 32] = qs
        scale_bits.append(sb)
    blob = bytearray()
    for s in range(n // 256):
        for g in range(8):
            b = scale_bits[8 * s + g]
            blob += bytes((b & 0xFF, b >> 8))
        for j in range(128):
            lo = q[256 * s + 2 * j] + 8
            hi = q[256 * s + 2 * j + 1] + 8
            blob.append((hi << 4) | lo)
    deq_bits = []
    deq_val = []
    for e in range(n):
        s = f16_value(scale_bits[e // 32])
        bits = f16_bits(q[e] * s)
        deq_bits.append(bits)
        deq_val.append(Fraction(f16_value(bits)))
    x = np.random.default_rng(xseed).standard_normal((N, K), dtype=np.float32).astype(np.float16)
    xv = [[Fraction(float(v)) for v in row] for row in x]
    y = np.zeros((N, M), dtype=np.float64)
    for r in range(N):
        for m in range(M):
            acc = Fraction(0)
            for k in range(K):
                acc += xv[r][k] * deq_val[k * M + m]
            y[r, m] = float(acc)
    return {
        "w": w,
        "q": np.array(q, dtype=np.int8),
        "scales": np.array(scale_bits, dtype=np.uint16),
        "blob": np.frombuffer(bytes(blob), dtype=np.uint8),
        "deq_bits": np.array(deq_bits, dtype=np.uint16),
        "x": x,
        "y": y,
        "shape": np.array([K, M, N], dtype=np.int64),
    }


def main() -> None:
    for name, K, M, N, ws, xs in CASES:
        d = make_case(K, M, N, ws, xs)
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **d)
        print(f"wrote {path}")


if __name__ == "__main__":
    main()
