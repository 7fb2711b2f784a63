"""CPU oracle for moat's INT4 superblock path: test infrastructure only.

This module is the *checker*. Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import it; the product
(``moat_amd``) never does, and has no CPU fallback.

It restates, in vectorised numpy, the arithmetic of the reference's two Python
surfaces and the byte layout its Metal kernels read:

* surface A  -- ``src/dequant.py`` (quantize any shape, LUT gather, 144-byte
  superblock decoder, footprint arithmetic);
* surface B  -- ``antigravity-engine/src/dequant.py`` (1-D quantizer with the
  fp16-rounded scale, nibble packing into per-superblock records, per-group
  LUT / arithmetic dequant);
* the superblock wire format -- ``antigravity-engine/src/shaders/batched_gemm.metal:16-20``
  (8 fp16 scales, then 128 bytes with element 2j in the LOW nibble of byte j
  and element 2j+1 in the HIGH nibble, stored as q+8), laid over the row-major
  flat index ``k*M + m`` of W[K][M] (``batched_gemm.metal:146-154``);
* the batched projection ``Y = f32(X) @ f32(deq(W))`` as the reference's CPU
  checks compute it (``antigravity-engine/tests/test_batched_speed.py:31-42``).

How each function is pinned (tests/test_oracle.py):

* dequant values: exhaustively, all 65,536 fp16 scale bit patterns x 16 nibbles,
  against Python's own IEEE binary16 packer (``struct`` format ``'e'``);
* quantizers: against an exact rational restatement (``fractions.Fraction``
  with hand-rolled binary32 round-to-nearest-even) on random and
  tie-constructed groups, and the reference tests' known answers;
* packing: the reference kernel test's byte 0x7F answer, the reference
  runner's 0x77 stream, round trips and Python-int bit arithmetic;
* tile order: a Python-loop index permutation on small shapes, and every
  tile's records decoding to that tile's 256 columns of W;
* strip order: a Python-loop byte permutation on small shapes over the row
  order's own offsets, and the strip decoder giving back W;
* GEMM: float64 accumulation of the same products, the closed-form
  -0.5*K answer of the reference runner's synthetic stream, and
  row-by-row GEMV equality.

NaN outputs are compared as a class, never by payload: the reference's own NaN
bits depend on the CPU it ran on (x86 and Arm produce different default NaNs).
"""

from __future__ import annotations

import numpy as np

# Quantisation constants, ``config/engine_config.yaml:1-5`` and
# ``batched_gemm.metal:12-14``.
GROUP = 32
GROUPS_PER_SB = 8
SB_ELEMS = GROUP * GROUPS_PER_SB  # 256
SB_HEADER_BYTES = 2 * GROUPS_PER_SB  # 16
SB_PAYLOAD_BYTES = SB_ELEMS // 2  # 128
SB_BYTES = SB_HEADER_BYTES + SB_PAYLOAD_BYTES  # 144


# --------------------------------------------------------------------------
# Quantizers
# --------------------------------------------------------------------------

def _group_absmax(groups_f32: np.ndarray) -> np.ndarray:
    return np.abs(groups_f32).max(axis=1)


def quantize_a(weights, group_size: int = GROUP):
    """Surface A quantizer, ``src/dequant.py:26-55``.

    Any shape, any float dtype; the values are cast to float32 and read in
    C order.  Per group: ``alpha = max|w|`` (f32), ``s = 1 if alpha == 0 else
    alpha / 7`` computed in float32, ``q = clip(rint_half_even(w / s), -8, 7)``.
    q keeps the input's shape; the scales are ``fp16(s)``, one per group.
    A length that is not a multiple of ``group_size`` raises AssertionError.
    """
    w = np.asarray(weights)
    flat = w.astype(np.float32).reshape(-1)
    assert flat.size % group_size == 0, (
        f"Weight array length ({flat.size}) must be a multiple of group_size ({group_size})."
    )
    groups = flat.reshape(-1, group_size)
    alpha = _group_absmax(groups)
    seven = np.float32(7.0)
    s32 = np.where(alpha == 0, np.float32(1.0), alpha / seven).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        r = np.rint(groups / s32[:, None])
    q = np.clip(r, -8, 7).astype(np.int8)
    return q.reshape(w.shape), s32.astype(np.float16)


def quantize_b(weights, group_size: int = GROUP):
    """Surface B quantizer, ``antigravity-engine/src/dequant.py:22-60``.

    1-D only (ValueError otherwise, and when the length is not a multiple of
    ``group_size``).  The scale is rounded to fp16 *before* dividing:
    ``s16 = fp16(1 if alpha == 0 else alpha / 7)``, then
    ``q = clip(rint_half_even(w_f32 / f32(s16)), -8, 7)``.
    """
    w = np.asarray(weights)
    if w.ndim != 1:
        raise ValueError(f"Expected 1D array, got shape {w.shape}")
    if w.shape[0] % group_size != 0:
        raise ValueError(
            f"Weight length {w.shape[0]} is not divisible by group_size={group_size}"
        )
    groups = w.astype(np.float32).reshape(-1, group_size)
    alpha = _group_absmax(groups)
    s16 = np.where(alpha == 0, np.float32(1.0), alpha / np.float32(7.0)).astype(np.float16)
    with np.errstate(invalid="ignore", divide="ignore"):
        r = np.rint(groups / s16.astype(np.float32)[:, None])
    q = np.clip(r, -8, 7).astype(np.int8)
    return q.reshape(-1), s16


# --------------------------------------------------------------------------
# Nibble packing and the 144-byte record
# --------------------------------------------------------------------------

def pack_nibbles(q) -> np.ndarray:
    """Nibble pairs, ``antigravity-engine/src/dequant.py:119-124``.

    Byte j holds ``(q[2j] + 8) & 15`` in its low nibble and
    ``(q[2j+1] + 8) & 15`` in its high nibble (integer wrap-around for values
    outside [-8, 7], as the reference's int16 -> uint8 casts give).
    """
    u = (np.asarray(q).astype(np.int64) + 8) & 0xF
    u = u.reshape(-1)
    return (u[0::2] | (u[1::2] << 4)).astype(np.uint8)


def unpack_nibbles(packed) -> np.ndarray:
    """Inverse of :func:`pack_nibbles`, ``antigravity-engine/src/dequant.py:135-156``."""
    p = np.asarray(packed).astype(np.int16).reshape(-1)
    out = np.empty(p.size * 2, dtype=np.int16)
    out[0::2] = p & 0xF
    out[1::2] = (p >> 4) & 0xF
    return (out - 8).astype(np.int8)


def superblock_records(q, scales, group_size: int = GROUP, groups_per_superblock: int = GROUPS_PER_SB):
    """Surface B's per-superblock records, ``antigravity-engine/src/dequant.py:69-132``.

    Returns a list of ``{'scales', 'packed_nibbles', 'raw_int4'}`` dicts;
    ValueError when the length is not a multiple of the superblock size.
    """
    q = np.asarray(q)
    per_sb = group_size * groups_per_superblock
    if len(q) % per_sb != 0:
        raise ValueError(f"Weight length {len(q)} not divisible by super-block size {per_sb}")
    packed = pack_nibbles(q).reshape(-1, per_sb // 2) if len(q) else np.zeros((0, per_sb // 2), np.uint8)
    out = []
    for i in range(len(q) // per_sb):
        out.append({
            "scales": np.asarray(scales)[i * groups_per_superblock:(i + 1) * groups_per_superblock].copy(),
            "packed_nibbles": packed[i].copy(),
            "raw_int4": q[i * per_sb:(i + 1) * per_sb].copy(),
        })
    return out


def serialize_superblocks(q, scales) -> np.ndarray:
    """The 144-byte wire records for a whole stream: ``uint8[S, 144]``.

    Layout of ``batched_gemm.metal:16-20``: bytes [0, 16) are the 8 group
    scales as little-endian fp16, bytes [16, 144) the nibble pairs of
    :func:`pack_nibbles`.  ``q`` is any-shape int (its C-order flat index is
    the element index), ``scales`` one fp16 per 32 elements.
    """
    qf = np.asarray(q).reshape(-1)
    if qf.size % SB_ELEMS != 0:
        raise ValueError(f"element count {qf.size} is not a multiple of {SB_ELEMS}")
    n_sb = qf.size // SB_ELEMS
    sc = np.asarray(scales, dtype=np.float16).reshape(-1)
    if sc.size != n_sb * GROUPS_PER_SB:
        raise ValueError(f"expected {n_sb * GROUPS_PER_SB} scales, got {sc.size}")
    blob = np.empty((n_sb, SB_BYTES), dtype=np.uint8)
    blob[:, :SB_HEADER_BYTES] = sc.astype("<f2").view(np.uint8).reshape(n_sb, SB_HEADER_BYTES)
    blob[:, SB_HEADER_BYTES:] = pack_nibbles(qf).reshape(n_sb, SB_PAYLOAD_BYTES)
    return blob


def quantize_pack_a(weights) -> np.ndarray:
    """Surface-A quantize then serialise, the load-time producer of the stream."""
    q, s = quantize_a(np.asarray(weights).reshape(-1))
    return serialize_superblocks(q, s)


# --------------------------------------------------------------------------
# Dequantisation
# --------------------------------------------------------------------------

def dequant_lut(scale) -> np.ndarray:
    """16-entry table, ``antigravity-engine/src/dequant.py:163-180``:
    ``fp16(f32(k) * f32(float(scale)))`` for k in -8..7."""
    ks = np.arange(-8, 8).astype(np.float32)
    return (ks * np.float32(float(scale))).astype(np.float16)


def group_dequant(q, scales, group_size: int = GROUP) -> np.ndarray:
    """``lut_dequantize`` / ``arithmetic_dequantize`` (``antigravity-engine/src/dequant.py:183-252``).

    Both give ``fp16(f32(q) * f32(float(scale_g)))`` per element of the
    first ``(len // group_size) * group_size`` elements; the tail stays 0.
    """
    q = np.asarray(q)
    n = len(q)
    n_groups = n // group_size
    out = np.zeros(n, dtype=np.float16)
    if n_groups == 0:
        return out
    sc = np.asarray([float(scales[g]) for g in range(n_groups)], dtype=np.float64).astype(np.float32)
    body = q[: n_groups * group_size].astype(np.float32).reshape(n_groups, group_size)
    with np.errstate(over="ignore", invalid="ignore"):
        out[: n_groups * group_size] = (body * sc[:, None]).astype(np.float16).reshape(-1)
    return out


def lut_indices(q) -> np.ndarray:
    """Index rule of ``src/dequant.py:87-95`` before clipping (int64)."""
    q = np.asarray(q)
    if q.dtype == np.int8:
        return q.astype(np.int64) + 8
    if np.issubdtype(q.dtype, np.signedinteger):
        qi = q.astype(np.int32)
        if np.min(q) < 0:  # empty input raises ValueError, as in the reference
            return (qi + np.int32(8)).astype(np.int64)
        return qi.astype(np.int64)
    return q.astype(np.int32).astype(np.int64)


def lut_gather(q, lut) -> np.ndarray:
    """``lut_dequantize_fp16``, ``src/dequant.py:79-112``: clipped table gather.

    1-D table: ``lut[idx]``; 2-D (rows x L): row r serves the r-th contiguous
    slice of q; 3-D (S x 8 x L) is the 2-D case with S*8 rows.  Output has q's
    shape, dtype fp16.
    """
    q = np.asarray(q)
    lut16 = np.asarray(lut)
    lut16 = lut16 if lut16.dtype == np.float16 else lut16.astype(np.float16)
    idx = np.clip(lut_indices(q), 0, lut16.shape[-1] - 1)
    if lut16.ndim == 1:
        return lut16[idx]
    if lut16.ndim in (2, 3):
        table = lut16.reshape(-1, lut16.shape[-1])
        rows = idx.reshape(table.shape[0], -1)
        return np.take_along_axis(table, rows, axis=1).reshape(q.shape)
    raise ValueError(f"Unsupported LUT shape {lut16.shape}. Must be 1D, 2D, or 3D.")


def decode_superblocks(blob, num_superblocks: int) -> np.ndarray:
    """The 144-byte decoder, ``src/dequant.py:116-147``: fp16 ``[S*256]``.

    Element e of superblock i is ``fp16(f32(nibble_e - 8) * f32(scale_{e // 32}))``
    (the f32 product is exact, so this is one round-to-nearest-even).
    """
    rec = np.asarray(blob, dtype=np.uint8).reshape(num_superblocks, SB_BYTES)
    scales = rec[:, :SB_HEADER_BYTES].copy().view("<f2").astype(np.float32)  # (S, 8)
    vals = unpack_nibbles(rec[:, SB_HEADER_BYTES:]).astype(np.float32).reshape(num_superblocks, GROUPS_PER_SB, GROUP)
    with np.errstate(over="ignore", invalid="ignore"):
        out = (vals * scales[:, :, None]).astype(np.float16)
    return out.reshape(-1)


def records_to_tiles(blob, K: int, M: int) -> np.ndarray:
    """The records of a row-major K x M stream (M % 256 == 0) in tile order:
    record (row r, 256-column tile j) moves from ``r * (M/256) + j`` to
    ``j * K + r`` (a storage order with no counterpart in the reference; the
    records themselves are unchanged)."""
    t = M // SB_ELEMS
    rec = np.asarray(blob, dtype=np.uint8).reshape(K, t, SB_BYTES)
    return np.ascontiguousarray(rec.transpose(1, 0, 2)).reshape(-1)


# Position of row 8b+i's byte inside the 8 bytes of one column pair of a
# strip-order record (rows 0-3 in the order 0, 2, 1, 3, rows 4-7 likewise):
# bytes 0 and 2 of each little-endian 32-bit word then hold two consecutive
# rows, and bytes 1 and 3 the next two.  The map is its own inverse.
STRIP_ROW_POS = np.array([0, 2, 1, 3, 4, 6, 5, 7])


def records_to_strips(blob, K: int, M: int) -> np.ndarray:
    """The quantized weights of a row-major K x M stream (K % 8 == 0,
    M % 32 == 0) in strip order: strip g = columns 32g..32g+31, strips in
    column order; inside strip g, record b (144 bytes) = [fp16 scales of rows
    8b..8b+7 for group g (16 B) | byte 8j + STRIP_ROW_POS[i] = byte j of row
    8b+i's 16 payload bytes of group g].  A storage order with no counterpart
    in the reference: every scale and payload byte of the row order appears
    once, regrouped into 8 x 32 blocks with the payload column pair by column
    pair."""
    G = M // GROUP
    rec = np.asarray(blob, dtype=np.uint8).reshape(-1, SB_BYTES)
    scales = rec[:, :SB_HEADER_BYTES].reshape(K, G, 2)  # flat group r*G + g
    payload = rec[:, SB_HEADER_BYTES:].reshape(K, G, 16)
    hdr = scales.reshape(K // 8, 8, G, 2).transpose(2, 0, 1, 3).reshape(G, K // 8, 16)
    pay = payload.reshape(K // 8, 8, G, 16).transpose(2, 0, 3, 1)  # [g, b, byte j, row i]
    pay = pay[:, :, :, STRIP_ROW_POS].reshape(G, K // 8, 128)      # position p holds row STRIP_ROW_POS[p]
    return np.ascontiguousarray(np.concatenate([hdr, pay], axis=2)).reshape(-1)


def decode_strips(strips, K: int, M: int) -> np.ndarray:
    """W[K][M] as fp16 from strip order: the records' row-major payload
    restored, then the 144-byte decoder (``src/dequant.py:116-147``) on each
    8 x 32 block."""
    G = M // GROUP
    rec = np.asarray(strips, dtype=np.uint8).reshape(G, K // 8, SB_BYTES)
    pay = rec[:, :, SB_HEADER_BYTES:].reshape(G, K // 8, 16, 8)[:, :, :, STRIP_ROW_POS]  # [g, b, byte j, row i]
    pay = pay.transpose(0, 1, 3, 2).reshape(G, K // 8, 128)
    rows = np.concatenate([rec[:, :, :SB_HEADER_BYTES], pay], axis=2).reshape(-1)
    blocks = decode_superblocks(rows, G * K // 8).reshape(G, K // 8, 8, GROUP)
    return np.ascontiguousarray(blocks.transpose(1, 2, 0, 3)).reshape(K, M)


# --------------------------------------------------------------------------
# Batched projection
# --------------------------------------------------------------------------

def gemm_ref(x, blob, K: int, M: int) -> np.ndarray:
    """``Y[N, M] = f32(X[N, K]) @ f32(deq(W)[K, M])`` (``test_batched_speed.py:39-42``
    semantics with the INT4 stream decoded first)."""
    w = decode_superblocks(blob, K * M // SB_ELEMS).astype(np.float32).reshape(K, M)
    return np.asarray(x).astype(np.float32) @ w


def gemv_stack(x, blob, K: int, M: int) -> np.ndarray:
    """N single-row products stacked (``test_batched_speed.py:31-36``)."""
    w = decode_superblocks(blob, K * M // SB_ELEMS).astype(np.float32).reshape(K, M)
    x32 = np.asarray(x).astype(np.float32)
    return np.vstack([x32[i:i + 1] @ w for i in range(x32.shape[0])])


def silu_mul(g, u) -> np.ndarray:
    """``silu(g) * u = g / (1 + exp(-g)) * u`` in float64: the SwiGLU step of
    ``antigravity-engine/src/shaders/transformer_ops.metal:216-232`` (which
    evaluates it in fp32 on fp16 inputs and rounds the result to fp16)."""
    g = np.asarray(g, dtype=np.float64)
    return g / (1.0 + np.exp(-g)) * np.asarray(u, dtype=np.float64)


def swiglu_ref(x, gate_blob, up_blob, K: int, M: int) -> np.ndarray:
    """``silu(X @ W_gate) * (X @ W_up)`` (float64) with both projections as
    :func:`gemm_ref`: the MLP front of ``transformer_engine.mm:694-713`` /
    ``transformer.py:133-134``."""
    return silu_mul(gemm_ref(x, gate_blob, K, M), gemm_ref(x, up_blob, K, M))


def footprint(num_params: int, group_size: int = GROUP, bits: int = 4) -> dict:
    """Closed forms of ``src/dequant.py:150-187``: 0.5 B/param + 2 B/group."""
    weight_bytes = num_params * (bits / 8.0)
    scale_bytes = (num_params // group_size) * 2.0
    total = weight_bytes + scale_bytes
    return {
        "num_params": num_params,
        "weight_bytes": weight_bytes,
        "scale_bytes": scale_bytes,
        "total_bytes": total,
        "total_mb": total / 1024 ** 2,
        "total_gb": total / 1024 ** 3,
        "ram_limit_gb": 4.5,
        "fits_in_ram": total / 1024 ** 3 <= 4.5,
        "bytes_per_param_effective": total / num_params,
    }


# --------------------------------------------------------------------------
# Synthetic workloads (shared by the tests and the benchmark)
# --------------------------------------------------------------------------

def synthetic_weights(K: int, M: int, std: float, seed: int, outlier_frac: float = 0.0,
                      outlier_sigma: float = 8.0) -> np.ndarray:
    """Row-major fp32 W[K][M] ~ N(0, std^2), optionally with a fraction of
    positions set to +-outlier_sigma*std (random sign)."""
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((K, M), dtype=np.float32) * np.float32(std)
    if outlier_frac > 0:
        n_out = int(round(outlier_frac * K * M))
        pos = rng.choice(K * M, size=n_out, replace=False)
        sign = rng.choice(np.array([-1.0, 1.0], dtype=np.float32), size=n_out)
        w.reshape(-1)[pos] = sign * np.float32(outlier_sigma * std)
    return w


def synthetic_activations(N: int, K: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.standard_normal((N, K), dtype=np.float32).astype(np.float16)
