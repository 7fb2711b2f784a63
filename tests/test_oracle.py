"""Pins the CPU oracle (CPU only).

Every oracle function is checked against something that does not share its
code: the reference tests' known answers (cited), Python's own binary16
packer, exact rational arithmetic, float64 accumulation, or closed forms.
"""

import numpy as np
import pytest

from ieee_exact import f16_bits, f16_value, quantize_group_exact
from oracle import superblock_oracle as O


def _group_bytes(nibbles):
    """16 payload bytes of one group from 32 nibble codes, by Python ints."""
    out = []
    for j in range(16):
        out.append(((int(nibbles[2 * j + 1]) & 0xF) << 4) | (int(nibbles[2 * j]) & 0xF))
    return out


# ---------------------------------------------------------------- dequant

def test_exhaustive_scale_by_nibble_table():
    """All 65,536 fp16 scale patterns x 16 nibbles against struct's binary16 rounding."""
    n_groups = 1 << 16
    nib = np.tile(np.arange(16, dtype=np.uint8), 2)  # element e has nibble e % 16
    payload = np.array(_group_bytes(nib), dtype=np.uint8)
    blob = np.zeros((n_groups // 8, 144), dtype=np.uint8)
    scale_bits = np.arange(n_groups, dtype=np.uint32).astype(np.uint16)
    blob[:, :16] = scale_bits.reshape(-1, 8).astype("<u2").view(np.uint8).reshape(-1, 16)
    blob[:, 16:] = np.tile(payload, 8)[None, :]
    got = O.decode_superblocks(blob, n_groups // 8).view(np.uint16).reshape(n_groups, 32)

    expected = np.empty((n_groups, 16), dtype=np.uint16)
    nan_mask = np.zeros((n_groups, 16), dtype=bool)
    for sb in range(n_groups):
        s = f16_value(sb)
        if s != s:
            nan_mask[sb, :] = True
            continue
        for n in range(16):
            v = (n - 8) * s
            if v != v:  # 0 * inf
                nan_mask[sb, n] = True
            else:
                expected[sb, n] = f16_bits(v)
    got16 = got[:, :16]
    assert np.array_equal(got16, got[:, 16:])
    got_nan = (got16 & 0x7C00 == 0x7C00) & (got16 & 0x03FF != 0)
    assert np.array_equal(got_nan, nan_mask)
    assert np.array_equal(got16[~nan_mask], expected[~nan_mask])


def test_kernel_kat_byte_0x7f():
    """``antigravity-engine/tests/test_metal_kernels.cpp:69-90``: scales 0.5, byte 0x7F ->
    element 0 (low nibble 15) = +3.5, element 1 (high nibble 7) = -0.5."""
    blob = np.zeros((1, 144), dtype=np.uint8)
    blob[0, :16] = np.full(8, 0.5, dtype="<f2").view(np.uint8)
    blob[0, 16:] = 0x7F
    out = O.decode_superblocks(blob, 1)
    assert out.dtype == np.float16 and out.shape == (256,)
    assert np.all(out[0::2] == np.float16(3.5))
    assert np.all(out[1::2] == np.float16(-0.5))


@pytest.mark.parametrize("K,M", [(256, 256), (2048, 2048)])
def test_runner_stream_closed_form(K, M):
    """``antigravity-engine/src/metal_runner.cpp:84-98``: scales 0x3800, bytes 0x77,
    X = 1 -> every weight is -0.5 and every output is -0.5*K."""
    S = K * M // 256
    blob = np.zeros((S, 144), dtype=np.uint8)
    blob[:, :16] = np.full(8, 0x3800, dtype="<u2").view(np.uint8)
    blob[:, 16:] = 0x77
    assert np.all(O.decode_superblocks(blob, S) == np.float16(-0.5))
    x = np.ones((8, K), dtype=np.float16)
    y = O.gemm_ref(x, blob, K, M)
    assert y.shape == (8, M) and np.all(y == np.float32(-0.5 * K))


def test_decoder_two_routes_agree():
    """Decoder (``src/dequant.py:116-147``) == unpack + per-group table gather
    (``antigravity-engine/src/dequant.py:135-220``) == arithmetic route."""
    rng = np.random.default_rng(5)
    q = rng.integers(-8, 8, size=256 * 12).astype(np.int8)
    scales = (rng.random(8 * 12) * 2 - 1).astype(np.float16)
    blob = O.serialize_superblocks(q, scales)
    dec = O.decode_superblocks(blob, 12)
    arith = O.group_dequant(q, scales)
    assert np.array_equal(dec.view(np.uint16), arith.view(np.uint16))
    luts = np.stack([O.dequant_lut(s) for s in scales])
    gathered = O.lut_gather(q.reshape(96, 32), luts).reshape(-1)
    assert np.array_equal(dec.view(np.uint16), gathered.view(np.uint16))
    exact = np.array([f16_bits(float(q[i]) * float(scales[i // 32])) for i in range(q.size)], dtype=np.uint16)
    assert np.array_equal(dec.view(np.uint16), exact)


# ---------------------------------------------------------------- packing

def test_pack_matches_python_int_bits():
    rng = np.random.default_rng(11)
    q = rng.integers(-8, 8, size=512).astype(np.int8)
    packed = O.pack_nibbles(q)
    expect = []
    for j in range(256):
        lo = (int(q[2 * j]) + 8) & 0xF
        hi = (int(q[2 * j + 1]) + 8) & 0xF
        expect.append(lo | (hi << 4))
    assert packed.tolist() == expect
    assert np.array_equal(O.unpack_nibbles(packed), q)


def test_boundary_values_survive_packing():
    """``antigravity-engine/tests/test_quantization.py:176-191``."""
    q = np.zeros(256, dtype=np.int8)
    q[:4] = [-8, 7, 0, -1]
    recs = O.superblock_records(q, np.ones(8, dtype=np.float16))
    back = O.unpack_nibbles(recs[0]["packed_nibbles"])
    assert back[:4].tolist() == [-8, 7, 0, -1]


def test_record_sizes_and_errors():
    """``antigravity-engine/tests/test_quantization.py:142-215``."""
    q = np.random.default_rng(0).integers(-8, 8, size=512).astype(np.int8)
    recs = O.superblock_records(q, np.ones(16, dtype=np.float16))
    assert len(recs) == 2
    for r in recs:
        assert r["packed_nibbles"].dtype == np.uint8 and r["packed_nibbles"].nbytes == 128
        assert r["scales"].dtype == np.float16 and r["scales"].nbytes == 16
    with pytest.raises(ValueError):
        O.superblock_records(q[:200], np.ones(7, dtype=np.float16))
    blob = O.serialize_superblocks(q, np.ones(16, dtype=np.float16))
    assert blob.shape == (2, 144)


@pytest.mark.parametrize("shape,n_sb", [((256, 256), 256), ((512, 512), 1024)])
def test_superblock_counts(shape, n_sb):
    """``antigravity-engine/tests/test_model_loader.py:70-83`` and
    ``test_batch_generator.py:159-171``: 256 SB / 36,864 B and 1024 SB / 147,456 B."""
    w = np.random.default_rng(1).standard_normal(shape).astype(np.float16)
    q, s = O.quantize_b(w.reshape(-1))
    blob = O.serialize_superblocks(q, s)
    assert blob.shape[0] == n_sb and blob.nbytes == n_sb * 144


# ---------------------------------------------------------------- quantizers

def _check_quantizer_exact(w, fp16_first):
    fn = O.quantize_b if fp16_first else O.quantize_a
    q, s = fn(w.reshape(-1))
    wf = w.astype(np.float32).reshape(-1, 32)
    for g in range(wf.shape[0]):
        qs, sbits = quantize_group_exact([float(v) for v in wf[g]], fp16_first)
        assert q.reshape(-1, 32)[g].tolist() == qs, g
        assert int(s.view(np.uint16)[g]) == sbits, g


@pytest.mark.parametrize("fp16_first", [False, True])
def test_quantizers_against_exact_rationals(fp16_first):
    rng = np.random.default_rng(3)
    w32 = rng.standard_normal(64 * 32).astype(np.float32) * np.float32(0.02)
    _check_quantizer_exact(w32, fp16_first)
    w16 = (rng.standard_normal(32 * 32) * 3).astype(np.float16)
    _check_quantizer_exact(w16, fp16_first)


@pytest.mark.parametrize("fp16_first", [False, True])
def test_quantizers_on_constructed_ties(fp16_first):
    """w = (k + 1/2) * s with a power-of-two s: every quotient is a tie."""
    rows = []
    for s in (0.25, 2.0 ** -10, 8.0):
        ties = [(k + 0.5) * s for k in range(-7, 7)]  # -6.5s .. 6.5s
        g = np.array(ties + [7 * s, -7 * s] + ties + [0.0, 7 * s], dtype=np.float32)
        rows.append(g)
    w = np.concatenate(rows)
    _check_quantizer_exact(w, fp16_first)
    q, _ = (O.quantize_b if fp16_first else O.quantize_a)(w)
    # half-to-even: -6.5 -> -6, -0.5 -> 0, 0.5 -> 0, 1.5 -> 2, 2.5 -> 2
    first = q[:32]
    assert first[0] == -6 and first[6] == 0 and first[7] == 0 and first[8] == 2 and first[9] == 2


def test_quantizers_differ_where_scale_rounding_matters():
    """A divides by the float32 scale, B by the fp16-rounded one; find a group
    where that changes q, so a mix-up of the two is caught."""
    rng = np.random.default_rng(17)
    w = rng.standard_normal(4096 * 32).astype(np.float32)
    qa, sa = O.quantize_a(w)
    qb, sb = O.quantize_b(w)
    assert np.array_equal(sa.view(np.uint16), sb.view(np.uint16))
    assert np.any(qa != qb)


def test_quantizer_known_answers():
    """Reference test answers: ``antigravity-engine/tests/test_quantization.py:69-111, 394-422``,
    ``tests/e2e/test_tier1_features.py:69-78``, ``tests/e2e/test_tier2_boundaries.py:51-57``."""
    z = np.zeros(32, dtype=np.float16)
    w = z.copy(); w[0] = 3.5
    assert O.quantize_b(w)[0][0] == 7
    w = z.copy(); w[0] = -3.5
    assert O.quantize_b(w)[0][0] == -7
    q, s = O.quantize_b(np.zeros(256, dtype=np.float16))
    assert np.all(q == 0) and np.all(s == np.float16(1.0))
    q, _ = O.quantize_b(np.full(256, 1.0, dtype=np.float16))
    assert np.all(q == 7)
    w = np.zeros(256, dtype=np.float16); w[0::2] = 10.0; w[1::2] = -10.0
    q, _ = O.quantize_b(w)
    assert np.all(q[0::2] == 7) and np.all(q[1::2] == -7)
    w = z.copy(); w[0] = 14.0; w[1] = -14.0
    _, s = O.quantize_a(w)
    assert s[0] == np.float16(2.0)
    q, s = O.quantize_a(np.full(32, 3.5, dtype=np.float16))
    assert s[0] == np.float16(0.5) and np.all(q == 7)
    with pytest.raises(ValueError):
        O.quantize_b(np.zeros(33, dtype=np.float16))
    with pytest.raises(ValueError):
        O.quantize_b(np.zeros((4, 32), dtype=np.float16))
    with pytest.raises(AssertionError):
        O.quantize_a(np.zeros(33, dtype=np.float16))
    q, _ = O.quantize_a(np.zeros((4, 64), dtype=np.float32))
    assert q.shape == (4, 64) and q.dtype == np.int8


def test_reconstruction_within_half_step():
    """``antigravity-engine/tests/test_quantization.py:311-332``."""
    np.random.seed(42)
    w = np.random.randn(1024).astype(np.float16)
    q, s = O.quantize_b(w)
    rec = O.group_dequant(q, s)
    err = np.abs(w.astype(np.float32) - rec.astype(np.float32)).reshape(-1, 32).max(axis=1)
    assert np.all(err <= s.astype(np.float32) / 2 + 1e-3)


# ---------------------------------------------------------------- tables

def test_table_known_answers():
    """``tests/test_quantization.py:100-112``, ``antigravity-engine/tests/test_quantization.py:221-305``,
    ``tests/e2e/test_tier1_features.py:56-65``, ``tests/e2e/test_tier2_boundaries.py:59-70``."""
    lut = np.arange(10, 26).astype(np.float16)
    out = O.lut_gather(np.array([-8, -7, 0, 7], dtype=np.int8), lut)
    assert out.tolist() == [10.0, 11.0, 18.0, 25.0]
    lut5 = np.array([-4.0, -2.0, 0.0, 2.0, 4.0], dtype=np.float16)
    idx = np.array([0, 2, 4, 1, 3], dtype=np.int32)
    assert np.array_equal(O.lut_gather(idx, lut5), lut5[idx])
    lin = np.linspace(-8.0, 7.0, 16, dtype=np.float16)
    out = O.lut_gather(np.clip(np.array([-10, 20, 5, 0], dtype=np.int32), 0, 15), lin)
    assert out[0] == lin[0] and out[1] == lin[-1]
    # signed non-int8 input with a negative entry shifts by 8 and clips
    out = O.lut_gather(np.array([-10, 20, 5, 0], dtype=np.int32), lin)
    assert out.tolist() == [lin[0], lin[15], lin[13], lin[8]]
    t = O.dequant_lut(np.float16(0.5))
    assert t.dtype == np.float16 and len(t) == 16 and t[15] == np.float16(3.5) and t[0] == np.float16(-4.0)
    assert O.dequant_lut(np.float16(1.0))[8] == 0
    q = np.full(32, 7, dtype=np.int8)
    assert np.all(O.group_dequant(q, np.array([0.5], dtype=np.float16)) == np.float16(3.5))
    q = np.full(32, -8, dtype=np.int8)
    assert np.all(O.group_dequant(q, np.array([0.5], dtype=np.float16)) == np.float16(-4.0))
    with pytest.raises(ValueError):
        O.lut_gather(q, np.zeros((2, 2, 2, 2), dtype=np.float16))


def test_group_dequant_float32_scale_double_rounding():
    """A float32 (not fp16) scale goes through f32 multiply then fp16 rounding."""
    s = np.float32(0.1)
    out = O.group_dequant(np.arange(-8, 8).astype(np.int8).repeat(2), np.array([s], dtype=np.float32), 32)
    for i, v in enumerate(out[:32]):
        k = -8 + i // 2
        prod32 = np.float32(k) * s  # reference does the product in float32
        assert v.view(np.uint16) == f16_bits(float(prod32))


# ---------------------------------------------------------------- GEMM

def test_gemm_against_float64_accumulation():
    rng = np.random.default_rng(7)
    K, M, N = 512, 96, 5
    w = rng.standard_normal((K, M)).astype(np.float32) * np.float32(0.02)
    blob = O.quantize_pack_a(w)
    x = rng.standard_normal((N, K)).astype(np.float16)
    y = O.gemm_ref(x, blob, K, M)
    # weights decoded independently of the oracle's decoder
    q, s = O.quantize_a(w.reshape(-1))
    wd = np.array([f16_value(f16_bits(float(q[i]) * float(s[i // 32]))) for i in range(K * M)]).reshape(K, M)
    y64 = x.astype(np.float64) @ wd
    rms = np.sqrt(np.mean(y64 ** 2))
    assert np.max(np.abs(y - y64)) <= 1e-5 * rms
    ys = O.gemv_stack(x, blob, K, M)
    assert np.max(np.abs(ys - y)) <= 1e-5 * rms


def test_serialize_layout_positions():
    """Scale g of superblock i at bytes [2g, 2g+2); element e in byte 16 + e//2."""
    q = np.zeros(512, dtype=np.int8)
    q[256 + 37] = 5  # superblock 1, element 37: byte 16 + 18, high nibble
    s = np.arange(16).astype(np.float16)
    blob = O.serialize_superblocks(q, s)
    assert blob[1, 16 + 18] == (((5 + 8) & 0xF) << 4) | 8
    assert blob[1, 2 * 3:2 * 3 + 2].view("<f2")[0] == np.float16(11)


# ---------------------------------------------------------------- footprint

def test_footprint_known_answers():
    """``tests/test_quantization.py:142-155``."""
    f = O.footprint(1_500_000_000)
    assert f["fits_in_ram"] and f["total_gb"] < 1.0
    assert abs(f["bytes_per_param_effective"] - 0.5625) < 1e-3
    assert O.footprint(3_000_000_000)["total_gb"] < 2.0
    assert O.footprint(7_000_000_000)["total_gb"] < 4.0
    assert O.footprint(256)["total_bytes"] == 144.0


def test_silu_mul_closed_forms():
    """silu(0) = 0; silu(1) = 1 / (1 + 1/e); silu(-1) = -1 / (1 + e); large |g|:
    silu(g) -> g (g > 0) and -> 0 (g < 0); the product scales with u."""
    import math
    g = np.array([0.0, 1.0, -1.0, 40.0, -40.0, 1.0])
    u = np.array([5.0, 2.0, 1.0, 0.5, 3.0, -3.0])
    got = O.silu_mul(g, u)
    want = [0.0, 2.0 / (1.0 + math.exp(-1.0)), -1.0 / (1.0 + math.e), 20.0, 0.0, -3.0 / (1.0 + math.exp(-1.0))]
    assert np.allclose(got, want, rtol=1e-15, atol=1e-15)
    assert abs(got[4]) < 1e-15


def test_records_to_tiles_is_the_tile_permutation():
    """Tile order (row r of 256-column tile j at record j*K + r), pinned by a
    plain index loop and by decoding: tile j's records hold columns
    256j .. 256j+255 of W, row by row."""
    for K, M in ((3, 512), (32, 768), (64, 256)):
        w = O.synthetic_weights(K, M, 0.05, 3 + K + M)
        blob = O.quantize_pack_a(w).reshape(-1)
        tiles = O.records_to_tiles(blob, K, M)
        assert tiles.shape == blob.shape and tiles.dtype == np.uint8
        t = M // 256
        for r in range(K):
            for j in range(t):
                src = (r * t + j) * 144
                dst = (j * K + r) * 144
                assert np.array_equal(tiles[dst:dst + 144], blob[src:src + 144])
        wdq = O.decode_superblocks(blob, K * M // 256).reshape(K, M)
        dec = O.decode_superblocks(tiles, K * M // 256).reshape(t, K, 256)
        for j in range(t):
            assert np.array_equal(dec[j].view(np.uint16), wdq[:, 256 * j:256 * (j + 1)].view(np.uint16))


def test_records_to_strips_is_the_strip_regrouping():
    """Strip order (record (g, b) = scales of rows 8b..8b+7 of group g, then
    byte 8j + pos(i) = byte j of row 8b+i's payload, pos = 0 2 1 3 4 6 5 7),
    pinned by a plain byte loop
    over the row-order format's own offsets (group f = r * M/32 + g: scale at
    byte 144*(f//8) + 2*(f%8), payload at 144*(f//8) + 16 + 16*(f%8)) and by
    decoding the strips back to W."""
    for K, M in ((8, 32), (16, 96), (40, 256), (64, 160)):
        w = O.synthetic_weights(K, M, 0.05, 11 + K + M)
        blob = O.quantize_pack_a(w).reshape(-1)
        strips = O.records_to_strips(blob, K, M)
        assert strips.shape == blob.shape and strips.dtype == np.uint8
        G = M // 32
        for g in range(G):
            for b in range(K // 8):
                dst = (g * (K // 8) + b) * 144
                for i in range(8):
                    f = (8 * b + i) * G + g
                    sc = 144 * (f // 8) + 2 * (f % 8)
                    pay = 144 * (f // 8) + 16 + 16 * (f % 8)
                    assert np.array_equal(strips[dst + 2 * i:dst + 2 * i + 2], blob[sc:sc + 2])
                    pos = (0, 2, 1, 3, 4, 6, 5, 7)[i]
                    for j in range(16):
                        assert strips[dst + 16 + 8 * j + pos] == blob[pay + j]
        wdq = O.decode_superblocks(blob, K * M // 256).reshape(K, M)
        assert np.array_equal(O.decode_strips(strips, K, M).view(np.uint16), wdq.view(np.uint16))
