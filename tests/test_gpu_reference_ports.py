"""The reference's unit tests for the two dequant surfaces, run against the
MI355X implementation (GPU).  Each test names the reference test it ports;
assertions are the reference's own."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


# ---------------------------------------------------------------- surface A: tests/test_quantization.py

def test_constants_match_engine_config():
    """tests/test_quantization.py:17-35 (quantization block of config/engine_config.yaml)."""
    from moat_amd import dequant as A
    assert A.GROUP_SIZE == 32 and A.SUPERBLOCK_ELEMS == 256 and A.SUPERBLOCK_BYTES == 144
    assert 4 * A.SUPERBLOCK_ELEMS // 8 + 2 * (A.SUPERBLOCK_ELEMS // A.GROUP_SIZE) == A.SUPERBLOCK_BYTES


def test_quantize_fp16_to_int4_correctness():
    """tests/test_quantization.py:38-49."""
    from moat_amd.dequant import quantize_fp16_to_int4
    np.random.seed(42)
    w = np.random.uniform(-2.0, 2.0, size=1024).astype(np.float16)
    q, s = quantize_fp16_to_int4(w, group_size=32)
    assert q.shape == (1024,) and s.shape == (32,)
    assert q.dtype == np.int8 and s.dtype == np.float16
    assert np.min(q) >= -8 and np.max(q) <= 7


def test_quantize_and_repack_superblock():
    """tests/test_quantization.py:52-64."""
    from moat_amd.dequant import quantize_fp16_to_int4, repack_weights_to_superblock
    np.random.seed(42)
    w = np.random.uniform(-2.0, 2.0, size=1024).astype(np.float16)
    q, _ = quantize_fp16_to_int4(w, group_size=32)
    rep = repack_weights_to_superblock(q, group_size=32)
    assert rep.shape == (4, 8, 32)
    assert rep.flags["C_CONTIGUOUS"]
    assert rep.ctypes.data % 128 == 0
    np.testing.assert_array_equal(rep.reshape(-1), q)


def test_repack_alignment_assertion():
    """tests/test_quantization.py:67-70; message pinned by tests/e2e/test_tier2_boundaries.py:26-30."""
    from moat_amd.dequant import repack_weights_to_superblock
    with pytest.raises(AssertionError, match="Weight array length must be a multiple of 256"):
        repack_weights_to_superblock(np.zeros(200, dtype=np.int8), group_size=32)


def test_ensure_aligned_array_utility():
    """tests/test_quantization.py:73-79."""
    from moat_amd.dequant import ensure_aligned_array
    arr = np.random.randint(-8, 8, size=256, dtype=np.int8)
    out = ensure_aligned_array(arr, alignment=128)
    assert out.ctypes.data % 128 == 0 and out.flags["C_CONTIGUOUS"]
    np.testing.assert_array_equal(out, arr)
    odd = np.zeros(300, dtype=np.int8)[1:257]
    assert ensure_aligned_array(odd).ctypes.data % 128 == 0


def test_lut_dequantization_correctness_and_precision():
    """tests/test_quantization.py:82-97."""
    from moat_amd.dequant import lut_dequantize_fp16, quantize_fp16_to_int4
    np.random.seed(42)
    w = np.random.uniform(-1.0, 1.0, size=256).astype(np.float16)
    q, s = quantize_fp16_to_int4(w, group_size=32)
    lut_2d = s[:, None] * np.arange(-8, 8, dtype=np.float32)[None, :]
    dq = lut_dequantize_fp16(q.reshape(8, 32), lut_2d)
    assert dq.shape == (8, 32) and dq.dtype == np.float16
    assert np.max(np.abs(w.astype(np.float32) - dq.astype(np.float32).flatten())) < 0.2


def test_lut_dequantization_signed_index_offset_mapping():
    """tests/test_quantization.py:100-112."""
    from moat_amd.dequant import lut_dequantize_fp16
    q = np.array([-8, -7, 0, 7], dtype=np.int8)
    lut = np.arange(10.0, 26.0, dtype=np.float16)
    np.testing.assert_array_equal(lut_dequantize_fp16(q, lut), np.array([10.0, 11.0, 18.0, 25.0], np.float16))


def test_memory_bounds_verification():
    """tests/test_quantization.py:142-172."""
    from moat_amd.dequant import calculate_memory_footprint
    f = calculate_memory_footprint(1_500_000_000)
    assert f["fits_in_ram"] and f["total_gb"] < 1.0
    assert pytest.approx(f["bytes_per_param_effective"], 0.001) == 0.5625
    assert calculate_memory_footprint(3_000_000_000)["total_gb"] < 2.0
    assert calculate_memory_footprint(7_000_000_000)["total_gb"] < 4.0
    kv = 8 * 2048 * 28 * 2 * 128 * 2 * 2
    assert (f["total_bytes"] + kv + 200 * 1024 * 1024) / 1024 ** 3 < 4.5


# ---------------------------------------------------------------- surface B: antigravity-engine/tests/test_quantization.py

def test_output_range_dtype_shape_scale():
    """antigravity-engine/tests/test_quantization.py:36-67, 112-121."""
    from moat_amd.engine_dequant import quantize_weights_int4
    np.random.seed(42)
    q, s = quantize_weights_int4(np.random.randn(1024).astype(np.float16), group_size=32)
    assert np.all(q >= -8) and np.all(q <= 7) and q.dtype == np.int8 and s.dtype == np.float16
    q, s = quantize_weights_int4(np.random.randn(512).astype(np.float16))
    assert len(q) == 512 and len(s) == 16
    np.random.seed(7)
    _, s = quantize_weights_int4(np.random.randn(256).astype(np.float16))
    assert np.all(s > 0)
    np.random.seed(99)
    q, s = quantize_weights_int4(np.random.randn(65536).astype(np.float16))
    assert len(q) == 65536 and len(s) == 2048 and np.all(q >= -8) and np.all(q <= 7)


def test_zero_max_and_errors():
    """antigravity-engine/tests/test_quantization.py:69-110."""
    from moat_amd.engine_dequant import quantize_weights_int4
    q, _ = quantize_weights_int4(np.zeros(32, dtype=np.float16))
    np.testing.assert_array_equal(q, np.zeros(32, dtype=np.int8))
    w = np.zeros(32, dtype=np.float16); w[0] = 1.0; w[1] = 0.1
    q, _ = quantize_weights_int4(w)
    assert abs(int(q[0])) > abs(int(q[1]))
    w = np.zeros(32, dtype=np.float16); w[0] = 3.5
    assert quantize_weights_int4(w)[0][0] == 7
    w = np.zeros(32, dtype=np.float16); w[0] = -3.5
    assert quantize_weights_int4(w)[0][0] == -7
    with pytest.raises(ValueError):
        quantize_weights_int4(np.random.randn(33).astype(np.float16))
    with pytest.raises(ValueError):
        quantize_weights_int4(np.random.randn(4, 32).astype(np.float16))


def test_superblock_repacking_suite():
    """antigravity-engine/tests/test_quantization.py:127-215."""
    from moat_amd.engine_dequant import quantize_weights_int4, repack_to_superblocks, unpack_superblock
    np.random.seed(42)
    q, s = quantize_weights_int4(np.random.randn(256).astype(np.float16))
    sbs = repack_to_superblocks(q, s)
    assert len(sbs) == 1
    np.testing.assert_array_equal(unpack_superblock(sbs[0]), q)
    q = np.random.randint(-8, 8, size=256, dtype=np.int8)
    sb = repack_to_superblocks(q, np.ones(8, dtype=np.float16))[0]
    assert len(sb["packed_nibbles"]) == 128 and sb["packed_nibbles"].dtype == np.uint8
    sb = repack_to_superblocks(q, np.random.rand(8).astype(np.float16))[0]
    assert len(sb["scales"]) == 8 and sb["scales"].dtype == np.float16
    q2 = np.random.randint(-8, 8, size=512, dtype=np.int8)
    sbs = repack_to_superblocks(q2, np.random.rand(16).astype(np.float16))
    assert len(sbs) == 2
    for i, b in enumerate(sbs):
        np.testing.assert_array_equal(unpack_superblock(b), q2[i * 256:(i + 1) * 256])
    qb = np.zeros(256, dtype=np.int8); qb[:4] = [-8, 7, 0, -1]
    u = unpack_superblock(repack_to_superblocks(qb, np.ones(8, dtype=np.float16))[0])
    assert (u[0], u[1], u[2], u[3]) == (-8, 7, 0, -1)
    with pytest.raises(ValueError):
        repack_to_superblocks(np.random.randint(-8, 8, size=200, dtype=np.int8), np.ones(7, dtype=np.float16))
    sb = repack_to_superblocks(q, np.ones(8, dtype=np.float16))[0]
    assert sb["scales"].nbytes == 16 and sb["packed_nibbles"].nbytes == 128
    assert sb["scales"].nbytes + sb["packed_nibbles"].nbytes == 144


def test_lut_dequantization_suite():
    """antigravity-engine/tests/test_quantization.py:221-305."""
    from moat_amd.engine_dequant import (arithmetic_dequantize, build_dequant_lut, lut_dequantize,
                                         quantize_weights_int4)
    lut = build_dequant_lut(np.float16(0.5))
    assert len(lut) == 16 and lut.dtype == np.float16
    assert abs(float(build_dequant_lut(np.float16(1.0))[8])) < 1e-5
    lut = build_dequant_lut(np.float16(0.75))
    for k in range(1, 8):
        assert abs(float(lut[8 + k]) + float(lut[8 - k])) < 1e-3
    for seed, n in ((42, 1024), (99, 65536)):
        np.random.seed(seed)
        q, s = quantize_weights_int4(np.random.randn(n).astype(np.float16), group_size=32)
        np.testing.assert_array_equal(lut_dequantize(q, s, group_size=32), arithmetic_dequantize(q, s, group_size=32))
    np.testing.assert_array_equal(lut_dequantize(np.zeros(32, np.int8), np.array([1.0], np.float16)),
                                  np.zeros(32, np.float16))
    r = lut_dequantize(np.full(32, 7, np.int8), np.array([0.5], np.float16))
    assert np.all(np.abs(r.astype(np.float32) - 3.5) < 1e-3)
    r = lut_dequantize(np.full(32, -8, np.int8), np.array([0.5], np.float16))
    assert np.all(np.abs(r.astype(np.float32) + 4.0) < 1e-3)


def test_roundtrip_suite():
    """antigravity-engine/tests/test_quantization.py:311-388."""
    from moat_amd.engine_dequant import lut_dequantize, quantize_weights_int4, repack_to_superblocks, unpack_superblock
    np.random.seed(42)
    w = np.random.randn(1024).astype(np.float16)
    q, s = quantize_weights_int4(w)
    rec = lut_dequantize(q, s)
    for g in range(32):
        err = np.abs(w[g * 32:(g + 1) * 32].astype(np.float32) - rec[g * 32:(g + 1) * 32].astype(np.float32))
        assert float(np.max(err)) <= float(s[g]) / 2.0 + 1e-3
    np.random.seed(7)
    w = np.random.randn(256).astype(np.float16)
    q, s = quantize_weights_int4(w)
    rec = lut_dequantize(q, s)
    mask = np.ones(256, dtype=bool)
    for g in range(8):
        mask[g * 32:(g + 1) * 32] &= np.abs(w[g * 32:(g + 1) * 32].astype(np.float32)) > float(s[g]) / 2.0 + 1e-3
    assert np.sum(np.sign(w[mask].astype(np.float32)) != np.sign(rec[mask].astype(np.float32))) == 0
    np.random.seed(42)
    w = np.random.randn(256).astype(np.float16)
    q, s = quantize_weights_int4(w)
    direct = lut_dequantize(q, s)
    sb = repack_to_superblocks(q, s)[0]
    np.testing.assert_array_equal(lut_dequantize(unpack_superblock(sb), sb["scales"]), direct)


def test_edge_case_suite():
    """antigravity-engine/tests/test_quantization.py:394-455."""
    from moat_amd.engine_dequant import lut_dequantize, quantize_weights_int4
    q, s = quantize_weights_int4(np.zeros(256, dtype=np.float16))
    np.testing.assert_array_equal(q, np.zeros(256, np.int8))
    np.testing.assert_array_equal(lut_dequantize(q, s), np.zeros(256, np.float16))
    q, _ = quantize_weights_int4(np.full(256, 1.0, dtype=np.float16))
    assert np.all(q == q[0]) and q[0] == 7
    w = np.zeros(256, dtype=np.float16); w[0::2] = 10.0; w[1::2] = -10.0
    q, _ = quantize_weights_int4(w)
    assert np.all(q[0::2] == 7) and np.all(q[1::2] == -7)
    q, s = quantize_weights_int4(np.full(256, 1e-4, dtype=np.float16))
    r = lut_dequantize(q, s)
    assert not np.any(np.isnan(r)) and not np.any(np.isinf(r))
    for seed in range(10):
        np.random.seed(seed)
        q, s = quantize_weights_int4(np.random.randn(1024).astype(np.float16))
        r = lut_dequantize(q, s)
        assert not np.any(np.isnan(s)) and not np.any(np.isnan(r))
        np.random.seed(seed)
        q, s = quantize_weights_int4((np.random.randn(1024) * 100).astype(np.float16))
        assert not np.any(np.isinf(lut_dequantize(q, s)))


def test_superblock_consumers():
    """antigravity-engine/tests/test_model_loader.py:67-99, test_batch_generator.py:156-171,
    test_fuzz_extreme_inputs.py:61-75: counts, bytes and MAE of the load-time pipeline
    (flatten -> pad to 256 -> quantize -> repack, model_loader.py:66-80)."""
    from moat_amd.engine_dequant import lut_dequantize, quantize_weights_int4, repack_to_superblocks, unpack_superblock
    for shape, n_sb in (((256, 256), 256), ((512, 512), 1024)):
        w = np.random.randn(*shape).astype(np.float16).reshape(-1)
        q, s = quantize_weights_int4(w)
        sbs = repack_to_superblocks(q, s)
        assert len(sbs) == n_sb and len(sbs) * 144 == n_sb * 144
    np.random.seed(99)
    orig = np.random.randn(128, 256).astype(np.float16)
    q, s = quantize_weights_int4(orig.reshape(-1))
    deq = lut_dequantize(q, s).reshape(orig.shape)
    assert float(np.mean(np.abs(orig.astype(np.float32) - deq.astype(np.float32)))) < 0.2
    for _ in range(100):
        w = (np.random.randn(256 * np.random.randint(1, 10)) * 5.0).astype(np.float16)
        q, s = quantize_weights_int4(w)
        sbs = repack_to_superblocks(q, s)
        assert len(sbs) == w.shape[0] // 256 and len(sbs[0]["packed_nibbles"]) == 128
        assert len(unpack_superblock(sbs[0])) == 256
