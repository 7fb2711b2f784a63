"""C ABI checks that need no GPU: the library loads, exports every symbol the
header declares, and rejects bad arguments before touching HIP."""

import ctypes
import os
import re

import pytest

from moat_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "moat_int4.h")


def _declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(moat_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libmoat_int4.so is not built (run `python -m moat_amd.build_lib`)")
    return _lib.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = _declared_symbols()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def _declared_arities():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for name, args in re.findall(r"\b(moat_\w+)\s*\(([^)]*)\)\s*;", text):
        args = args.strip()
        out[name] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_bindings_match_header_arity():
    arities = _declared_arities()
    assert set(arities) == set(_lib.SIGNATURES)
    for name, n in arities.items():
        assert len(_lib.SIGNATURES[name][1]) == n, name


def test_version_and_status_strings(lib):
    assert lib.moat_int4_version() == 1
    assert lib.moat_int4_status_string(0) == b"ok"
    assert b"invalid" in lib.moat_int4_status_string(-2)
    assert b"workspace" in lib.moat_int4_status_string(-4)


FAKE = ctypes.c_void_p(0x10000)  # never dereferenced: validation fails first


@pytest.mark.parametrize("n,k,m", [(0, 256, 256), (33, 256, 256), (1, 256, 48), (1, 3, 32), (1, 0, 256), (1, 256, 16)])
def test_gemm_rejects_bad_shapes(lib, n, k, m):
    assert lib.moat_int4_gemm(FAKE, FAKE, FAKE, n, k, m, None, 0, None) == _lib.MOAT_ERR_INVALID
    assert lib.moat_int4_gemm_workspace_size(n, k, m) == -1


def test_gemm_rejects_null_and_misaligned(lib):
    assert lib.moat_int4_gemm(None, FAKE, FAKE, 1, 256, 256, None, 0, None) == _lib.MOAT_ERR_INVALID
    assert lib.moat_int4_gemm(FAKE, None, FAKE, 1, 256, 256, None, 0, None) == _lib.MOAT_ERR_INVALID
    assert lib.moat_int4_gemm(FAKE, FAKE, None, 1, 256, 256, None, 0, None) == _lib.MOAT_ERR_INVALID
    odd = ctypes.c_void_p(0x10001)
    assert lib.moat_int4_gemm(odd, FAKE, FAKE, 1, 256, 256, None, 0, None) == _lib.MOAT_ERR_INVALID
    sb_misaligned = ctypes.c_void_p(0x10008)
    assert lib.moat_int4_gemm(FAKE, sb_misaligned, FAKE, 1, 256, 256, None, 0, None) == _lib.MOAT_ERR_INVALID
    # dot2 kernel only up to N = 8; unknown algo / batch / finish values are refused
    for opt in (_lib.GemmOptions(_lib.GEMM_DOT2, 1, 0, 0),):
        assert lib.moat_int4_gemm_ex(FAKE, FAKE, FAKE, 9, 256, 256, ctypes.byref(opt), None, 0, None) == _lib.MOAT_ERR_INVALID
    for opt in (_lib.GemmOptions(7, 1, 0, 0), _lib.GemmOptions(0, 1, 6, 0), _lib.GemmOptions(0, 1, -1, 0),
                _lib.GemmOptions(0, 1, 0, 4), _lib.GemmOptions(0, 1, 0, 0, 5), _lib.GemmOptions(0, -1, 0, 0),
                _lib.GemmOptions(0, 1, 0, 0, 4, 3), _lib.GemmOptions(0, 1, 0, 0, 4, 8),
                _lib.GemmOptions(0, 1, 0, 0, 4, 1, 6), _lib.GemmOptions(0, 1, 0, 0, 4, 1, 16),
                _lib.GemmOptions(0, 1, 0, 0, 4, 1, -4)):
        assert lib.moat_int4_gemm_ex(FAKE, FAKE, FAKE, 1, 256, 256, ctypes.byref(opt), None, 0, None) == _lib.MOAT_ERR_INVALID
        assert lib.moat_int4_gemm_ex_workspace_size(1, 256, 256, ctypes.byref(opt)) == -1


def test_gemm_workspace_contract(lib):
    # a split-K plan needs a workspace; a missing or short one is refused before launch
    opt = _lib.GemmOptions(_lib.GEMM_MFMA, 8, 0, 0, _lib.FRONT_LDS)  # general kernel
    size = lib.moat_int4_gemm_ex_workspace_size(1, 2048, 5504, ctypes.byref(opt))
    assert size == 64 * 1024 + 8 * 1 * 5504 * 4  # fixed counter block + partials
    # record-stream kernel: `splits` workgroups per 256-column tile (22 tiles),
    # two partial slots of N x 256 floats per workgroup, after the counter block
    # (which every call leaves zero for the calls that share the workspace)
    rec = _lib.GemmOptions(_lib.GEMM_MFMA, 8, 0, 0, _lib.FRONT_RECORDS, 1)
    assert lib.moat_int4_gemm_ex_workspace_size(4, 2048, 5504, ctypes.byref(rec)) == 64 * 1024 + 2 * 22 * 8 * 4 * 256 * 4
    # four tiles per workgroup: 6 tile groups, partial slots of 4 tiles
    rec4 = _lib.GemmOptions(_lib.GEMM_MFMA, 8, 0, 0, _lib.FRONT_RECORDS, 4)
    assert lib.moat_int4_gemm_ex_workspace_size(4, 2048, 5504, ctypes.byref(rec4)) == 64 * 1024 + 2 * 6 * 8 * 4 * 4 * 256 * 4
    st = lib.moat_int4_gemm_ex(FAKE, FAKE, FAKE, 4, 2048, 5504, ctypes.byref(rec), None, 0, None)
    assert st == _lib.MOAT_ERR_WORKSPACE
    # 8 waves per workgroup: the same workgroups and partial slots
    rec8 = _lib.GemmOptions(_lib.GEMM_MFMA, 8, 0, 0, _lib.FRONT_RECORDS, 1, 8)
    assert lib.moat_int4_gemm_ex_workspace_size(4, 2048, 5504, ctypes.byref(rec8)) == 64 * 1024 + 2 * 22 * 8 * 4 * 256 * 4
    assert lib.moat_int4_gemm_ex_workspace_size(32, 2048, 5504, ctypes.byref(rec8)) == 64 * 1024 + 2 * 22 * 8 * 32 * 256 * 4
    # one workgroup per tile: nothing shared, no workspace
    one_rec = _lib.GemmOptions(_lib.GEMM_MFMA, 1, 0, 0, _lib.FRONT_RECORDS, 2)
    assert lib.moat_int4_gemm_ex_workspace_size(4, 2048, 5504, ctypes.byref(one_rec)) == 0
    st = lib.moat_int4_gemm_ex(FAKE, FAKE, FAKE, 1, 2048, 5504, ctypes.byref(opt), None, 0, None)
    assert st == _lib.MOAT_ERR_WORKSPACE
    st = lib.moat_int4_gemm_ex(FAKE, FAKE, FAKE, 1, 2048, 5504, ctypes.byref(opt), FAKE, size - 1, None)
    assert st == _lib.MOAT_ERR_WORKSPACE
    one = _lib.GemmOptions(_lib.GEMM_MFMA, 1, 0, 0, _lib.FRONT_LDS)
    assert lib.moat_int4_gemm_ex_workspace_size(4, 2048, 2048, ctypes.byref(one)) == 0
    assert lib.moat_int4_gemm_ex_workspace_size(4, 2048, 2048, None) >= 0
    # automatic plans at the benchmark shapes: splits shrink as N grows
    sizes = [lib.moat_int4_gemm_workspace_size(n, 2048, 5504) for n in (1, 2, 4, 8, 16, 32)]
    assert all(s >= 0 for s in sizes)


def test_other_entry_points_validate(lib):
    I = _lib.MOAT_ERR_INVALID
    assert lib.moat_int4_dequant(FAKE, -1, FAKE, None) == I
    assert lib.moat_int4_dequant(None, 4, FAKE, None) == I
    assert lib.moat_int4_dequant(ctypes.c_void_p(0x10004), 4, FAKE, None) == I
    assert lib.moat_int4_dequant(FAKE, 0, FAKE, None) == _lib.MOAT_OK  # nothing to do, no launch
    assert lib.moat_int4_quantize(FAKE, 0, 33, 32, 0, FAKE, FAKE, None) == I
    assert lib.moat_int4_quantize(FAKE, 9, 32, 32, 0, FAKE, FAKE, None) == I
    assert lib.moat_int4_quantize(FAKE, 0, 32, 32, 5, FAKE, FAKE, None) == I
    assert lib.moat_int4_quantize(FAKE, 0, 32, 0, 0, FAKE, FAKE, None) == I
    assert lib.moat_int4_quantize_pack(FAKE, 0, 255, 0, FAKE, None) == I
    assert lib.moat_int4_pack_superblocks(None, FAKE, 1, FAKE, None) == I
    assert lib.moat_int4_pack_nibbles(FAKE, 3, FAKE, None) == I
    assert lib.moat_int4_unpack_nibbles(None, 3, FAKE, None) == I
    assert lib.moat_int4_group_dequant(FAKE, 0, FAKE, 0, 1, 32, 1, FAKE, FAKE, None) == I  # table mode needs ints
    assert lib.moat_int4_group_dequant(FAKE, 2, FAKE, 2, 1, 32, 0, FAKE, None, None) == I  # int8 scales
    assert lib.moat_int4_group_dequant(FAKE, 2, FAKE, 1, 1, 32, 1, FAKE, None, None) == I  # no flag in table mode
    assert lib.moat_int4_lut_gather(FAKE, 10, 0, FAKE, 3, 16, FAKE, None) == I  # 10 % 3
    assert lib.moat_int4_lut_gather(FAKE, 10, 3, FAKE, 1, 16, FAKE, None) == I
    assert lib.moat_int4_any_negative(FAKE, 4, None, None) == I
    assert lib.moat_int4_to_f16(FAKE, 2, 4, FAKE, None) == I
    assert lib.moat_int4_workspace_clear(None, 16, None) == I


def test_fused_entry_points_validate(lib):
    I = _lib.MOAT_ERR_INVALID
    P2 = ctypes.c_void_p * 2
    sbs, ys = P2(FAKE.value, FAKE.value), P2(FAKE.value, FAKE.value)
    # count 1..4, the record-stream kernel's shapes only (m % 128, k % 32)
    assert lib.moat_int4_gemm_multi_workspace_size(0, 1, 2048, 2048) == -1
    assert lib.moat_int4_gemm_multi_workspace_size(5, 1, 2048, 2048) == -1
    assert lib.moat_int4_gemm_multi_workspace_size(2, 1, 2048, 2016) == -1  # m % 128
    assert lib.moat_int4_gemm_multi_workspace_size(2, 1, 40, 2048) == -1    # k % 32
    assert lib.moat_int4_gemm_multi_workspace_size(2, 33, 2048, 2048) == -1
    assert lib.moat_int4_gemm_multi_workspace_size(3, 1, 2048, 2048) >= 0
    assert lib.moat_int4_gemm_swiglu_workspace_size(1, 2048, 2016) == -1
    assert lib.moat_int4_gemm_swiglu_workspace_size(16, 2048, 5632) >= 0
    assert lib.moat_int4_gemm_multi(FAKE, sbs, ys, 2, 1, 2048, 2016, None, 0, None) == I
    assert lib.moat_int4_gemm_multi(None, sbs, ys, 2, 1, 2048, 2048, None, 0, None) == I
    assert lib.moat_int4_gemm_multi(FAKE, None, ys, 2, 1, 2048, 2048, None, 0, None) == I
    assert lib.moat_int4_gemm_multi(FAKE, P2(FAKE.value, None), ys, 2, 1, 2048, 2048, None, 0, None) == I
    assert lib.moat_int4_gemm_multi(FAKE, P2(FAKE.value, 0x10008), ys, 2, 1, 2048, 2048, None, 0, None) == I
    assert lib.moat_int4_gemm_multi(ctypes.c_void_p(0x10008), sbs, ys, 2, 1, 2048, 2048, None, 0, None) == I  # x 16 B
    assert lib.moat_int4_gemm_swiglu(FAKE, FAKE, FAKE, ctypes.c_void_p(0x10004), 1, 2048, 2048, None, 0, None) == I
    assert lib.moat_int4_gemm_swiglu(FAKE, None, FAKE, FAKE, 1, 2048, 2048, None, 0, None) == I
    # the SwiGLU step alone: m % 4, ld >= 2m and ld % 4, 16 B gate/up rows, 8 B h
    assert lib.moat_int4_swiglu_f32(FAKE, 1, 6, 12, FAKE, None) == I
    assert lib.moat_int4_swiglu_f32(FAKE, 1, 8, 12, FAKE, None) == I
    assert lib.moat_int4_swiglu_f32(FAKE, 1, 8, 18, FAKE, None) == I
    assert lib.moat_int4_swiglu_f32(ctypes.c_void_p(0x10008), 1, 8, 16, FAKE, None) == I
    assert lib.moat_int4_swiglu_f32(FAKE, 1, 8, 16, ctypes.c_void_p(0x10004), None) == I
    assert lib.moat_int4_swiglu_f32(FAKE, -1, 8, 16, FAKE, None) == I
    assert lib.moat_int4_swiglu_f32(None, 0, 8, 16, None, None) == _lib.MOAT_OK
    # a shared-tile plan needs the workspace: refused before any launch
    size = lib.moat_int4_gemm_swiglu_workspace_size(16, 2048, 5632)
    if size > 0:
        assert lib.moat_int4_gemm_swiglu(FAKE, FAKE, FAKE, FAKE, 16, 2048, 5632, None, 0, None) == _lib.MOAT_ERR_WORKSPACE
    size = lib.moat_int4_gemm_multi_workspace_size(3, 1, 2048, 2048)
    if size > 0:
        P3 = ctypes.c_void_p * 3
        assert lib.moat_int4_gemm_multi(FAKE, P3(*[FAKE.value] * 3), P3(*[FAKE.value] * 3), 3, 1, 2048, 2048,
                                        FAKE, size - 1, None) == _lib.MOAT_ERR_WORKSPACE


def test_sampling_entry_points_validate(lib):
    I, W = _lib.MOAT_ERR_INVALID, _lib.MOAT_ERR_WORKSPACE
    F = ctypes.c_float
    step = F(10.0 / 32767)
    # workspace sizes: n rows of v logits, -1 outside the limits
    ws = lib.moat_sample_workspace_size(2, 1000)
    sws = lib.moat_lut_softmax_workspace_size(2, 1000)
    assert 2 * 2 * 1000 < ws and 0 < sws < ws
    assert lib.moat_sample_workspace_size(0, 1000) == 0 and lib.moat_lut_softmax_workspace_size(0, 5) == 0
    assert lib.moat_sample_workspace_size(2, 0) == -1 and lib.moat_sample_workspace_size(-1, 10) == -1
    assert lib.moat_sample_workspace_size(1, 524288) > 2 * 524288
    assert lib.moat_sample_workspace_size(1, 524289) == -1 and lib.moat_lut_softmax_workspace_size(1, 524289) == -1
    assert lib.moat_sample_workspace_size((1 << 21) + 1, 10) == -1
    big = lib.moat_sample_workspace_size(1 << 21, 1 << 19)  # 64-bit byte counts
    assert big > 2 * (1 << 21) * (1 << 19)

    # moat_lut_softmax(x, dtype, n, v, lut, lut_size, step, probs, workspace, bytes, stream)
    def sm(x, dtype, n, v, lut_size, st, probs, w=FAKE, nbytes=sws):
        return lib.moat_lut_softmax(x, dtype, n, v, FAKE, lut_size, st, probs, w, nbytes, None)
    assert sm(FAKE, 0, 2, 1000, 32768, step, None) == I  # no output
    assert sm(FAKE, 2, 2, 1000, 32768, step, FAKE) == I  # int8 logits
    assert sm(FAKE, 0, 2, 524289, 32768, step, FAKE) == I  # row above 64 chunks of 8192
    assert sm(FAKE, 0, 2, 0, 32768, step, FAKE) == I
    assert sm(FAKE, 0, 2, 1000, (1 << 24) + 1, step, FAKE) == I  # table index past float32's integers
    assert sm(FAKE, 0, 2, 1000, 1, step, FAKE) == I
    assert sm(FAKE, 0, 2, 1000, 32768, F(0.0), FAKE) == I
    assert sm(FAKE, 0, 2, 1000, 32768, F(float("inf")), FAKE) == I
    assert sm(ctypes.c_void_p(0x10002), 0, 2, 1000, 32768, step, FAKE) == I
    assert sm(ctypes.c_void_p(0x10004), 3, 2, 1000, 32768, step, FAKE) == I  # f64: 8 B
    assert sm(FAKE, 0, 2, 1000, 32768, step, FAKE, w=None) == W
    assert sm(FAKE, 0, 2, 1000, 32768, step, FAKE, nbytes=sws - 1) == W
    assert sm(FAKE, 0, 2, 1000, 32768, step, FAKE, w=ctypes.c_void_p(0x10080)) == W  # 256-byte alignment
    assert sm(FAKE, 0, 0, 1000, 32768, step, None, w=None, nbytes=0) == _lib.MOAT_OK  # no rows

    # moat_sample_tokens(x, dtype, n, v, T, top_k, seed, lut, lut_size, step, tokens, logprobs, workspace,
    #                    bytes, stream)
    def st(dtype, n, v, t, k, tok=FAKE, lp=FAKE, w=FAKE, nbytes=ws):
        return lib.moat_sample_tokens(FAKE, dtype, n, v, t, k, 1, FAKE, 32768, step, tok, lp, w, nbytes, None)
    assert st(0, 2, 1000, 0.7, 0) == I
    assert st(0, 2, 1000, 0.7, 65) == I
    assert st(0, 2, 1000, float("nan"), 50) == I
    assert st(0, 2, 1000, 0.7, 50, tok=None) == I
    assert st(0, 2, 1000, 0.7, 50, lp=ctypes.c_void_p(0x10002)) == I
    assert st(1, 2, 600000, 0.0, 50) == I
    assert st(0, 2, 1000, 0.7, 50, nbytes=sws) == W  # the softmax's size lacks the table values
    assert st(0, 2, 1000, 0.0, 50, w=None) == W
    assert lib.moat_lut_lookup(FAKE, -1, FAKE, 32768, step, FAKE, None) == I
    assert lib.moat_lut_lookup(FAKE, 4, FAKE, 1, step, FAKE, None) == I
    assert lib.moat_lut_lookup(ctypes.c_void_p(0x10002), 4, FAKE, 32768, step, FAKE, None) == I
    assert lib.moat_lut_lookup(FAKE, 0, FAKE, 32768, step, FAKE, None) == _lib.MOAT_OK


def test_sampling_python_checks_first():
    import numpy as np
    from moat_amd import sampling
    with pytest.raises(ValueError):
        sampling.ExponentialLUT(size=1)
    with pytest.raises(ValueError):
        sampling.ExponentialLUT(range_max=-1.0)
    with pytest.raises(ValueError):
        sampling.TokenSampler(top_k=65)
    with pytest.raises(ValueError):
        sampling.TokenSampler(exp_lut_size=(1 << 24) + 1)
    lut = sampling.ExponentialLUT()
    assert lut.memory_bytes == 65536 and lut.lut.dtype == np.float16 and lut.size == 32768


def test_fused_python_shapes_checked_first():
    import numpy as np
    from moat_amd import dequant
    with pytest.raises(ValueError):
        dequant.batched_int4_matmul_multi(np.zeros((1, 40), np.float16), [np.zeros(15 * 144, np.uint8)], 40, 96)
    with pytest.raises(ValueError):
        dequant.batched_int4_matmul_multi(np.zeros((1, 64), np.float16), [], 64, 128)
    with pytest.raises(ValueError):
        dequant.int4_swiglu(np.zeros((1, 64), np.float16), None, None, 64, 96)


def test_product_refuses_to_run_without_gpu():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    import numpy as np
    from moat_amd import dequant
    with pytest.raises(RuntimeError, match="GPU"):
        dequant.unpack_superblock_weights(np.zeros(144, dtype=np.uint8), 1)


def test_tile_order_entry_points_validate(lib):
    I = _lib.MOAT_ERR_INVALID
    opt = _lib.GemmOptions(0, 0, 0, 0, 0, 0, 0)
    # moat_int4_records_to_tiles(sb, k, m, tiles, stream)
    assert lib.moat_int4_records_to_tiles(FAKE, 64, 384, ctypes.c_void_p(0x90000000), None) == I  # m % 256
    assert lib.moat_int4_records_to_tiles(FAKE, 0, 512, ctypes.c_void_p(0x90000000), None) == I
    assert lib.moat_int4_records_to_tiles(FAKE, 64, 512, FAKE, None) == I  # overlapping copies
    assert lib.moat_int4_records_to_tiles(ctypes.c_void_p(0x10008), 64, 512, ctypes.c_void_p(0x90000000),
                                          None) == I  # 16-byte alignment
    assert lib.moat_int4_records_to_tiles(None, 64, 512, ctypes.c_void_p(0x90000000), None) == I
    # moat_int4_gemm_tiles(x, tiles, y, n, k, m, options, workspace, bytes, stream): the record-stream kernel only
    big = ctypes.c_void_p(0x90000000)
    assert lib.moat_int4_gemm_tiles(FAKE, FAKE, big, 1, 2048, 5504, ctypes.byref(opt), big, 1 << 30, None) == I
    assert lib.moat_int4_gemm_tiles(FAKE, FAKE, big, 1, 48, 512, ctypes.byref(opt), big, 1 << 30, None) == I
    assert lib.moat_int4_gemm_tiles(ctypes.c_void_p(0x10008), FAKE, big, 1, 2048, 2048, ctypes.byref(opt), big,
                                    1 << 30, None) == I  # X rows need 16-byte loads
    dot2 = _lib.GemmOptions(_lib.GEMM_DOT2, 0, 0, 0, 0, 0, 0)
    assert lib.moat_int4_gemm_tiles(FAKE, FAKE, big, 1, 2048, 2048, ctypes.byref(dot2), big, 1 << 30, None) == I
    assert lib.moat_int4_gemm_tiles(FAKE, FAKE, big, 33, 2048, 2048, ctypes.byref(opt), big, 1 << 30, None) == I


def test_strip_swiglu_entry_points_validate(lib):
    I = _lib.MOAT_ERR_INVALID
    opt = _lib.GemmOptions(0, 0, 0, 0, 0, 0, 0)
    big = ctypes.c_void_p(0x90000000)
    # moat_int4_gemm_strips_swiglu(x, gate_up_strips, h, n, k, m, options, stream)
    f = lib.moat_int4_gemm_strips_swiglu
    assert f(FAKE, FAKE, big, 0, 2048, 5632, ctypes.byref(opt), None) == I     # n < 1
    assert f(FAKE, FAKE, big, 33, 2048, 5632, ctypes.byref(opt), None) == I    # n > 32
    assert f(FAKE, FAKE, big, 1, 2016, 5632, ctypes.byref(opt), None) == I     # k < 2048
    assert f(FAKE, FAKE, big, 1, 2056, 5632, ctypes.byref(opt), None) == I     # k % 32
    assert f(FAKE, FAKE, big, 1, 2048, 5616, ctypes.byref(opt), None) == I     # m % 32
    assert f(FAKE, FAKE, big, 1, 2048, 0, ctypes.byref(opt), None) == I
    assert f(FAKE, FAKE, big, 1, 2048, 1 << 30, ctypes.byref(opt), None) == I  # 2m columns too many
    assert f(ctypes.c_void_p(0x10008), FAKE, big, 1, 2048, 5632, ctypes.byref(opt), None) == I  # x 16 B
    assert f(FAKE, ctypes.c_void_p(0x10008), big, 1, 2048, 5632, ctypes.byref(opt), None) == I  # strips 16 B
    assert f(FAKE, FAKE, ctypes.c_void_p(0x90000004), 1, 2048, 5632, ctypes.byref(opt), None) == I  # h 8 B
    assert f(None, FAKE, big, 1, 2048, 5632, ctypes.byref(opt), None) == I
    assert f(FAKE, None, big, 1, 2048, 5632, ctypes.byref(opt), None) == I
    assert f(FAKE, FAKE, None, 1, 2048, 5632, ctypes.byref(opt), None) == I
    bad = _lib.GemmOptions(0, -1, 0, 0, 0, 0, 0)
    assert f(FAKE, FAKE, big, 1, 2048, 5632, ctypes.byref(bad), None) == I     # negative splits
    # moat_int4_interleave_strips(gate, up, k, m, out, stream)
    g = lib.moat_int4_interleave_strips
    assert g(FAKE, ctypes.c_void_p(0x20000000), 2044, 64, big, None) == I      # k % 8
    assert g(FAKE, ctypes.c_void_p(0x20000000), 2048, 48, big, None) == I      # m % 32
    assert g(None, ctypes.c_void_p(0x20000000), 2048, 64, big, None) == I
    assert g(FAKE, ctypes.c_void_p(0x20000000), 2048, 64, None, None) == I
    assert g(FAKE, ctypes.c_void_p(0x20000000), 2048, 64, FAKE, None) == I     # output overlaps gate
    assert g(FAKE, ctypes.c_void_p(0x20000000), 2048, 64, ctypes.c_void_p(0x20000000 - 4096), None) == I  # and up


def test_strip_swiglu_python_checks_first():
    import numpy as np
    from moat_amd import dequant
    with pytest.raises(ValueError):
        dequant.int4_swiglu_strips(np.zeros((1, 1024), np.float16), None, 1024, 64)
    with pytest.raises(ValueError):
        dequant.interleave_strips(None, None, 2048, 40)


def test_tile_order_python_checks_first():
    import numpy as np
    from moat_amd import dequant
    with pytest.raises(ValueError):
        dequant.records_to_tiles(np.zeros(21 * 144, np.uint8), 1, 5376 - 128)


def test_gemm_unaligned_x_is_validated_against_its_own_plan(lib):
    """x only 2-byte aligned on a record-stream shape: the call plans the
    general kernel (the record-stream kernel reads X 16 bytes at a time) and
    checks the workspace against that plan; the size query covers both."""
    odd_x = ctypes.c_void_p(0x10002)
    for n in (1, 8):
        general = _lib.GemmOptions(0, 0, 0, 0, _lib.FRONT_LDS)
        g_size = lib.moat_int4_gemm_ex_workspace_size(n, 2048, 5504, ctypes.byref(general))
        a_size = lib.moat_int4_gemm_workspace_size(n, 2048, 5504)
        assert g_size > 0 and a_size >= g_size
        st = lib.moat_int4_gemm(odd_x, FAKE, FAKE, n, 2048, 5504, FAKE, g_size - 1, None)
        assert st == _lib.MOAT_ERR_WORKSPACE
        # the same explicit record-stream request also falls back to the general plan
        rec = _lib.GemmOptions(0, 0, 0, 0, _lib.FRONT_RECORDS)
        st = lib.moat_int4_gemm_ex(odd_x, FAKE, FAKE, n, 2048, 5504, ctypes.byref(rec), FAKE, g_size - 1, None)
        assert st == _lib.MOAT_ERR_WORKSPACE
    # tile order has no general kernel: refused outright
    assert lib.moat_int4_gemm_tiles(odd_x, FAKE, FAKE, 1, 2048, 8192, None, FAKE, 1 << 30, None) == _lib.MOAT_ERR_INVALID


def test_workspace_status_rejects_bad_arguments(lib):
    st = ctypes.c_int32(0)
    assert lib.moat_int4_workspace_status(None, 1 << 20, ctypes.byref(st), None) == _lib.MOAT_ERR_INVALID
    assert lib.moat_int4_workspace_status(FAKE, 255, ctypes.byref(st), None) == _lib.MOAT_ERR_INVALID
    assert lib.moat_int4_workspace_status(FAKE, 1 << 20, None, None) == _lib.MOAT_ERR_INVALID


def test_gemm_noalloc_validates_before_any_hip_call(lib):
    assert lib.moat_int4_gemm_noalloc(FAKE, FAKE, FAKE, 0, 256, 256, None) == _lib.MOAT_ERR_INVALID
    assert lib.moat_int4_gemm_noalloc(None, FAKE, FAKE, 1, 256, 256, None) == _lib.MOAT_ERR_INVALID
    assert lib.moat_int4_gemm_noalloc(FAKE, ctypes.c_void_p(0x10008), FAKE, 1, 256, 256, None) == _lib.MOAT_ERR_INVALID
    # 32 rows over 128 tile groups: 256 workgroups with 32 KB of partials
    # each, more than the 16 MB scratch: refused with its own status
    size = lib.moat_int4_gemm_ex_workspace_size(32, 8192, 32768, ctypes.byref(_lib.GemmOptions(0, 0, 0, 3)))
    assert size > 16 << 20
    st = lib.moat_int4_gemm_noalloc(FAKE, FAKE, FAKE, 32, 8192, 32768, None)
    assert st == _lib.MOAT_ERR_TOO_LARGE
    assert b"16 MB" in lib.moat_int4_status_string(st)


def test_dense_entry_points_validate(lib):
    I, W = _lib.MOAT_ERR_INVALID, _lib.MOAT_ERR_WORKSPACE
    big = ctypes.c_void_p(0x90000000)
    sz = lib.moat_dense_gemm_workspace_size
    assert sz(0, 2048, 2048, 0) == -1                       # n < 1
    assert sz(1, 2044, 2048, 0) == -1                       # k % 8
    assert sz(1, 2048, 2052, 0) == -1                       # m % 8
    assert sz(1, 2048, 2048, -1) == -1                      # negative splits
    assert sz(1, 2048, 2048, 1025) == -1                    # too many splits
    assert sz(1, 2048, 2048, 1) == 0                        # one split: no workspace
    assert sz(1, 2048, 2048, 0) > 0                         # 32 blocks split over 8: counters + sums
    assert sz(32, 2048, 2048, 0) == 16384 + 32 * 8 * 4 * 2 * 4096  # counter area, then the sums
    assert sz(1, 2048, 256 * 4097, 2) == 0                  # more blocks than counter words: one split
    assert sz(17, 2048, 2048, 0) == sz(33, 2048, 2048, 0)   # 32 rows a launch
    # moat_dense_gemm(x, w, y, n, k, m, splits, workspace, workspace_bytes, stream)
    f = lib.moat_dense_gemm
    assert f(FAKE, ctypes.c_void_p(0x20000000), big, 0, 2048, 2048, 1, None, 0, None) == I
    assert f(FAKE, ctypes.c_void_p(0x20000000), big, 1, 2044, 2048, 1, None, 0, None) == I
    assert f(FAKE, ctypes.c_void_p(0x20000000), big, 1, 2048, 2052, 1, None, 0, None) == I
    assert f(ctypes.c_void_p(0x10008), ctypes.c_void_p(0x20000000), big, 1, 2048, 2048, 1, None, 0, None) == I
    assert f(FAKE, ctypes.c_void_p(0x20000008), big, 1, 2048, 2048, 1, None, 0, None) == I   # w 16 B
    assert f(FAKE, ctypes.c_void_p(0x20000000), ctypes.c_void_p(0x90000001), 1, 2048, 2048, 1, None, 0, None) == I
    assert f(None, ctypes.c_void_p(0x20000000), big, 1, 2048, 2048, 1, None, 0, None) == I
    assert f(FAKE, None, big, 1, 2048, 2048, 1, None, 0, None) == I
    assert f(FAKE, ctypes.c_void_p(0x20000000), None, 1, 2048, 2048, 1, None, 0, None) == I
    # the output overlaps w
    assert f(FAKE, ctypes.c_void_p(0x20000000), ctypes.c_void_p(0x20001000), 1, 2048, 2048, 1, None, 0, None) == I
    # split plans need a workspace of the reported size
    need = sz(1, 2048, 2048, 0)
    assert f(FAKE, ctypes.c_void_p(0x20000000), big, 1, 2048, 2048, 0, None, 0, None) == W
    assert f(FAKE, ctypes.c_void_p(0x20000000), big, 1, 2048, 2048, 0, ctypes.c_void_p(0x70000000), need - 1,
             None) == W
    assert f(FAKE, ctypes.c_void_p(0x20000000), big, 1, 2048, 2048, 0, ctypes.c_void_p(0x70000008), need,
             None) == W
