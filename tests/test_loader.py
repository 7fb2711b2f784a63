"""Quantize-on-load (``moat_amd/loader.py``): the record file and the
safetensors reader on the CPU; the GPU loader against the oracle (surface B's
fp16-scale quantizer on the fp16-rounded, zero-padded tensor, then the
144-byte records), bit for bit."""

import os

import numpy as np
import pytest
import torch

from oracle import superblock_oracle as O


def _oracle_layer(w):
    """model_loader.py:66-80 with the oracle: fp16 cast, zero pad to 256,
    surface-B quantize, 144-byte records."""
    flat = np.asarray(w).reshape(-1).astype(np.float16)
    rem = flat.size % 256
    if rem:
        flat = np.pad(flat, (0, 256 - rem))
    q, s = O.quantize_b(flat)
    return q.reshape(-1), s, O.serialize_superblocks(q, s).reshape(-1, 144), flat


def test_record_file_round_trip(tmp_path):
    import struct
    from moat_amd.loader import RECORD_FILE_MAGIC_V1, load_superblocks, save_superblocks
    w = O.synthetic_weights(64, 96, 0.02, 5)
    blob = O.quantize_pack_a(w).reshape(-1, 144)
    path = os.path.join(tmp_path, "layer.i4r")
    save_superblocks(path, blob, (64, 96))
    got, shape = load_superblocks(path)
    assert shape == (64, 96) and got.shape == blob.shape and np.array_equal(got, blob)
    strips = O.records_to_strips(blob.reshape(-1), 64, 96).reshape(-1, 144)
    save_superblocks(path, strips, (64, 96), layout="strip")
    got, shape, layout = load_superblocks(path, with_layout=True)
    assert layout == "strip" and shape == (64, 96) and np.array_equal(got, strips)
    with pytest.raises(ValueError):
        save_superblocks(path, blob, (64, 96), layout="tiles")
    # a file of the first version (no layout byte) reads as row order
    with open(path, "wb") as f:
        f.write(RECORD_FILE_MAGIC_V1 + struct.pack("<I", 2) + struct.pack("<2Q", 64, 96)
                + struct.pack("<Q", blob.shape[0]) + blob.tobytes())
    got, shape, layout = load_superblocks(path, with_layout=True)
    assert layout == "row" and np.array_equal(got, blob)
    with open(path, "r+b") as f:
        f.write(b"NOTMOAT!")
    with pytest.raises(ValueError):
        load_superblocks(path)
    with pytest.raises(ValueError):
        save_superblocks(path, blob, (64, 97 * 256))  # more elements than records


def test_safetensors_reader_rounds_to_fp16(tmp_path):
    from safetensors.torch import save_file
    from moat_amd.loader import SafetensorsWeightReader
    g = torch.Generator().manual_seed(3)
    tensors = {"a.weight": torch.randn(8, 32, generator=g) * 0.02,
               "b.weight": (torch.randn(4, 64, generator=g) * 0.02).to(torch.bfloat16)}
    path = os.path.join(tmp_path, "m.safetensors")
    save_file(tensors, path)
    r = SafetensorsWeightReader(path)
    assert sorted(r.list_tensor_names()) == ["a.weight", "b.weight"]
    assert r.get_total_parameter_count() == 8 * 32 + 4 * 64
    a = r.read_tensor("a.weight")
    assert a.dtype == np.float16 and np.array_equal(a, tensors["a.weight"].numpy().astype(np.float16))
    b = r.read_tensor("b.weight")  # bf16 -> fp32 is exact, then one rounding to fp16
    assert np.array_equal(b, tensors["b.weight"].to(torch.float32).numpy().astype(np.float16))
    with pytest.raises(KeyError):
        r.read_tensor("missing")
    with pytest.raises(FileNotFoundError):
        SafetensorsWeightReader(os.path.join(tmp_path, "none.safetensors"))


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [(256, 512), (100, 30), (2048, 2048), (3072, 256)])
def test_gpu_loader_matches_oracle(shape):
    """Row order for shapes the strip GEMM cannot read, strip order (the
    oracle's regrouping of the same records) for those it can; codes and
    scales read back from the records equal the quantizer's."""
    from moat_amd.loader import ModelWeightLoader, strip_layout_ok
    print(f"case: loader shape={shape}", flush=True)
    w = O.synthetic_weights(int(np.prod(shape)), 1, 0.02, 11).reshape(shape)
    q, s, records, _ = _oracle_layer(w)
    loader = ModelWeightLoader()
    layer = loader.load_and_repack_layer("x", w)
    assert layer["original_shape"] == shape and layer["n_elements"] == int(np.prod(shape))
    assert layer["memory_bytes"] == records.shape[0] * 144
    if strip_layout_ok(shape):
        assert layer["layout"] == "strip"
        want = O.records_to_strips(records.reshape(-1), *shape).reshape(-1, 144)
        assert np.array_equal(layer["superblocks"].cpu().numpy(), want)
    else:
        assert layer["layout"] == "row"
        assert np.array_equal(layer["superblocks"].cpu().numpy(), records)
    assert np.array_equal(loader.row_records("x").cpu().numpy(), records)
    assert np.array_equal(layer["q_weights"], q) and np.array_equal(layer["scales"].view(np.uint16), s.view(np.uint16))
    deq = loader.dequantize_layer("x")  # numpy in, numpy out
    assert isinstance(deq, np.ndarray)
    want = O.decode_superblocks(records, records.shape[0])[: int(np.prod(shape))].reshape(shape)
    assert deq.shape == shape and np.array_equal(deq.view(np.uint16), want.view(np.uint16))
    assert loader.total_loaded_bytes == records.shape[0] * 144


@pytest.mark.gpu
def test_gpu_loader_layout_choice_and_strip_round_trip():
    """layout='row' keeps row order for a strip-eligible shape; layout='strip'
    on a shape only the conversion accepts; the strip -> row kernel inverts
    the row -> strip kernel; a bad layout is a ValueError."""
    from moat_amd.dequant import records_to_strips, strips_to_records
    from moat_amd.loader import ModelWeightLoader
    print("case: loader layouts", flush=True)
    w = O.synthetic_weights(2048 * 64, 1, 0.02, 21).reshape(2048, 64)
    _, _, records, _ = _oracle_layer(w)
    row = ModelWeightLoader(layout="row").load_and_repack_layer("x", w)
    assert row["layout"] == "row" and np.array_equal(row["superblocks"].cpu().numpy(), records)
    w2 = O.synthetic_weights(64 * 96, 1, 0.02, 22).reshape(64, 96)
    _, _, rec2, _ = _oracle_layer(w2)
    loader = ModelWeightLoader()
    st = loader.load_and_repack_layer("y", w2, layout="strip")
    assert st["layout"] == "strip"
    assert np.array_equal(st["superblocks"].cpu().numpy().reshape(-1), O.records_to_strips(rec2.reshape(-1), 64, 96))
    deq = loader.dequantize_layer("y")
    want = O.decode_superblocks(rec2, rec2.shape[0]).reshape(64, 96)
    assert np.array_equal(deq.view(np.uint16), want.view(np.uint16))
    with pytest.raises(ValueError):
        loader.load_and_repack_layer("z", np.zeros((60, 96), np.float16), layout="strip")
    with pytest.raises(ValueError):
        ModelWeightLoader(layout="tiles")
    for K, M in ((8, 32), (40, 256), (2048, 5504)):
        blob = O.quantize_pack_a(O.synthetic_weights(K, M, 0.02, K + M)).reshape(-1)
        d = torch.from_numpy(blob).cuda()
        back = strips_to_records(records_to_strips(d, K, M), K, M)
        assert torch.equal(back.reshape(-1), d), (K, M)


@pytest.mark.gpu
def test_gpu_to_f16_rounds_once():
    """float64 -> fp16 in one nearest-even rounding (numpy's astype): values
    just above an fp16 midpoint whose even neighbour is below -- a float64 ->
    float32 -> float16 chain lands on the midpoint and rounds down -- plus
    float32, bfloat16 and integer inputs; and the loader packs the
    single-rounded values."""
    from moat_amd.dequant import to_f16
    from moat_amd.loader import ModelWeightLoader
    print("case: to_f16 rounding", flush=True)
    rng = np.random.default_rng(31)
    lo = (rng.integers(0, 1 << 15, 4096) & ~1).astype(np.uint16)  # even positive fp16 patterns
    lo = lo[np.isfinite(lo.view(np.float16)) & (lo.view(np.float16) != np.float16(65504))]
    a = lo.view(np.float16).astype(np.float64)
    b = (lo + 1).view(np.float16).astype(np.float64)
    mid = (a + b) / 2
    v = mid + np.abs(b - a) * 2.0 ** -40  # above the midpoint, below a float32 half-ulp of it
    want = v.astype(np.float16)  # numpy: one rounding
    assert np.array_equal(want.view(np.uint16), (lo + 1))  # the single rounding goes up
    v = np.concatenate([v, -v])  # and the same magnitudes negative
    want = v.astype(np.float16)
    got = to_f16(torch.from_numpy(v).cuda()).cpu().numpy()
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    chained = torch.from_numpy(v).to(torch.float32).to(torch.float16).numpy()
    assert not np.array_equal(chained.view(np.uint16), want.view(np.uint16))  # what the chain would give
    f32 = (rng.standard_normal(1000) * 3).astype(np.float32)
    assert np.array_equal(to_f16(torch.from_numpy(f32).cuda()).cpu().numpy(), f32.astype(np.float16))
    bf = torch.from_numpy(f32).to(torch.bfloat16)
    assert np.array_equal(to_f16(bf.cuda()).cpu().numpy(), bf.to(torch.float32).numpy().astype(np.float16))
    ints = np.arange(-3000, 3000, 7, dtype=np.int64)
    assert np.array_equal(to_f16(torch.from_numpy(ints).cuda()).cpu().numpy(), ints.astype(np.float16))
    w = np.resize(v, 256 * 8).reshape(8, 256) * 1e-3
    _, _, records, _ = _oracle_layer(w)
    layer = ModelWeightLoader().load_and_repack_layer("f64", w)
    assert np.array_equal(layer["superblocks"].cpu().numpy(), records)


@pytest.mark.gpu
def test_gpu_loader_budget_and_safetensors(tmp_path):
    from safetensors.torch import save_file
    from moat_amd.loader import ModelWeightLoader, load_superblocks, save_superblocks
    print("case: loader budget + safetensors", flush=True)
    loader = ModelWeightLoader(memory_budget_bytes=144 * 10)
    loader.load_and_repack_layer("small", np.zeros(256 * 10, np.float16))
    with pytest.raises(MemoryError):
        loader.load_and_repack_layer("over", np.zeros(256, np.float16))
    g = torch.Generator().manual_seed(4)
    tensors = {"q_proj.weight": (torch.randn(64, 256, generator=g) * 0.02).to(torch.bfloat16),
               "up_proj.weight": torch.randn(96, 128, generator=g) * 0.02}
    path = os.path.join(tmp_path, "m.safetensors")
    save_file(tensors, path)
    layers = ModelWeightLoader().load_safetensors(path)
    for name, t in tensors.items():
        _, _, records, _ = _oracle_layer(t.to(torch.float32).numpy())
        assert np.array_equal(layers[name]["superblocks"].cpu().numpy(), records), name
        rec_path = os.path.join(tmp_path, name + ".i4r")
        save_superblocks(rec_path, layers[name]["superblocks"], layers[name]["original_shape"],
                         layout=layers[name]["layout"])
        back, shape, layout = load_superblocks(rec_path, device=True, with_layout=True)
        assert shape == tuple(t.shape) and torch.equal(back, layers[name]["superblocks"])
        assert layout == layers[name]["layout"]


# ---------------------------------------------------------------------------
# GGUF files (written here with the GGUF layout: little-endian header, typed
# key/values, tensor table, data aligned to general.alignment)

def _gguf_bytes(kvs, tensors, alignment=None):
    """kvs: [(key, vtype, value)] (vtype 9 = (elem_type, [values])); tensors:
    [(name, dims, ttype, payload bytes)].  Returns the file bytes and the
    expected data offset."""
    import struct

    def s(text):
        b = text.encode()
        return struct.pack("<Q", len(b)) + b

    scalar = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}

    def val(vt, v):
        if vt in scalar:
            return struct.pack(scalar[vt], v)
        if vt == 8:
            return s(v)
        et, items = v
        return struct.pack("<I", et) + struct.pack("<Q", len(items)) + b"".join(val(et, i) for i in items)

    kvs = list(kvs)
    if alignment is not None:
        kvs.append(("general.alignment", 4, alignment))
    align = alignment or 32
    head = b"GGUF" + struct.pack("<I", 3) + struct.pack("<Q", len(tensors)) + struct.pack("<Q", len(kvs))
    for k, vt, v in kvs:
        head += s(k) + struct.pack("<I", vt) + val(vt, v)
    offsets, off = [], 0
    for _, _, _, payload in tensors:
        offsets.append(off)
        off += len(payload) + (-len(payload)) % align
    for (name, dims, tt, _), o in zip(tensors, offsets):
        head += s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<I", tt) + struct.pack("<Q", o)
    data_off = len(head) + (-len(head)) % align
    body = bytearray(head + b"\0" * (data_off - len(head)))
    for (_, _, _, payload), o in zip(tensors, offsets):
        body += b"\0" * (data_off + o - len(body)) + payload
    return bytes(body), data_off


def test_gguf_header_parse(tmp_path):
    from moat_amd.loader import ModelWeightLoader
    kvs = [("general.name", 8, "tiny"), ("u8", 0, 250), ("i8", 1, -5), ("u16", 2, 65000), ("i16", 3, -300),
           ("u32", 4, 4000000000), ("i32", 5, -7), ("f32", 6, 0.5), ("flag", 7, True), ("u64", 10, 2 ** 40),
           ("i64", 11, -2 ** 40), ("f64", 12, 0.125), ("arr", 9, (5, [1, -2, 3])), ("names", 9, (8, ["a", "bc"]))]
    w = np.arange(12, dtype=np.float32)
    blob, data_off = _gguf_bytes(kvs, [("w", [3, 4], 0, w.tobytes()), ("h", [8], 1, np.ones(8, np.float16).tobytes())],
                                 alignment=64)
    path = os.path.join(tmp_path, "m.gguf")
    open(path, "wb").write(blob)
    info = ModelWeightLoader().parse_gguf_file(path)
    md = info["metadata"]
    assert info["version"] == 3 and info["n_tensors"] == 2
    assert md["general.name"] == "tiny" and md["u8"] == 250 and md["i8"] == -5 and md["u16"] == 65000
    assert md["i16"] == -300 and md["u32"] == 4000000000 and md["i32"] == -7 and md["f32"] == 0.5
    assert md["flag"] is True and md["u64"] == 2 ** 40 and md["i64"] == -2 ** 40 and md["f64"] == 0.125
    assert md["arr"] == [1, -2, 3] and md["names"] == ["a", "bc"] and md["general.alignment"] == 64
    assert info["tensors"]["w"] == {"name": "w", "dims": [3, 4], "type": 0, "offset": 0}
    assert info["tensors"]["h"]["offset"] == 64 and info["tensors"]["h"]["type"] == 1
    assert info["tensor_data_offset"] == data_off and data_off % 64 == 0
    # default alignment 32
    blob32, off32 = _gguf_bytes([("k", 8, "v")], [("w", [4], 0, w[:4].tobytes())])
    open(path, "wb").write(blob32)
    assert ModelWeightLoader().parse_gguf_file(path)["tensor_data_offset"] == off32 and off32 % 32 == 0


def test_gguf_header_errors(tmp_path):
    from moat_amd.loader import ModelWeightLoader
    loader = ModelWeightLoader()
    path = os.path.join(tmp_path, "bad.gguf")
    with pytest.raises(FileNotFoundError):
        loader.parse_gguf_file(path)
    with pytest.raises(FileNotFoundError):
        loader.auto_load_gguf(path)
    open(path, "wb").write(b"GGML" + bytes(20))
    with pytest.raises(ValueError, match="magic"):
        loader.parse_gguf_file(path)
    blob, _ = _gguf_bytes([("k", 8, "v")], [])
    open(path, "wb").write(blob.replace(b"\x08\x00\x00\x00", b"\x0d\x00\x00\x00", 1))  # value type 13
    with pytest.raises(ValueError, match="Unknown value type: 13"):
        loader.parse_gguf_file(path)


def test_memory_estimates():
    """model_loader.py:281-318 and :378-403, with the reference tests' cases
    (test_batch_generator.py:192-199, test_model_loader.py:106-149) and the
    closed forms."""
    from moat_amd.loader import MODEL_WEIGHT_BUDGET_BYTES, MemoryBudgetValidator, estimate_model_superblock_memory
    est = estimate_model_superblock_memory(1_500_000_000)
    assert est["superblock_memory_mb"] * 2 ** 20 == 5_859_375 * 144          # 1.5e9 / 256 records exactly
    assert est["superblock_memory_gb"] <= 2.5 and est["fits_ios_4_5gb_ceiling"] and est["bits_per_weight"] == 4.5
    assert est["compression_ratio"] == 3e9 / (5_859_375 * 144) and est["fp16_memory_mb"] == 3e9 / 2 ** 20
    assert estimate_model_superblock_memory(257)["superblock_memory_mb"] * 2 ** 20 == 2 * 144  # ceil
    big = MODEL_WEIGHT_BUDGET_BYTES // 144 * 256 + 256
    assert not estimate_model_superblock_memory(big)["fits_ios_4_5gb_ceiling"]
    assert MODEL_WEIGHT_BUDGET_BYTES == 2500 * 2 ** 20
    gb = MemoryBudgetValidator.calculate_weight_memory_gb(1_540_000_000)
    assert gb == 6_015_625 * 144 / 2 ** 30 and 0.7 < gb <= 2.5
    rep = MemoryBudgetValidator.validate_memory_budget(1_540_000_000, num_traces=8, seq_len=2048,
                                                       runtime_overhead_gb=0.5)
    assert rep["total_app_memory_gb"] == gb + 8 * 2048 * 16 * 64 * 4 / 2 ** 30 + 0.5
    assert rep["weight_budget_passed"] and rep["total_app_budget_passed"] and rep["is_valid"]
    with pytest.raises(ValueError):
        MemoryBudgetValidator.validate_memory_budget(num_params=6_000_000_000)
    with pytest.raises(ValueError):  # weights fit, the KV cache does not
        MemoryBudgetValidator.validate_memory_budget(1_000_000_000, num_traces=512)


@pytest.mark.gpu
def test_gpu_auto_load_gguf(tmp_path):
    """F32 rounded to fp16, F16 as stored, and the int8 fallback over all 256
    byte values (fp16 of int8 / 7, computed here as numpy computes it), each
    packed bit-exactly like the oracle; a short tensor is zero-filled."""
    from moat_amd.loader import ModelWeightLoader
    print("case: auto_load_gguf", flush=True)
    rng = np.random.default_rng(12)
    f32 = (rng.standard_normal((16, 48)) * 0.05).astype(np.float32)
    f32[0, :4] = [1000.0, -1e-8, 0.0, 65504.0]  # fp16 max, and a value that rounds to -0
    f16 = (rng.standard_normal(320) * 0.1).astype(np.float16)
    i8 = np.arange(-128, 128, dtype=np.int8)
    short = np.tile(i8, 2)[:300]
    tensors = [("a", [16, 48], 0, f32.tobytes()), ("b", [320], 1, f16.tobytes()), ("c", [256], 24, i8.tobytes()),
               ("d", [2, 256], 30, short.tobytes())]  # last tensor: 300 of 512 bytes in the file
    blob, _ = _gguf_bytes([("general.name", 8, "t")], tensors)
    path = os.path.join(tmp_path, "m.gguf")
    open(path, "wb").write(blob)
    loader = ModelWeightLoader()
    hdr = loader.parse_gguf_file(path)
    open(path, "wb").write(blob[: hdr["tensor_data_offset"] + hdr["tensors"]["d"]["offset"] + 300])
    info = loader.auto_load_gguf(path)
    assert sorted(info["tensors"]) == ["a", "b", "c", "d"]
    d = np.concatenate([short, np.zeros(212, np.int8)])
    want = {"a": f32.astype(np.float16), "b": f16, "c": i8.astype(np.float16) / 7.0,
            "d": (d.astype(np.float16) / 7.0).reshape(2, 256)}
    for name, w in want.items():
        assert w.dtype == np.float16
        _, _, records, _ = _oracle_layer(w)
        layer = loader.layers[name]
        assert layer["original_shape"] == w.shape, name
        assert np.array_equal(layer["superblocks"].cpu().numpy(), records), name


@pytest.mark.gpu
def test_gpu_repacker_and_layer_bookkeeping():
    """SuperBlockRepacker / QuantizedSuperBlockTensor (test_model_loader.py:70-99
    cases, plus the oracle's bits), host-in/host-out dequantize_layer, and
    unload_layer / clear returning bytes to the budget."""
    from moat_amd.loader import ModelWeightLoader, SuperBlockRepacker
    print("case: repacker + bookkeeping", flush=True)
    matrix = np.random.default_rng(42).standard_normal((256, 256)).astype(np.float16)
    qt = SuperBlockRepacker.repack_matrix(matrix, group_size=32, groups_per_superblock=8)
    assert qt.validate_structure() and qt.bytes_per_superblock == 144
    assert len(qt.superblocks) == 256 and qt.memory_bytes == 256 * 144
    _, _, records, _ = _oracle_layer(matrix)
    assert np.array_equal(qt.superblocks.cpu().numpy(), records)
    original = np.random.default_rng(99).standard_normal((128, 256)).astype(np.float16)
    deq = SuperBlockRepacker.repack_matrix(original).dequantize()
    assert isinstance(deq, np.ndarray) and deq.shape == original.shape and deq.dtype == np.float16
    _, _, rec2, _ = _oracle_layer(original)
    assert np.array_equal(deq.reshape(-1).view(np.uint16), O.decode_superblocks(rec2, rec2.shape[0]).view(np.uint16))
    assert float(np.mean(np.abs(original.astype(np.float32) - deq.astype(np.float32)))) < 0.2
    with pytest.raises(ValueError):
        SuperBlockRepacker.repack_matrix(original, group_size=64)

    loader = ModelWeightLoader()
    w = np.random.default_rng(5).standard_normal((256, 256)).astype(np.float16)
    loader.load_and_repack_layer("layer_0", w)
    out = loader.dequantize_layer("layer_0")
    assert isinstance(out, np.ndarray) and out.shape == (256, 256) and out.dtype == np.float16
    loader.load_and_repack_layer("layer_1", torch.from_numpy(w).cuda())
    assert loader.dequantize_layer("layer_1").is_cuda
    assert loader.total_loaded_bytes == 2 * 256 * 144
    loader.unload_layer("layer_0")
    loader.unload_layer("missing")
    assert loader.total_loaded_bytes == 256 * 144 and list(loader.layers) == ["layer_1"]
    loader.clear()
    assert loader.total_loaded_bytes == 0 and not loader.layers
