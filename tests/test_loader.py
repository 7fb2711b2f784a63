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
    from moat_amd.loader import load_superblocks, save_superblocks
    w = O.synthetic_weights(64, 96, 0.02, 5)
    blob = O.quantize_pack_a(w).reshape(-1, 144)
    path = os.path.join(tmp_path, "layer.i4r")
    save_superblocks(path, blob, (64, 96))
    got, shape = load_superblocks(path)
    assert shape == (64, 96) and got.shape == blob.shape and np.array_equal(got, blob)
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
@pytest.mark.parametrize("shape", [(256, 512), (100, 30), (2048, 2048)])
def test_gpu_loader_matches_oracle(shape):
    from moat_amd.loader import ModelWeightLoader
    print(f"case: loader shape={shape}", flush=True)
    w = O.synthetic_weights(int(np.prod(shape)), 1, 0.02, 11).reshape(shape)
    q, s, records, _ = _oracle_layer(w)
    loader = ModelWeightLoader()
    layer = loader.load_and_repack_layer("x", w)
    assert layer["original_shape"] == shape and layer["n_elements"] == int(np.prod(shape))
    assert layer["memory_bytes"] == records.shape[0] * 144
    assert np.array_equal(layer["superblocks"].cpu().numpy(), records)
    assert np.array_equal(layer["q_weights"], q) and np.array_equal(layer["scales"].view(np.uint16), s.view(np.uint16))
    deq = loader.dequantize_layer("x").cpu().numpy()
    want = O.decode_superblocks(records, records.shape[0])[: int(np.prod(shape))].reshape(shape)
    assert deq.shape == shape and np.array_equal(deq.view(np.uint16), want.view(np.uint16))
    assert loader.total_loaded_bytes == records.shape[0] * 144


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
        save_superblocks(rec_path, layers[name]["superblocks"], layers[name]["original_shape"])
        back, shape = load_superblocks(rec_path, device=True)
        assert shape == tuple(t.shape) and torch.equal(back, layers[name]["superblocks"])
