"""Quantize-on-load: weights from a checkpoint file (or arrays) to the
144-byte INT4 records on the GPU, and a record file for the quantized result.

GPU counterpart of ``antigravity-engine/src/model_loader.py``:

* :class:`ModelWeightLoader` keeps the interface of the reference's loader
  (``model_loader.py:33-134``): ``load_and_repack_layer`` casts to fp16,
  zero-pads to a multiple of 256 (``:66-74``), quantizes with the fp16-scale
  rule of ``quantize_weights_int4`` (``antigravity-engine/src/dequant.py:22-62``),
  checks the memory budget (``:86-92``, same ``MemoryError``) and returns the
  same keys.  ``'superblocks'`` holds the device record stream ``uint8[S,
  144]`` (what the projection kernels read) instead of the reference's list
  of per-superblock dicts; ``moat_amd.engine_dequant.repack_to_superblocks``
  still produces that list when a caller needs it.
* :class:`SafetensorsWeightReader` is the reference's reader (``:321-343``):
  safetensors' own loader (no pickle), fp16 out.
* :func:`save_superblocks` / :func:`load_superblocks`: a record file (magic,
  original shape, then the records as written) so that quantization runs once.
"""

from __future__ import annotations

import os
import struct
from typing import Dict, Iterable, Optional, Tuple

import numpy as np
import torch

from . import _device as D
from .dequant import SUPERBLOCK_BYTES, SUPERBLOCK_ELEMS, quantize_to_superblocks, unpack_superblock_weights
from .engine_dequant import quantize_weights_int4

MODEL_WEIGHT_BUDGET_BYTES = int(2.5 * 1024 ** 3)  # model_loader.py's default budget (2.5 GB)
RECORD_FILE_MAGIC = b"MOATI4R1"


class ModelWeightLoader:
    """Loads weight tensors as INT4 records on the GPU (``model_loader.py:33-134``)."""

    def __init__(self, memory_budget_bytes: int = MODEL_WEIGHT_BUDGET_BYTES):
        self.memory_budget_bytes = memory_budget_bytes
        self.layers: Dict[str, Dict] = {}
        self.total_loaded_bytes = 0

    def load_and_repack_layer(self, layer_name: str, weights_fp16, group_size: int = 32,
                              keep_q: bool = True) -> Dict:
        """Quantize and pack one weight tensor (any shape, any float dtype,
        numpy or torch).  Returns ``layer_name``, ``original_shape``,
        ``n_elements`` (before padding), ``superblocks`` (device ``uint8[S,
        144]``), ``memory_bytes`` (S * 144) and, with ``keep_q``, the int8
        codes ``q_weights`` and fp16 ``scales`` of the padded tensor (as numpy
        arrays, like the reference)."""
        if group_size != 32:
            raise ValueError("the 144-byte records hold groups of 32 weights (group_size=32)")
        original_shape = tuple(weights_fp16.shape)
        w = D.to_device(weights_fp16).reshape(-1).to(torch.float16)  # round to nearest even, as astype
        n_elements = w.numel()
        rem = n_elements % SUPERBLOCK_ELEMS
        if rem:
            w = torch.cat([w, torch.zeros(SUPERBLOCK_ELEMS - rem, dtype=torch.float16, device=w.device)])
        n_sb = w.numel() // SUPERBLOCK_ELEMS
        layer_memory_bytes = n_sb * SUPERBLOCK_BYTES
        if self.total_loaded_bytes + layer_memory_bytes > self.memory_budget_bytes:
            raise MemoryError(
                f"Loading layer '{layer_name}' ({layer_memory_bytes / 1e6:.1f} MB) exceeds "
                f"memory budget of {self.memory_budget_bytes / 1e9:.2f} GB. "
                f"Currently loaded: {self.total_loaded_bytes / 1e9:.2f} GB.")
        records = quantize_to_superblocks(w, scale_rule="f16")
        layer = {
            "layer_name": layer_name,
            "original_shape": original_shape,
            "n_elements": n_elements,
            "superblocks": records,
            "memory_bytes": layer_memory_bytes,
        }
        if keep_q:
            q, s = quantize_weights_int4(w)
            layer["q_weights"] = D.to_host(q)
            layer["scales"] = D.to_host(s)
        self.layers[layer_name] = layer
        self.total_loaded_bytes += layer_memory_bytes
        return layer

    def dequantize_layer(self, layer_name: str) -> torch.Tensor:
        """fp16 weights of a loaded layer in its original shape, decoded on the
        GPU from the records (``model_loader.py:110-134``; same bits as its
        LUT route)."""
        if layer_name not in self.layers:
            raise KeyError(f"Layer '{layer_name}' not found in loader")
        layer = self.layers[layer_name]
        flat = unpack_superblock_weights(layer["superblocks"], layer["superblocks"].shape[0])
        return flat[: layer["n_elements"]].reshape(layer["original_shape"])

    def load_safetensors(self, path: str, names: Optional[Iterable[str]] = None) -> Dict[str, Dict]:
        """Quantize-on-load of a safetensors checkpoint: every tensor (or those
        named) read with safetensors' loader, moved to the GPU, rounded to fp16
        and packed; returns {name: layer dict}."""
        reader = SafetensorsWeightReader(path)
        out = {}
        for name in (list(names) if names is not None else reader.list_tensor_names()):
            out[name] = self.load_and_repack_layer(name, reader.read_tensor_device(name))
        return out

    @property
    def total_memory_mb(self) -> float:
        return self.total_loaded_bytes / (1024 * 1024)

    @property
    def total_memory_gb(self) -> float:
        return self.total_loaded_bytes / (1024 ** 3)


class SafetensorsWeightReader:
    """``model_loader.py:321-343``: safetensors' torch loader (no pickle)."""

    def __init__(self, model_path: str):
        from safetensors.torch import load_file
        self.model_path = model_path
        if not os.path.exists(self.model_path):
            raise FileNotFoundError(f"Model weight file not found at '{self.model_path}'.")
        self.f = load_file(self.model_path)

    def list_tensor_names(self):
        return list(self.f.keys())

    def get_total_parameter_count(self):
        return int(sum(int(np.prod(tuple(t.shape))) for t in self.f.values()))

    def read_tensor(self, name) -> np.ndarray:
        if name not in self.f:
            raise KeyError(f"Tensor '{name}' not found in Safetensors file {self.model_path}.")
        return self.f[name].to(dtype=torch.float16).numpy()

    def read_tensor_device(self, name) -> torch.Tensor:
        """The tensor on the GPU in its stored dtype (bf16 included); the
        loader rounds it to fp16 there."""
        if name not in self.f:
            raise KeyError(f"Tensor '{name}' not found in Safetensors file {self.model_path}.")
        return D.to_device(self.f[name])


def save_superblocks(path: str, records, original_shape: Tuple[int, ...]) -> None:
    """Write a record file: 8-byte magic, uint32 rank, rank x uint64 dims,
    uint64 record count, then the records as stored (144 bytes each)."""
    data = D.to_host(records) if D.is_tensor(records) else np.asarray(records)
    data = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
    if data.size % SUPERBLOCK_BYTES:
        raise ValueError(f"record bytes {data.size} are not a multiple of {SUPERBLOCK_BYTES}")
    n_sb = data.size // SUPERBLOCK_BYTES
    dims = tuple(int(d) for d in original_shape)
    if int(np.prod(dims, dtype=np.int64)) > n_sb * SUPERBLOCK_ELEMS:
        raise ValueError("shape holds more elements than the records")
    with open(path, "wb") as f:
        f.write(RECORD_FILE_MAGIC)
        f.write(struct.pack("<I", len(dims)))
        f.write(struct.pack(f"<{len(dims)}Q", *dims))
        f.write(struct.pack("<Q", n_sb))
        f.write(data.tobytes())


def load_superblocks(path: str, device: bool = False):
    """Read a record file: (records ``uint8[S, 144]``, original shape); the
    records on the GPU when ``device`` is true."""
    with open(path, "rb") as f:
        if f.read(8) != RECORD_FILE_MAGIC:
            raise ValueError(f"{path} is not a record file")
        (rank,) = struct.unpack("<I", f.read(4))
        dims = struct.unpack(f"<{rank}Q", f.read(8 * rank))
        (n_sb,) = struct.unpack("<Q", f.read(8))
        data = np.frombuffer(f.read(n_sb * SUPERBLOCK_BYTES), dtype=np.uint8)
    if data.size != n_sb * SUPERBLOCK_BYTES:
        raise ValueError(f"{path}: truncated record file")
    records = data.reshape(n_sb, SUPERBLOCK_BYTES).copy()
    return (D.to_device(records) if device else records), tuple(int(d) for d in dims)
