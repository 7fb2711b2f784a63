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
* :meth:`ModelWeightLoader.parse_gguf_file` / :meth:`ModelWeightLoader.auto_load_gguf`:
  the reference's GGUF header parser and loader (``:137-251``): F32 and F16
  tensors, and its int8 fallback for every other tensor type.
* :func:`estimate_model_superblock_memory`, :class:`SuperBlockRepacker`,
  :class:`QuantizedSuperBlockTensor` and :class:`MemoryBudgetValidator`: the
  reference's helpers (``:281-403``) with the records on the GPU.
* :func:`save_superblocks` / :func:`load_superblocks`: a record file (magic,
  original shape, layout, then the records as written) so that quantization
  runs once.

Storage order.  A 2-D weight ``W[K][M]`` that the strip GEMM can read (K >=
2048, K % 32 == 0, M % 32 == 0) is stored in strip order by default (the
loader's ``layout="auto"``; :func:`moat_amd.dequant.records_to_strips`): the
order the batched decode GEMM streams fastest.  Every other tensor, or
``layout="row"``, keeps the reference's row order.  The layer dict says which
(``'layout'``); :meth:`ModelWeightLoader.row_records` gives row order either
way.

Rounding.  Float inputs are rounded to fp16 once, nearest-even, by a library
kernel (numpy's ``astype(float16)``), float64 included.
"""

from __future__ import annotations

import os
import struct
from typing import Dict, Iterable, Optional, Tuple

import numpy as np
import torch

from . import _device as D
from .dequant import (GROUP_SIZE, SUPERBLOCK_BYTES, SUPERBLOCK_ELEMS, i8_div_to_f16, quantize_to_superblocks,
                      records_to_strips, strips_to_records, to_f16, unpack_superblock_weights)

IOS_APP_MEMORY_CEILING_BYTES = 4500 * 1024 * 1024  # model_loader.py:21
MODEL_WEIGHT_BUDGET_BYTES = 2500 * 1024 * 1024  # model_loader.py:22, the loader's default budget
RECORD_FILE_MAGIC = b"MOATI4R2"      # with a layout byte
RECORD_FILE_MAGIC_V1 = b"MOATI4R1"   # row order, no layout byte (still read)
LAYOUTS = ("row", "strip")


def strip_layout_ok(shape) -> bool:
    """Whether the strip GEMM can read a weight of this shape: 2-D ``(K, M)``
    with K >= 2048, K % 32 == 0 and M % 32 == 0."""
    return len(shape) == 2 and shape[0] >= 2048 and shape[0] % 32 == 0 and shape[1] % 32 == 0


def _codes_from_records(records: torch.Tensor):
    """int8 codes (q, one per element, in [-8, 7]) and fp16 scales (one per 32
    elements) of a row-order record stream: the quantizer's output read back
    from the records it wrote (low nibble = element 2j, high = 2j+1, each
    stored as q + 8)."""
    rec = records.reshape(-1, SUPERBLOCK_BYTES)
    scales = rec[:, :16].contiguous().view(torch.float16).reshape(-1)
    pay = rec[:, 16:].reshape(-1)
    lo = (pay & 15).to(torch.int8) - 8
    hi = (pay >> 4).to(torch.int8) - 8
    q = torch.stack([lo, hi], dim=1).reshape(-1)
    return q, scales


class ModelWeightLoader:
    """Loads weight tensors as INT4 records on the GPU (``model_loader.py:33-134``)."""

    def __init__(self, memory_budget_bytes: int = MODEL_WEIGHT_BUDGET_BYTES, layout: str = "auto"):
        if layout not in ("auto",) + LAYOUTS:
            raise ValueError(f"layout must be 'auto', 'row' or 'strip' (got {layout!r})")
        self.memory_budget_bytes = memory_budget_bytes
        self.layout = layout
        self.layers: Dict[str, Dict] = {}
        self.total_loaded_bytes = 0
        self._host_io = set()

    def load_and_repack_layer(self, layer_name: str, weights_fp16, group_size: int = 32,
                              keep_q: bool = True, layout: Optional[str] = None) -> Dict:
        """Quantize and pack one weight tensor (any shape, any float dtype,
        numpy or torch).  Returns ``layer_name``, ``original_shape``,
        ``n_elements`` (before padding), ``superblocks`` (device ``uint8[S,
        144]``, in ``layout`` order), ``layout`` (``'row'`` or ``'strip'``),
        ``memory_bytes`` (S * 144) and, with ``keep_q``, the int8 codes
        ``q_weights`` and fp16 ``scales`` of the padded tensor in row order
        (numpy arrays, like the reference), read back from the records rather
        than quantized a second time.

        ``group_size``: the reference's parameter; the 144-byte record holds
        groups of 32 weights, so 32 is the only value (ValueError otherwise).
        ``layout``: ``'auto'`` (the loader's default: strip order when
        :func:`strip_layout_ok`), ``'row'``, or ``'strip'`` (2-D with K % 8 == 0
        and M % 32 == 0, else ValueError)."""
        if group_size != 32:
            raise ValueError("the 144-byte records hold groups of 32 weights (group_size=32)")
        layout = layout or self.layout
        if layout not in ("auto",) + LAYOUTS:
            raise ValueError(f"layout must be 'auto', 'row' or 'strip' (got {layout!r})")
        original_shape = tuple(weights_fp16.shape)
        if layout == "strip" and not (len(original_shape) == 2 and original_shape[0] % 8 == 0
                                      and original_shape[0] > 0 and original_shape[1] % 32 == 0
                                      and original_shape[1] > 0):
            raise ValueError(f"strip order needs a 2-D (K, M) weight with K % 8 == 0 and M % 32 == 0 "
                             f"(got {original_shape})")
        if layout == "auto":
            layout = "strip" if strip_layout_ok(original_shape) else "row"
        w = to_f16(weights_fp16).reshape(-1)  # one nearest-even rounding, as astype
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
        q_codes = _codes_from_records(records) if keep_q else None
        if layout == "strip":
            records = records_to_strips(records, original_shape[0], original_shape[1]).reshape(n_sb, SUPERBLOCK_BYTES)
        if D.is_tensor(weights_fp16) and weights_fp16.is_cuda:
            self._host_io.discard(layer_name)
        else:
            self._host_io.add(layer_name)  # numpy in: dequantize_layer hands numpy back
        layer = {
            "layer_name": layer_name,
            "original_shape": original_shape,
            "n_elements": n_elements,
            "superblocks": records,
            "layout": layout,
            "memory_bytes": layer_memory_bytes,
        }
        if keep_q:
            layer["q_weights"] = D.to_host(q_codes[0])
            layer["scales"] = D.to_host(q_codes[1])
        self.layers[layer_name] = layer
        self.total_loaded_bytes += layer_memory_bytes
        return layer

    def dequantize_layer(self, layer_name: str) -> torch.Tensor:
        """fp16 weights of a loaded layer in its original shape, decoded on the
        GPU from the records (``model_loader.py:110-134``; same bits as its
        LUT route): numpy when the layer was loaded from host data, else a
        GPU tensor."""
        if layer_name not in self.layers:
            raise KeyError(f"Layer '{layer_name}' not found in loader")
        layer = self.layers[layer_name]
        rows = self.row_records(layer_name)
        flat = unpack_superblock_weights(rows, rows.shape[0])
        out = flat[: layer["n_elements"]].reshape(layer["original_shape"])
        return D.to_host(out) if layer_name in self._host_io else out

    def row_records(self, layer_name: str) -> torch.Tensor:
        """The layer's records in row order (the stored stream itself when the
        layer is in row order)."""
        if layer_name not in self.layers:
            raise KeyError(f"Layer '{layer_name}' not found in loader")
        layer = self.layers[layer_name]
        if layer.get("layout", "row") == "strip":
            K, M = layer["original_shape"]
            return strips_to_records(layer["superblocks"], K, M)
        return layer["superblocks"]

    def unload_layer(self, layer_name: str) -> None:
        """Drop a layer (its records are freed with the last reference) and
        return its bytes to the budget (``model_loader.py:264-269``)."""
        if layer_name in self.layers:
            self.total_loaded_bytes -= self.layers.pop(layer_name)["memory_bytes"]
            self._host_io.discard(layer_name)

    def clear(self) -> None:
        """Drop every layer (``model_loader.py:271-274``)."""
        self.layers.clear()
        self._host_io.clear()
        self.total_loaded_bytes = 0

    def parse_gguf_file(self, gguf_path: str) -> Dict:
        """GGUF header: metadata key/values, tensor table (name, dims as
        stored, type, offset) and the aligned start of the tensor data
        (``model_loader.py:137-214``).  Raises FileNotFoundError for a missing
        file and ValueError for a bad magic or an unknown value type."""
        if not os.path.exists(gguf_path):
            raise FileNotFoundError(f"GGUF weight file not found at: {gguf_path}")
        with open(gguf_path, "rb") as f:
            return _GGUFHeader(f).parse()

    def auto_load_gguf(self, gguf_path: str) -> Dict:
        """Load every tensor of a GGUF file as INT4 records
        (``model_loader.py:217-251``): F32 (type 0) is rounded to fp16 on the
        GPU, F16 (type 1) is taken as stored, and any other type is read as
        one int8 per element (zero-filled past the end of the file) and
        mapped to fp16(int8 / 7) as the reference's numpy float16 division
        computes it (library kernels for both conversions).  The shape is the
        dims in stored order.  Returns the parsed header."""
        if not os.path.exists(gguf_path):
            raise FileNotFoundError(f"GGUF model file not found at '{gguf_path}'. Please provide a valid file path.")
        info = self.parse_gguf_file(gguf_path)
        base = info.get("tensor_data_offset", 0)
        dev = D.require_gpu()
        with open(gguf_path, "rb") as f:
            for name, t in info["tensors"].items():
                shape = tuple(int(d) for d in t["dims"])
                n = int(np.prod(shape, dtype=np.int64)) if shape else 1
                f.seek(base + t["offset"])
                if t["type"] == 0:
                    host = np.frombuffer(f.read(4 * n), dtype=np.float32)
                    w = to_f16(torch.from_numpy(host.copy()).to(dev))
                elif t["type"] == 1:
                    w = torch.from_numpy(np.frombuffer(f.read(2 * n), dtype=np.float16).copy()).to(dev)
                else:
                    raw = f.read(n)
                    raw = raw + b"\x00" * (n - len(raw))
                    w = i8_div_to_f16(torch.from_numpy(np.frombuffer(raw, dtype=np.int8).copy()).to(dev), 7.0)
                self.load_and_repack_layer(name, w.reshape(shape))
        return info

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


class _GGUFHeader:
    """Reader of a GGUF header (little-endian): magic, version, tensor count,
    key/value count, the key/values, the tensor table."""

    # value type -> struct code of the scalar types (GGUF value-type table)
    _SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
    _STRING, _ARRAY = 8, 9

    def __init__(self, f):
        self.f = f

    def _unpack(self, code: str):
        size = struct.calcsize(code)
        data = self.f.read(size)
        if len(data) != size:
            raise ValueError("GGUF header is truncated")
        return struct.unpack(code, data)[0]

    def _string(self) -> str:
        return self.f.read(self._unpack("<Q")).decode("utf-8", errors="replace")

    def _value(self, vtype: int):
        if vtype in self._SCALAR:
            return self._unpack(self._SCALAR[vtype])
        if vtype == self._STRING:
            return self._string()
        if vtype == self._ARRAY:
            etype = self._unpack("<I")
            count = self._unpack("<Q")
            return [self._value(etype) for _ in range(count)]
        raise ValueError(f"Unknown value type: {vtype}")

    def parse(self) -> Dict:
        magic = self.f.read(4)
        if magic != b"GGUF":
            raise ValueError(f"Invalid GGUF magic header: {magic}")
        version = self._unpack("<I")
        n_tensors = self._unpack("<Q")
        n_kv = self._unpack("<Q")
        metadata = {}
        for _ in range(n_kv):
            key = self._string()
            metadata[key] = self._value(self._unpack("<I"))
        tensors = {}
        for _ in range(n_tensors):
            name = self._string()
            dims = [self._unpack("<Q") for _ in range(self._unpack("<I"))]
            ttype = self._unpack("<I")
            tensors[name] = {"name": name, "dims": dims, "type": ttype, "offset": self._unpack("<Q")}
        end = self.f.tell()
        align = int(metadata.get("general.alignment", 32))
        return {"metadata": metadata, "tensors": tensors, "version": version, "n_tensors": n_tensors,
                "tensor_data_offset": end + (-end) % align}


def estimate_model_superblock_memory(n_parameters: int, group_size: int = 32) -> Dict[str, float]:
    """Footprint of a model stored as 144-byte records (``model_loader.py:281-318``):
    ceil(P / 256) records against 2 bytes per fp16 weight."""
    records_bytes = -(-int(n_parameters) // SUPERBLOCK_ELEMS) * SUPERBLOCK_BYTES
    fp16_bytes = int(n_parameters) * 2
    mib = 1024.0 * 1024.0
    return {
        "n_parameters": n_parameters,
        "fp16_memory_mb": fp16_bytes / mib,
        "superblock_memory_mb": records_bytes / mib,
        "superblock_memory_gb": records_bytes / mib / 1024.0,
        "compression_ratio": fp16_bytes / records_bytes,
        "bits_per_weight": SUPERBLOCK_BYTES * 8 / SUPERBLOCK_ELEMS,
        "fits_ios_4_5gb_ceiling": records_bytes <= MODEL_WEIGHT_BUDGET_BYTES,
    }


class QuantizedSuperBlockTensor:
    """A weight tensor held as 144-byte records on the GPU with its original
    shape (``model_loader.py:344-360``)."""

    def __init__(self, superblocks, shape, group_size: int = 32, host_io: bool = False):
        self.superblocks = superblocks
        self.shape = tuple(shape)
        self.group_size = group_size
        self.bytes_per_superblock = SUPERBLOCK_BYTES
        self.memory_bytes = len(superblocks) * SUPERBLOCK_BYTES
        self._host_io = host_io

    def validate_structure(self) -> bool:
        """Every record is 144 bytes: 8 fp16 scales (16 bytes) then 128
        payload bytes, and the records cover the shape."""
        sb = self.superblocks
        ok = sb.dim() == 2 and sb.shape[1] == SUPERBLOCK_BYTES and sb.dtype == torch.uint8
        return bool(ok and sb.shape[0] * SUPERBLOCK_ELEMS >= int(np.prod(self.shape, dtype=np.int64)))

    def dequantize(self):
        """fp16 weights in the original shape (numpy when packed from host data)."""
        flat = unpack_superblock_weights(self.superblocks, self.superblocks.shape[0])
        out = flat[: int(np.prod(self.shape, dtype=np.int64))].reshape(self.shape)
        return D.to_host(out) if self._host_io else out


class SuperBlockRepacker:
    """``model_loader.py:363-375``: fp16 cast, zero pad to 256, fp16-scale
    quantizer, records -- one GPU kernel after the cast."""

    @staticmethod
    def repack_matrix(matrix, group_size: int = 32, groups_per_superblock: int = 8) -> QuantizedSuperBlockTensor:
        if group_size != GROUP_SIZE or groups_per_superblock != SUPERBLOCK_ELEMS // GROUP_SIZE:
            raise ValueError("the 144-byte records hold 8 groups of 32 weights")
        shape = tuple(matrix.shape)
        w = to_f16(matrix).reshape(-1)  # one nearest-even rounding, as astype
        rem = w.numel() % SUPERBLOCK_ELEMS
        if rem:
            w = torch.cat([w, torch.zeros(SUPERBLOCK_ELEMS - rem, dtype=torch.float16, device=w.device)])
        records = quantize_to_superblocks(w, scale_rule="f16")
        host_io = not (D.is_tensor(matrix) and matrix.is_cuda)
        return QuantizedSuperBlockTensor(records, shape, group_size=group_size, host_io=host_io)


class MemoryBudgetValidator:
    """``model_loader.py:378-403``: weights as records plus an fp16 KV cache
    (16 heads x 64 dims, keys and values) against 2.5 GB / 4.5 GB."""

    @staticmethod
    def calculate_weight_memory_gb(num_params: int) -> float:
        return (-(-int(num_params) // SUPERBLOCK_ELEMS) * SUPERBLOCK_BYTES) / 1024.0 ** 3

    @staticmethod
    def validate_memory_budget(num_params: int, num_traces: int = 8, seq_len: int = 2048,
                               runtime_overhead_gb: float = 0.5) -> Dict:
        weight_gb = MemoryBudgetValidator.calculate_weight_memory_gb(num_params)
        kv_gb = num_traces * seq_len * 16 * 64 * 2 * 2 / 1024.0 ** 3
        total_gb = weight_gb + kv_gb + runtime_overhead_gb
        weight_ok = weight_gb <= 2.5
        app_ok = total_gb <= 4.5
        if not (weight_ok and app_ok):
            raise ValueError(f"Memory budget breached: weight={weight_gb:.2f}GB, total={total_gb:.2f}GB")
        return {"weight_memory_gb": weight_gb, "total_app_memory_gb": total_gb,
                "weight_budget_passed": weight_ok, "total_app_budget_passed": app_ok, "is_valid": True}


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


GGUFWeightReader = SafetensorsWeightReader  # model_loader.py:341, the same reader under the GGUF name


def save_superblocks(path: str, records, original_shape: Tuple[int, ...], layout: str = "row") -> None:
    """Write a record file: 8-byte magic, uint32 rank, rank x uint64 dims,
    uint64 record count, one layout byte (0 row order, 1 strip order), then
    the records as stored (144 bytes each)."""
    if layout not in LAYOUTS:
        raise ValueError(f"layout must be 'row' or 'strip' (got {layout!r})")
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
        f.write(struct.pack("<B", LAYOUTS.index(layout)))
        f.write(data.tobytes())


def load_superblocks(path: str, device: bool = False, with_layout: bool = False):
    """Read a record file: (records ``uint8[S, 144]``, original shape), plus the
    layout (``'row'`` or ``'strip'``) when ``with_layout``; the records on the
    GPU when ``device`` is true.  Files of the first version (no layout
    byte) are row order."""
    with open(path, "rb") as f:
        magic = f.read(8)
        if magic not in (RECORD_FILE_MAGIC, RECORD_FILE_MAGIC_V1):
            raise ValueError(f"{path} is not a record file")
        (rank,) = struct.unpack("<I", f.read(4))
        dims = struct.unpack(f"<{rank}Q", f.read(8 * rank))
        (n_sb,) = struct.unpack("<Q", f.read(8))
        layout = "row"
        if magic == RECORD_FILE_MAGIC:
            (code,) = struct.unpack("<B", f.read(1))
            if code >= len(LAYOUTS):
                raise ValueError(f"{path}: unknown layout code {code}")
            layout = LAYOUTS[code]
        data = np.frombuffer(f.read(n_sb * SUPERBLOCK_BYTES), dtype=np.uint8)
    if data.size != n_sb * SUPERBLOCK_BYTES:
        raise ValueError(f"{path}: truncated record file")
    records = data.reshape(n_sb, SUPERBLOCK_BYTES).copy()
    out = (D.to_device(records) if device else records), tuple(int(d) for d in dims)
    return out + (layout,) if with_layout else out
