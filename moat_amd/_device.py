"""Device plumbing: numpy/torch inputs to device tensors, pointers, streams,
and the per-stream workspaces.  torch provides memory and streams only;
all arithmetic of the path runs in libmoat_int4.so."""

from __future__ import annotations

import ctypes
import threading

import numpy as np
import torch

from . import _lib

_DEVICE_DTYPES = {
    np.dtype(np.float32): torch.float32,
    np.dtype(np.float16): torch.float16,
    np.dtype(np.float64): torch.float64,
    np.dtype(np.int8): torch.int8,
    np.dtype(np.uint8): torch.uint8,
    np.dtype(np.int16): torch.int16,
    np.dtype(np.int32): torch.int32,
    np.dtype(np.int64): torch.int64,
    np.dtype(np.bool_): torch.bool,
}


def require_gpu() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("moat_amd needs a ROCm GPU (MI355X / gfx950); there is no CPU path")
    return torch.device("cuda", torch.cuda.current_device())


def is_tensor(a) -> bool:
    return isinstance(a, torch.Tensor)


def to_device(a, dtype: torch.dtype | None = None) -> torch.Tensor:
    """A contiguous device tensor with a's values (a copy for host data).
    `dtype`, when given, is applied on the device after the copy."""
    dev = require_gpu()
    if is_tensor(a):
        t = a.to(dev)
    else:
        arr = np.ascontiguousarray(a)
        if arr.dtype not in _DEVICE_DTYPES:
            kind = arr.dtype.kind
            if kind in "iu":
                arr = arr.astype(np.int64)  # value-preserving widening
            elif kind == "f":
                arr = arr.astype(np.float64)
            else:
                raise TypeError(f"unsupported dtype {arr.dtype}")
        t = torch.from_numpy(arr).to(dev)
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous()


def aligned(t: torch.Tensor, a: int) -> torch.Tensor:
    """t itself when its data pointer is a-byte aligned, else an aligned copy."""
    if t.numel() == 0 or t.data_ptr() % a == 0:
        return t
    return t.clone()


def ptr(t: torch.Tensor | None) -> int | None:
    if t is None or t.numel() == 0:
        return None
    return t.data_ptr()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def to_host(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy()


def out_like(t: torch.Tensor, want_tensor: bool):
    return t if want_tensor else to_host(t)


class _Workspaces:
    """One zero-initialised workspace per (device, stream), grown on demand.
    The kernels leave its counter words at zero after every call."""

    def __init__(self) -> None:
        self._lock = threading.Lock()
        self._bufs: dict[tuple[int, int], torch.Tensor] = {}

    def get(self, nbytes: int) -> torch.Tensor | None:
        if nbytes <= 0:
            return None
        dev = require_gpu()
        key = (dev.index, stream())
        with self._lock:
            buf = self._bufs.get(key)
            if buf is None or buf.numel() < nbytes:
                size = max(nbytes, 1 << 20)
                buf = torch.empty(size, dtype=torch.uint8, device=dev)
                _lib.check(_lib.load().moat_int4_workspace_clear(buf.data_ptr(), size, stream()),
                           "moat_int4_workspace_clear")
                self._bufs[key] = buf
            return buf

    def check(self, what: str) -> None:
        """Raise if an in-kernel hand-off on this stream's workspace ran out
        of time since it was last cleared (its sticky status word is set:
        those calls and every later one on it wrote NaN).  The workspace is
        cleared before raising, so later calls produce results again.  Waits
        for the stream's queued work."""
        dev = require_gpu()
        key = (dev.index, stream())
        with self._lock:
            buf = self._bufs.get(key)
        if buf is None:
            return
        lib = _lib.load()
        st = ctypes.c_int32(0)
        _lib.check(lib.moat_int4_workspace_status(buf.data_ptr(), buf.numel(), ctypes.byref(st), stream()),
                   "moat_int4_workspace_status")
        if st.value:
            _lib.check(lib.moat_int4_workspace_clear(buf.data_ptr(), buf.numel(), stream()),
                       "moat_int4_workspace_clear")
            raise RuntimeError(f"{what}: a hand-off between workgroups ran out of time (workspace status "
                               f"{st.value}); the results of that call and of later calls on this stream were "
                               "NaN; the workspace has been cleared")


workspaces = _Workspaces()  # GEMM calls
sample_workspaces = _Workspaces()  # sampling calls: their own (they rewrite their counter words)
dense_workspaces = _Workspaces()  # dense fp16 products: their own (their split sums stay behind)
