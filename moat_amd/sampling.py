"""Batched token sampling from LM-head logits on the GPU.

GPU counterpart of the reference's numpy sampler and the table softmax it
uses:

* :class:`ExponentialLUT` -- ``antigravity-engine/src/attention.py:21-94``: the
  fp16 table of exp over [-range_max, 0] (built on the host exactly as the
  reference builds it, then kept on the GPU) and its ``lookup``;
* :func:`safe_softmax_lut` -- ``attention.py:97-135``, along any axis;
* :class:`TokenSampler` / :func:`sample_tokens` --
  ``BatchedRolloutCoordinator.sample_tokens``
  (``antigravity-engine/src/batch_generator.py:187-253``, its numpy path):
  greedy at temperature <= 0, otherwise one draw per row from the 50 most
  probable tokens of the table softmax of logits / T.

All arithmetic runs in ``libmoat_int4.so`` (one workgroup per 8192-logit
chunk of a row, V up to 524288).  Where the reference leaves a choice open the GPU fixes it: the top-k
set and its order are (probability descending, index ascending) -- the
reference takes ``np.argpartition``'s order -- and row r's uniform draw comes
from a counter-based generator keyed by ``seed`` (drawn from numpy's global
generator when not given, so ``np.random.seed`` still makes runs repeatable).
``top_p`` is accepted and unused, as in the reference.

numpy logits give numpy results with the reference's dtypes (greedy: int64
tokens and fp16 log-probabilities; sampling: int32 and float32); a GPU tensor
gives GPU tensors of the same dtypes.
"""

from __future__ import annotations

from typing import Optional, Tuple

import numpy as np
import torch

from . import _device as D
from . import _lib

MAX_VOCAB = 64 * 8192  # logits per row: 64 chunks of numpy's 8192-element sum pieces
MAX_TABLE = 1 << 24  # table entries (indices exact in float32)
MAX_TOP_K = 64
_MAX_ROWS = 1 << 21  # rows per call (rows x 1024 threads stay below 2^32)
DEFAULT_TOP_K = 50  # batch_generator.py:241

_DTYPES = {torch.float32: _lib.DTYPE_F32, torch.float16: _lib.DTYPE_F16, torch.float64: _lib.DTYPE_F64}


class ExponentialLUT:
    """fp16 exp(x) for x in [-range_max, 0] at ``size`` evenly spaced points
    (``attention.py:21-94``)."""

    def __init__(self, size: int = 32768, range_max: float = 10.0):
        if size < 2:
            raise ValueError(f"LUT size must be >= 2, got {size}")
        if range_max <= 0:
            raise ValueError(f"range_max must be positive, got {range_max}")
        self.size = size
        self.range_max = range_max
        # the table's definition (attention.py:52-53): float32 grid, fp16 exp
        self.inputs = np.linspace(-range_max, 0.0, size, dtype=np.float32)
        self.lut = np.exp(self.inputs).astype(np.float16)
        self.step = range_max / (size - 1)
        if abs(float(self.lut[-1]) - 1.0) >= 0.01:
            raise ValueError(f"LUT endpoint should be ~1.0, got {self.lut[-1]}")
        self._tables = {}

    @property
    def step_f32(self) -> float:
        """The step as the lookup divides by it (a float32 array / Python float)."""
        return float(np.float32(self.step))

    @property
    def memory_bytes(self) -> int:
        return self.lut.nbytes

    def table(self) -> torch.Tensor:
        """The table on the current GPU (copied once per device)."""
        dev = D.require_gpu()
        t = self._tables.get(dev.index)
        if t is None:
            t = torch.from_numpy(self.lut.view(np.int16).copy()).to(dev)
            self._tables[dev.index] = t
        return t

    def lookup(self, x_shifted):
        """Table exp of non-positive inputs, ``lut[size-1-trunc(clip(|x| / step,
        0, size-1))]`` (``attention.py:60-85``); fp16, the shape of the input."""
        host = not (D.is_tensor(x_shifted) and x_shifted.is_cuda)
        x = D.to_device(x_shifted, torch.float32)
        out = torch.empty(x.shape, dtype=torch.float16, device=x.device)
        _lib.check(_lib.load().moat_lut_lookup(D.ptr(x), x.numel(), D.ptr(self.table()), self.size,
                                               self.step_f32, D.ptr(out), D.stream()), "ExponentialLUT.lookup")
        return D.to_host(out) if host else out


def _logits_dtype(t: torch.Tensor) -> torch.Tensor:
    # float16/32/64 as they are; integers and other floats through float64
    # (exact for integers below 2**53), which the kernels round to float32
    return t if t.dtype in _DTYPES else t.to(torch.float64)


def _workspace(n: int, v: int, softmax: bool = False):
    """The calling stream's sampling workspace for n rows of v logits."""
    lib = _lib.load()
    nbytes = int((lib.moat_lut_softmax_workspace_size if softmax else lib.moat_sample_workspace_size)(n, v))
    if nbytes < 0:
        raise ValueError(f"{n} rows of {v} logits: outside the sampler's limits")
    ws = D.sample_workspaces.get(nbytes)
    return ws, (ws.numel() if ws is not None else 0)


def _check_table(exp_lut: ExponentialLUT) -> None:
    if exp_lut.size > MAX_TABLE:
        raise ValueError(f"table of {exp_lut.size} entries: the GPU softmax indexes at most {MAX_TABLE}")


def safe_softmax_lut(x, exp_lut: ExponentialLUT, axis: int = -1):
    """Softmax along ``axis`` with the table exp (``attention.py:97-135``):
    float32 row max, table lookup of x - max, numpy's float32 sum, fp16
    quotient.  At most 524288 values along ``axis``."""
    _check_table(exp_lut)
    host = not (D.is_tensor(x) and x.is_cuda)
    t = _logits_dtype(D.to_device(x))
    if t.dim() == 0:
        raise ValueError("softmax needs at least one axis")
    t = torch.movedim(t, axis, -1).contiguous()
    v = t.shape[-1]
    if v == 0:
        raise ValueError("zero-size array to reduction operation maximum which has no identity")
    if v > MAX_VOCAB:
        raise ValueError(f"{v} values along the softmax axis: at most {MAX_VOCAB}")
    rows = t.numel() // v
    out = torch.empty(t.shape, dtype=torch.float16, device=t.device)
    flat_in, flat_out = t.reshape(rows, v), out.reshape(rows, v)
    for r0 in range(0, rows, _MAX_ROWS):
        r1 = min(rows, r0 + _MAX_ROWS)
        ws, ws_bytes = _workspace(r1 - r0, v, softmax=True)
        _lib.check(_lib.load().moat_lut_softmax(D.ptr(flat_in[r0:r1]), _DTYPES[t.dtype], r1 - r0, v,
                                                D.ptr(exp_lut.table()), exp_lut.size, exp_lut.step_f32,
                                                D.ptr(flat_out[r0:r1]), D.ptr(ws), ws_bytes, D.stream()),
                   "safe_softmax_lut")
    out = torch.movedim(out, -1, axis)
    return D.to_host(out.contiguous()) if host else out


class TokenSampler:
    """The sampling part of ``BatchedRolloutCoordinator`` (``batch_generator.py:161-253``):
    its exp table (``exp_lut_size`` entries over [-10, 0]) and ``sample_tokens``."""

    def __init__(self, exp_lut_size: int = 32768, top_k: int = DEFAULT_TOP_K):
        if not 1 <= top_k <= MAX_TOP_K:
            raise ValueError(f"top_k must be in [1, {MAX_TOP_K}], got {top_k}")
        self.exp_lut = ExponentialLUT(size=exp_lut_size, range_max=10.0)
        _check_table(self.exp_lut)
        self.top_k = top_k

    def sample_tokens(self, logits_batch, temperature: float = 0.7, top_p: float = 0.9,
                      seed: Optional[int] = None) -> Tuple:
        """Next token and its log-probability for each of the N rows of
        ``logits_batch`` [N, V] (``batch_generator.py:187-253``)."""
        host = not (D.is_tensor(logits_batch) and logits_batch.is_cuda)
        t = _logits_dtype(D.to_device(logits_batch))
        if t.dim() != 2:
            raise ValueError(f"logits_batch must be [N, V], got shape {tuple(t.shape)}")
        n, v = t.shape
        if v == 0 or v > MAX_VOCAB:
            raise ValueError(f"vocabulary of {v}: 1 to {MAX_VOCAB} logits per row")
        temperature = float(temperature)
        if seed is None:
            seed = int(np.random.randint(0, 2 ** 63 - 1, dtype=np.int64))
        tokens = torch.empty(n, dtype=torch.int32, device=t.device)
        logprobs = torch.empty(n, dtype=torch.float32, device=t.device)
        ws, ws_bytes = _workspace(n, v)
        _lib.check(_lib.load().moat_sample_tokens(D.ptr(t), _DTYPES[t.dtype], n, v, temperature, self.top_k,
                                                  int(seed) & (2 ** 64 - 1), D.ptr(self.exp_lut.table()),
                                                  self.exp_lut.size, self.exp_lut.step_f32, D.ptr(tokens),
                                                  D.ptr(logprobs), D.ptr(ws), ws_bytes, D.stream()),
                   "sample_tokens")
        if temperature <= 0.0:
            tokens, logprobs = tokens.to(torch.int64), logprobs.to(torch.float16)
        if host:
            return D.to_host(tokens), D.to_host(logprobs)
        return tokens, logprobs


_default_sampler: Optional[TokenSampler] = None


def sample_tokens(logits_batch, temperature: float = 0.7, top_p: float = 0.9, seed: Optional[int] = None):
    """:meth:`TokenSampler.sample_tokens` with the default table (32768 entries)."""
    global _default_sampler
    if _default_sampler is None:
        _default_sampler = TokenSampler()
    return _default_sampler.sample_tokens(logits_batch, temperature, top_p, seed)
