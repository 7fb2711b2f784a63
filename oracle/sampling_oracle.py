"""CPU oracle for moat's batched token sampler: test infrastructure only.

This module is the *checker*. Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import it; the product
(``moat_amd``) never does, and has no CPU fallback.

It restates the numpy path of the reference's sampler,
``BatchedRolloutCoordinator.sample_tokens``
(``antigravity-engine/src/batch_generator.py:187-253``), and the LUT softmax it
calls (``antigravity-engine/src/attention.py:21-135``):

* ``exp_table``: the 32768-entry fp16 table of exp over [-range_max, 0]
  (``attention.py:32-58``);
* ``numpy_sum_f32`` / ``pairwise_sum_f32``: numpy's float32 ``np.sum`` along
  a contiguous axis -- 8192-element pieces (the ufunc buffer) added in order,
  each summed with the pairwise algorithm of numpy's reduction loops (blocks
  of at most 128 summed with 8 strided accumulators, halves split at
  multiples of 8).  The reference's softmax denominator (``attention.py:129``)
  and top-k mass (``batch_generator.py:244``) are such sums, so their bits
  depend on it;
* ``softmax_lut``: ``safe_softmax_lut`` (``attention.py:97-135``);
* ``sample_tokens``: greedy (temperature <= 0: argmax, log of the LUT-softmax
  probability in fp16) and temperature sampling (LUT softmax of logits / T,
  the 50 most probable, renormalised, one draw, log of the full-softmax
  probability in fp32).

A row whose maximum (after the temperature) is NaN or infinite, where the
reference's table index is undefined (numpy raises IndexError), gets NaN
probabilities, the first maximum of the raw logits (np.argmax's rule) as its
token and a NaN log-probability.

Where the reference leaves a choice open this oracle fixes it, as the GPU
sampler does: the top-k set and the order of its cumulative distribution are
(probability descending, index ascending) -- the reference takes whatever
order ``np.argpartition`` returns -- and the uniform draw of row r comes from
a counter-based generator (SplitMix64 of ``seed + (r + 1) * 0x9E3779B97F4A7C15``)
instead of numpy's global generator. Logarithms are the correctly rounded
float32 log (float64 log rounded once); numpy's own float32 log may differ from
it by an ulp on some CPUs.

How each function is pinned (tests/test_sampling_oracle.py):

* ``numpy_sum_f32``: bit for bit against ``np.sum`` itself on random float32
  rows of every length class (short, one block, many blocks, odd tails, more
  than one 8192-element piece), 1-D and along the last axis of a 2-D array;
* ``exp_table`` / ``lut_index``: the reference tests' known answers
  (``tests/test_attention.py``: LUT[-1] = 1, LUT[0] = exp(-10) > 0, monotone,
  lookup(-1) and lookup(-5) within 2 % / 5 %, batch mean error < 0.01) and
  float64 exp within fp16 rounding;
* ``softmax_lut``: uniform rows (all probabilities fp16(1/V)), one-hot rows,
  sums within fp16 rounding of 1, monotone in the logit, and the exact
  softmax within the table's quantisation bound;
* ``sample_tokens``: the reference's greedy answer (``tests/test_batch_generator.py:97-109``),
  the extreme-input cases of ``tests/test_fuzz_extreme_inputs.py:32-60`` (no
  NaN), and a chi-square test of the draws against the renormalised top-k
  distribution.
"""

from __future__ import annotations

import math
from typing import Tuple

import numpy as np

PW_BLOCK = 128  # numpy's pairwise block (elements summed with 8 accumulators)
GOLDEN = 0x9E3779B97F4A7C15
MASK64 = (1 << 64) - 1
LOG_1E_10_F32 = np.float32(math.log(1e-10))  # log(max(p, 1e-10)) for p == 0 (batch_generator.py:250)


def exp_table(size: int = 32768, range_max: float = 10.0) -> np.ndarray:
    """fp16 exp over ``linspace(-range_max, 0, size)`` in float32 (``attention.py:52-53``)."""
    if size < 2:
        raise ValueError(f"LUT size must be >= 2, got {size}")
    if range_max <= 0:
        raise ValueError(f"range_max must be positive, got {range_max}")
    return np.exp(np.linspace(-range_max, 0.0, size, dtype=np.float32)).astype(np.float16)


def table_step_f32(size: int = 32768, range_max: float = 10.0) -> np.float32:
    """The index step as the lookup uses it: range_max / (size - 1) in float64,
    rounded to float32 when it divides a float32 array (``attention.py:56, 82``)."""
    return np.float32(range_max / (size - 1))


def lut_index(shifted_f32: np.ndarray, size: int, step: np.float32) -> np.ndarray:
    """Table row of exp(shifted): ``size - 1 - trunc(clip(|x| / step, 0, size - 1))``
    (``attention.py:80-85``), for finite or -inf x <= 0."""
    a = np.abs(shifted_f32.astype(np.float32)) / step
    return (size - 1) - np.clip(a, 0, size - 1).astype(np.int64)


def pairwise_sum_f32(a: np.ndarray) -> np.float32:
    """numpy's float32 sum of a contiguous 1-D array, in numpy's order."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    n = a.size
    if n < 8:
        res = np.float32(0.0)
        for v in a:
            res = np.float32(res + v)
        return res
    if n <= PW_BLOCK:
        r = a[:8].copy()
        i = 8
        while i < n - (n % 8):
            r = (r + a[i:i + 8]).astype(np.float32)
            i += 8
        res = np.float32(np.float32(np.float32(r[0] + r[1]) + np.float32(r[2] + r[3]))
                         + np.float32(np.float32(r[4] + r[5]) + np.float32(r[6] + r[7])))
        for v in a[i:]:
            res = np.float32(res + v)
        return res
    n2 = n // 2
    n2 -= n2 % 8
    return np.float32(pairwise_sum_f32(a[:n2]) + pairwise_sum_f32(a[n2:]))


def numpy_sum_f32(a: np.ndarray, bufsize: int = 8192) -> np.float32:
    """``np.sum`` of a contiguous float32 row: the reduction runs over
    ``bufsize``-element pieces (numpy's ufunc buffer, ``np.getbufsize()``),
    each summed pairwise, accumulated in order from 0."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    res = np.float32(0.0)
    for i in range(0, a.size, bufsize):
        res = np.float32(res + pairwise_sum_f32(a[i:i + bufsize]))
    return res


def softmax_lut(x: np.ndarray, table: np.ndarray, step: np.float32) -> np.ndarray:
    """``safe_softmax_lut`` along the last axis of a 2-D array (``attention.py:97-135``):
    float32 max, shift, table lookup, numpy-order float32 sum, divide, fp16."""
    x32 = np.asarray(x).astype(np.float32)
    size = table.size
    out = np.empty(x32.shape, dtype=np.float16)
    for r in range(x32.shape[0]):
        row = x32[r]
        if not np.isfinite(row.max()):
            out[r] = np.nan  # the reference's table index is undefined here (IndexError)
            continue
        shifted = row - row.max()
        e = table[lut_index(shifted, size, step)].astype(np.float32)
        s = numpy_sum_f32(e)
        s = s if s > 0 else np.float32(1.0)
        out[r] = (e / s).astype(np.float16)
    return out


def scale_logits(logits: np.ndarray, temperature: float) -> np.ndarray:
    """``logits / max(T, 1e-5)`` in the logits' own dtype (``batch_generator.py:231``):
    T is rounded to that dtype first; fp16 divides in float32 and rounds back."""
    x = np.asarray(logits)
    if x.dtype.kind != "f":
        x = x.astype(np.float64)  # integer / Python float is float64
    t = max(temperature, 1e-5)
    if x.dtype == np.float16:
        return (x.astype(np.float32) / np.float32(np.float16(t))).astype(np.float16)
    return x / x.dtype.type(t)


def uniform(seed: int, row: int) -> float:
    """Row ``row``'s draw in [0, 1): 53 bits of SplitMix64's output mix."""
    z = (seed + GOLDEN * (row + 1)) & MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    z ^= z >> 31
    return (z >> 11) * 2.0 ** -53


def log_f32(p: float) -> np.float32:
    """Correctly rounded float32 log of a float32 value (float64 log, one rounding)."""
    if np.isnan(p):
        return np.float32(np.nan)
    return np.float32(math.log(float(p))) if p > 0 else np.float32(-np.inf)


def first_argmax(row: np.ndarray) -> int:
    """``np.argmax``: the first maximum, a NaN counting as the maximum."""
    nan = np.isnan(row)
    if nan.any():
        return int(np.argmax(nan))
    return int(np.argmax(row))


def top_k_order(p_row: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest probabilities, probability descending then
    index ascending."""
    order = np.lexsort((np.arange(p_row.size), -p_row.astype(np.float64)))
    return order[:k]


def sample_tokens(logits: np.ndarray, temperature: float = 0.7, top_k: int = 50, seed: int = 0,
                  size: int = 32768, range_max: float = 10.0) -> Tuple[np.ndarray, np.ndarray]:
    """The reference's numpy sampler with the choices above fixed. Greedy:
    (int64 tokens, fp16 logprobs); sampling: (int32 tokens, float32 logprobs)."""
    x = np.asarray(logits)
    n, v = x.shape
    table = exp_table(size, range_max)
    step = table_step_f32(size, range_max)
    if temperature <= 0.0:
        tokens = np.array([first_argmax(x[r]) for r in range(n)], dtype=np.int64)
        probs = softmax_lut(x, table, step)
        lp = np.array([log_f32(probs[r, tokens[r]]) for r in range(n)], dtype=np.float32)
        return tokens, lp.astype(np.float16)
    scaled = scale_logits(x, temperature)
    uniq, inv = np.unique(scaled, axis=0, return_inverse=True)  # repeated rows: one softmax each
    probs = softmax_lut(uniq, table, step).astype(np.float32)[inv.reshape(-1)]
    k = min(top_k, v)
    tokens = np.zeros(n, dtype=np.int32)
    logprobs = np.zeros(n, dtype=np.float32)
    for r in range(n):
        p = probs[r]
        if np.isnan(p).any():  # a row whose maximum is not finite
            tokens[r] = first_argmax(x[r])
            logprobs[r] = np.nan
            continue
        idx = top_k_order(p, k)
        pk = p[idx]
        s = pairwise_sum_f32(pk)
        pk = (pk / s).astype(np.float32) if s > 0 else np.full(k, 1.0 / k)
        cdf = np.cumsum(pk.astype(np.float64))
        cdf /= cdf[-1]
        j = int(np.searchsorted(cdf, uniform(seed, r), side="right"))
        tokens[r] = idx[min(j, k - 1)]
        pc = p[tokens[r]]
        logprobs[r] = log_f32(pc) if pc >= 1e-10 else LOG_1E_10_F32
    return tokens, logprobs
