"""Pins of the sampling oracle (``oracle/sampling_oracle.py``) on the CPU:
numpy's own float32 sum, the reference tests' known answers for the exp table
and the sampler, closed forms of the table softmax, and the distribution of
the draws."""

import math

import numpy as np
import pytest

from oracle import sampling_oracle as S


def test_numpy_sum_order_matches_np_sum():
    """The restated order gives np.sum's bits: 1-D, and along the last axis of
    2-D arrays, for every length class."""
    assert np.getbufsize() == 8192
    rng = np.random.default_rng(0)
    lengths = list(range(0, 140)) + [255, 256, 257, 519, 540, 1000, 1023, 4096, 8191, 8192, 8193, 9000,
                                     16385, 24577, 32000, 32768]
    for n in lengths:
        for scale in (1e-3, 1.0, 1e4):
            a = (rng.standard_normal(n) * scale).astype(np.float32)
            assert S.numpy_sum_f32(a).tobytes() == np.float32(np.sum(a)).tobytes(), n
            m = np.stack([a, np.abs(a), a[::-1]])
            want = np.sum(m, axis=-1, keepdims=True)
            for r in range(3):
                assert S.numpy_sum_f32(m[r]).tobytes() == want[r, 0].tobytes(), (n, r)
    # a plausible mistake fails: one pairwise pass over the whole row
    a = (rng.standard_normal(32000) * 100).astype(np.float32)
    wrong = [S.pairwise_sum_f32(b) for b in (a, a * 3, a + 1)]
    right = [np.sum(b) for b in (a, (a * 3).astype(np.float32), (a + 1).astype(np.float32))]
    assert any(w.tobytes() != np.float32(r).tobytes() for w, r in zip(wrong, right))


def test_exp_table_known_answers():
    """tests/test_attention.py of the reference (construction and lookup)."""
    t = S.exp_table()
    assert t.size == 32768 and t.dtype == np.float16 and t.nbytes == 65536
    assert abs(float(t[-1]) - 1.0) < 0.01 and float(t[-1]) == 1.0
    assert 0.0 < float(t[0]) < 0.001
    assert np.all(np.diff(t.astype(np.float32)) >= 0)
    step = S.table_step_f32()
    look = lambda x: t[S.lut_index(np.asarray(x, np.float32), t.size, step)]
    assert abs(float(look([0.0])[0]) - 1.0) < 0.01
    assert abs(float(look([-1.0])[0]) - math.exp(-1)) / math.exp(-1) < 0.02
    assert abs(float(look([-5.0])[0]) - math.exp(-5)) / math.exp(-5) < 0.05
    x = np.linspace(-10, 0, 10000, dtype=np.float32)
    assert np.mean(np.abs(look(x).astype(np.float32) - np.exp(x))) < 0.01
    assert np.all(np.isfinite(look([-20.0, -100.0, -1e6, -np.inf]).astype(np.float32)))
    # every entry is exp of its grid point within fp16 rounding
    grid = np.linspace(-10.0, 0.0, 32768, dtype=np.float32).astype(np.float64)
    assert np.all(np.abs(t.astype(np.float64) - np.exp(grid)) <= 2.0 ** -11 * np.exp(grid) + 2.0 ** -25)
    with pytest.raises(ValueError):
        S.exp_table(size=1)
    with pytest.raises(ValueError):
        S.exp_table(range_max=-1.0)


def test_softmax_lut_closed_forms():
    t = S.exp_table()
    step = S.table_step_f32()
    for v in (1, 7, 100, 1000, 8193, 32000):
        # uniform rows: every probability is fp16(1 / V) (exact sum of ones)
        p = S.softmax_lut(np.full((2, v), 3.25, np.float32), t, step)
        assert np.all(p == np.float16(np.float32(1.0) / np.float32(v)))
    # one-hot rows: the peak against V-1 tail entries of exp(-10)
    x = np.zeros((1, 1000), np.float32)
    x[0, 17] = 50.0
    p = S.softmax_lut(x, t, step)
    tail = np.float32(t[0])
    assert p[0, 17] == np.float16(np.float32(1.0) / S.numpy_sum_f32(np.r_[np.ones(1), np.full(999, tail)]))
    # random rows: sums near 1, monotone in the logit, the exact softmax within
    # the table's quantisation (one step of exp's argument) and fp16 rounding
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((4, 5000)) * 2).astype(np.float32)
    p = S.softmax_lut(x, t, step).astype(np.float64)
    assert np.all(np.abs(p.sum(axis=1) - 1) < 5e-3)
    for r in range(4):
        o = np.argsort(x[r], kind="stable")
        assert np.all(np.diff(p[r][o]) >= 0)
        sh = x[r].astype(np.float64) - x[r].max()
        ex = np.exp(np.maximum(sh, -10.0))  # the table clamps below -range_max
        ex /= ex.sum()
        assert np.all(np.abs(p[r] - ex) <= ex * (float(step) + 2e-3) + 2.0 ** -24)
        assert np.all(p[r][sh < -10.0] == p[r][np.argmin(x[r])])


def test_greedy_known_answer_and_logprob():
    """tests/test_batch_generator.py:97-109 of the reference."""
    x = np.zeros((4, 100), np.float32)
    x[0, 10], x[1, 42], x[2, 7], x[3, 99] = 5.0, 10.0, 8.0, 12.0
    tok, lp = S.sample_tokens(x, temperature=0.0)
    assert tok.dtype == np.int64 and lp.dtype == np.float16
    assert np.array_equal(tok, [10, 42, 7, 99])
    p = S.softmax_lut(x, S.exp_table(), S.table_step_f32())
    assert np.all(lp == np.log(p[np.arange(4), tok]))
    # first maximum wins, and a NaN counts as the maximum (np.argmax)
    y = np.array([[1.0, 3.0, 3.0, 2.0], [1.0, np.nan, 5.0, np.nan]], np.float32)
    assert S.first_argmax(y[0]) == 1 and S.first_argmax(y[1]) == 1


def test_fp16_log_is_f32_log_rounded():
    """numpy's fp16 log (the greedy log-probability's dtype) equals the
    correctly rounded float32 log rounded to fp16, for every fp16 value in (0, 1]."""
    bits = np.arange(1, 0x3C01, dtype=np.uint16)
    p = bits.view(np.float16)
    mine = np.array([S.log_f32(v) for v in p.astype(np.float32)], np.float32).astype(np.float16)
    assert np.array_equal(np.log(p).view(np.uint16), mine.view(np.uint16))


def test_sampling_extreme_inputs():
    """tests/test_fuzz_extreme_inputs.py:32-60 of the reference: huge, tiny and
    zero logits and temperatures from 0 to 100 give no NaN."""
    rng = np.random.default_rng(1337)
    for logits in (rng.standard_normal((8, 1000)) * 1e8, -np.abs(rng.standard_normal((8, 1000))) * 1e8,
                   np.zeros((8, 1000), np.float32)):
        tok, lp = S.sample_tokens(logits, temperature=0.7, seed=5)
        assert not np.any(np.isnan(lp)) and not np.any(np.isinf(lp)) and np.all((tok >= 0) & (tok < 1000))
    logits = rng.standard_normal((8, 1000)).astype(np.float32)
    for temp in (0.0, 1e-10, 1e-5, 0.01, 1.0, 10.0, 100.0):
        tok, lp = S.sample_tokens(logits, temperature=temp, seed=6)
        assert len(tok) == 8 and not np.any(np.isnan(lp))
    # diversity at T = 1 over 16 channels (tests/test_batch_generator.py:111-125)
    tok, _ = S.sample_tokens(rng.standard_normal((16, 1000)).astype(np.float32), temperature=1.0, seed=7)
    assert len(set(tok.tolist())) > 1


def test_draws_follow_the_top_k_distribution():
    """Chi-square of 20000 draws of one row against its renormalised top-50
    probabilities; every draw inside the top-50 set; log-probabilities are the
    full softmax's."""
    rng = np.random.default_rng(11)
    row = (rng.standard_normal(300) * 1.5).astype(np.float32)
    reps = 20000
    logits = np.tile(row, (reps, 1))
    tok, lp = S.sample_tokens(logits, temperature=0.8, seed=2024)
    p = S.softmax_lut(S.scale_logits(row[None], 0.8), S.exp_table(), S.table_step_f32())[0].astype(np.float64)
    top = S.top_k_order(p.astype(np.float32), 50)
    assert set(tok.tolist()) <= set(top.tolist())
    assert np.all(p[top].min() >= np.delete(p, top).max())
    q = p[top] / p[top].sum()
    counts = np.array([np.sum(tok == i) for i in top], np.float64)
    keep = q * reps >= 5
    chi2 = np.sum((counts[keep] - q[keep] * reps) ** 2 / (q[keep] * reps))
    dof = int(keep.sum()) - 1
    assert chi2 < dof + 6 * math.sqrt(2 * dof), (chi2, dof)
    assert np.all(lp == np.array([S.log_f32(p[t]) for t in tok], np.float32))
    # the generator: uniform on [0, 1), rows independent
    u = np.array([S.uniform(99, r) for r in range(20000)])
    assert 0 <= u.min() and u.max() < 1 and abs(u.mean() - 0.5) < 0.01 and abs(np.corrcoef(u[:-1], u[1:])[0, 1]) < 0.03


def test_ties_taken_lowest_index_first():
    """With more equal probabilities than k, the k lowest indices form the set."""
    x = np.zeros((1, 200), np.float32)
    x[0, 150] = 1.0
    p = S.softmax_lut(S.scale_logits(x, 1.0), S.exp_table(), S.table_step_f32())[0]
    top = S.top_k_order(p.astype(np.float32), 50)
    assert top[0] == 150 and list(top[1:]) == list(range(49))
