"""Token sampling on the GPU (``moat_amd/sampling.py`` -> ``moat_lut_softmax``,
``moat_sample_tokens``, ``moat_lut_lookup``) against the sampling oracle, bit
for bit: table lookups, fp16 probabilities, greedy tokens and fp16
log-probabilities, sampled tokens and float32 log-probabilities for the same
seed; the reference tests' known answers and extreme inputs; the LM head's
logits sampled straight from the GPU."""

import numpy as np
import pytest

from oracle import sampling_oracle as S

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def _rows(n, v, seed, dtype=np.float32, scale=3.0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, v)) * scale
    if n > 1:
        x[1] = x[1] * 10  # much of the row clamped at the table's end
    if n > 2 and v > 3:
        x[2, ::3] = -np.inf  # -inf logits are exp(-10) entries
    if n > 3:
        x[3] = 0.5  # uniform row: all ties
    if n > 4 and v > 2:
        # 60 equal maxima spread over the row (across its 8192-logit chunks
        # when it has several): the top 50 are the 50 lowest indices among them
        x[4, np.unique(np.linspace(v - 1, 0, 60).astype(np.int64))] = np.abs(x[4]).max() + 1.0
    return x.astype(dtype)


VOCABS = [1, 2, 7, 8, 9, 50, 100, 128, 129, 136, 540, 1000, 4096, 8192, 8193, 16385, 32000, 32768]
# GPT-2, Llama-3 and Qwen-2.5 vocabularies and the largest row (64 chunks)
LARGE_VOCABS = [50257, 128256, 151936, 524288]


def test_lookup_matches_oracle():
    import torch
    from moat_amd.sampling import ExponentialLUT
    say("case: lookup")
    for size, rmax in ((32768, 10.0), (1000, 4.0), (2, 1.0)):
        lut = ExponentialLUT(size, rmax)
        x = -np.abs(np.random.default_rng(size).standard_normal(20000).astype(np.float32)) * rmax * 1.2
        x[:4] = [0.0, -0.0, -np.inf, -rmax]
        got = lut.lookup(x)
        table = S.exp_table(size, rmax)
        assert np.array_equal(lut.lut.view(np.uint16), table.view(np.uint16))
        want = table[S.lut_index(x, size, S.table_step_f32(size, rmax))]
        assert got.dtype == np.float16 and np.array_equal(got.view(np.uint16), want.view(np.uint16))
        dev = lut.lookup(torch.from_numpy(x).cuda())
        assert dev.is_cuda and torch.equal(dev.cpu(), torch.from_numpy(got))


@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.float64])
def test_softmax_matches_oracle(dtype):
    from moat_amd.sampling import ExponentialLUT, safe_softmax_lut
    lut = ExponentialLUT()
    table, step = S.exp_table(), S.table_step_f32()
    for v in VOCABS:
        say(f"case: softmax dtype={np.dtype(dtype).name} v={v}")
        x = _rows(5, v, 100 + v, dtype)
        got = safe_softmax_lut(x, lut)
        want = S.softmax_lut(x, table, step)
        assert got.dtype == np.float16 and got.shape == x.shape
        bad = np.flatnonzero(got.view(np.uint16) != want.view(np.uint16))
        assert bad.size == 0, (v, bad[:10], got.reshape(-1)[bad[:5]], want.reshape(-1)[bad[:5]])


def test_softmax_axes_and_small_tables():
    from moat_amd.sampling import ExponentialLUT, safe_softmax_lut
    say("case: softmax axes")
    x = np.random.default_rng(5).standard_normal((3, 300, 4)).astype(np.float32) * 4
    lut = ExponentialLUT()
    got = safe_softmax_lut(x, lut, axis=1)
    want = np.moveaxis(S.softmax_lut(np.moveaxis(x, 1, -1).reshape(-1, 300), S.exp_table(), S.table_step_f32())
                       .reshape(3, 4, 300), -1, 1)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    small = ExponentialLUT(size=512, range_max=6.0)
    got = safe_softmax_lut(x[0], small, axis=0)
    want = S.softmax_lut(x[0].T, S.exp_table(512, 6.0), S.table_step_f32(512, 6.0)).T
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    with pytest.raises(ValueError):
        safe_softmax_lut(np.zeros((2, 0), np.float32), lut)
    with pytest.raises(ValueError):
        safe_softmax_lut(np.zeros((1, 524289), np.float32), lut)


def test_large_vocabularies():
    """Rows of many chunks: softmax (float32), greedy (fp16) and sampling
    (float32 at T = 0.7, float64 at T = 3) bit for bit against the oracle."""
    from moat_amd.sampling import ExponentialLUT, TokenSampler, safe_softmax_lut
    lut, sampler = ExponentialLUT(), TokenSampler()
    table, step = S.exp_table(), S.table_step_f32()
    for v in LARGE_VOCABS:
        say(f"case: large v={v} softmax")
        x = _rows(5, v, 700 + v)
        got = safe_softmax_lut(x, lut)
        assert np.array_equal(got.view(np.uint16), S.softmax_lut(x, table, step).view(np.uint16)), v
        say(f"case: large v={v} greedy")
        x = _rows(6, v, 800 + v, np.float16)
        tok, lp = sampler.sample_tokens(x, temperature=0.0)
        wt, wl = S.sample_tokens(x, temperature=0.0)
        assert np.array_equal(tok, wt) and np.array_equal(lp.view(np.uint16), wl.view(np.uint16)), (v, tok, wt)
        for dtype, temp in ((np.float32, 0.7), (np.float64, 3.0)):
            say(f"case: large v={v} sample dtype={np.dtype(dtype).name} T={temp}")
            x = _rows(7, v, 900 + v, dtype)
            tok, lp = sampler.sample_tokens(x, temperature=temp, seed=99 + v)
            wt, wl = S.sample_tokens(x, temperature=temp, seed=99 + v)
            assert np.array_equal(tok, wt), (v, temp, tok, wt)
            assert np.array_equal(lp.view(np.uint32), wl.view(np.uint32)), (v, temp, lp, wl)


@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.float64])
def test_greedy_matches_oracle(dtype):
    from moat_amd.sampling import TokenSampler
    sampler = TokenSampler()
    for v in VOCABS:
        say(f"case: greedy dtype={np.dtype(dtype).name} v={v}")
        x = _rows(6, v, 300 + v, dtype)
        tok, lp = sampler.sample_tokens(x, temperature=0.0)
        wt, wl = S.sample_tokens(x, temperature=0.0)
        assert tok.dtype == np.int64 and lp.dtype == np.float16
        assert np.array_equal(tok, wt), (v, tok, wt)
        assert np.array_equal(lp.view(np.uint16), wl.view(np.uint16)), (v, lp, wl)
    # the reference's known answer (tests/test_batch_generator.py:97-109)
    x = np.zeros((4, 100), np.float32)
    x[0, 10], x[1, 42], x[2, 7], x[3, 99] = 5.0, 10.0, 8.0, 12.0
    tok, _ = sampler.sample_tokens(x, temperature=0.0)
    assert np.array_equal(tok, [10, 42, 7, 99])


def test_greedy_argmax_in_the_input_dtype():
    """float64 logits that float32 cannot tell apart: the argmax is float64's."""
    from moat_amd.sampling import TokenSampler
    say("case: greedy f64 argmax")
    x = np.zeros((2, 1000), np.float64)
    x[0, 10], x[0, 20] = 1.0, 1.0 + 2.0 ** -40
    x[1, 5], x[1, 900] = 7.0, 7.0
    tok, lp = TokenSampler().sample_tokens(x, temperature=0.0)
    assert list(tok) == [20, 5]
    wt, wl = S.sample_tokens(x, temperature=0.0)
    assert list(wt) == [20, 5] and np.array_equal(lp.view(np.uint16), wl.view(np.uint16))


@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.float64])
def test_sampling_matches_oracle(dtype):
    from moat_amd.sampling import TokenSampler
    sampler = TokenSampler()
    for v in VOCABS:
        for temp in (0.7, 1e-10, 3.0):
            say(f"case: sample dtype={np.dtype(dtype).name} v={v} T={temp}")
            x = _rows(7, v, 500 + v, dtype)
            seed = 1234567 + v
            tok, lp = sampler.sample_tokens(x, temperature=temp, seed=seed)
            wt, wl = S.sample_tokens(x, temperature=temp, seed=seed)
            assert tok.dtype == np.int32 and lp.dtype == np.float32
            assert np.array_equal(tok, wt), (v, temp, tok, wt)
            assert np.array_equal(lp.view(np.uint32), wl.view(np.uint32)), (v, temp, lp, wl)


def test_sampling_distribution_and_seeds():
    """20000 rows of one distribution: every draw equals the oracle's for the
    same seed (so the chi-square of the oracle's draws carries over); seeds
    from numpy's global generator repeat under np.random.seed."""
    import torch
    from moat_amd.sampling import TokenSampler, sample_tokens
    say("case: distribution")
    rng = np.random.default_rng(11)
    row = (rng.standard_normal(300) * 1.5).astype(np.float32)
    logits = np.tile(row, (20000, 1))
    sampler = TokenSampler()
    tok, lp = sampler.sample_tokens(torch.from_numpy(logits).cuda(), temperature=0.8, seed=2024)
    assert tok.is_cuda and tok.dtype == torch.int32 and lp.dtype == torch.float32
    wt, wl = S.sample_tokens(logits, temperature=0.8, seed=2024)
    assert np.array_equal(tok.cpu().numpy(), wt) and np.array_equal(lp.cpu().numpy(), wl)
    assert len(set(wt.tolist())) > 20
    np.random.seed(7)
    a = sample_tokens(logits[:64], temperature=1.0)
    np.random.seed(7)
    b = sample_tokens(logits[:64], temperature=1.0)
    c = sample_tokens(logits[:64], temperature=1.0)
    assert np.array_equal(a[0], b[0]) and not np.array_equal(b[0], c[0])


def test_extreme_inputs():
    """tests/test_fuzz_extreme_inputs.py:32-60 and test_batch_generator.py:111-125
    of the reference, through the GPU sampler, and bit-equal to the oracle."""
    from moat_amd.sampling import TokenSampler
    say("case: extreme inputs")
    sampler = TokenSampler()
    rng = np.random.default_rng(1337)
    for i, logits in enumerate((rng.standard_normal((8, 1000)) * 1e8, -np.abs(rng.standard_normal((8, 1000))) * 1e8,
                                np.zeros((8, 1000), np.float32))):
        tok, lp = sampler.sample_tokens(logits, temperature=0.7, seed=i)
        assert not np.any(np.isnan(lp)) and not np.any(np.isinf(lp))
        wt, wl = S.sample_tokens(logits, temperature=0.7, seed=i)
        assert np.array_equal(tok, wt) and np.array_equal(lp, wl)
    logits = rng.standard_normal((8, 1000)).astype(np.float32)
    for temp in (0.0, 1e-10, 1e-5, 0.01, 1.0, 10.0, 100.0):
        tok, lp = sampler.sample_tokens(logits, temperature=temp, seed=3)
        assert len(tok) == 8 and not np.any(np.isnan(lp))
    tok, _ = sampler.sample_tokens(rng.standard_normal((16, 1000)).astype(np.float32), temperature=1.0, seed=4)
    assert len(set(tok.tolist())) > 1


def test_non_finite_rows():
    """A row whose maximum is NaN or +inf: NaN probabilities, the argmax
    rule's token and a NaN log-probability; other rows unaffected."""
    from moat_amd.sampling import ExponentialLUT, TokenSampler, safe_softmax_lut
    say("case: non-finite rows")
    x = np.random.default_rng(2).standard_normal((4, 500)).astype(np.float32)
    x[0, 30], x[0, 40] = np.nan, np.nan
    x[1, 7] = np.inf
    x[2, :] = -np.inf
    p = safe_softmax_lut(x, ExponentialLUT())
    assert np.all(np.isnan(p[:3].astype(np.float32)))
    want = S.softmax_lut(x[3:], S.exp_table(), S.table_step_f32())
    assert np.array_equal(p[3:].view(np.uint16), want.view(np.uint16))
    sampler = TokenSampler()
    for temp in (0.0, 0.7):
        tok, lp = sampler.sample_tokens(x, temperature=temp, seed=1)
        assert list(tok[:3]) == [30, 7, 0] and np.all(np.isnan(lp[:3].astype(np.float32)))
        wt, wl = S.sample_tokens(x, temperature=temp, seed=1)
        assert np.array_equal(tok, wt) and np.array_equal(lp, wl, equal_nan=True)
    # the same over a row of three 8192-logit chunks: the first NaN, the
    # first +inf and the first of equal maxima in different chunks
    say("case: non-finite rows, three chunks")
    x = np.random.default_rng(3).standard_normal((4, 20000)).astype(np.float32)
    x[0, 17000], x[0, 9000] = np.nan, np.nan
    x[1, 19999], x[1, 12000] = np.inf, np.inf
    x[2, 300], x[2, 8200], x[2, 16500] = 49.0, 50.0, 50.0
    p = safe_softmax_lut(x, ExponentialLUT())
    assert np.all(np.isnan(p[:2].astype(np.float32)))
    want = S.softmax_lut(x[2:], S.exp_table(), S.table_step_f32())
    assert np.array_equal(p[2:].view(np.uint16), want.view(np.uint16))
    for temp in (0.0, 0.7):
        tok, lp = sampler.sample_tokens(x, temperature=temp, seed=5)
        assert list(tok[:2]) == [9000, 12000] and np.all(np.isnan(lp[:2].astype(np.float32)))
        if temp == 0.0:
            assert tok[2] == 8200
        wt, wl = S.sample_tokens(x, temperature=temp, seed=5)
        assert np.array_equal(tok, wt) and np.array_equal(lp, wl, equal_nan=True)


def test_lm_head_logits_sampled_on_the_gpu():
    """The INT4 LM head (K=2048, V=32000, N=16) feeding the sampler without
    leaving the GPU: tokens equal the oracle's on the same logits."""
    import torch
    from oracle import superblock_oracle as O
    from moat_amd.dequant import batched_int4_matmul
    from moat_amd.sampling import TokenSampler
    say("case: lm head -> sampler")
    K, V, N = 2048, 32000, 16
    w = O.synthetic_weights(K, V, 0.02, 77)
    blob = torch.from_numpy(O.quantize_pack_a(w).reshape(-1)).cuda()
    x = torch.from_numpy(O.synthetic_activations(N, K, 78)).cuda()
    logits = batched_int4_matmul(x, blob, K, V)
    sampler = TokenSampler()
    host = logits.cpu().numpy()
    for temp in (0.0, 0.7):
        tok, lp = sampler.sample_tokens(logits, temperature=temp, seed=99)
        wt, wl = S.sample_tokens(host, temperature=temp, seed=99)
        assert np.array_equal(tok.cpu().numpy(), wt)
        assert np.array_equal(lp.cpu().numpy().view(np.uint16 if temp == 0 else np.uint32),
                              wl.view(np.uint16 if temp == 0 else np.uint32))


def test_workspace_counters_return_to_zero():
    """The per-row counters at the start of the sampling workspace (the last
    of a row's chunk workgroups takes over the row) are zero after every
    call, so one workspace serves calls of any shape in turn."""
    import torch
    from moat_amd import _device as D
    from moat_amd.sampling import TokenSampler
    say("case: workspace counters")
    sampler = TokenSampler()
    x = _rows(9, 20000, 31)  # three chunks per row
    for temp in (0.0, 0.7, 0.0, 2.0):
        tok, lp = sampler.sample_tokens(x, temperature=temp, seed=8)
        wt, wl = S.sample_tokens(x, temperature=temp, seed=8)
        assert np.array_equal(tok, wt) and np.array_equal(lp.view(np.uint16 if temp == 0 else np.uint32),
                                                          wl.view(np.uint16 if temp == 0 else np.uint32))
        torch.cuda.synchronize()
        ws = D.sample_workspaces.get(1)
        assert int(torch.count_nonzero(ws[:4 * 9])) == 0, temp
    # a workspace full of stale bytes: every call sets up its own counters
    ws.fill_(0xAB)
    for temp in (0.0, 0.7):
        tok, lp = sampler.sample_tokens(x, temperature=temp, seed=9)
        wt, wl = S.sample_tokens(x, temperature=temp, seed=9)
        assert np.array_equal(tok, wt) and np.array_equal(lp.view(np.uint16 if temp == 0 else np.uint32),
                                                          wl.view(np.uint16 if temp == 0 else np.uint32))
        ws.fill_(0xAB)


def test_softmax_rows_past_one_call():
    """More rows than one call takes (2^21): the softmax runs in slices of
    rows; rows on both sides of the slice boundary and a sample of the rest
    equal the oracle."""
    import torch
    from moat_amd.sampling import ExponentialLUT, safe_softmax_lut, _MAX_ROWS
    say("case: softmax rows past one call")
    rows = _MAX_ROWS + 3
    x = torch.randn((rows, 2), dtype=torch.float32, device="cuda") * 3
    got = safe_softmax_lut(x, ExponentialLUT()).cpu().numpy()
    xh = x.cpu().numpy()
    pick = np.concatenate([np.arange(_MAX_ROWS - 3, rows), np.random.default_rng(4).integers(0, rows, 200)])
    want = S.softmax_lut(xh[pick], S.exp_table(), S.table_step_f32())
    assert np.array_equal(got[pick].view(np.uint16), want.view(np.uint16))
