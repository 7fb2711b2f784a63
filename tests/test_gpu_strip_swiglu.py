"""The gate/up projections with SwiGLU in one strip-order launch
(``moat_int4_gemm_strips_swiglu``) on the GPU: against the oracle
(``swiglu_ref``: silu(X @ W_gate) * (X @ W_up) in float64), against the same
activation on this library's own strip-order GEMM of ``[W_gate | W_up]``, and
over workgroup counts that give every workgroup one or several gate/up pairs
and the last one fewer."""

import numpy as np
import pytest

from oracle import superblock_oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3


def say(msg):
    print(msg, flush=True)


_cache = {}


def _problem(K, M, seed):
    """Row-order records of W_gate and W_up, their decoded float32 weights,
    and the interleaved strip stream on the GPU."""
    import torch
    from moat_amd.dequant import interleave_strips, records_to_strips
    key = (K, M, seed)
    if key not in _cache:
        out = []
        for i in range(2):
            w = O.synthetic_weights(K, M, 0.02, seed + 31 * i)
            blob = O.quantize_pack_a(w).reshape(-1)
            wdq = O.decode_superblocks(blob, K * M // 256).astype(np.float32).reshape(K, M)
            out.append((blob, wdq))
        (gb, gw), (ub, uw) = out
        gs = records_to_strips(torch.from_numpy(gb).cuda(), K, M)
        us = records_to_strips(torch.from_numpy(ub).cuda(), K, M)
        _cache[key] = (gb, gw, ub, uw, gs, us, interleave_strips(gs, us, K, M))
    return _cache[key]


def test_interleave_strips_places_gate_and_up_strips():
    import torch
    from moat_amd.dequant import interleave_strips
    K, M = 2048, 96
    strip = K * 18
    g = torch.arange(K * M // 256 * 144, dtype=torch.int64).remainder(251).to(torch.uint8).cuda()
    u = torch.arange(K * M // 256 * 144, dtype=torch.int64).remainder(241).to(torch.uint8).cuda()
    out = interleave_strips(g, u, K, M).cpu().numpy()
    gh, uh = g.cpu().numpy(), u.cpu().numpy()
    for c in range(M // 32):
        assert np.array_equal(out[2 * c * strip:(2 * c + 1) * strip], gh[c * strip:(c + 1) * strip])
        assert np.array_equal(out[(2 * c + 1) * strip:(2 * c + 2) * strip], uh[c * strip:(c + 1) * strip])


@pytest.mark.parametrize("K,M", [(2048, 5632), (3072, 8192), (2048, 14336), (2048, 8224), (2048, 32)])
def test_strip_swiglu_matches_oracle(K, M):
    import torch
    from moat_amd.dequant import batched_int4_matmul, int4_swiglu_strips
    gb, gw, ub, uw, gs, us, gu = _problem(K, M, 800 + K + M)
    pairs = M // 32
    cat = torch.cat([gs, us])  # [W_gate | W_up] in strip order: the unfused path's matrix
    for N in (1, 5, 8, 9, 16, 17, 32):
        x = O.synthetic_activations(N, K, 90 + N)
        xd = torch.from_numpy(x).cuda()
        x32 = x.astype(np.float32)
        ref = O.silu_mul(x32 @ gw, x32 @ uw)
        bound = 2.0 ** -11 * np.abs(ref) + TOL * np.sqrt(np.mean(ref ** 2))
        y = batched_int4_matmul(xd, cat, K, 2 * M, strip_order=True).cpu().numpy()
        mine = O.silu_mul(y[:, :M], y[:, M:]).astype(np.float16).astype(np.float64)
        for splits in (0, 1, 3, 100, 256):
            if splits > pairs:
                continue
            say(f"case: strip swiglu K={K} M={M} N={N} workgroups={splits}")
            h = int4_swiglu_strips(xd, gu, K, M, splits=splits)
            assert h.dtype == torch.float16 and tuple(h.shape) == (N, M)
            hh = h.cpu().numpy().astype(np.float64)
            assert np.all(np.abs(hh - ref) <= bound), (K, M, N, splits, float(np.max(np.abs(hh - ref) - bound)))
            # the same activation on this library's own unfused strip GEMM: equal
            # up to float32 summation order and one fp16 rounding
            assert np.all(np.abs(hh - mine) <= 2.0 ** -10 * np.abs(mine) + 1e-5 * np.sqrt(np.mean(mine ** 2))), \
                (K, M, N, splits)


def test_strip_swiglu_repeated_calls_and_row_slices():
    """N above 32 goes in slices of 32 rows; calls in a row on one stream
    leave nothing behind (no workspace)."""
    import torch
    from moat_amd.dequant import int4_swiglu_strips
    K, M = 2048, 5632
    gb, gw, ub, uw, gs, us, gu = _problem(K, M, 800 + K + M)
    for N in (40, 3, 64):
        say(f"case: strip swiglu rows={N}")
        x = O.synthetic_activations(N, K, 300 + N)
        x32 = x.astype(np.float32)
        ref = O.silu_mul(x32 @ gw, x32 @ uw)
        h = int4_swiglu_strips(torch.from_numpy(x).cuda(), gu, K, M).cpu().numpy().astype(np.float64)
        assert np.all(np.abs(h - ref) <= 2.0 ** -11 * np.abs(ref) + TOL * np.sqrt(np.mean(ref ** 2))), N
