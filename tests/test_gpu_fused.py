"""Fused record-stream launches on the GPU: several projections of one shape
sharing X (``moat_int4_gemm_multi``) and the SwiGLU gate/up pair
(``moat_int4_gemm_swiglu``), against the oracle (``gemm_ref`` /
``swiglu_ref``), against the single-matrix path, and sharing one workspace
with it."""

import numpy as np
import pytest

from oracle import superblock_oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3


def say(msg):
    print(msg, flush=True)


def rel_err(y, ref):
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.max(np.abs(np.asarray(y, dtype=np.float64) - ref)) / np.sqrt(np.mean(ref ** 2)))


def _blobs(K, M, count, seed):
    import torch
    out = []
    for i in range(count):
        w = O.synthetic_weights(K, M, 0.02, seed + 17 * i)
        b = O.quantize_pack_a(w)
        out.append((b, torch.from_numpy(b.reshape(-1)).cuda()))
    return out


@pytest.mark.parametrize("K,M,count", [(2048, 2048, 3), (2048, 5632, 2), (96, 640, 4), (64, 384, 1), (32, 128, 3)])
def test_multi_matches_oracle(K, M, count):
    import torch
    from moat_amd.dequant import batched_int4_matmul, batched_int4_matmul_multi
    blobs = _blobs(K, M, count, 300 + K + M)
    for N in (1, 5, 16, 17, 32):
        say(f"case: multi K={K} M={M} count={count} N={N}")
        x = O.synthetic_activations(N, K, 40 + N)
        xd = torch.from_numpy(x).cuda()
        ys = batched_int4_matmul_multi(xd, [b for _, b in blobs], K, M)
        assert len(ys) == count
        for (bh, bd), y in zip(blobs, ys):
            yh = y.cpu().numpy()
            assert rel_err(yh, O.gemm_ref(x, bh, K, M)) <= TOL, (K, M, count, N)
            single = batched_int4_matmul(xd, bd, K, M).cpu().numpy()
            assert rel_err(yh, single) <= 1e-5, (K, M, count, N)


@pytest.mark.parametrize("K,M", [(2048, 5632), (96, 640), (64, 384), (3072, 8192)])
def test_swiglu_matches_oracle(K, M):
    import torch
    from moat_amd.dequant import batched_int4_matmul, int4_swiglu
    (gh, gd), (uh, ud) = _blobs(K, M, 2, 500 + K + M)
    for N in (1, 3, 16, 17, 32):
        say(f"case: swiglu K={K} M={M} N={N}")
        x = O.synthetic_activations(N, K, 60 + N)
        xd = torch.from_numpy(x).cuda()
        h = int4_swiglu(xd, gd, ud, K, M)
        assert h.dtype == torch.float16 and tuple(h.shape) == (N, M)
        hh = h.cpu().numpy().astype(np.float64)
        ref = O.swiglu_ref(x, gh, uh, K, M)
        # fp16 output: half an ulp of each value on top of the GEMM tolerance
        bound = 2.0 ** -11 * np.abs(ref) + TOL * np.sqrt(np.mean(ref ** 2))
        assert np.all(np.abs(hh - ref) <= bound), (K, M, N, float(np.max(np.abs(hh - ref) - bound)))
        # the same activation on our own two projections, rounded to fp16 once
        g = batched_int4_matmul(xd, gd, K, M).cpu().numpy()
        u = batched_int4_matmul(xd, ud, K, M).cpu().numpy()
        mine = O.silu_mul(g, u).astype(np.float16).astype(np.float64)
        assert np.all(np.abs(hh - mine) <= 2.0 ** -10 * np.abs(mine) + 1e-5 * np.sqrt(np.mean(mine ** 2))), (K, M, N)


def test_fused_and_single_share_a_workspace():
    """Fused and single calls alternate on one stream (one workspace): every
    hand-off leaves the workspace zero for the next."""
    import torch
    from moat_amd.dequant import batched_int4_matmul, batched_int4_matmul_multi, int4_swiglu
    K, M = 2048, 2048
    blobs = _blobs(K, M, 3, 900)
    for rep in range(3):
        for N in (1, 4, 16, 32):
            say(f"case: shared workspace rep={rep} N={N}")
            x = O.synthetic_activations(N, K, 70 + N)
            xd = torch.from_numpy(x).cuda()
            refs = [O.gemm_ref(x, bh, K, M) for bh, _ in blobs]
            ys = batched_int4_matmul_multi(xd, [b for _, b in blobs], K, M)
            for y, r in zip(ys, refs):
                assert rel_err(y.cpu().numpy(), r) <= TOL
            y0 = batched_int4_matmul(xd, blobs[0][1], K, M)
            assert rel_err(y0.cpu().numpy(), refs[0]) <= TOL
            h = int4_swiglu(xd, blobs[1][1], blobs[2][1], K, M).cpu().numpy().astype(np.float64)
            ref = O.silu_mul(refs[1], refs[2])
            assert np.all(np.abs(h - ref) <= 2.0 ** -11 * np.abs(ref) + TOL * np.sqrt(np.mean(ref ** 2)))
