"""Strip order on the GPU: the conversion kernel against the oracle's
byte-level restatement, and the strip GEMM against the oracle (dequantize the
row-order stream, float32 matmul) within 1e-3 of the output RMS -- every
plan shape (one whole strip per workgroup, strips shared by several
workgroups, ranges over several strips), N from 1 to 32 (the strip kernel
up to 8 rows, the wide strip kernel beyond; on request the strip-group
kernel or 8-row launches), every ring depth, wave count and forced
workgroup counts -- plus determinism, GEMM(N)
against stacked single-row products, and a workspace shared with the
row-order kernels."""

import sys

import numpy as np
import pytest
import torch

from oracle import superblock_oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def rel_err(y, yref):
    rms = float(np.sqrt(np.mean(yref.astype(np.float64) ** 2)))
    return float(np.max(np.abs(y.astype(np.float64) - yref))) / max(rms, 1e-30)


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from moat_amd import _lib
    _lib.load()


_cache = {}


def problem(K, M, seed):
    key = (K, M, seed)
    if key not in _cache:
        w = O.synthetic_weights(K, M, 0.02, seed)
        blob = O.quantize_pack_a(w).reshape(-1)
        wdq = O.decode_superblocks(blob, K * M // 256).astype(np.float32).reshape(K, M)
        _cache[key] = (blob, wdq)
    return _cache[key]


@pytest.mark.parametrize("K,M", [(8, 32), (40, 256), (64, 160), (2048, 5504), (3072, 8192)])
def test_records_to_strips_matches_oracle(K, M):
    from moat_amd.dequant import records_to_strips
    blob, _ = problem(K, M, 5 + K + M)
    say(f"case: records_to_strips K={K} M={M}")
    got = records_to_strips(torch.from_numpy(blob).cuda(), K, M).cpu().numpy()
    assert np.array_equal(got, O.records_to_strips(blob, K, M))


CASES = [
    (2048, 2048, [1, 2, 3, 4, 5, 8, 16, 32]),   # 64 strips: four workgroups per strip
    (3072, 8192, [1, 2, 4, 8, 32]),             # 256 strips: one whole strip per workgroup
    (2048, 5504, [1, 4, 8]),                    # 172 strips: one whole strip per workgroup
    (2048, 32, [1, 8]),                         # one strip over four workgroups
    (2048, 32000, [1, 8]),                      # 1000 strips: ranges of about four strips
    (5632, 2048, [1, 16]),                      # the down projection's shape
]


@pytest.mark.parametrize("K,M,ns", CASES)
def test_strip_gemm_matches_oracle(K, M, ns):
    from moat_amd.dequant import batched_int4_matmul, records_to_strips
    blob, wdq = problem(K, M, 7 + K + M)
    strips = records_to_strips(torch.from_numpy(blob).cuda(), K, M)
    for N in ns:
        x = O.synthetic_activations(N, K, 30 + N)
        yref = x.astype(np.float32) @ wdq
        say(f"case: strip gemm K={K} M={M} N={N}")
        y = batched_int4_matmul(torch.from_numpy(x).cuda(), strips, K, M, strip_order=True)
        assert rel_err(y.cpu().numpy(), yref) <= TOL, (K, M, N)


@pytest.mark.parametrize("K,M", [(2048, 2048), (3072, 8192), (2048, 1024)])
def test_strip_gemm_forced_plans(K, M):
    """Workgroup counts that make ranges start and end anywhere in a strip,
    ring depths 2 and 3 and every wave count (N=8 always runs on 4 waves)."""
    from moat_amd.dequant import batched_int4_matmul, records_to_strips
    blob, wdq = problem(K, M, 9 + K + M)
    strips = records_to_strips(torch.from_numpy(blob).cuda(), K, M)
    for N in (1, 3, 8):
        x = O.synthetic_activations(N, K, 50 + N)
        yref = x.astype(np.float32) @ wdq
        xd = torch.from_numpy(x).cuda()
        for splits in (1, 2, 3, 7, 33, 100, 255, 256):
            for depth in (2, 3):
                for waves in (4, 8, 12):
                    say(f"case: strip gemm K={K} M={M} N={N} workgroups={splits} depth={depth} waves={waves}")
                    y = batched_int4_matmul(xd, strips, K, M, strip_order=True, splits=splits, batch=depth,
                                            waves=waves)
                    assert rel_err(y.cpu().numpy(), yref) <= TOL, (K, M, N, splits, depth, waves)


@pytest.mark.parametrize("K,M", [(2048, 2048), (3072, 8192), (2048, 1056), (2048, 5504), (5632, 2048)])
def test_strip_wide_gemm_forced_plans(K, M):
    """N > 8 runs the wide strip kernel (all rows in one launch, one or two
    16-row tiles): the automatic plan and workgroup counts that make ranges
    start and end anywhere in a strip (several workgroups per strip, ranges
    over several strips, one workgroup for everything)."""
    from moat_amd.dequant import batched_int4_matmul, records_to_strips
    blob, wdq = problem(K, M, 17 + K + M)
    strips = records_to_strips(torch.from_numpy(blob).cuda(), K, M)
    total = (M // 32) * (K // 32)
    for N in (9, 16, 17, 24, 32):
        x = O.synthetic_activations(N, K, 170 + N)
        yref = x.astype(np.float32) @ wdq
        xd = torch.from_numpy(x).cuda()
        for splits in (0, 1, 2, 3, 7, 33, 100, 255, 256):
            if splits > total:
                continue
            say(f"case: wide strip gemm K={K} M={M} N={N} workgroups={splits}")
            y = batched_int4_matmul(xd, strips, K, M, strip_order=True, splits=splits)
            assert rel_err(y.cpu().numpy(), yref) <= TOL, (K, M, N, splits)
        say(f"case: strip gemm K={K} M={M} N={N} as 8-row launches")
        y = batched_int4_matmul(xd, strips, K, M, strip_order=True, group=2)
        assert rel_err(y.cpu().numpy(), yref) <= TOL, (K, M, N, "slices")
        for su, depth in ((1, 2), (1, 4), (2, 3), (4, 2)):
            say(f"case: wide strip gemm K={K} M={M} N={N} units a stage={su} depth={depth}")
            y = batched_int4_matmul(xd, strips, K, M, strip_order=True, group=3, front=su, batch=depth)
            assert rel_err(y.cpu().numpy(), yref) <= TOL, (K, M, N, su, depth)
    for N in (1, 3, 5, 8):  # 8 rows staged
        x = O.synthetic_activations(N, K, 270 + N)
        yref = x.astype(np.float32) @ wdq
        xd = torch.from_numpy(x).cuda()
        for splits in (0, 3, 100, 256):
            for su in (0, 2, 8):
                if splits > total:
                    continue
                say(f"case: wide strip gemm K={K} M={M} N={N} workgroups={splits} units a stage={su}")
                y = batched_int4_matmul(xd, strips, K, M, strip_order=True, group=3, splits=splits, front=su)
                assert rel_err(y.cpu().numpy(), yref) <= TOL, (K, M, N, splits, su)


@pytest.mark.parametrize("K,M", [(2048, 2048), (3072, 8192), (2048, 1056), (2048, 32000)])
def test_strip_dot2_variant_matches_oracle(K, M):
    """The strip kernel's vector-ALU variant (algo=MOAT_GEMM_DOT2: v_dot2 and
    a reduction across the four lanes of a column pair), N = 1..4, with the
    automatic and forced workgroup counts and every wave count; N = 5 is
    refused."""
    from moat_amd import _lib as L
    from moat_amd.dequant import batched_int4_matmul, records_to_strips
    blob, wdq = problem(K, M, 19 + K + M)
    strips = records_to_strips(torch.from_numpy(blob).cuda(), K, M)
    total = (M // 32) * (K // 32)
    for N in (1, 2, 3, 4):
        x = O.synthetic_activations(N, K, 190 + N)
        yref = x.astype(np.float32) @ wdq
        xd = torch.from_numpy(x).cuda()
        for splits in (0, 1, 7, 100, 256):
            for waves in (0, 4, 8, 12):
                if splits > total:
                    continue
                say(f"case: dot2 strip gemm K={K} M={M} N={N} workgroups={splits} waves={waves}")
                y = batched_int4_matmul(xd, strips, K, M, strip_order=True, algo=L.GEMM_DOT2, splits=splits,
                                        waves=waves)
                assert rel_err(y.cpu().numpy(), yref) <= TOL, (K, M, N, splits, waves)
    with pytest.raises(ValueError):
        batched_int4_matmul(torch.zeros((5, K), dtype=torch.float16, device="cuda"), strips, K, M, strip_order=True,
                            algo=L.GEMM_DOT2)


@pytest.mark.parametrize("K,M", [(2048, 2048), (3072, 8192), (2048, 1056)])
def test_strip_group_gemm_forced_plans(K, M):
    """On request (group=1) N > 8 runs the strip-group kernel (8 strips a
    group, one launch): workgroup counts that split groups anywhere, a
    partial last group (M/32 not a multiple of 8), both ring depths, one and
    two 16-row tiles."""
    from moat_amd.dequant import batched_int4_matmul, records_to_strips
    blob, wdq = problem(K, M, 13 + K + M)
    strips = records_to_strips(torch.from_numpy(blob).cuda(), K, M)
    groups = (M // 32 + 7) // 8
    for N in (9, 16, 17, 32):
        x = O.synthetic_activations(N, K, 70 + N)
        yref = x.astype(np.float32) @ wdq
        xd = torch.from_numpy(x).cuda()
        for splits in (1, 2, 3, 7, 33, 100, 255, 256):
            if splits > groups * (K // 32):
                continue
            for depth in (2, 3):
                say(f"case: strip group gemm K={K} M={M} N={N} workgroups={splits} depth={depth}")
                y = batched_int4_matmul(xd, strips, K, M, strip_order=True, splits=splits, batch=depth, group=1)
                assert rel_err(y.cpu().numpy(), yref) <= TOL, (K, M, N, splits, depth)


def test_strip_gemm_is_deterministic_and_equals_stacked_gemv():
    from moat_amd.dequant import batched_int4_matmul, records_to_strips
    K, M = 2048, 2048
    blob, _ = problem(K, M, 77)
    strips = records_to_strips(torch.from_numpy(blob).cuda(), K, M)
    for N in (8, 32):
        x = torch.from_numpy(O.synthetic_activations(N, K, 78 + N)).cuda()
        say(f"case: strip gemm determinism and stacked GEMVs N={N}")
        ref = batched_int4_matmul(x, strips, K, M, strip_order=True)
        for _ in range(20):
            assert torch.equal(batched_int4_matmul(x, strips, K, M, strip_order=True), ref)
        rows = torch.cat([batched_int4_matmul(x[i:i + 1], strips, K, M, strip_order=True) for i in range(N)])
        assert rel_err(ref.cpu().numpy(), rows.cpu().numpy()) <= TOL


def test_strip_gemm_shares_the_workspace_with_row_order_calls():
    from moat_amd import _lib as L
    from moat_amd.dequant import batched_int4_matmul, records_to_strips
    K, M = 2048, 5504
    blob, wdq = problem(K, M, 91)
    blob_d = torch.from_numpy(blob).cuda()
    strips = records_to_strips(blob_d, K, M)
    for N in (1, 4, 8):
        x = O.synthetic_activations(N, K, 92 + N)
        yref = x.astype(np.float32) @ wdq
        xd = torch.from_numpy(x).cuda()
        for rep in range(3):
            for kind in ("strips", "records", "groups", "strips64", "wide", "general", "groups64", "wide64",
                         "strips"):
                say(f"case: shared workspace N={N} rep={rep} {kind}")
                if kind == "strips":
                    y = batched_int4_matmul(xd, strips, K, M, strip_order=True)
                elif kind == "strips64":
                    y = batched_int4_matmul(xd, strips, K, M, strip_order=True, splits=64)
                elif kind in ("groups", "groups64", "wide", "wide64"):  # 16 rows, first N compared
                    x16 = torch.cat([xd, xd.new_zeros((16 - N, K))]) if N < 16 else xd
                    y = batched_int4_matmul(x16, strips, K, M, strip_order=True,
                                            splits=64 if kind.endswith("64") else 0,
                                            group=1 if kind.startswith("groups") else 0)[:N]
                elif kind == "records":
                    y = batched_int4_matmul(xd, blob_d, K, M, algo=L.GEMM_MFMA, splits=8, front=L.FRONT_RECORDS)
                else:
                    y = batched_int4_matmul(xd, blob_d, K, M, algo=L.GEMM_MFMA, splits=3, finish=1, front=L.FRONT_LDS)
                assert rel_err(y.cpu().numpy(), yref) <= TOL, (N, rep, kind)


def test_strip_gemm_largest_projection_matches_row_order():
    """K=8192 x M=28672 (0.1 % outliers at 8 sigma): the strip GEMM equals the
    row-order GEMM (itself checked against the oracle at this shape)."""
    from moat_amd.dequant import batched_int4_matmul, quantize_to_superblocks, records_to_strips
    K, M = 8192, 28672
    w = O.synthetic_weights(K, M, 0.01, 1005, outlier_frac=0.001)
    blob = quantize_to_superblocks(torch.from_numpy(w).cuda()).reshape(-1)
    del w
    strips = records_to_strips(blob, K, M)
    for N in (1, 8, 32):
        x = torch.from_numpy(O.synthetic_activations(N, K, 60 + N)).cuda()
        say(f"case: strip gemm K={K} M={M} N={N} against row order")
        y = batched_int4_matmul(x, strips, K, M, strip_order=True).cpu().numpy()
        yr = batched_int4_matmul(x, blob, K, M).cpu().numpy()
        assert rel_err(y, yr) <= TOL, N


def test_strip_shape_errors():
    from moat_amd.dequant import batched_int4_matmul, records_to_strips
    with pytest.raises(ValueError):
        records_to_strips(np.zeros(144, np.uint8), 4, 64)
    with pytest.raises(ValueError):  # K below 2048: use the row order
        batched_int4_matmul(np.zeros((1, 1024), np.float16), np.zeros(1024 * 256 // 256 * 144, np.uint8), 1024, 256,
                            strip_order=True)
