"""Tile-order weight stream (``moat_int4_records_to_tiles``,
``moat_int4_gemm_tiles`` through ``moat_amd.dequant``): the permutation bit
for bit against the oracle, and the GEMM over tile order bit for bit equal to
the GEMM over the row order (same plan, same kernel, same summation order) at
every N and launch choice, within tolerance of the oracle, and at the
8192 x 28672 shape."""

import numpy as np
import pytest
import torch

from oracle import superblock_oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3
SHAPES = [(32, 256), (96, 768), (2048, 2048), (3072, 8192), (2048, 32000)]


def say(msg):
    print(msg, flush=True)


def rel_err(y, ref):
    return float(np.max(np.abs(y - ref)) / max(float(np.sqrt(np.mean(ref.astype(np.float64) ** 2))), 1e-30))


def _blob(K, M):
    w = O.synthetic_weights(K, M, 0.03, 40 + K + M)
    return O.quantize_pack_a(w).reshape(-1)


def test_records_to_tiles_matches_oracle():
    from moat_amd.dequant import records_to_tiles
    for K, M in SHAPES:
        say(f"case: records_to_tiles K={K} M={M}")
        blob = _blob(K, M)
        tiles = records_to_tiles(torch.from_numpy(blob).cuda(), K, M)
        assert tiles.is_cuda and tiles.dtype == torch.uint8 and tiles.numel() == blob.size
        assert np.array_equal(tiles.cpu().numpy(), O.records_to_tiles(blob, K, M))
        # a host stream gives the same tensor
        assert torch.equal(records_to_tiles(blob, K, M), tiles)


def test_gemm_tiles_equals_row_order():
    from moat_amd import _lib as L
    from moat_amd.dequant import batched_int4_matmul, records_to_tiles
    for K, M in SHAPES:
        blob = _blob(K, M)
        blob_d = torch.from_numpy(blob).cuda()
        tiles = records_to_tiles(blob_d, K, M)
        wdq = O.decode_superblocks(blob, K * M // 256).astype(np.float32).reshape(K, M)
        for N in (1, 2, 8, 16, 17, 32):
            say(f"case: gemm tiles K={K} M={M} N={N}")
            x = O.synthetic_activations(N, K, 60 + N)
            xd = torch.from_numpy(x).cuda()
            y_rows = batched_int4_matmul(xd, blob_d, K, M)
            y_tiles = batched_int4_matmul(xd, tiles, K, M, tile_order=True)
            assert torch.equal(y_rows.view(torch.int32), y_tiles.view(torch.int32)), (K, M, N)
            assert rel_err(y_tiles.cpu().numpy(), x.astype(np.float32) @ wdq) <= TOL
        # launch choices: stream-K splits, tile groups, 8-wave workgroups, fix-up kernel
        rounds = K // 32
        x = O.synthetic_activations(3, K, 7)
        xd = torch.from_numpy(x).cuda()
        for waves in (4, 8):
            for group in (1, 2):
                for splits in sorted({1, 2, min(5, rounds)}):
                    for finish in (L.FINISH_AUTO, L.FINISH_SECOND_KERNEL):
                        say(f"case: gemm tiles K={K} M={M} waves={waves} group={group} splits={splits} "
                            f"finish={finish}")
                        kw = dict(algo=L.GEMM_MFMA, splits=splits, finish=finish, front=L.FRONT_RECORDS,
                                  group=group, waves=waves)
                        y_rows = batched_int4_matmul(xd, blob_d, K, M, **kw)
                        y_tiles = batched_int4_matmul(xd, tiles, K, M, tile_order=True, **kw)
                        assert torch.equal(y_rows.view(torch.int32), y_tiles.view(torch.int32))


def test_gemm_tiles_refuses_other_kernels():
    from moat_amd import _lib as L
    from moat_amd.dequant import batched_int4_matmul
    say("case: gemm tiles refusals")
    x = torch.zeros((1, 2048), dtype=torch.float16, device="cuda")
    w = torch.zeros(2048 * 2048 // 256 * 144, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError):
        batched_int4_matmul(x, w, 2048, 2048, tile_order=True, front=L.FRONT_LDS)
    w2 = torch.zeros(2048 * 5504 // 256 * 144, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError):  # M % 256 == 128: rows start half-way into records
        batched_int4_matmul(x, w2, 2048, 5504, tile_order=True)


def test_large_projection_tile_order():
    """8192 x 28672 (132 MB of records) at N = 1 and 32: tile order equals row order."""
    from moat_amd.dequant import batched_int4_matmul, quantize_to_superblocks, records_to_tiles
    K, M = 8192, 28672
    say("case: tiles 8192x28672 quantize on GPU")
    g = torch.Generator(device="cpu").manual_seed(5)
    w = (torch.randn((K, M), generator=g) * 0.01).cuda()
    blob_d = quantize_to_superblocks(w)
    del w
    tiles = records_to_tiles(blob_d, K, M)
    for N in (1, 32):
        say(f"case: tiles 8192x28672 gemm N={N}")
        x = torch.from_numpy(O.synthetic_activations(N, K, 90 + N)).cuda()
        y_rows = batched_int4_matmul(x, blob_d, K, M)
        y_tiles = batched_int4_matmul(x, tiles, K, M, tile_order=True)
        assert torch.equal(y_rows.view(torch.int32), y_tiles.view(torch.int32)), N
