"""moat_int4_gemm_noalloc (the GEMM entry point without a workspace, for
callers that cannot allocate): called through the C ABI, two calls in a
row -- the second on a smaller input -- each equal to moat_int4_gemm_ex with
the same plan (the fix-up hand-off), bit for bit, and within 1e-3 of the
output RMS of the oracle."""

import ctypes
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


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from moat_amd import _lib
    return _lib.load()


def _problem(K, M, seed):
    """Records quantized on the GPU (bit-exact with the oracle's quantizer,
    tested elsewhere); the decoded weights for the oracle check only for
    shapes the host decodes quickly."""
    from moat_amd.dequant import quantize_to_superblocks
    w = O.synthetic_weights(K, M, 0.02, seed)
    blob = quantize_to_superblocks(torch.from_numpy(w).cuda()).reshape(-1)
    wdq = None
    if K * M <= 3072 * 8192:
        wdq = O.decode_superblocks(blob.cpu().numpy(), K * M // 256).astype(np.float32).reshape(K, M)
    return blob, wdq


def _x(N, K, seed, offset_elems=0):
    x = O.synthetic_activations(N, K, seed)
    if not offset_elems:
        return torch.from_numpy(x).cuda(), x
    base = torch.zeros(N * K + 8, dtype=torch.float16, device="cuda")
    xv = base[offset_elems:offset_elems + N * K].view(N, K)
    xv.copy_(torch.from_numpy(x).cuda())
    return xv, x


def _call_noalloc(lib, xd, blob, y, N, K, M):
    return lib.moat_int4_gemm_noalloc(xd.data_ptr(), blob.data_ptr(), y.data_ptr(), N, K, M,
                                      torch.cuda.current_stream().cuda_stream)


def _call_ex(lib, xd, blob, N, K, M):
    from moat_amd import _lib as L
    opt = L.GemmOptions(0, 0, 0, L.FINISH_SECOND_KERNEL)
    ws_bytes = lib.moat_int4_gemm_ex_workspace_size(N, K, M, ctypes.byref(opt))
    ws = torch.zeros(max(ws_bytes, 16), dtype=torch.uint8, device="cuda")
    y = torch.empty((N, M), dtype=torch.float32, device="cuda")
    st = lib.moat_int4_gemm_ex(xd.data_ptr(), blob.data_ptr(), y.data_ptr(), N, K, M, ctypes.byref(opt),
                               ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
    assert st == 0
    return y


# (K, M, N) of the first call, then the second call's smaller input; the
# last field shifts X by one element (2-byte aligned: the general kernel)
CASES = [
    ((2048, 5504, 32), (2048, 5504, 4), 0),
    ((3072, 8192, 16), (2048, 2048, 1), 0),
    ((8192, 28672, 32), (3072, 8192, 8), 0),
    ((2048, 5504, 8), (512, 384, 3), 1),
    ((64, 256, 3), (32, 128, 1), 0),
]


@pytest.mark.parametrize("first,second,shift", CASES)
def test_noalloc_matches_the_workspace_entry_point(lib, first, second, shift):
    for call_no, (K, M, N) in enumerate((first, second)):
        say(f"case: noalloc call {call_no + 1}: K={K} M={M} N={N} x shifted by {shift}")
        blob, wdq = _problem(K, M, 300 + K + M)
        xd, x = _x(N, K, 400 + N, shift)
        y = torch.full((N, M), float("nan"), dtype=torch.float32, device="cuda")
        assert _call_noalloc(lib, xd, blob, y, N, K, M) == 0
        ref_ex = _call_ex(lib, xd, blob, N, K, M)
        torch.cuda.synchronize()
        assert torch.equal(y, ref_ex), (K, M, N)
        if wdq is not None:
            assert rel_err(y.cpu().numpy(), x.astype(np.float32) @ wdq) <= TOL


def test_noalloc_refuses_plans_beyond_its_scratch(lib):
    from moat_amd import _lib as L
    blob = torch.zeros(1, dtype=torch.uint8, device="cuda")  # never read: refused before any launch
    x = torch.zeros(16, dtype=torch.float16, device="cuda")
    y = torch.zeros(16, dtype=torch.float32, device="cuda")
    st = lib.moat_int4_gemm_noalloc(x.data_ptr(), blob.data_ptr(), y.data_ptr(), 32, 8192, 32768,
                                    torch.cuda.current_stream().cuda_stream)
    assert st == L.MOAT_ERR_TOO_LARGE
