"""Dense fp16 product on the GPU (``moat_dense_gemm``) against the reference's
known answers, exact integer products and the CPU oracle."""

import ctypes

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _gemm(x, w, splits=0):
    from moat_amd.dense import dense_gemm
    return dense_gemm(x, w, splits=splits)


def test_reference_gemm_known_answer():
    """antigravity-engine/tests/test_metal_kernels.cpp:94-131 (8 x 16 ones @
    16 x 16 halves = 8.0), the shape the reference's test launches."""
    x = np.ones((8, 16), np.float16)
    w = np.full((16, 16), 0.5, np.float16)
    y = _gemm(x, w)
    assert y.dtype == np.float16 and y.shape == (8, 16)
    assert np.all(y == np.float16(8.0))


@pytest.mark.parametrize("splits", [0, 1, 2, 8])
def test_benchmark_harness_known_answer(splits):
    """antigravity-engine/src/metal_runner.cpp:84-98 and :120-143: X = 1,
    W = -0.5 (scales 0.5, bytes 0x77), N = 8, K = M = 2048 -> -1024 everywhere."""
    x = torch.ones((8, 2048), dtype=torch.float16, device="cuda")
    w = torch.full((2048, 2048), -0.5, dtype=torch.float16, device="cuda")
    y = _gemm(x, w, splits)
    assert torch.all(y == -1024.0).item()


@pytest.mark.parametrize("K,M", [(8, 8), (40, 72), (96, 200), (264, 136), (2048, 2048)])
@pytest.mark.parametrize("N", [1, 5, 16, 17, 32, 40])
def test_integer_products_exact(N, K, M):
    """Small integers: every path is exact (|sums| <= 2048), so the result
    must equal the integer product bit for bit -- ragged K (a partial
    32-row round), M not a multiple of 64 (a partial block), N across the
    16- and 32-row tiles and past 32 rows."""
    rng = np.random.default_rng(1000 * N + K + M)
    hi = 2 if K >= 1024 else 4
    x = rng.integers(-hi, hi + 1, size=(N, K)).astype(np.float16)
    w = rng.integers(-1, 2, size=(K, M)).astype(np.float16)
    want = (x.astype(np.int64) @ w.astype(np.int64))
    assert np.abs(want).max() <= 2048
    for splits in (0, 1, 3):
        y = _gemm(x, w, splits)
        np.testing.assert_array_equal(y.astype(np.int64), want)


@pytest.mark.parametrize("K,M", [(2048, 2048), (2048, 5504), (3072, 8192)])
@pytest.mark.parametrize("N", [1, 8, 32])
def test_float_products_within_bound(N, K, M):
    """Random fp16 weights and activations: |y - exact| <= one fp16 ulp of
    the exact value + K float32 roundings of sum |x||w| (the bound any
    float32 summation order meets), against float64 on the CPU."""
    rng = np.random.default_rng(N + K + M)
    x = rng.standard_normal((N, K)).astype(np.float16)
    w = (0.02 * rng.standard_normal((K, M))).astype(np.float16)
    y = _gemm(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()).cpu().numpy()
    assert np.all(np.isfinite(y))
    exact = x.astype(np.float64) @ w.astype(np.float64)
    tol = O.dense_tolerance(x, w)
    err = np.abs(y.astype(np.float64) - exact)
    assert np.all(err <= tol), float((err - tol).max())
    # and the reference CPU product (fp32 BLAS, then fp16) within 1e-3 of the RMS
    ref = O.dense_gemm_ref(x, w).astype(np.float64)
    rms = np.sqrt(np.mean(ref ** 2))
    assert np.abs(y.astype(np.float64) - ref).max() <= 1e-3 * rms + O.fp16_ulp(ref).max()


def test_rows_equal_one_row_calls():
    """GEMM(N) row r equals the N = 1 call on x[r] bit for bit (the GEMV of
    antigravity-engine/tests/test_batched_speed.py:55-86, N = 8, 2048 x 2048),
    and the GEMV oracle (k-order float32 sums) within the bound."""
    from moat_amd.dense import dense_gemv
    rng = np.random.default_rng(77)
    x = torch.from_numpy(rng.standard_normal((8, 2048)).astype(np.float16)).cuda()
    w = torch.from_numpy((0.02 * rng.standard_normal((2048, 2048))).astype(np.float16)).cuda()
    y = _gemm(x, w)
    for r in range(8):
        g = dense_gemv(x[r], w)
        assert torch.equal(g, y[r])
    xn, wn = x.cpu().numpy(), w.cpu().numpy()
    g0 = O.gemv_ref(xn[0], wn).astype(np.float64)
    assert np.all(np.abs(y[0].cpu().numpy().astype(np.float64) - g0) <= 2 * O.dense_tolerance(xn[:1], wn)[0])


def test_repeated_calls_and_split_changes():
    """The block counters return to zero after every call: calls in a row
    (different inputs, different split counts, a smaller shape after a
    larger one) each give their own product."""
    rng = np.random.default_rng(3)
    shapes = [(8, 2048, 2048, 0), (3, 1024, 512, 4), (32, 2048, 2048, 8), (1, 256, 64, 0), (8, 2048, 2048, 0)]
    for n, k, m, sp in shapes:
        x = rng.integers(-2, 3, size=(n, k)).astype(np.float16)
        w = rng.integers(-1, 2, size=(k, m)).astype(np.float16)
        want = x.astype(np.int64) @ w.astype(np.int64)
        assert np.abs(want).max() <= 2048
        y = _gemm(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), sp).cpu().numpy()
        np.testing.assert_array_equal(y.astype(np.int64), want)


def test_python_checks():
    from moat_amd.dense import dense_gemm
    x = torch.ones((2, 16), dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        dense_gemm(x, torch.ones((16, 12), dtype=torch.float16, device="cuda"))   # M % 8
    with pytest.raises(ValueError):
        dense_gemm(torch.ones((2, 12), dtype=torch.float16, device="cuda"),
                   torch.ones((12, 16), dtype=torch.float16, device="cuda"))      # K % 8
    with pytest.raises(ValueError):
        dense_gemm(x, torch.ones((8, 16), dtype=torch.float16, device="cuda"))    # K mismatch
    with pytest.raises(ValueError):
        dense_gemm(x.float(), torch.ones((16, 16), dtype=torch.float16, device="cuda"))  # dtype
    with pytest.raises(ValueError):
        dense_gemm(x, torch.ones((16, 16), dtype=torch.float16, device="cuda"),
                   torch.empty((2, 16), dtype=torch.float16))                      # out on the host
    with pytest.raises(ValueError):
        dense_gemm(x, torch.ones((16, 16), dtype=torch.float16, device="cuda"),
                   torch.empty((2, 8), dtype=torch.float16, device="cuda"))        # out shape
    out = torch.empty((2, 16), dtype=torch.float16, device="cuda")
    y = dense_gemm(x, torch.full((16, 16), 0.25, dtype=torch.float16, device="cuda"), out)
    assert y is out and torch.all(out == 4.0).item()


def test_c_abi_workspace_errors():
    """A split plan without its workspace is refused before any launch."""
    from moat_amd import _lib
    lib = _lib.load()
    x = torch.ones((1, 2048), dtype=torch.float16, device="cuda")
    w = torch.ones((2048, 2048), dtype=torch.float16, device="cuda")
    y = torch.empty((1, 2048), dtype=torch.float16, device="cuda")
    assert lib.moat_dense_gemm_workspace_size(1, 2048, 2048, 0) > 0
    st = lib.moat_dense_gemm(x.data_ptr(), w.data_ptr(), y.data_ptr(), 1, 2048, 2048, 0, None, 0,
                             torch.cuda.current_stream().cuda_stream)
    assert st == _lib.MOAT_ERR_WORKSPACE
    # one split needs none
    st = lib.moat_dense_gemm(x.data_ptr(), w.data_ptr(), y.data_ptr(), 1, 2048, 2048, 1, None, 0,
                             torch.cuda.current_stream().cuda_stream)
    assert st == _lib.MOAT_OK
    torch.cuda.synchronize()
    assert torch.all(y == 2048.0).item()


def test_graph_replays_match_eager():
    """Captured in a HIP graph (split plan: the block counters must return to
    zero every replay), replayed three times with eager calls of another
    shape in between; every replay equals the eager result bit for bit."""
    from moat_amd.dense import dense_gemm
    rng = np.random.default_rng(12)
    x = torch.from_numpy(rng.standard_normal((8, 2048)).astype(np.float16)).cuda()
    w = torch.from_numpy((0.02 * rng.standard_normal((2048, 2048))).astype(np.float16)).cuda()
    x2 = torch.from_numpy(rng.standard_normal((3, 1024)).astype(np.float16)).cuda()
    w2 = torch.from_numpy((0.02 * rng.standard_normal((1024, 512))).astype(np.float16)).cuda()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        want = dense_gemm(x, w).clone()  # eager, and the stream's workspace exists before capture
        want2 = dense_gemm(x2, w2).clone()
        y = torch.empty((8, 2048), dtype=torch.float16, device="cuda")
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            dense_gemm(x, w, y)
        for _ in range(3):
            y.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, want)
            assert torch.equal(dense_gemm(x2, w2), want2)
    torch.cuda.synchronize()
