"""The dense fp16 oracle against the reference's known answers and exact
integer products (CPU)."""

import numpy as np

import oracle as O


def test_reference_gemm_known_answer():
    """antigravity-engine/tests/test_metal_kernels.cpp:94-131: ones(8 x 16) @
    0.5 * ones(16 x 16) -> every output 8.0."""
    x = np.ones((8, 16), np.float16)
    w = np.full((16, 16), 0.5, np.float16)
    for y in (O.dense_gemm_ref(x, w), O.dense_exact(x, w), np.vstack([O.gemv_ref(r, w) for r in x])):
        assert y.dtype == np.float16 and y.shape == (8, 16)
        assert np.all(y == np.float16(8.0))


def test_benchmark_harness_known_answer():
    """antigravity-engine/src/metal_runner.cpp:84-98: scales 0.5, bytes 0x77
    (q = -1) and X = 1.0, so every output is -0.5 * K = -1024 at K = 2048."""
    x = np.ones((8, 2048), np.float16)
    w = np.full((2048, 64), -0.5, np.float16)
    assert np.all(O.dense_gemm_ref(x, w) == np.float16(-1024.0))
    assert np.all(O.gemv_ref(x[0], w) == np.float16(-1024.0))


def test_integer_products_are_exact_and_not_transposed():
    rng = np.random.default_rng(5)
    x = rng.integers(-3, 4, size=(5, 40)).astype(np.float16)
    w = rng.integers(-3, 4, size=(40, 24)).astype(np.float16)
    want = (x.astype(np.int64) @ w.astype(np.int64)).astype(np.float16)
    np.testing.assert_array_equal(O.dense_gemm_ref(x, w), want)
    np.testing.assert_array_equal(O.dense_exact(x, w), want)
    np.testing.assert_array_equal(np.vstack([O.gemv_ref(r, w) for r in x]), want)
    # a transposed or shifted operand does not give the same numbers
    assert not np.array_equal((x.astype(np.int64) @ np.roll(w, 1, axis=0).astype(np.int64)).astype(np.float16), want)


def test_gemv_sums_in_k_order():
    """gemv_kernel adds in k order in float32: 1 + 2^-24 + ... stays 1,
    while the exact sum, 1 + 2^-10 - 2^-24, rounds to the next fp16 value."""
    k = 16384
    x = np.ones(k, np.float16)
    w = np.zeros((k, 8), np.float16)
    w[0] = 1.0
    w[1:] = np.float16(2.0 ** -24)  # the smallest fp16 subnormal
    g = O.gemv_ref(x, w).astype(np.float64)
    assert np.all(g == 1.0)
    assert np.all(O.dense_exact(x.reshape(1, -1), w).astype(np.float64) == 1.0 + 2.0 ** -10)


def test_tolerance_covers_float32_orders():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((4, 512)).astype(np.float16)
    w = (0.05 * rng.standard_normal((512, 96))).astype(np.float16)
    tol = O.dense_tolerance(x, w)
    exact = x.astype(np.float64) @ w.astype(np.float64)
    for y in (O.dense_gemm_ref(x, w), np.vstack([O.gemv_ref(r, w) for r in x])):
        assert np.all(np.abs(y.astype(np.float64) - exact) <= tol)
    # and is tighter than a wrong answer: one product dropped
    y_bad = (x[:, 1:].astype(np.float32) @ w[1:].astype(np.float32)).astype(np.float16)
    assert np.any(np.abs(y_bad.astype(np.float64) - exact) > tol)


def test_fp16_ulp():
    assert O.fp16_ulp(1.0) == 2.0 ** -10
    assert O.fp16_ulp(1024.0) == 1.0
    assert O.fp16_ulp(-3.0) == 2.0 ** -9
    assert O.fp16_ulp(0.0) == 2.0 ** -24
