"""GPU parity of the gfx950 kernels against the CPU oracle.

Bars: bit-exact for nibbles, quantized codes and dequantized fp16 weights
(NaN compared as a class: the reference's NaN payloads depend on its CPU);
GEMM within max|Y - Y_ref| <= 1e-3 * RMS(Y_ref), and GEMM(N) against N
single-row products within the same bound.
"""

import sys

import numpy as np
import pytest
import torch

from oracle import superblock_oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3  # max-abs error relative to the reference output's RMS


def _lib():
    from moat_amd import _lib as L
    return L


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def bits16(a):
    return np.asarray(a).view(np.uint16)


def assert_f16_equal(got, exp):
    g, e = bits16(got), bits16(exp)
    gn = ((g & 0x7C00) == 0x7C00) & ((g & 0x3FF) != 0)
    en = ((e & 0x7C00) == 0x7C00) & ((e & 0x3FF) != 0)
    assert np.array_equal(gn, en), "NaN positions differ"
    bad = np.flatnonzero(g[~en] != e[~en])
    assert bad.size == 0, f"{bad.size} fp16 mismatches, first at {bad[:5]}"


def rel_err(y, yref):
    rms = float(np.sqrt(np.mean(yref.astype(np.float64) ** 2)))
    return float(np.max(np.abs(y.astype(np.float64) - yref))) / max(rms, 1e-30)


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    _lib().load()
    return torch.device("cuda", 0)


# ------------------------------------------------------------------ dequant

def test_dequant_exhaustive_scale_nibble_table():
    from moat_amd.dequant import unpack_superblock_weights
    n_groups = 1 << 16
    nib = np.tile(np.arange(16, dtype=np.uint8), 2)
    payload = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
    blob = np.zeros((n_groups // 8, 144), dtype=np.uint8)
    blob[:, :16] = np.arange(n_groups, dtype=np.uint32).astype("<u2").view(np.uint8).reshape(-1, 16)
    blob[:, 16:] = np.tile(payload, 8)[None, :]
    say("case: exhaustive 65536 scales x 16 nibbles")
    got = unpack_superblock_weights(blob.reshape(-1), n_groups // 8)
    assert_f16_equal(got, O.decode_superblocks(blob, n_groups // 8))


def test_dequant_kernel_kat_0x7f():
    """antigravity-engine/tests/test_metal_kernels.cpp:69-90."""
    from moat_amd.dequant import unpack_superblock_weights
    blob = np.zeros(144, dtype=np.uint8)
    blob[:16] = np.full(8, 0.5, dtype="<f2").view(np.uint8)
    blob[16:] = 0x7F
    out = unpack_superblock_weights(blob, 1)
    assert out.dtype == np.float16 and out.shape == (256,)
    assert np.all(out[0::2] == np.float16(3.5)) and np.all(out[1::2] == np.float16(-0.5))


SHAPES = {
    "proj 2048x2048": (2048, 2048, 0.02, 1001, 0.0),
    "ffn 2048x5504": (2048, 5504, 0.02, 1002, 0.0),
    "ffn 3072x8192": (3072, 8192, 0.02, 1003, 0.0),
    "layer qkvo 2048x2048": (2048, 2048, 0.02, 1004, 0.0),
    "layer gate/up 2048x5632": (2048, 5632, 0.02, 1014, 0.0),
    "layer down 5632x2048": (5632, 2048, 0.02, 1024, 0.0),
    "lm head 2048x32000": (2048, 32000, 0.02, 1006, 0.0),
}

_cache = {}


def workload(name):
    if name not in _cache:
        K, M, std, seed, outl = SHAPES[name] if name in SHAPES else BIG[name]
        w = O.synthetic_weights(K, M, std, seed, outlier_frac=outl)
        _cache[name] = (K, M, w, O.quantize_pack_a(w))
    return _cache[name]


@pytest.mark.parametrize("name", list(SHAPES))
def test_quantize_pack_and_dequant_bit_exact(name):
    from moat_amd.dequant import quantize_to_superblocks, unpack_superblock_weights
    K, M, w, blob_ref = workload(name)
    say(f"case: quantize+pack+dequant {name}")
    blob = quantize_to_superblocks(w)
    assert blob.shape == blob_ref.shape and np.array_equal(blob, blob_ref)
    dq = unpack_superblock_weights(blob.reshape(-1), K * M // 256)
    assert_f16_equal(dq, O.decode_superblocks(blob_ref, K * M // 256))


# ------------------------------------------------------------------ GEMM

def _x(N, K, seed):
    return O.synthetic_activations(N, K, seed)


GEMM_CASES = [
    ("proj 2048x2048", [8]),
    ("ffn 2048x5504", [1, 2, 4, 8, 16, 32]),
    ("ffn 3072x8192", [1, 8, 32]),
    ("layer qkvo 2048x2048", [16]),
    ("layer gate/up 2048x5632", [16]),
    ("layer down 5632x2048", [16]),
    ("lm head 2048x32000", [1, 16, 32]),
]


@pytest.mark.parametrize("name,ns", GEMM_CASES)
def test_gemm_matches_oracle_all_kernels(name, ns):
    from moat_amd.dequant import batched_int4_matmul
    L = _lib()
    K, M, _, blob = workload(name)
    wdq = O.decode_superblocks(blob, K * M // 256).astype(np.float32).reshape(K, M)
    blob_d = torch.from_numpy(blob.reshape(-1)).cuda()
    for N in ns:
        x = _x(N, K, 2000 + N)
        yref = x.astype(np.float32) @ wdq
        xd = torch.from_numpy(x).cuda()
        algos = [L.GEMM_AUTO, L.GEMM_MFMA] + ([L.GEMM_DOT2] if N <= 8 else [])
        for algo in algos:
            for splits, batch, finish, front in ((0, 0, 0, 0), (1, 0, 0, 1), (1, 0, 0, 2), (1, 0, 0, 3), (3, 1, 1, 1),
                                                 (3, 2, 2, 2), (7, 4, 3, 1), (5, 4, 1, 2), (6, 4, 1, 3), (2, 2, 3, 3)):
                say(f"case: gemm {name} N={N} algo={algo} splits={splits} batch={batch} finish={finish} front={front}")
                y = batched_int4_matmul(xd, blob_d, K, M, algo=algo, splits=splits, batch=batch, finish=finish,
                                        front=front)
                e = rel_err(y.cpu().numpy(), yref)
                assert e <= TOL, (name, N, algo, splits, batch, finish, front, e)


@pytest.mark.parametrize("K,M", [(2048, 5504), (3072, 8192), (32, 128), (64, 384), (96, 640), (32, 256),
                                 (160, 1152)])
def test_gemm_record_stream_kernel(K, M):
    """The record-stream kernel (256-column tiles of whole records; rows that
    start half-way into a record when M % 256 == 128; a 128-column last tile;
    a short last tile group; waves with no round when K is short) at every
    tile-group size, workgroup size (4 or 8 waves), ring depth (deeper
    than the LDS holds: clamped), stream-K split and hand-off (last
    workgroup in the kernel, or the fix-up kernel)."""
    from moat_amd.dequant import batched_int4_matmul
    L = _lib()
    w = O.synthetic_weights(K, M, 0.03, 11 + K + M)
    blob = O.quantize_pack_a(w)
    wdq = O.decode_superblocks(blob, K * M // 256).astype(np.float32).reshape(K, M)
    blob_d = torch.from_numpy(blob.reshape(-1)).cuda()
    rounds = K // 32
    for N in (1, 3, 16, 17, 32):
        x = _x(N, K, 21 + N)
        yref = x.astype(np.float32) @ wdq
        xd = torch.from_numpy(x).cuda()
        for waves, depths in ((4, (1, 2, 3, 5)), (8, (1, 2, 5))):
            for group in (1, 2, 4):
                for depth in depths:
                    for splits in sorted({1, 2, min(5, rounds), min(16, rounds)}):
                        for finish in (L.FINISH_AUTO, L.FINISH_SECOND_KERNEL):
                            say(f"case: records K={K} M={M} N={N} waves={waves} group={group} depth={depth} "
                                f"splits={splits} finish={finish}")
                            y = batched_int4_matmul(xd, blob_d, K, M, algo=L.GEMM_MFMA, splits=splits, batch=depth,
                                                    finish=finish, front=L.FRONT_RECORDS, group=group, waves=waves)
                            e = rel_err(y.cpu().numpy(), yref)
                            assert e <= TOL, (K, M, N, waves, group, depth, splits, finish, e)


def test_gemm_workspace_shared_between_kernels():
    """Calls of both kernels and of every hand-off alternate on one stream,
    hence one workspace: each must leave it all at zero (the record-stream
    kernel's in-kernel hand-off reads zero as "partial not written")."""
    from moat_amd.dequant import batched_int4_matmul
    L = _lib()
    K, M = 2048, 5504
    w = O.synthetic_weights(K, M, 0.02, 77)
    blob = O.quantize_pack_a(w)
    wdq = O.decode_superblocks(blob, K * M // 256).astype(np.float32).reshape(K, M)
    blob_d = torch.from_numpy(blob.reshape(-1)).cuda()
    for N in (4, 32):
        x = _x(N, K, 5 + N)
        yref = x.astype(np.float32) @ wdq
        xd = torch.from_numpy(x).cuda()
        for rep in range(3):
            for front, splits, finish in ((L.FRONT_RECORDS, 8, 0), (L.FRONT_LDS, 3, 1), (L.FRONT_RECORDS, 3, 0),
                                          (L.FRONT_DIRECT, 5, 2), (L.FRONT_RECORDS, 176, 0), (L.FRONT_LDS, 4, 3),
                                          (L.FRONT_RECORDS, 5, 3), (L.FRONT_RECORDS, 44, 0)):
                say(f"case: shared workspace N={N} rep={rep} front={front} splits={splits} finish={finish}")
                y = batched_int4_matmul(xd, blob_d, K, M, algo=L.GEMM_MFMA, splits=splits, finish=finish, front=front)
                assert rel_err(y.cpu().numpy(), yref) <= TOL, (N, rep, front, splits, finish)


def test_gemm_equals_stacked_gemv():
    """GEMM(N) == N single-row products (antigravity-engine/tests/test_batched_speed.py:55-86)."""
    from moat_amd.dequant import batched_int4_matmul
    K, M, _, blob = workload("ffn 3072x8192")
    blob_d = torch.from_numpy(blob.reshape(-1)).cuda()
    for N in (8, 32):
        x = torch.from_numpy(_x(N, K, 77 + N)).cuda()
        say(f"case: gemm vs stacked gemv N={N}")
        y = batched_int4_matmul(x, blob_d, K, M).cpu().numpy()
        rows = np.vstack([batched_int4_matmul(x[i:i + 1], blob_d, K, M).cpu().numpy() for i in range(N)])
        assert rel_err(y, rows) <= TOL


@pytest.mark.parametrize("seed,ns", [(42, [8]), (7, [1, 2, 4, 8, 16])])
def test_gemm_equals_sequential_gemvs_2048(seed, ns):
    """The reference's must-pass invariant at its own shape, K = M = 2048
    (antigravity-engine/tests/test_batched_speed.py:55-86): W and the
    activations drawn as there (np.random.seed, randn as fp16), W quantized
    to superblocks; GEMM(N) equals N sequential N=1 calls and the oracle."""
    from moat_amd.dequant import batched_int4_matmul
    K = M = 2048
    np.random.seed(seed)
    w = np.random.randn(K, M).astype(np.float16)
    blob = O.quantize_pack_a(w)
    wdq = O.decode_superblocks(blob, K * M // 256).astype(np.float32).reshape(K, M)
    blob_d = torch.from_numpy(blob.reshape(-1)).cuda()
    for N in ns:
        acts = np.random.randn(N, K).astype(np.float16)
        xd = torch.from_numpy(acts).cuda()
        say(f"case: 2048x2048 seed={seed} N={N}: GEMM vs {N} sequential GEMVs")
        y = batched_int4_matmul(xd, blob_d, K, M).cpu().numpy()
        seq = np.vstack([batched_int4_matmul(xd[i:i + 1], blob_d, K, M).cpu().numpy() for i in range(N)])
        yref = acts.astype(np.float32) @ wdq
        assert rel_err(y, seq) <= TOL
        assert rel_err(y, yref) <= TOL and rel_err(seq, yref) <= TOL
        assert np.all(np.isfinite(y))


def test_gemm_unaligned_x_on_record_stream_shape_through_abi():
    """x only 2-byte aligned on a shape the record-stream kernel takes: the
    call plans the general kernel, and the workspace the size query gives
    covers that plan (called through the C ABI, no Python re-alignment)."""
    import ctypes
    L = _lib()
    lib = L.load()
    K, M, _, blob = workload("ffn 2048x5504")
    wdq = O.decode_superblocks(blob, K * M // 256).astype(np.float32).reshape(K, M)
    blob_d = torch.from_numpy(blob.reshape(-1)).cuda()
    for N in (1, 8, 32):
        x = _x(N, K, 600 + N)
        yref = x.astype(np.float32) @ wdq
        base = torch.zeros(N * K + 8, dtype=torch.float16, device="cuda")
        xv = base[1:1 + N * K]
        xv.copy_(torch.from_numpy(x.reshape(-1)).cuda())
        assert xv.data_ptr() % 16 == 2
        y = torch.full((N, M), float("nan"), dtype=torch.float32, device="cuda")
        for opt in (None, L.GemmOptions(0, 0, 0, 0, L.FRONT_RECORDS)):
            ref = ctypes.byref(opt) if opt is not None else None
            ws_bytes = lib.moat_int4_gemm_ex_workspace_size(N, K, M, ref)
            ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
            say(f"case: unaligned x through the ABI N={N} options={'front records' if opt else 'auto'}")
            st = lib.moat_int4_gemm_ex(xv.data_ptr(), blob_d.data_ptr(), y.data_ptr(), N, K, M, ref,
                                       ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
            assert st == 0
            assert rel_err(y.cpu().numpy(), yref) <= TOL


def test_gemm_runner_stream_closed_form():
    """antigravity-engine/src/metal_runner.cpp:84-98: every output is -0.5*K, exactly."""
    from moat_amd.dequant import batched_int4_matmul
    L = _lib()
    K = M = 2048
    S = K * M // 256
    blob = np.zeros((S, 144), dtype=np.uint8)
    blob[:, :16] = np.full(8, 0x3800, dtype="<u2").view(np.uint8)
    blob[:, 16:] = 0x77
    x = np.ones((8, K), dtype=np.float16)
    for algo in (L.GEMM_MFMA, L.GEMM_DOT2):
        for splits in (1, 4, 16):
            for finish in (1, 2, 3):
                say(f"case: runner stream algo={algo} splits={splits} finish={finish}")
                y = batched_int4_matmul(x, blob, K, M, algo=algo, splits=splits, finish=finish)
                assert np.all(y == np.float32(-0.5 * K)), (algo, splits, finish)


@pytest.mark.parametrize("K,M", [(3, 256), (64, 160), (12, 64), (40, 96), (256, 32), (1000, 224), (24, 192),
                                 (100, 448), (293, 256), (1000, 448), (518, 128)])
def test_gemm_ragged_shapes(K, M):
    """K not a multiple of 32 or 8, M not a multiple of the 128-column tile."""
    from moat_amd.dequant import batched_int4_matmul
    L = _lib()
    w = O.synthetic_weights(K, M, 0.05, 5 + K + M)
    blob = O.quantize_pack_a(w)
    wdq = O.decode_superblocks(blob, K * M // 256).astype(np.float32).reshape(K, M)
    for N in (1, 5, 16, 17, 32):
        x = _x(N, K, 9 + N)
        yref = x.astype(np.float32) @ wdq
        for algo in (L.GEMM_MFMA, L.GEMM_DOT2):
            if algo == L.GEMM_DOT2 and N > 8:
                continue
            for splits, batch, front in ((1, 1, 1), (2, 2, 1), (2, 4, 1), (1, 1, 2), (2, 4, 2), (1, 2, 3), (2, 4, 3)):
                say(f"case: ragged K={K} M={M} N={N} algo={algo} splits={splits} batch={batch} front={front}")
                y = batched_int4_matmul(x, blob, K, M, algo=algo, splits=splits, batch=batch, front=front)
                assert rel_err(y, yref) <= TOL, (K, M, N, algo, splits, batch, front)


def test_gemm_unaligned_activations_and_zero_rows():
    from moat_amd.dequant import batched_int4_matmul
    K, M = 512, 384
    w = O.synthetic_weights(K, M, 0.02, 31)
    blob = O.quantize_pack_a(w)
    wdq = O.decode_superblocks(blob, K * M // 256).astype(np.float32).reshape(K, M)
    base = torch.from_numpy(_x(5, K + 1, 4)).cuda()
    x = base.reshape(-1)[1:1 + 4 * K].reshape(4, K)  # 2-byte aligned only
    assert x.data_ptr() % 16 != 0
    say("case: unaligned X")
    y = batched_int4_matmul(x, torch.from_numpy(blob).cuda(), K, M).cpu().numpy()
    assert rel_err(y, x.cpu().numpy().astype(np.float32) @ wdq) <= TOL
    z = batched_int4_matmul(np.zeros((3, K), np.float16), blob, K, M)
    assert np.all(z == 0)


def test_gemm_split_k_handoff_is_deterministic():
    """Every split-K hand-off gives the same bits on every call (partials are
    added in split order), and the hand-offs agree with each other."""
    from moat_amd.dequant import batched_int4_matmul
    K, M, _, blob = workload("ffn 2048x5504")
    blob_d = torch.from_numpy(blob.reshape(-1)).cuda()
    L = _lib()
    for front, splits in ((L.FRONT_RECORDS, 16), (L.FRONT_RECORDS, 176), (L.FRONT_RECORDS, 500),
                          (L.FRONT_LDS, 16)):
        for N in (1, 4, 32):
            x = torch.from_numpy(_x(N, K, 3)).cuda()
            ref = batched_int4_matmul(x, blob_d, K, M, algo=2, splits=splits, finish=3, front=front)
            for finish in (0, 1, 2, 3):
                say(f"case: split-K hand-off front={front} splits={splits} N={N} finish={finish}")
                for _ in range(20):
                    y = batched_int4_matmul(x, blob_d, K, M, algo=2, splits=splits, finish=finish, front=front)
                    assert torch.equal(y, ref), (front, splits, N, finish)


def test_gemm_n_above_32_is_sliced():
    from moat_amd.dequant import batched_int4_matmul
    K, M = 256, 256
    w = O.synthetic_weights(K, M, 0.02, 8)
    blob = O.quantize_pack_a(w)
    x = _x(70, K, 1)
    y = batched_int4_matmul(x, blob, K, M)
    assert rel_err(y, O.gemm_ref(x, blob, K, M)) <= TOL


BIG = {"proj 8192x28672": (8192, 28672, 0.01, 1005, 0.001)}


def test_large_projection_with_outliers():
    """8192 x 28672 (132 MB of records), 0.1% outliers at 8 sigma, N = 1 and 32."""
    from moat_amd.dequant import batched_int4_matmul, quantize_to_superblocks
    K, M = 8192, 28672
    w = O.synthetic_weights(K, M, 0.01, 1005, outlier_frac=0.001)
    say("case: 8192x28672 quantize on GPU")
    blob_d = quantize_to_superblocks(torch.from_numpy(w).cuda())
    blob = blob_d.cpu().numpy()
    q, s = O.quantize_a(w.reshape(-1))
    assert np.array_equal(blob, O.serialize_superblocks(q, s))
    del q, s
    wdq = O.decode_superblocks(blob, K * M // 256).astype(np.float32).reshape(K, M)
    for N in (1, 32):
        x = _x(N, K, 2500 + N)
        say(f"case: 8192x28672 gemm N={N}")
        y = batched_int4_matmul(torch.from_numpy(x).cuda(), blob_d, K, M).cpu().numpy()
        assert rel_err(y, x.astype(np.float32) @ wdq) <= TOL


# ------------------------------------------------------------------ quantizers

QUANT_INPUTS = {
    "f32 normal": lambda r: r.standard_normal(4096 * 32).astype(np.float32) * np.float32(0.02),
    "f16 wide": lambda r: (r.standard_normal(1024 * 32) * 5).astype(np.float16),
    "f64": lambda r: r.standard_normal(512 * 32) * 0.3,
    "ties": lambda r: np.tile(np.array([(k + 0.5) * 0.25 for k in range(-7, 7)] + [1.75, -1.75] * 9, np.float32), 64),
    "zeros+subnormal": lambda r: np.concatenate([np.zeros(64, np.float32), np.full(64, 1e-40, np.float32),
                                                 (r.standard_normal(128) * 1e-39).astype(np.float32)]),
}


@pytest.mark.parametrize("kind", list(QUANT_INPUTS))
@pytest.mark.parametrize("gs", [32, 64, 16])
def test_quantizers_bit_exact(kind, gs):
    from moat_amd import dequant as A
    from moat_amd import engine_dequant as B
    w = QUANT_INPUTS[kind](np.random.default_rng(42))
    w = w[: (w.size // gs) * gs]
    say(f"case: quantize {kind} gs={gs}")
    qa, sa = A.quantize_fp16_to_int4(w, group_size=gs)
    qa_ref, sa_ref = O.quantize_a(w, group_size=gs)
    assert np.array_equal(qa, qa_ref) and np.array_equal(bits16(sa), bits16(sa_ref))
    qb, sb = B.quantize_weights_int4(w, group_size=gs)
    qb_ref, sb_ref = O.quantize_b(w, group_size=gs)
    assert np.array_equal(qb, qb_ref) and np.array_equal(bits16(sb), bits16(sb_ref))


def test_quantizer_shape_and_errors():
    from moat_amd import dequant as A
    from moat_amd import engine_dequant as B
    w = np.random.default_rng(1).standard_normal((64, 96)).astype(np.float32)
    q, s = A.quantize_fp16_to_int4(w)
    qr, sr = O.quantize_a(w)
    assert q.shape == (64, 96) and np.array_equal(q, qr) and np.array_equal(bits16(s), bits16(sr))
    with pytest.raises(AssertionError):
        A.quantize_fp16_to_int4(np.zeros(33, np.float16))
    with pytest.raises(ValueError):
        B.quantize_weights_int4(np.zeros((4, 32), np.float16))
    with pytest.raises(ValueError):
        B.quantize_weights_int4(np.zeros(33, np.float16))


# ------------------------------------------------------------------ surfaces

def test_pack_unpack_and_records():
    from moat_amd import dequant as A
    from moat_amd import engine_dequant as B
    rng = np.random.default_rng(2)
    q = rng.integers(-8, 8, size=256 * 40).astype(np.int8)
    s = (rng.standard_normal(8 * 40) * 0.1).astype(np.float16)
    blob = A.pack_superblocks_bytes(q, s)
    assert np.array_equal(blob, O.serialize_superblocks(q, s))
    recs = B.repack_to_superblocks(q, s)
    recs_ref = O.superblock_records(q, s)
    assert len(recs) == len(recs_ref) == 40
    for r, rr in zip(recs, recs_ref):
        assert np.array_equal(r["packed_nibbles"], rr["packed_nibbles"])
        assert np.array_equal(bits16(r["scales"]), bits16(rr["scales"]))
        assert np.array_equal(r["raw_int4"], rr["raw_int4"])
        assert np.array_equal(B.unpack_superblock(r), O.unpack_nibbles(rr["packed_nibbles"]))
    wide = np.array([-9, 8, 20, -30] * 64, dtype=np.int32)  # wraps mod 16 like the reference
    assert np.array_equal(B.repack_to_superblocks(wide, np.ones(8, np.float16))[0]["packed_nibbles"],
                          O.pack_nibbles(wide))
    with pytest.raises(ValueError):
        B.repack_to_superblocks(q[:200], s)


def test_table_and_arithmetic_dequant():
    from moat_amd import engine_dequant as B
    rng = np.random.default_rng(3)
    q = rng.integers(-8, 8, size=32 * 50 + 7).astype(np.int8)
    s16 = (rng.standard_normal(50) * 0.3).astype(np.float16)
    s32 = (rng.standard_normal(50) * 0.3).astype(np.float32)
    for s in (s16, s32, s32.astype(np.float64)):
        exp = O.group_dequant(q, s)
        assert_f16_equal(B.arithmetic_dequantize(q, s), exp)
        assert_f16_equal(B.lut_dequantize(q, s), exp)
    for sc in (0.5, np.float16(0.75), 0.1, np.float32(1e-3)):
        assert_f16_equal(B.build_dequant_lut(sc), O.dequant_lut(sc))
    wrapped = np.array([-9] * 32, dtype=np.int8)  # index -1: Python wraps to the last entry
    assert_f16_equal(B.lut_dequantize(wrapped, s16[:1]), np.full(32, O.dequant_lut(s16[0])[15]))
    with pytest.raises(IndexError):
        B.lut_dequantize(np.array([8] * 32, dtype=np.int8), s16[:1])
    with pytest.raises(IndexError):
        B.lut_dequantize(q, s16[:3])


def test_lut_gather_modes():
    from moat_amd.dequant import lut_dequantize_fp16
    rng = np.random.default_rng(4)
    lut1 = np.arange(10, 26).astype(np.float16)
    cases = [
        (np.array([-8, -7, 0, 7], np.int8), lut1),
        (np.array([-10, 20, 5, 0], np.int32), np.linspace(-8.0, 7.0, 16, dtype=np.float16)),
        (np.array([0, 2, 4, 1, 3], np.int32), np.array([-4.0, -2.0, 0.0, 2.0, 4.0], np.float16)),
        (rng.integers(0, 20, 64).astype(np.uint8), lut1),
        (rng.integers(-8, 8, 8 * 32).astype(np.int8).reshape(8, 32), rng.standard_normal((8, 16)).astype(np.float32)),
        (rng.integers(-8, 8, 4 * 8 * 32).astype(np.int8), (rng.standard_normal((4, 8, 16)) * 0.1)),
        (rng.integers(0, 15, 96).astype(np.int64), rng.standard_normal((3, 16)).astype(np.float32)),
        (rng.random(40).astype(np.float32) * 15, lut1),
    ]
    for q, lut in cases:
        say(f"case: lut gather q={q.dtype}{q.shape} lut={np.asarray(lut).dtype}{np.asarray(lut).shape}")
        got = lut_dequantize_fp16(q, lut)
        exp = O.lut_gather(q, lut)
        assert got.shape == exp.shape
        assert_f16_equal(got, exp)
    with pytest.raises(ValueError):
        lut_dequantize_fp16(np.zeros(4, np.int8), np.zeros((1, 1, 1, 16), np.float16))


def test_f64_table_single_rounding():
    """float64 -> fp16 must round once (a float32 step in between can double-round)."""
    from moat_amd.dequant import lut_dequantize_fp16
    # 1 + 2^-11 + 2^-40 is just above the fp16 halfway point; via float32 it lands exactly on it
    vals = np.array([1 + 2.0 ** -11 + 2.0 ** -40, 1 + 2.0 ** -11, -(2.0 ** -25) * 1.0000001, 65519.99, 1e-300, np.inf],
                    dtype=np.float64)
    got = lut_dequantize_fp16(np.arange(len(vals), dtype=np.uint8), vals)
    assert_f16_equal(got, vals.astype(np.float16))
