"""The golden fixtures of ``tests/golden`` (written by ``tests/golden/make_golden.py``
from the format and exact IEEE rounding, independent of the oracle) against
the oracle on the CPU and against the HIP path on the GPU: quantize + pack
bytes, dequantized binary16 bits, and Y = X @ W within 1e-3 of RMS(Y)
(measured errors are far smaller: fp32 accumulation of exact products)."""

import glob
import os

import numpy as np
import pytest

from oracle import superblock_oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))
TOL = 1e-3


def _load(path):
    with np.load(path, allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def _rel(y, ref):
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.max(np.abs(np.asarray(y, dtype=np.float64) - ref)) / np.sqrt(np.mean(ref ** 2)))


def test_fixtures_present():
    names = {os.path.basename(p) for p in FIXTURES}
    assert {"aligned_k64_m256_n3.npz", "shifted_k96_m384_n17.npz", "ragged_k40_m96_n5.npz"} <= names


@pytest.mark.parametrize("path", FIXTURES, ids=os.path.basename)
def test_oracle_matches_golden(path):
    d = _load(path)
    K, M, N = (int(v) for v in d["shape"])
    n_sb = K * M // 256
    q, s = O.quantize_a(d["w"].reshape(-1))
    assert np.array_equal(q.reshape(-1), d["q"])
    assert np.array_equal(s.view(np.uint16), d["scales"])
    assert np.array_equal(O.quantize_pack_a(d["w"]).reshape(-1), d["blob"])
    assert np.array_equal(O.decode_superblocks(d["blob"], n_sb).view(np.uint16).reshape(-1), d["deq_bits"])
    y = O.gemm_ref(d["x"], d["blob"], K, M)
    assert _rel(y, d["y"]) <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("path", FIXTURES, ids=os.path.basename)
def test_hip_path_matches_golden(path):
    import torch
    from moat_amd import _lib
    from moat_amd.dequant import batched_int4_matmul, quantize_to_superblocks, unpack_superblock_weights

    d = _load(path)
    K, M, N = (int(v) for v in d["shape"])
    n_sb = K * M // 256
    print(f"case: golden {os.path.basename(path)} K={K} M={M} N={N}", flush=True)
    blob_d = quantize_to_superblocks(torch.from_numpy(d["w"]).cuda())
    assert np.array_equal(blob_d.cpu().numpy().reshape(-1), d["blob"])
    deq = unpack_superblock_weights(blob_d, n_sb)
    assert np.array_equal(deq.cpu().numpy().view(np.uint16).reshape(-1), d["deq_bits"])
    x = torch.from_numpy(d["x"]).cuda()
    choices = [dict(), dict(algo=_lib.GEMM_MFMA, front=_lib.FRONT_RECORDS), dict(algo=_lib.GEMM_MFMA, front=_lib.FRONT_LDS),
               dict(algo=_lib.GEMM_MFMA, front=_lib.FRONT_DIRECT), dict(algo=_lib.GEMM_MFMA, splits=2, finish=3),
               dict(algo=_lib.GEMM_MFMA, front=_lib.FRONT_RECORDS, splits=3, finish=1)]
    if N <= 8:
        choices.append(dict(algo=_lib.GEMM_DOT2))
    for opts in choices:
        y = batched_int4_matmul(x, blob_d, K, M, **opts)
        e = _rel(y.cpu().numpy(), d["y"])
        assert e <= TOL, (os.path.basename(path), opts, e)
