"""The record-stream GEMM's hand-off protocol on the host: the word
encoding over every fp32 bit pattern, the chunk and stop rules, and a
simulated workspace through a late store, a give-up, the sticky status that
turns later calls' results into NaN, and a clear (tests/handoff_sim.cpp,
built with g++ against moat_amd/csrc/handoff.h, the header the kernel uses)."""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_handoff_protocol_on_host(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path / "handoff_sim"
    subprocess.run([gxx, "-O2", "-std=c++17", "-I", os.path.join(ROOT, "moat_amd", "csrc"),
                    os.path.join(ROOT, "tests", "handoff_sim.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    for name in ("chunk_rules", "protocol", "encoding_exhaustive"):
        assert f"ok {name}" in out.stdout, out.stdout
