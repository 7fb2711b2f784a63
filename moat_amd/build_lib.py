"""Builds libmoat_int4.so (the gfx950 kernels + C ABI) in-tree with hipcc.

``python -m moat_amd.build_lib`` or ``moat_amd.build_lib.build()``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libmoat_int4.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = ["abi.hip", "dense.hip", "dequant.hip", "gemm.hip", "probe.hip", "quant.hip", "sample.hip", "strips.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",  # keep every rounding step explicit (bit-exact dequant/quantize)
    "-fno-gpu-flush-denormals-to-zero",  # fp32/fp16 subnormals are values of the format
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libmoat_int4.so)")


def build(verbose: bool = False) -> str:
    """Compile every HIP source into ``moat_amd/libmoat_int4.so``; returns its path."""
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    out = (proc.stdout or "") + (proc.stderr or "")
    # hipcc's host pass does not know the packed-fp32 feature flag; that note is harmless
    noise = "is not a recognized feature for this target"
    lines = [ln for ln in out.splitlines() if noise not in ln and ln.strip()]
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(lines))
    if verbose and lines:
        print("\n".join(lines), flush=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
