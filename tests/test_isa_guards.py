"""Compiles each HIP source to gfx950 assembly with the library's own flags and
checks what must never appear in it (CPU only).

* packed fp32 VALU ops (v_pk_add/mul/fma_f32) are excluded by the build flags;
* mixed-precision multiply+convert (v_fma_mix / v_mad_mix) would round once
  where the reference rounds twice (float32 product, then fp16);
* the kernels never write through the scalar data cache.
"""

import os
import re
import subprocess

import pytest

from moat_amd import build_lib

FORBIDDEN = {
    "packed fp32": re.compile(r"\bv_pk_(add|mul|fma|mov)_f32\b"),
    "mixed fma": re.compile(r"\bv_(fma|mad)_mix"),
    "scalar memory write": re.compile(r"\bs_(store|buffer_store|atomic|buffer_atomic|dcache_wb|dcache_discard)"),
}


@pytest.mark.parametrize("src", build_lib.SOURCES)
def test_device_code_free_of_forbidden_instructions(src, tmp_path):
    out = tmp_path / (src + ".s")
    flags = [f for f in build_lib.HIPCC_FLAGS if f not in ("-shared", "-fPIC")]
    cmd = [build_lib.hipcc(), *flags, "--cuda-device-only", "-S", os.path.join(build_lib.CSRC, src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    text = out.read_text()
    assert "v_mfma" in text or src != "gemm.hip"
    for what, rx in FORBIDDEN.items():
        hits = sorted(set(m.group(0) for m in rx.finditer(text)))
        assert not hits, f"{src}: {what}: {hits}"
