"""Compiles each HIP source to gfx950 assembly with the library's own flags and
checks what must never appear in it (CPU only).

* packed fp32 VALU ops (v_pk_add/mul/fma_f32) are excluded by the build flags;
* mixed-precision multiply+convert (v_fma_mix / v_mad_mix) would round once
  where the reference rounds twice (float32 product, then fp16);
* the kernels never write through the scalar data cache;
* inline assembly that reads scalar registers in a vector memory instruction
  sees at least 5 wait states after a VALU instruction writes one of them (a
  gfx9 hazard the compiler does not fix inside inline assembly: a spilled
  base address reloaded by v_readlane right before such a block is read
  stale, and the load goes to a wrong address).
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


def _sgprs(tok):
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"s(\d+)", tok)
    return {int(m.group(1))} if m else set()


def sgpr_vmem_hazards(text):
    """(line, instruction, writer) for each vector memory instruction inside
    an inline-assembly block that reads an SGPR written by a VALU instruction
    fewer than 5 wait states earlier (an s_nop k counts k + 1)."""
    lines = text.splitlines()
    in_asm, hits = False, []
    for i, ln in enumerate(lines):
        if ";;#ASMSTART" in ln:
            in_asm = True
            continue
        if ";;#ASMEND" in ln:
            in_asm = False
            continue
        t = ln.strip()
        if not in_asm or not (t.startswith("global_") or t.startswith("buffer_")) or " " not in t:
            continue
        used = set()
        for op in t.split(None, 1)[1].split(","):
            op = op.strip()
            if op:
                used |= _sgprs(op.split()[0])
        if not used:
            continue
        ws, j = 0, i - 1
        while j >= 0 and ws < 5:
            u = lines[j].strip()
            j -= 1
            if not u or u.startswith(";") or u.startswith(".") or u.endswith(":"):
                continue
            m = re.match(r"s_nop (\d+)", u)
            if m:
                ws += int(m.group(1)) + 1
                continue
            if u.startswith("v_") and " " in u and _sgprs(u.split(None, 1)[1].split(",")[0].strip()) & used:
                hits.append((i + 1, t, u))
                break
            ws += 1
    return hits


def test_hazard_scan_finds_the_pattern():
    bad = "\tv_readlane_b32 s42, v253, 59\n\t;;#ASMSTART\n\tglobal_load_dwordx4 v[0:3], v4, s[42:43] sc1\n\t;;#ASMEND"
    good = bad.replace(";;#ASMSTART\n", ";;#ASMSTART\n\ts_nop 4\n")
    assert len(sgpr_vmem_hazards(bad)) == 1 and not sgpr_vmem_hazards(good)


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
    hazards = sgpr_vmem_hazards(text)
    assert not hazards, f"{src}: VALU-written SGPR read by inline-asm VMEM too soon: {hazards[:3]}"
