"""Properties of the built gfx950 code object that the GEMV kernels rely on
but the compiler decides, checked on this build's own code object with the
ROCm LLVM tools:
  - no kernel spills VGPRs or SGPRs to scratch memory.  A spill inside the
    GEMV kernels' load sequences turns their exact per-row load waits into
    full drains (one such kernel ran at twice the time of its spill-free
    neighbour), and the compiler's choice depends on unroll depth and loads
    in flight, so every configuration is checked;
  - no kernel has a private (scratch) segment at all: a stack object that is
    not a spill -- a struct whose fields are chosen through a conditional on
    the fields themselves, which selects their addresses -- puts every access
    to it through scratch memory;
  - in the CU-resident kernels whose staging waves issue their first weight
    loads before converting x, the explicit s_waitcnt vmcnt(n) that waits
    for x counts exactly the weight loads issued after the workgroup barrier
    (the x copies precede them in the in-order load count), so it covers x
    and nothing else."""
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HSACO = ROOT / "_build" / "er_kernels.hsaco"
LLVM = Path("/opt/rocm/llvm/bin")


def _elf(tmp_path):
    bundler = LLVM / "clang-offload-bundler"
    if not HSACO.exists() or not bundler.exists():
        pytest.skip("built code object or ROCm LLVM tools not present")
    elf = tmp_path / "er_kernels_gfx950.elf"
    subprocess.run([str(bundler), "--unbundle", "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                    f"--input={HSACO}", f"--output={elf}"], check=True)
    return elf


def _kernel_metadata(tmp_path):
    readobj = LLVM / "llvm-readobj"
    if not readobj.exists():
        pytest.skip("llvm-readobj not present")
    notes = subprocess.run([str(readobj), "--notes", str(_elf(tmp_path))], check=True, capture_output=True,
                           text=True).stdout
    # Each kernel's map lists .args (whose entries carry their own .name) before
    # the kernel's .name, and the register counts after it.
    kernels, name = {}, None
    for line in notes.splitlines():
        m = re.match(r"\s+\.name:\s+(\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.match(r"\s+\.(vgpr_spill_count|sgpr_spill_count|vgpr_count|private_segment_fixed_size):\s+(\d+)",
                     line)
        if m and name is not None:
            kernels.setdefault(name, {})[m.group(1)] = int(m.group(2))
    return kernels


def test_no_kernel_spills(tmp_path):
    kernels = _kernel_metadata(tmp_path)
    gemv = [k for k in kernels if k.startswith("er_gemv_")]
    assert len(gemv) > 100 and any("_cu_" in k for k in gemv)
    spills = {k: v for k, v in kernels.items()
              if v.get("vgpr_spill_count", 0) or v.get("sgpr_spill_count", 0)}
    assert not spills, spills


def test_no_private_segment(tmp_path):
    kernels = _kernel_metadata(tmp_path)
    assert any(k.startswith("er_gemv_q8_0_silu_cuk") for k in kernels)
    private = {k: v["private_segment_fixed_size"] for k, v in kernels.items()
               if v.get("private_segment_fixed_size", 0)}
    assert not private, private


def test_cu_early_weight_loads_match_x_wait(tmp_path):
    objdump = LLVM / "llvm-objdump"
    if not objdump.exists():
        pytest.skip("llvm-objdump not present")
    text = subprocess.run([str(objdump), "-d", str(_elf(tmp_path))], check=True, capture_output=True,
                          text=True).stdout
    # kernels with 1 or >= 5 slots per lane stage x in all waves and issue early
    early = re.compile(r"er_gemv_(q4k|q8_0|q6k)(_top1)?_cu_l\d+_n([15678])_j\w+$")
    checked = 0
    for block in re.split(r"\n(?=[0-9a-f]+ <)", text):
        m = re.match(r"[0-9a-f]+ <([^>]+)>:", block)
        if not m or not early.match(m.group(1)):
            continue
        lines = block.splitlines()
        bar = next(i for i, l in enumerate(lines) if re.search(r"\bs_barrier\b", l))
        loads = 0
        for l in lines[bar + 1:]:
            w = re.search(r"\bs_waitcnt\b.*vmcnt\((\d+)\)", l)
            if w:
                assert int(w.group(1)) == loads, (m.group(1), int(w.group(1)), loads)
                break
            if re.search(r"\b(global|buffer)_load", l):
                loads += 1
        else:
            raise AssertionError(f"{m.group(1)}: no vmcnt wait after the staging barrier")
        checked += 1
    assert checked >= 50
