"""Register use of the built gfx950 code object: no kernel spills VGPRs or
SGPRs to scratch memory.  A spill inside the GEMV kernels' load sequences
turns their exact per-row load waits into full drains (one such kernel ran at
twice the time of its spill-free neighbour), and the compiler's choice depends
on unroll depth and loads in flight, so every configuration is checked.  Reads
the AMDGPU metadata of this build's own code object with the ROCm LLVM
tools."""
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HSACO = ROOT / "_build" / "er_kernels.hsaco"
LLVM = Path("/opt/rocm/llvm/bin")


def _kernel_metadata(tmp_path):
    bundler, readobj = LLVM / "clang-offload-bundler", LLVM / "llvm-readobj"
    if not HSACO.exists() or not bundler.exists() or not readobj.exists():
        pytest.skip("built code object or ROCm LLVM tools not present")
    elf = tmp_path / "er_kernels_gfx950.elf"
    subprocess.run([str(bundler), "--unbundle", "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                    f"--input={HSACO}", f"--output={elf}"], check=True)
    notes = subprocess.run([str(readobj), "--notes", str(elf)], check=True, capture_output=True,
                           text=True).stdout
    # Each kernel's map lists .args (whose entries carry their own .name) before
    # the kernel's .name, and the register counts after it.
    kernels, name = {}, None
    for line in notes.splitlines():
        m = re.match(r"\s+\.name:\s+(\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.match(r"\s+\.(vgpr_spill_count|sgpr_spill_count|vgpr_count):\s+(\d+)", line)
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
