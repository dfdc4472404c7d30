"""Build the gfx950 code object and the host libraries in-tree.

Produces (next to this file, so they travel with the source tree):
  libedgerunner_hip.so   -- the C-ABI library (include/er_hip.h, er_gguf.h) with
                            the gfx950 code object embedded
  libedgerunner_probe.so -- the measurement library: the same sources built with
                            -DER_WITH_PROBES (every er_hip.h entry point plus
                            csrc/er_hip_probe.h); bench.py's ceilings and GEMM
                            clock legs only
  liber_synth.so         -- seeded synthetic workload generator (host only)

Usage: python -m edgerunner_amd.build
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = ROOT / "_build"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")

# Device flags.  Packed-FP32 instruction selection is disabled for every
# kernel (the hardware's packed fp32 forms are not used by this library);
# 128-bit LDS accesses are enabled (ds_read_b128 / ds_write_b128).
DEVICE_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Xclang", "-target-feature", "-Xclang", "+enable-ds128",
    "-munsafe-fp-atomics",
]

LIB = PKG / "libedgerunner_hip.so"
PROBE_LIB = PKG / "libedgerunner_probe.so"
SYNTH = PKG / "liber_synth.so"
CODE_OBJECT = BUILD / "er_kernels.hsaco"
PROBE_CODE_OBJECT = BUILD / "er_kernels_probe.hsaco"
PROBE_DEFINES = ["-DER_WITH_PROBES=1"]


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def _code_object_cmd(out: Path, extra: list[str] | None = None) -> list[str]:
    return [HIPCC, *DEVICE_FLAGS, *(extra or []), "--genco", "-I", str(CSRC),
            str(CSRC / "er_kernels.hip"), "-o", str(out)]


def build_code_object(extra: list[str] | None = None, out: Path = CODE_OBJECT) -> Path:
    BUILD.mkdir(exist_ok=True)
    _run(_code_object_cmd(out, extra))
    return out


def build_code_objects() -> None:
    """The product and the measurement code objects, compiled concurrently
    (one hipcc process each)."""
    BUILD.mkdir(exist_ok=True)
    cmds = [_code_object_cmd(CODE_OBJECT), _code_object_cmd(PROBE_CODE_OBJECT, PROBE_DEFINES)]
    procs = []
    for c in cmds:
        print("+", " ".join(c), flush=True)
        procs.append(subprocess.Popen(c))
    bad = [c for c, p in zip(cmds, procs) if p.wait() != 0]
    if bad:
        raise subprocess.CalledProcessError(1, bad[0])


def _blob_source(code_object: Path) -> str:
    """Assembly that embeds the code object as er_kernels_blob[_end]."""
    return ("    .section .rodata\n"
            "    .balign 4096\n"
            "    .globl er_kernels_blob\n"
            "er_kernels_blob:\n"
            f"    .incbin \"{code_object}\"\n"
            "    .globl er_kernels_blob_end\n"
            "er_kernels_blob_end:\n"
            "    .byte 0\n"
            "    .section .note.GNU-stack,\"\",@progbits\n")


def build_host_library(code_object: Path = CODE_OBJECT, out: Path = LIB, defines: list[str] | None = None) -> Path:
    BUILD.mkdir(exist_ok=True)
    tag = out.stem
    blob = BUILD / f"{tag}_blob.S"
    blob.write_text(_blob_source(code_object))
    blob_o = BUILD / f"{tag}_blob.o"
    host_o = BUILD / f"{tag}_er_hip.o"
    _run(["gcc", "-c", str(blob), "-o", str(blob_o)])
    gguf_o = BUILD / f"{tag}_er_gguf.o"
    for src, obj in ((CSRC / "er_hip.cpp", host_o), (CSRC / "er_gguf.cpp", gguf_o)):
        _run(["g++", "-O2", "-fPIC", "-std=c++17", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__", *(defines or []),
              "-I", str(ROCM / "include"), "-I", str(ROOT / "include"), "-I", str(CSRC),
              "-c", str(src), "-o", str(obj)])
    tmp = out.with_suffix(".so.tmp")
    _run(["g++", "-shared", "-o", str(tmp), str(host_o), str(gguf_o), str(blob_o), "-pthread",
          "-L", str(ROCM / "lib"), "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}",
          "-Wl,--version-script=" + str(CSRC / "er_hip.map")])
    os.replace(tmp, out)
    return out


# Host-side sanitizer flags (g++/gcc only; no device code is built with them).
SAN_FLAGS = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer",
             "-g", "-O1"]


def build_sanitized(out_dir: Path) -> tuple[Path, Path]:
    """AddressSanitizer + UndefinedBehaviorSanitizer builds of the host code:
    the C-ABI library (er_hip.cpp, er_gguf.cpp, with the gfx950 code object
    embedded unchanged) and the CPU oracle.  For CPU runs of the host-side
    tests (argument validation, GGUF parsing); the GPU kernels are never
    built with a sanitizer.  Returns (library, oracle library)."""
    out_dir.mkdir(parents=True, exist_ok=True)
    if not CODE_OBJECT.exists():
        build_code_object()
    blob = out_dir / "er_blob.S"
    blob.write_text(_blob_source(CODE_OBJECT))
    blob_o = out_dir / "er_blob.o"
    _run(["gcc", "-c", str(blob), "-o", str(blob_o)])
    objs = []
    for src in (CSRC / "er_hip.cpp", CSRC / "er_gguf.cpp"):
        obj = out_dir / (src.stem + ".o")
        _run(["g++", *SAN_FLAGS, "-fPIC", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I", str(ROCM / "include"),
              "-I", str(ROOT / "include"), "-I", str(CSRC), "-c", str(src), "-o", str(obj)])
        objs.append(str(obj))
    lib = out_dir / "libedgerunner_hip.so"
    _run(["g++", *SAN_FLAGS, "-shared", "-o", str(lib), *objs, str(blob_o), "-pthread", "-L", str(ROCM / "lib"),
          "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}", "-Wl,--version-script=" + str(CSRC / "er_hip.map")])
    oracle = out_dir / "liber_oracle.so"
    _run(["gcc", *SAN_FLAGS, "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-fopenmp", "-std=c11", "-shared",
          "-o", str(oracle), str(ROOT / "oracle" / "er_oracle.c"), "-lm"])
    return lib, oracle


def build_synth() -> Path:
    tmp = SYNTH.with_suffix(".so.tmp")
    _run(["gcc", "-O2", "-fPIC", "-shared", "-std=c11", "-Wall", "-Wextra",
          str(CSRC / "er_synth.c"), "-o", str(tmp), "-lm"])
    os.replace(tmp, SYNTH)
    return SYNTH


def build_all() -> None:
    build_code_objects()
    build_host_library()
    build_host_library(PROBE_CODE_OBJECT, PROBE_LIB, PROBE_DEFINES)
    build_synth()


if __name__ == "__main__":
    build_all()
    sys.exit(0)
