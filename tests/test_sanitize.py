"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer.  Builds the
C-ABI library (er_hip.cpp, er_gguf.cpp; the gfx950 code object is embedded
unchanged) and the CPU oracle with -fsanitize=address,undefined
(edgerunner_amd.build.build_sanitized) and runs the host-side tests against
those builds in a child process: GGUF parsing with every truncation and
corruption case (test_gguf.py), the C-ABI's argument validation without a
device (test_abi.py), and the oracle against its known answers and the golden
fixtures.  A sanitizer report aborts the child (abort_on_error /
halt_on_error), which fails this test."""
import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HOST_TESTS = ["tests/test_gguf.py", "tests/test_abi.py", "tests/test_oracle_known_answers.py",
              "tests/test_oracle_gemv.py", "tests/test_golden.py"]


def _runtime(name: str) -> str:
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not present")
    path = subprocess.run([gxx, f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(path) or not Path(path).exists():
        pytest.skip(f"{name} not installed")
    return path


def test_host_code_under_sanitizers(tmp_path):
    sys.path.insert(0, str(ROOT))
    from edgerunner_amd import build as b
    preload = f"{_runtime('libasan.so')}:{_runtime('libubsan.so')}"
    lib, oracle = b.build_sanitized(tmp_path / "asan")
    env = dict(os.environ, LD_PRELOAD=preload,
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=1:verify_asan_link_order=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               ER_HIP_LIB=str(lib), ER_ORACLE_LIB=str(oracle))
    # the child really runs the instrumented builds
    check = ("import ctypes, sys; sys.path.insert(0, sys.argv[1]); ctypes.CDLL(None).__asan_init; "
             "from edgerunner_amd import _ffi; from oracle import ref; import numpy as np; "
             "import edgerunner_amd.synth as s; _ffi.load(); ref.gemv('q4_k', s.q4_k(1, 1, 256), "
             "np.ones(256, np.float32), 1, 256); "
             "maps = open('/proc/self/maps').read(); "
             "assert sys.argv[2] in maps and sys.argv[3] in maps, 'sanitized builds not loaded'")
    r = subprocess.run([sys.executable, "-c", check, str(ROOT), str(lib), str(oracle)], cwd=ROOT, env=env,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    r = subprocess.run([sys.executable, "-m", "pytest", *HOST_TESTS, "-q", "-m", "not gpu", "-p", "no:cacheprovider"],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-4000:]
    assert " passed" in r.stdout
