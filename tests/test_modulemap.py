"""The Swift-facing module: include/module.modulemap must expose every C
entry point the drop-in boundary declares (er_hip.h, er_gguf.h) and every
function INTEGRATION.md's Swift binding calls.  Checked with clang's own
module loader: a C translation unit that does `@import EdgeRunnerHIP;` and
takes the address of each function must compile (what a Swift
`import EdgeRunnerHIP` resolves goes through the same module map).  The
translation unit is Objective-C because `@import` is that language's module
syntax; the headers themselves are plain C."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CLANG = Path("/opt/rocm/llvm/bin/clang")
BOUNDARY_HEADERS = ("er_hip.h", "er_gguf.h")


def header_functions(name):
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / name).read_text(), flags=re.S)
    return set(re.findall(r"\b(er_\w+)\s*\(", text))


def header_types(name):
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / name).read_text(), flags=re.S)
    return set(re.findall(r"}\s*(er_\w+)\s*;", text)) | set(re.findall(r"typedef\s+struct\s+\w+\s+(er_\w+)\s*;", text))


def swift_calls():
    """C functions (and C struct initialisers) called in INTEGRATION.md's
    swift code blocks."""
    doc = (ROOT / "INTEGRATION.md").read_text()
    calls = set()
    for block in re.findall(r"```swift\n(.*?)```", doc, flags=re.S):
        calls |= set(re.findall(r"\b(er_[a-z0-9_]+)\s*\(", block))
    return calls


def compile_against_module(tmp_path, names):
    src = tmp_path / "uses_module.m"
    refs = ",\n    ".join(f"(void (*)(void))&{n}" for n in sorted(names))
    src.write_text("@import EdgeRunnerHIP;\n\n"
                   f"void (*const every_entry[])(void) = {{\n    {refs}\n}};\n"
                   "int status_ok(void) { return ER_OK; }\n")
    return subprocess.run([str(CLANG), "-fmodules", "-fimplicit-module-maps",
                           f"-fmodules-cache-path={tmp_path / 'mcache'}", "-I", str(ROOT / "include"),
                           "-fsyntax-only", "-x", "objective-c", str(src)],
                          capture_output=True, text=True)


needs_clang = pytest.mark.skipif(not CLANG.exists() and shutil.which("clang") is None,
                                 reason="clang with module support not found")


def test_module_lists_the_boundary_headers_only():
    text = (ROOT / "include" / "module.modulemap").read_text()
    headers = re.findall(r'header\s+"([^"]+)"', text)
    assert sorted(headers) == sorted(BOUNDARY_HEADERS)
    assert 'link "edgerunner_hip"' in text


def test_integration_swift_calls_are_declared():
    funcs = set().union(*(header_functions(h) for h in BOUNDARY_HEADERS))
    types = set().union(*(header_types(h) for h in BOUNDARY_HEADERS))
    calls = swift_calls()
    assert {"er_gguf_open", "er_hip_gguf_upload", "er_hip_create"} <= calls
    assert calls <= funcs | types, sorted(calls - funcs - types)


@needs_clang
def test_module_import_resolves_every_entry_point(tmp_path):
    types = set().union(*(header_types(h) for h in BOUNDARY_HEADERS))
    names = set().union(*(header_functions(h) for h in BOUNDARY_HEADERS)) | (swift_calls() - types)
    r = compile_against_module(tmp_path, names)
    assert r.returncode == 0, r.stderr[-4000:]


@needs_clang
def test_module_import_rejects_an_undeclared_name(tmp_path):
    """The check has teeth: a name outside the module fails to resolve."""
    r = compile_against_module(tmp_path, {"er_hip_create", "er_hip_not_an_entry_point"})
    assert r.returncode != 0 and "er_hip_not_an_entry_point" in r.stderr
