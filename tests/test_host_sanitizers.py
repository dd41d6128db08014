"""CPU: the host-side code under AddressSanitizer and UndefinedBehaviorSanitizer.

Counterpart of the reference's host ASan/UBSan build preset (cmake/Sanitizers.cmake:10-24,
CMakePresets.json:24-29). Each part is built here into a temporary directory with
-fsanitize=address,undefined and -fno-sanitize-recover (any report aborts the run) and run as
its own process, so the sanitizer runtimes come first without any preloading:

* tests/sanitize/host_checks.cpp, parts "geom" and "oracle": every function of
  csrc/fa_geometry.h over its domain and the tile arithmetic up to N = 2^30 (g++), and the C
  fp64 oracle (oracle/attention_fp64.c) on seeded inputs and edge arguments;
* the same program, part "abi", linked to a build of csrc/flash_fwd.hip whose host code is
  sanitized (hipcc, sanitizer flags for the host pass only): argument validation, tile choice
  and split-KV planning of every C entry point over a grid of valid and invalid shapes, none
  of which touches the GPU;
* dev/fa_dev built the same way, on the command lines it must reject (exit 2, before any GPU
  call).

GPU code is never built with a sanitizer here: the device pass of every hipcc line is plain.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "flash-attention-from-scratch_amd"
CSRC = PKG / "csrc"
CHECKS = REPO / "tests" / "sanitize" / "host_checks.cpp"
ORACLE_C = REPO / "oracle" / "attention_fp64.c"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]
ENV = {**os.environ, "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0",
       "UBSAN_OPTIONS": "print_stacktrace=1"}


def _host_only(flags):
    """Sanitizer flags for hipcc's host pass only (each one behind -Xarch_host)."""
    out = []
    for f in flags:
        out += ["-Xarch_host", f]
    return out


def _run(cmd, cwd, timeout=300, env=None):
    return subprocess.run(cmd, cwd=cwd, capture_output=True, text=True, timeout=timeout, env=env)


def _clean(res):
    text = res.stdout + res.stderr
    assert "runtime error:" not in text, text[-4000:]
    assert "AddressSanitizer" not in text, text[-4000:]
    return text


def test_geometry_and_oracle_under_sanitizers(tmp_path):
    exe = tmp_path / "host_checks"
    b = _run(["g++", "-std=c++17", "-O1", "-g", *SAN, f"-I{CSRC}", str(CHECKS), "-x", "c",
              str(ORACLE_C), "-x", "none", "-o", str(exe), "-lm"], tmp_path)
    assert b.returncode == 0, b.stderr
    r = _run([str(exe), "geom", "oracle"], tmp_path, env=ENV)
    text = _clean(r)
    assert r.returncode == 0 and "0 failures" in text, text[-4000:]


@pytest.fixture(scope="module")
def hip_tools():
    hipcc = ROCM / "bin" / "hipcc"
    clangxx = ROCM / "llvm" / "bin" / "clang++"
    clang = ROCM / "llvm" / "bin" / "clang"
    if not (hipcc.exists() and clangxx.exists() and clang.exists()):
        pytest.skip("ROCm compilers not found")
    return hipcc, clangxx, clang


def _hip_flags():
    import sys

    sys.path.insert(0, str(PKG))
    import fa_build

    # the library's own flags, with -O1 -g for readable reports
    return [f for f in fa_build.HIP_FLAGS if f not in ("-O3", "-Wall")] + ["-O1", "-g"]


def test_c_abi_host_paths_under_sanitizers(tmp_path, hip_tools):
    hipcc, clangxx, clang = hip_tools
    lib = tmp_path / "libfa_hip_san.so"
    b = _run([str(hipcc), *_hip_flags(), "-shared", *_host_only(SAN), f"-I{REPO / 'include'}",
              f"-I{CSRC}", str(CSRC / "flash_fwd.hip"), "-o", str(lib)], tmp_path, timeout=600)
    assert b.returncode == 0, b.stderr[-4000:]
    b = _run([str(clang), "-O1", "-g", *SAN, "-c", str(ORACLE_C), "-o",
              str(tmp_path / "oracle.o")], tmp_path)
    assert b.returncode == 0, b.stderr
    exe = tmp_path / "host_checks_abi"
    b = _run([str(clangxx), "-std=c++17", "-O1", "-g", *SAN, "-DWITH_ABI",
              f"-I{REPO / 'include'}", f"-I{CSRC}", str(CHECKS), str(tmp_path / "oracle.o"),
              f"-L{tmp_path}", "-lfa_hip_san", f"-Wl,-rpath,{tmp_path}",
              f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}", "-lm",
              "-o", str(exe)], tmp_path)
    assert b.returncode == 0, b.stderr[-4000:]
    r = _run([str(exe), "abi"], tmp_path, env=ENV)
    text = _clean(r)
    assert r.returncode == 0 and "0 failures" in text, text[-4000:]


BAD_COMMAND_LINES = [
    ["--splitkv"], ["--splitkv", "-1"], ["--boost-keys", "2:1"], ["--boost-keys", "0.5"],
    ["--seed", "abc"], ["1", "2", "3", "4", "5", "0"], ["1", "2", "3", "4", "5", "6", "opt", "x"],
    ["--std"], ["--help"], ["99999999999", "1", "1", "1", "1", "1"],
    ["1", "1", "16", "64", "0", "1", "opt", "--lib", "/nonexistent/libfa_hip.so"],
]


def test_fa_dev_rejects_bad_command_lines_under_sanitizers(tmp_path, hip_tools):
    hipcc, _, _ = hip_tools
    exe = tmp_path / "fa_dev_san"
    b = _run([str(hipcc), *_hip_flags(), *_host_only(SAN), f"-I{REPO / 'include'}",
              str(PKG / "dev" / "fa_dev.cpp"), "-o", str(exe), "-ldl"], tmp_path, timeout=600)
    assert b.returncode == 0, b.stderr[-4000:]
    for args in BAD_COMMAND_LINES:
        r = _run([str(exe), *args], tmp_path, timeout=60, env=ENV)
        text = _clean(r)
        assert r.returncode == 2 and "error:" in r.stderr, (args, text[-2000:])
    # a bad head_dim reaches the library's own validation (no GPU call before it)
    lib = PKG / "fa" / "libfa_hip.so"
    if lib.exists():
        r = _run([str(exe), "1", "1", "16", "96", "0", "1", "opt", "--lib", str(lib)], tmp_path,
                 timeout=60, env=ENV)
        _clean(r)
        assert r.returncode == 2 and "head_dim must be 64 or 128" in r.stderr, r.stderr[-2000:]
    assert shutil.which("g++")
