"""Builds the native parts in-tree, for gfx950 only.

    python flash-attention-from-scratch_amd/fa_build.py            # everything
    python flash-attention-from-scratch_amd/fa_build.py --only lib # one target

Targets (outputs are git-ignored; they travel to the GPU box with the source tree):
  lib     fa/libfa_hip.so        HIP kernels + the C ABI of include/fa_hip.h (hipcc, gfx950)
  ext     fa/_C.<abi>.so         PyTorch-ROCm binding (g++ against torch's headers), links lib
  blocks  tests/blocks/libfa_blocks.so   building-block kernels for the GPU unit tests
  oracle  oracle/liboracle_fp64.so       the C fp64 oracle (gcc), test infrastructure only
  geom    tests/geometry/libfa_geom.so   host build of the tile geometry, for the CPU tests
  dev     dev/fa_dev             standalone C++ driver (no Python) over the C ABI, for
          rocprofv3 counter runs and tile tuning (dev/counters.sh, dev/tune.py); and
          dev/tile_ceiling, the synthetic ceiling of the d=64 simple tile

Counterpart of the reference's setup.py / CMakeLists.txt / Makefile build targets
(setup.py:12-33, CMakeLists.txt:56-87, Makefile:21-32): the kernel library is compiled by
hipcc directly (no CUDAExtension, no hipify) and the binding is a plain C++ extension.
"""

from __future__ import annotations

import argparse
import os
import shlex
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = REPO / "include"
FA = PKG / "fa"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"

# Every HIP compile: gfx950 only, and no packed-fp32 VALU instructions (v_pk_fma_f32 and
# friends), which this fleet has seen give silently wrong results.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Keep MFMA accumulators in ordinary VGPRs: with AGPR accumulators every VALU touch of O
    # (the softmax rescale) costs a v_accvgpr_read/write round trip per register.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wall",
]


def _run(cmd: list[str], quiet: bool = False) -> None:
    if not quiet:
        print("+", " ".join(shlex.quote(c) for c in cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: drop that noise.
    err = "\n".join(
        line for line in res.stderr.splitlines() if "packed-fp32-ops" not in line and line.strip()
    )
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if err and not quiet:
        print(err, file=sys.stderr)


def _hipcc() -> str:
    return str(ROCM / "bin" / "hipcc")


def _kernel_resources(remarks: str) -> dict:
    """Per-kernel VGPRs, AGPRs, scratch bytes per lane, occupancy (waves per SIMD) and LDS
    bytes, from hipcc's -Rpass-analysis=kernel-resource-usage remarks."""
    import re

    out: dict = {}
    name = None
    fields = {"VGPRs": "vgpr", "AGPRs": "agpr", "ScratchSize [bytes/lane]": "scratch",
              "Occupancy [waves/SIMD]": "occupancy", "LDS Size [bytes/block]": "lds"}
    for line in remarks.splitlines():
        m = re.search(r"remark: (.*?) \[-Rpass-analysis=kernel-resource-usage\]", line)
        if not m:
            continue
        text = m.group(1).strip()
        if text.startswith("Function Name: "):
            name = text[len("Function Name: "):]
            out[name] = {}
        elif name is not None and ":" in text:
            key, _, val = text.rpartition(":")
            if key.strip() in fields and val.strip().lstrip("-").isdigit():
                out[name][fields[key.strip()]] = int(val)
    return out


def build_lib(extra: list[str] | None = None) -> Path:
    """Builds fa/libfa_hip.so and records each kernel's register, scratch, occupancy and LDS
    use in fa/libfa_hip.resources.json (checked by tests/test_kernel_resources.py)."""
    import json

    out = FA / "libfa_hip.so"
    cmd = [_hipcc(), *HIP_FLAGS, "-shared", f"-I{INCLUDE}", f"-I{CSRC}",
           "-Rpass-analysis=kernel-resource-usage", str(CSRC / "flash_fwd.hip"), "-o", str(out),
           *(extra or [])]
    print("+", " ".join(shlex.quote(c) for c in cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        err = "\n".join(ln for ln in res.stderr.splitlines() if "remark:" not in ln)
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    (FA / "libfa_hip.resources.json").write_text(
        json.dumps(_kernel_resources(res.stderr), indent=1, sort_keys=True) + "\n")
    return out


def _ext_suffix() -> str:
    return sysconfig.get_config_var("EXT_SUFFIX") or ".so"


def build_ext() -> Path:
    import torch
    from torch.utils import cpp_extension

    out = FA / f"_C{_ext_suffix()}"
    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [f"-I{p}" for p in cpp_extension.include_paths()]
    pyinc = sysconfig.get_paths()["include"]
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *incs, f"-I{pyinc}", f"-I{ROCM / 'include'}", f"-I{INCLUDE}",
        str(CSRC / "bindings.cpp"),
        f"-L{FA}", "-lfa_hip",
        f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
        "-Wl,-rpath,$ORIGIN",
        "-o", str(out),
    ]
    _run(cmd)
    return out


def build_blocks() -> Path:
    src = REPO / "tests" / "blocks" / "fa_blocks.hip"
    out = src.parent / "libfa_blocks.so"
    cmd = [_hipcc(), *HIP_FLAGS, "-shared", f"-I{CSRC}", str(src), "-o", str(out)]
    _run(cmd)
    return out


def build_oracle() -> Path:
    src = REPO / "oracle" / "attention_fp64.c"
    out = REPO / "oracle" / "liboracle_fp64.so"
    _run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-Wextra", str(src),
          "-o", str(out), "-lm"])
    return out


def build_geom() -> Path:
    src = REPO / "tests" / "geometry" / "geom_shim.cpp"
    out = src.parent / "libfa_geom.so"
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra", f"-I{CSRC}",
          str(src), "-o", str(out)])
    return out


def build_dev() -> Path:
    src = PKG / "dev" / "fa_dev.cpp"
    out = src.parent / "fa_dev"
    _run([_hipcc(), *HIP_FLAGS, "-Wextra", f"-I{INCLUDE}", str(src), "-o", str(out), "-ldl"])
    probe = PKG / "dev" / "tile_ceiling.hip"
    _run([_hipcc(), *HIP_FLAGS, "-Wextra", str(probe), "-o", str(probe.with_suffix(""))])
    return out


TARGETS = {"lib": build_lib, "ext": build_ext, "blocks": build_blocks, "oracle": build_oracle,
           "geom": build_geom, "dev": build_dev}
ALL = ("lib", "ext", "blocks", "oracle", "geom", "dev")


def build_all() -> None:
    for name in ALL:
        TARGETS[name]()


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--only", choices=sorted(TARGETS), action="append")
    ap.add_argument("--define", action="append", default=[], metavar="NAME=VALUE",
                    help="a kernel build option of libfa_hip.so (a macro of csrc/flash_fwd.hip), "
                         "e.g. FA_PP16_UNCHECKED=0 for the per-tile checked softmax")
    args = ap.parse_args()
    for d in args.define:
        if not d.split("=", 1)[0].startswith("FA_"):
            ap.error(f"--define takes the library's FA_* options, got {d}")
    for name in args.only or ALL:
        if name == "lib":
            build_lib([f"-D{d}" for d in args.define])
        else:
            TARGETS[name]()


if __name__ == "__main__":
    main()
