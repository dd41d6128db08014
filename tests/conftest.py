"""Shared pytest setup.

Markers: `gpu` = needs a ROCm GPU (run on the MI355X box with `-m gpu`); everything else runs
on the CPU. Native libraries are built in-tree by flash-attention-from-scratch_amd/fa_build.py;
a test session only builds the CPU-side helpers if they are missing (the GPU box runs with the
prebuilt libraries that travel with the tree).
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "flash-attention-from-scratch_amd"
for p in (str(PKG), str(REPO)):
    if p not in sys.path:
        sys.path.insert(0, p)

# |out - ref| <= ATOL + RTOL * |ref|, elementwise.
ATOL = 2e-3
RTOL = 1e-2


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")


def _ensure_built(*targets: str) -> None:
    import importlib

    fa_build = importlib.import_module("fa_build")
    paths = {
        "lib": PKG / "fa" / "libfa_hip.so",
        "oracle": REPO / "oracle" / "liboracle_fp64.so",
        "geom": REPO / "tests" / "geometry" / "libfa_geom.so",
        "blocks": REPO / "tests" / "blocks" / "libfa_blocks.so",
    }
    for t in targets:
        if not paths[t].exists():
            fa_build.TARGETS[t]()


@pytest.fixture(scope="session", autouse=True)
def _native_helpers():
    _ensure_built("oracle", "geom")
    yield


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()
