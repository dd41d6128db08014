"""CPU: register, scratch and occupancy budget of every kernel in the built library.

fa_build.py records hipcc's kernel-resource-usage remarks for libfa_hip.so in
fa/libfa_hip.resources.json. The schedules are designed for a number of waves per SIMD
(the ping-pong pairs two waves on a SIMD, the simple d=64 tile runs two 8-wave workgroups per
CU, ...); a code change that makes the compiler spill or drop a kernel below its occupancy
costs far more than any instruction it saves (an innocuous-looking early exit once cost the
causal d=64 tile 30 VGPRs and half its occupancy). This test pins the budget.
"""

from __future__ import annotations

import json
import re
from pathlib import Path

import pytest

RES = Path(__file__).resolve().parents[1] / "flash-attention-from-scratch_amd" / "fa" / \
    "libfa_hip.resources.json"
TILE = re.compile(r"TileILi(\d+)ELi(\d+)ELi(\d+)ELb(\d)ELi(\d)E")
SIMPLE, KSPLIT, PINGPONG16, KSPLIT4, SIMPLE16 = 0, 3, 4, 5, 6


def _load():
    if not RES.exists():
        pytest.skip("library not built (fa_build.py --only lib)")
    return json.loads(RES.read_text())


def _family(mangled: str) -> str:
    """Kernel function name of a mangled symbol (_ZN2fa12_GLOBAL__N_1<len><name>I...)."""
    m = re.search(r"_GLOBAL__N_1(\d+)", mangled)
    assert m, mangled
    start = m.end()
    return mangled[start:start + int(m.group(1))]


def _min_occupancy(name: str) -> int:
    family = _family(name)
    if family == "flash_fwd_combine":
        return 4
    d, bc, nw, _lazy, sched = (int(x) for x in TILE.search(name).groups())
    if family == "flash_fwd_pingpong16":
        return 2                      # waves w and w+4 share a SIMD
    if family == "flash_fwd_ksplit":
        return 2                      # two 4-wave workgroups (64 KiB) or one 8-wave (128 KiB)
    assert (family, sched) in (("flash_fwd_kernel", SIMPLE), ("flash_fwd_simple16", SIMPLE16)), name
    if d == 64 and bc == 128:
        return 2                      # one-round causal grids: one 8-wave workgroup per CU
    return 4 if d == 64 else 2        # d=64: two 8-wave workgroups per CU


def test_every_kernel_is_recorded():
    families = {_family(k) for k in _load()}
    assert families == {"flash_fwd_kernel", "flash_fwd_simple16", "flash_fwd_pingpong16",
                        "flash_fwd_ksplit", "flash_fwd_combine"}, families


def test_no_kernel_spills_to_scratch():
    for name, r in _load().items():
        assert r.get("scratch", 0) == 0, (name, r)


def test_kernels_keep_their_occupancy():
    """Occupancy, and at most 64 KiB of LDS per workgroup (the four-way key split aside): on
    gfx950 K/V tiles placed above the first 64 KiB of a workgroup's LDS measured 2.9 % slower on
    the causal pair kernels (an unused 64 KiB array declared before them; placed after them, the
    same 112 KiB cost nothing)."""
    for name, r in _load().items():
        want = _min_occupancy(name)
        assert r["occupancy"] >= want, (name, r, want)
        four_way = (_family(name) == "flash_fwd_ksplit"
                    and int(TILE.search(name).group(5)) == KSPLIT4)
        assert r["lds"] <= (160 if four_way else 64) * 1024, (name, r)
