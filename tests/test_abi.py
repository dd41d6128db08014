"""CPU: the C ABI of include/fa_hip.h and the Python binding, without a GPU.

* libfa_hip.so loads and exports every function the header declares;
* the header is valid C and the ctypes struct mirrors its layout;
* every argument check of fa_flash_fwd runs before any HIP call and returns FA_EINVAL with
  the reference's message keywords (csrc/kernels/flash_fwd.cu:626-651,
  tests/cpp/test_flash_fwd.cu:64-83);
* the torch extension imports, and rejects host tensors with the reference's "CUDA" message
  (csrc/bindings.cpp:31-33).
"""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from fa import native

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "fa_hip.h"

GOOD = dict(q=0x1000, k=0x2000, v=0x3000, o=0x4000, batch=1, heads=1, seqlen=64, head_dim=64,
            softmax_scale=0.125, causal=False, variant="opt")


def _declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(fa_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_function():
    names = _declared_functions()
    assert {"fa_flash_fwd", "fa_last_error", "fa_tile_config", "fa_version", "fa_flash_fwd_lse",
            "fa_splitkv_plan", "fa_flash_fwd_splitkv"} <= set(names)
    so = native.lib()
    for name in names:
        assert hasattr(so, name), name


def test_header_is_c_and_struct_layout_matches(tmp_path):
    src = tmp_path / "abi.c"
    src.write_text(
        '#include <stddef.h>\n#include <stdio.h>\n#include "fa_hip.h"\n'
        "int main(void){printf(\"%zu %zu %zu %zu %zu %zu\\n\", sizeof(fa_params),"
        " offsetof(fa_params, batch), offsetof(fa_params, softmax_scale),"
        " offsetof(fa_params, causal), offsetof(fa_params, variant), sizeof(fa_tile_info));"
        " return 0;}\n")
    exe = tmp_path / "abi"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{REPO / 'include'}", str(src),
                    "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True,
                                          check=True).stdout.split()]
    P = native.FaParams
    assert got == [ctypes.sizeof(P), P.batch.offset, P.softmax_scale.offset, P.causal.offset,
                   P.variant.offset, ctypes.sizeof(native.FaTileInfo)]


def _call(**over):
    args = dict(GOOD)
    args.update(over)
    return native.flash_fwd(native.make_params(**args))


@pytest.mark.parametrize("over, words", [
    (dict(batch=0), "batch, heads and seqlen must be positive"),
    (dict(heads=-1), "batch, heads and seqlen must be positive"),
    (dict(seqlen=0), "batch, heads and seqlen must be positive"),
    (dict(head_dim=32), "head_dim must be 64 or 128, got 32"),
    (dict(head_dim=96), "head_dim must be 64 or 128, got 96"),
    (dict(variant=3), "unknown variant"),
    (dict(q=0), "non-null"),
    (dict(o=0), "non-null"),
    (dict(k=0x2008), "16-byte aligned"),
    (dict(o=0x4002), "16-byte aligned"),
    (dict(softmax_scale=float("nan")), "finite"),
    (dict(softmax_scale=float("inf")), "finite"),
    (dict(seqlen=2**24, head_dim=128), "below 2^31"),
    (dict(batch=2**20, heads=2**10, seqlen=2**10), "grid limit"),
])
def test_invalid_arguments_return_einval(over, words):
    rc, msg = _call(**over)
    assert rc == native.FA_EINVAL
    assert words in msg


def test_null_params_and_reserved_bytes():
    so = native.lib()
    assert so.fa_flash_fwd(None, None) == native.FA_EINVAL
    assert b"NULL" in so.fa_last_error()
    p = native.make_params(**GOOD)
    p.reserved[0] = 1
    assert native.flash_fwd(p)[0] == native.FA_EINVAL
    p = native.make_params(**GOOD)
    p.causal = 2
    assert native.flash_fwd(p)[0] == native.FA_EINVAL


def _tile(d, causal, var, n, b=16, h=32):
    t = native.tile_config(d, causal, var, n, b, h)
    return t["block_q"], t["block_k"], t["waves"], t["lds_bytes"], t["schedule"]


def test_tile_config_invariants():
    for d in (64, 128):
        for causal in (False, True):
            for var in ("baseline", "opt", "fp16acc"):
                for n in (1, 1000, 2048, 2049, 3072, 3073, 4096, 4097, 8192, 8193, 16384):
                    for b, h in ((1, 1), (2, 8), (16, 32)):
                        bq, bk, waves, lds, sched = _tile(d, causal, var, n, b, h)
                        # 32 query rows per wave, or per two or four waves (key split)
                        split = {"ksplit": 2, "ksplit4": 4}.get(sched, 1)
                        assert bq == 32 * waves // split and bk % 32 == 0
                        # two or three K/V tile buffers each, per key part
                        assert lds in (4 * bk * 2 * d * split, 6 * bk * 2 * d * split)
                        # above 64 KiB only the four-way key split (one workgroup per CU)
                        assert lds <= 64 * 1024 or (sched == "ksplit4" and lds <= 160 * 1024)
                        # the 16x16x32 layouts: 32-key tiles at d=128, 64-key tiles at d=64
                        if sched in ("simple16", "pingpong16"):
                            assert bk == 4096 // d
                        assert _tile(d, causal, "fp16acc", n, b, h) == _tile(d, causal, "opt", n, b, h)


def test_tile_config_rows():
    """The opt rows by N for a large grid (16 x 32 heads), and the small-grid rows."""
    simple64x8, simple16_64x8 = (256, 64, 8, 32768, "simple"), (256, 64, 8, 32768, "simple16")
    simple128x4, simple16_128x4 = (128, 32, 4, 32768, "simple"), (128, 32, 4, 32768, "simple16")
    pingpong128 = (256, 32, 8, 49152, "pingpong16")                   # three K + three V tiles
    for n in (1, 2048, 4096, 8192, 16384):                            # d=64: simple16 ...
        assert _tile(64, False, "opt", n) == simple16_64x8
    for n in (1, 2048):                                               # ... causal from 2049 keys
        assert _tile(64, True, "opt", n) == simple64x8
    for n in (2049, 4096, 16384):
        assert _tile(64, True, "opt", n) == simple16_64x8
    # one round of one workgroup per CU (256 items) from 4096 keys: the d=64 ping-pong
    pingpong64 = (256, 64, 8, 49152, "pingpong16")
    assert _tile(64, False, "opt", 4096, 1, 16) == pingpong64
    assert _tile(64, False, "opt", 16384, 1, 4) == pingpong64
    assert _tile(64, False, "opt", 4000, 1, 16) == simple16_64x8
    assert _tile(64, False, "opt", 4096, 1, 17) == simple16_64x8
    # causal grids of at most 512 items from 1536 keys: 128-key simple tiles
    round64 = (256, 128, 8, 65536, "simple")
    assert _tile(64, True, "opt", 4096, 1, 16) == round64
    assert _tile(64, True, "opt", 4096, 2, 16) == round64
    assert _tile(64, True, "opt", 4096, 2, 17) == simple16_64x8
    assert _tile(64, True, "opt", 1536, 4, 16) == round64
    assert _tile(64, True, "opt", 1535, 4, 16) == simple64x8
    assert _tile(128, False, "opt", 256) == simple128x4
    assert _tile(128, False, "opt", 257) == simple16_128x4
    assert _tile(128, False, "opt", 1536) == simple16_128x4
    assert _tile(128, False, "opt", 1537) == pingpong128
    assert _tile(128, True, "opt", 512) == simple128x4
    assert _tile(128, True, "opt", 513) == simple16_128x4
    assert _tile(128, True, "opt", 3072) == simple16_128x4
    # above 3072 keys the ping-pong, except grids that run in head groups (256 heads or more:
    # fa::geom::causal_group_heads) up to 4096 keys
    assert _tile(128, True, "opt", 3073, 4, 16) == pingpong128        # 64 heads
    assert _tile(128, True, "opt", 4096, 8, 16) == pingpong128        # 128 heads
    assert _tile(128, True, "opt", 3073) == simple16_128x4            # 512 heads
    assert _tile(128, True, "opt", 4096, 16, 16) == simple16_128x4    # 256 heads
    assert _tile(128, True, "opt", 4097) == pingpong128
    # fewer 8-wave workgroups than CUs: B*H*ceil(N/256) < 256 -> key-split tiles (64 rows,
    # two waves on each 32 rows)
    assert _tile(64, True, "opt", 900, 2, 8) == (64, 64, 4, 65536, "ksplit")
    # at most 256 query blocks of 64 rows and at least 16 key tiles: four waves per 32 rows
    assert _tile(64, True, "opt", 1000, 2, 8) == (64, 64, 8, 131072, "ksplit4")
    assert _tile(128, False, "opt", 1500, 1, 2) == (64, 32, 8, 131072, "ksplit4")
    assert _tile(64, False, "opt", 256, 1, 4) == (64, 64, 4, 65536, "ksplit")
    assert _tile(128, False, "opt", 16384, 1, 3) == (64, 32, 4, 65536, "ksplit")
    assert _tile(128, True, "opt", 16384, 1, 3) == (64, 32, 4, 65536, "ksplit")
    assert _tile(128, False, "opt", 16384, 1, 4) == pingpong128        # 4 * 64 = 256 WGs
    for n in (1, 5000, 16384):
        assert _tile(64, n > 1, "baseline", n) == (128, 64, 4, 32768, "simple")


def test_tile_config_errors():
    with pytest.raises(ValueError, match="seqlen"):
        native.tile_config(128, True, "opt", 0)
    with pytest.raises(ValueError, match="positive"):
        native.tile_config(128, True, "opt", 64, 0, 1)
    with pytest.raises(ValueError, match="head_dim"):
        native.tile_config(96, False)
    with pytest.raises(ValueError, match="variant"):
        native.tile_config(64, False, 7)


def test_version():
    assert "gfx950" in native.version()


def test_extension_imports_and_rejects_host_tensors():
    import torch

    import fa

    assert set(fa.__all__) >= {"forward", "forward_variant", "attention_reference"}
    assert "gfx950" in fa._C.version()
    q = torch.zeros(1, 1, 64, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="CUDA"):
        fa.forward(q, q, q)
    with pytest.raises(RuntimeError, match="CUDA"):
        fa.forward_variant(q, q, q, variant="nope")


# ---- LSE and split-KV entry points: host-side checks (all fail before any HIP call) ---------
def test_lse_entry_rejects_bad_lse_pointer():
    p = native.make_params(**GOOD)
    assert native.flash_fwd_lse(p, 0) == (native.FA_EINVAL, native.flash_fwd_lse(p, 0)[1])
    rc, msg = native.flash_fwd_lse(p, 0x1002)
    assert rc == native.FA_EINVAL and "4-byte aligned" in msg
    rc, msg = native.flash_fwd_lse(native.make_params(**{**GOOD, "head_dim": 96}), 0x1000)
    assert rc == native.FA_EINVAL and "head_dim must be 64 or 128, got 96" in msg


@pytest.mark.parametrize("b,h,n,d,causal", [(1, 2, 16384, 128, False), (1, 2, 16384, 128, True),
                                            (1, 2, 32768, 128, True), (1, 8, 8192, 128, True),
                                            (1, 8, 8192, 64, True), (1, 4, 32768, 128, True),
                                            (2, 8, 1000, 64, True), (1, 1, 1, 64, False),
                                            (16, 32, 2048, 64, True)])
def test_splitkv_plan(b, h, n, d, causal):
    p = native.make_params(**{**GOOD, "batch": b, "heads": h, "seqlen": n, "head_dim": d,
                              "causal": causal})
    # Partial-pass rows: the 16x16x32 ping-pong (256 query rows; 32 keys per tile at d=128, 64 at
    # d=64) except causal d=64 (simple tile, 128 rows, 64 keys) and causal d=128 on grids of
    # fewer 256-row blocks than CUs (simple 4-wave tile, 128 rows, 32 keys); the automatic plan
    # keeps at least 512 keys per range when not causal, 1024 causal d=128 (512 on small
    # grids), 256 causal d=64.
    small = b * h * -(-n // 256) < 256
    bq, bc, min_keys = {(128, False): (256, 32, 512),
                        (128, True): (128, 32, 512) if small else (256, 32, 1024),
                        (64, False): (256, 64, 512), (64, True): (128, 64, 256)}[(d, causal)]
    max_tiles = -(-n // bc)
    for req in (0, 1, 2, 3, 7, 100000):
        plan = native.splitkv_plan(p, req)
        ns, tps = plan["num_splits"], plan["tiles_per_split"]
        assert plan["block_k"] == bc and plan["block_q"] == bq
        assert ns * tps >= max_tiles > (ns - 1) * tps       # ranges cover the keys, none empty
        assert plan["workspace_bytes"] == ns * b * h * n * (d + 1) * 4
        if req:
            assert ns <= req
        else:
            assert tps >= min(min_keys // bc, max_tiles)
    known = {
        # 2 heads x 64 query blocks x 512 key tiles / 256 target workgroups = 256 tiles
        (1, 2, 16384, 128, False): 256,
        # causal, small grid: 2 heads x 4 x (1 + ... + 128) = 66048 (block, tile) pairs / 1024
        # target workgroups -> 65 tiles
        (1, 2, 16384, 128, True): 65,
        # causal, one round of 256 query blocks from 8192 keys: two ranges of the 1024 tiles
        (1, 2, 32768, 128, True): 512, (1, 8, 8192, 128, True): 128,
        # causal: 4 heads x 8 x (1 + ... + 128) = 264192 pairs / 512 -> 516 tiles
        (1, 4, 32768, 128, True): 516,
    }
    if (b, h, n, d, causal) in known:
        assert native.splitkv_plan(p, 0)["tiles_per_split"] == known[(b, h, n, d, causal)]


def test_splitkv_entry_rejects_bad_workspace():
    p = native.make_params(**{**GOOD, "heads": 2, "seqlen": 3000, "head_dim": 128})
    need = native.splitkv_plan(p, 3)["workspace_bytes"]
    rc, msg = native.flash_fwd_splitkv(p, None, 3, 0x10000, need - 1)
    assert rc == native.FA_EINVAL and f"need {need} bytes" in msg
    rc, msg = native.flash_fwd_splitkv(p, None, 3, 0, need)
    assert rc == native.FA_EINVAL and "workspace must be non-null" in msg
    rc, msg = native.flash_fwd_splitkv(p, None, 3, 0x10008, need)
    assert rc == native.FA_EINVAL and "16-byte aligned" in msg
    rc, msg = native.flash_fwd_splitkv(p, None, -1, 0x10000, need)
    assert rc == native.FA_EINVAL and "num_splits" in msg
    rc, msg = native.flash_fwd_splitkv(p, 0x1001, 3, 0x10000, need)
    assert rc == native.FA_EINVAL and "lse must be 4-byte aligned" in msg
    with pytest.raises(ValueError, match="num_splits"):
        native.splitkv_plan(p, -2)



@pytest.mark.parametrize("b,h,n,d,causal,variant,want", [
    # few heads of long sequences: the split-KV path
    (1, 1, 16384, 128, False, "opt", 1), (1, 2, 16384, 128, True, "opt", 1),
    (1, 1, 32768, 128, True, "fp16acc", 1), (1, 2, 4096, 128, True, "opt", 1),
    (1, 4, 8192, 64, False, "opt", 1),
    # causal grids of 256 to 288 query blocks of 256 rows from 8192 keys
    (1, 8, 8192, 128, True, "opt", 1), (1, 9, 8192, 128, True, "opt", 1),
    (1, 4, 16384, 64, True, "opt", 1), (1, 8, 8192, 64, True, "fp16acc", 1),
    (1, 10, 8192, 128, True, "opt", 0),        # 320 blocks
    (1, 16, 4096, 128, True, "opt", 0),        # N below 8192
    (1, 8, 8191, 64, True, "opt", 0),
    (1, 8, 8192, 128, False, "opt", 0),        # not causal
    (1, 8, 8192, 128, True, "baseline", 0),
    # one step past each boundary of the rule
    (1, 2, 4095, 128, True, "opt", 0),         # N below 4096
    (1, 4, 8192, 64, True, "opt", 0),          # causal d = 64
    (1, 16, 4096, 128, False, "opt", 0),       # 256 workgroups of 8 waves fill the GPU
    (1, 15, 4096, 128, False, "opt", 1),       # 240 do not
    (1, 2, 16384, 128, False, "baseline", 0),  # the baseline build is never re-routed
    (2, 8, 1000, 64, True, "opt", 0), (16, 32, 2048, 64, True, "opt", 0),
    (1, 16, 16384, 128, False, "opt", 0),      # the headline shape
])
def test_splitkv_preferred_flag(b, h, n, d, causal, variant, want):
    p = native.make_params(**{**GOOD, "batch": b, "heads": h, "seqlen": n, "head_dim": d,
                              "causal": causal, "variant": variant})
    for req in (0, 3):   # independent of the requested split count
        plan = native.splitkv_plan(p, req)
        assert plan["preferred"] == want and plan["reserved"] == 0


def test_splitkv_info_layout_matches_header(tmp_path):
    src = tmp_path / "info.c"
    src.write_text(
        '#include <stddef.h>\n#include <stdio.h>\n#include "fa_hip.h"\n'
        "int main(void){printf(\"%zu %zu %zu\\n\", sizeof(fa_splitkv_info),"
        " offsetof(fa_splitkv_info, workspace_bytes), offsetof(fa_splitkv_info, preferred));"
        " return 0;}\n")
    exe = tmp_path / "info"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{REPO / 'include'}", str(src),
                    "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True,
                                          check=True).stdout.split()]
    S = native.FaSplitKvInfo
    assert got == [ctypes.sizeof(S), S.workspace_bytes.offset, S.preferred.offset]


def _tail(b, h, n, d, causal=False, variant="opt"):
    p = native.make_params(0x1000, 0x1000, 0x1000, 0x1000, b, h, n, d, d ** -0.5, causal, variant)
    return native.tail_plan(p)


def test_tail_plan_head_split():
    """fa_tail_plan: non-causal ping-pong grids with two or more whole rounds of 256 items and a
    last round at most half full keep the heads that fill the whole rounds in one launch."""
    measured = {(1, 20, 10000): 19, (1, 40, 5000): 38, (1, 17, 8192): 16, (1, 36, 4096): 32,
                (1, 17, 4096): 16, (1, 9, 8192): 8}
    for (b, h, n), want in measured.items():
        assert _tail(b, h, n, 128) == want
    for b, h, n in [(1, 20, 10000), (2, 12, 9000), (3, 16, 6144), (1, 40, 5000), (1, 17, 8192),
                    (1, 36, 4096), (5, 7, 9999), (1, 17, 4096), (1, 9, 8192), (1, 19, 4500)]:
        heads = _tail(b, h, n, 128)
        nqb = -(-n // 256)
        items = b * h * nqb
        if heads:
            assert 0 < heads < b * h
            assert heads * nqb <= items // 256 * 256 < (heads + 1) * nqb
            assert heads * nqb >= 256                 # the first launch keeps the ping-pong row
            assert 3 * (items % 256) <= 256           # the last round was at most 1/3 full
    # full rounds, causal, baseline, short, few-head (split-KV) and d=64 simple rows: no split
    assert _tail(1, 16, 16384, 128) == 0
    assert _tail(4, 16, 4096, 128) == 0
    assert _tail(1, 20, 10000, 128, causal=True) == 0
    assert _tail(1, 20, 10000, 128, variant="baseline") == 0
    assert _tail(1, 45, 3000, 128) == 0
    assert _tail(1, 2, 16384, 128) == 0
    assert _tail(1, 20, 10000, 64) == 19              # d=64: the first heads take the ping-pong
    assert _tail(1, 20, 3000, 64) == 0                # d=64 below 4096 keys: simple tile only
    assert _tail(1, 45, 4096, 128) == 0               # last round 81 % full: one launch
    assert _tail(3, 16, 6144, 128) == 0               # half full: the split measured slower
    assert _tail(2, 12, 9000, 128) == 0               # 3/8 full: within noise, one launch


def test_tail_plan_errors():
    so = native.lib()
    heads = ctypes.c_int64(7)
    assert so.fa_tail_plan(None, ctypes.byref(heads)) == native.FA_EINVAL
    p = native.make_params(0x1000, 0x1000, 0x1000, 0x1000, 1, 1, 64, 96, 1.0, False, "opt")
    assert so.fa_tail_plan(ctypes.byref(p), ctypes.byref(heads)) == native.FA_EINVAL
    assert b"head_dim" in so.fa_last_error() and heads.value == 0
    p = native.make_params(0x1000, 0x1000, 0x1000, 0x1000, 1, 1, 64, 64, 1.0, False, "opt")
    assert so.fa_tail_plan(ctypes.byref(p), None) == native.FA_EINVAL
