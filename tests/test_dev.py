"""The standalone driver (dev/fa_dev), the counter summariser and the tuning sweep.

CPU: argument handling of fa_dev before any device call, the summariser on a synthetic
rocprofv3 output, and that every tuning slot names a macro of the tile table.
GPU: fa_dev runs the kernel through the C ABI and its sampled-row fp64 check passes.
"""

from __future__ import annotations

import csv
import json
import re
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
DEV = REPO / "flash-attention-from-scratch_amd" / "dev"
FA_DEV = DEV / "fa_dev"


def _need_driver():
    if not FA_DEV.exists():
        pytest.skip("dev/fa_dev not built (fa_build.py --only dev)")


@pytest.mark.parametrize("args,msg", [
    (["1", "1", "64", "96"], "head_dim must be 64 or 128, got 96"),
    (["1", "1", "64", "64", "0", "1", "bogus"], "variant must be base, opt or fp16acc"),
    (["1", "1", "64", "64", "0", "0"], "iters must be >= 1"),
    (["1", "1", "0", "64"], "seqlen"),
    (["1", "1", "64", "64", "--lib", "/nonexistent/libfa_hip.so"], "dlopen"),
])
def test_fa_dev_rejects_bad_arguments(args, msg):
    _need_driver()
    res = subprocess.run([str(FA_DEV), *args], capture_output=True, text=True, timeout=60)
    assert res.returncode == 2
    assert msg in res.stderr


def _write_csv(path: Path, header: list[str], rows: list[list]):
    path.parent.mkdir(parents=True, exist_ok=True)
    with path.open("w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


@pytest.mark.parametrize("kname, fpm, shape", [("_ZN2fa16flash_fwd_kernelE", 32768, "32x32x16"),
                                               ("_ZN2fa20flash_fwd_pingpong16E", 16384, "16x16x32")])
def test_counters_summary(tmp_path, kname, fpm, shape):
    """Two dispatches of a kernel: the first (the checked launch) is dropped, and the derived
    figures follow from the second one's counters; MFMA FLOPs per instruction follow the
    kernel (flash_fwd_pingpong16 issues 16x16x32 MFMAs)."""
    b, h, n, d = 1, 2, 1024, 128
    flops = 4.0 * b * h * n * n * d
    hdr = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    second = {"SQ_INSTS_MFMA": flops / fpm, "SQ_VALU_MFMA_BUSY_CYCLES": 1024 * 500.0,
              "GRBM_GUI_ACTIVE": 8 * 1000.0, "SQ_INSTS_VALU": 4 * flops / fpm,
              "SQ_LDS_BANK_CONFLICT": 0.0, "SQ_LDS_IDX_ACTIVE": 10.0}
    rows = [[1, kname, k, 7 * v] for k, v in second.items()]
    rows += [[2, kname, k, v] for k, v in second.items()]
    rows += [[3, "other_kernel", "SQ_INSTS_MFMA", 1e12]]
    _write_csv(tmp_path / "pmcA" / "run_counter_collection.csv", hdr, rows)
    alg = 4 * b * h * n * d * 2
    _write_csv(tmp_path / "fetch" / "x_counter_collection.csv", hdr,
               [[1, kname, "FETCH_SIZE", 1.0], [2, kname, "FETCH_SIZE", 3 * alg / 4 / 1024 / 2]])
    _write_csv(tmp_path / "write" / "x_counter_collection.csv", hdr,
               [[1, kname, "WRITE_SIZE", 1.0], [2, kname, "WRITE_SIZE", alg / 4 / 1024]])
    _write_csv(tmp_path / "trace" / "run_kernel_trace.csv",
               ["Kernel_Name", "Start_Timestamp", "End_Timestamp"],
               [[kname, 0, 5_000_000], [kname, 10_000_000, 11_000_000]])
    res = subprocess.run(
        [sys.executable, str(DEV / "counters.py"), str(tmp_path), "--shape", str(b), str(h),
         str(n), str(d), "0", "--fetch-scale", "2.0"], capture_output=True, text=True, timeout=60)
    assert res.returncode == 0, res.stderr
    out = res.stdout
    assert "| MFMA FLOPs / algorithmic FLOPs | 1.0000 |" in out
    assert "= 50.0 %" in out                      # 500 busy cycles per SIMD of 1000
    assert f"| non-MFMA VALU instructions per MFMA ({shape}) | 3.00 |" in out
    assert f"{flops / 1e-3 / 1e12:.1f}" in out    # 1 ms, the second launch only
    assert f"= 1.00 x algorithmic {alg:,}" in out


def test_tune_slots_name_tile_macros():
    src = (REPO / "flash-attention-from-scratch_amd" / "csrc" / "flash_fwd.hip").read_text()
    sys.path.insert(0, str(DEV))
    try:
        import tune
    finally:
        sys.path.remove(str(DEV))
    for slot, (macro, variant, d, causal, extra) in tune.SLOTS.items():
        assert re.search(rf"#ifndef {macro}\n#define {macro} ", src), slot
        assert variant in ("opt", "base") and d in (64, 128) and causal in (0, 1)
        for e in extra:
            assert e.split("=")[0][2:] in src
    assert tune._build_one("opt_d64", "32,4,true") == ("32,4,true",
                                                       "bad candidate (want BC,NW,LAZY,SCHED)")


@pytest.mark.gpu
@pytest.mark.parametrize("args", [["2", "3", "300", "64", "1", "3", "opt"],
                                  ["1", "2", "1000", "128", "0", "3", "base"]])
def test_fa_dev_runs_and_checks(args):
    _need_driver()
    print(f"case fa_dev {' '.join(args)}", flush=True)
    res = subprocess.run([str(FA_DEV), *args, "--json", "--warmup-ms", "20"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    rec = json.loads(res.stdout.splitlines()[0])
    assert rec["check"] == "ok" and rec["max_abs_err"] < 2e-2 and rec["tflops"] > 0
