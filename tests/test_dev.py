"""The standalone driver (dev/fa_dev), the counter summariser, the tuning sweep and the tile
ceiling probe (dev/tile_ceiling).

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


@pytest.mark.parametrize("iters", ["0", "-3", "2000000"])
def test_tile_ceiling_rejects_bad_iteration_counts(iters):
    """dev/tile_ceiling checks its argument before any HIP call."""
    probe = DEV / "tile_ceiling"
    if not probe.exists():
        pytest.skip("dev/tile_ceiling not built (fa_build.py --only dev)")
    res = subprocess.run([str(probe), iters], capture_output=True, text=True, timeout=60)
    assert res.returncode == 1 and "usage" in res.stderr


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


def _stamps(wgs):
    """A synthetic timeline dump: per workgroup (cu, xcc, entry, [item phase lengths in
    ticks]) -> 32 uint64 slots as the FA_PROBE build writes them (the phase stamps only)."""
    import numpy as np

    out = np.zeros((len(wgs), 32), dtype=np.uint64)
    for w, (cu, xcc, entry, items) in enumerate(wgs):
        out[w, 0] = entry
        t = entry
        for i, (lead, *phases) in enumerate(items):
            t += lead
            out[w, 1 + 5 * i] = t
            for k, dt in enumerate(phases):
                t += dt
                out[w, 2 + 5 * i + k] = t
        out[w, 14] = cu << 8
        out[w, 15] = xcc
    return out


def test_probe_summary_of_synthetic_stamps(tmp_path):
    """dev/probe.py on a dump whose phases are known: two CUs of XCD 0 and one of XCD 1, two
    workgroups in turn on each CU, 150 ticks (1.5 us) apart; phases of 300, 10000, 100, 150
    ticks after an entry-to-item lead of 10."""
    sys.path.insert(0, str(DEV))
    import probe

    item = [(10, 300, 10000, 100, 150)]
    span = 10 + 300 + 10000 + 100 + 150
    wgs = []
    for cu, xcc, skew in [(0, 0, 0), (1, 0, 50), (0, 1, 400)]:
        wgs.append((cu, xcc, 1000 + skew, item))
        wgs.append((cu, xcc, 1000 + skew + span + 150, item))
    path = tmp_path / "stamps.bin"
    _stamps(wgs).tofile(path)
    s = probe.summarize(probe.load(path))
    assert (s["workgroups"], s["cus"], s["pairs"], s["second_passes"]) == (6, 3, False, 0)
    approx = pytest.approx
    assert s["items"][0] == approx({"prologue": 3.0, "steady": 100.0, "last_tile": 1.0,
                                    "final_and_store": 1.5})
    assert s["entry_to_item"] == approx(0.1)
    assert s["gap_between_workgroups_on_a_cu"] == approx(1.5)
    end = (2 * span + 150) / 100.0
    assert s["cu_end"] == approx({"min": end, "median": end + 0.5, "max": end + 4.0})
    assert s["xcd_end"] == approx([end + 0.5, end + 4.0])
    assert "launch" in probe.report(s)


def test_probe_summary_of_pairs(tmp_path):
    """A causal pair workgroup: the second item's phases and the gap between the items."""
    sys.path.insert(0, str(DEV))
    import probe

    path = tmp_path / "pairs.bin"
    _stamps([(0, 0, 500, [(10, 300, 20000, 40, 200), (120, 280, 5000, 30, 190)])]).tofile(path)
    s = probe.summarize(probe.load(path))
    assert s["pairs"] and s["gap_between_items"] == pytest.approx(1.2)
    assert s["items"][1] == pytest.approx({"prologue": 2.8, "steady": 50.0, "last_tile": 0.3,
                                           "final_and_store": 1.9})


def test_library_has_no_probe_symbols():
    """The timeline probe is a development build (FA_PROBE=1): the library as built exports
    neither of its functions, and its kernels hold no stamp array."""
    import ctypes

    lib = REPO / "flash-attention-from-scratch_amd" / "fa" / "libfa_hip.so"
    if not lib.exists():
        pytest.skip("library not built")
    so = ctypes.CDLL(str(lib))
    assert not hasattr(so, "fa_probe_read") and not hasattr(so, "fa_probe_clear")


def test_probe_xcd_clocks(tmp_path):
    """The XCD clock from the shader cycle counts (slots 11 and 13) over the 100 MHz stamps:
    a workgroup of XCD 0 that runs 10,000 ticks (100 us) and 200,000 cycles is at 2.0 GHz, one
    of XCD 1 with 190,000 cycles at 1.9 GHz."""
    sys.path.insert(0, str(DEV))
    import probe

    item = [(10, 300, 9440, 100, 150)]  # 10,000 ticks from entry to the O stores
    a = _stamps([(0, 0, 1000, item), (0, 1, 1000, item)])
    a[0, 11], a[0, 13] = 5_000, 205_000
    a[1, 11], a[1, 13] = 7_000, 197_000
    path = tmp_path / "clocks.bin"
    a.tofile(path)
    s = probe.summarize(probe.load(path))
    assert s["xcd_clock_ghz"] == pytest.approx([2.0, 1.9])
    assert "GHz" in probe.report(s)


def test_probe_summary_of_item_steps(tmp_path):
    """The steps inside an item (slots 16-20): load issue 40 ticks, load wait 110, barrier wait
    60 (the prologue's 210 ticks split), first S 70, first tile 130, the rest of the steady
    tiles 9800 (the 10000 ticks of the steady phase split), last tile 100, final test 40 and
    O-store issue 110 (the 150 ticks of the final phase split)."""
    sys.path.insert(0, str(DEV))
    import probe

    a = _stamps([(0, 0, 1000, [(10, 210, 10000, 100, 150)])])
    start = 1010
    a[0, 16] = start + 40
    a[0, 17] = start + 150
    a[0, 18] = start + 210 + 70
    a[0, 19] = start + 210 + 200
    a[0, 20] = start + 210 + 10000 + 100 + 40
    path = tmp_path / "steps.bin"
    a.tofile(path)
    s = probe.summarize(probe.load(path))
    assert s["detail"][0] == pytest.approx({
        "issue_loads": 0.4, "load_wait": 1.1, "barrier_wait": 0.6, "first_s": 0.7,
        "first_tile": 1.3, "steady_rest": 98.0, "last_tile": 1.0, "final_test": 0.4,
        "store_issue": 1.1})
    assert "steps:" in probe.report(s)
    # a dump without the step stamps has no detail
    b = _stamps([(0, 0, 1000, [(10, 210, 10000, 100, 150)])])
    b.tofile(path)
    assert "detail" not in probe.summarize(probe.load(path))
