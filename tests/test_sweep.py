"""The FA2-paper benchmark sweep (fa/sweep.py), counterpart of the reference's
bench/benchmark.py.

CPU: the shape rule (B = 16384 / N, H = 2048 / d, bench/benchmark.py:165), the FLOP rule
(4 B H N^2 d, halved for causal, :142), the correctness gate and the table writers.
GPU: one small sweep end to end, whose fa rows must pass the gate against the fp32 reference.
"""

from __future__ import annotations

import csv
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from fa import sweep

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "flash-attention-from-scratch_amd"


def test_paper_shape_rule():
    # bench/benchmark.py:165 -- batch = 16384 // seqlen, nheads = 2048 // headdim
    for n in (512, 1024, 2048, 4096, 8192, 16384):
        for d in (64, 128):
            b, h = sweep.paper_shape(n, d)
            assert b * n == 16384 and h * d == 2048
    # the two benchmark configurations that sit on the rule
    assert sweep.paper_shape(4096, 128) == (4, 16)     # cfg2
    assert sweep.paper_shape(16384, 128) == (1, 16)    # cfg4
    assert sweep.paper_shape(32768, 64) == (1, 32)     # B never drops below 1
    assert sweep.paper_shape(1000, 64, tokens=2000, hidden=512) == (2, 8)


def test_flop_rule():
    assert sweep.attention_flops(1, 16, 16384, 128, False) == 4 * 16 * 16384 ** 2 * 128
    assert sweep.attention_flops(1, 16, 16384, 128, True) == 2 * 16 * 16384 ** 2 * 128
    # two matmuls of 2*N*N*d each per head: Q K^T and P V
    b, h, n, d = 3, 5, 7, 64
    assert sweep.attention_flops(b, h, n, d, False) == b * h * 2 * (2 * n * n * d)
    # the cfg4 figure every roofline in this repository uses
    assert sweep.attention_flops(1, 16, 16384, 128, False) == pytest.approx(2.199023e12, rel=1e-6)


def test_gate_uses_the_library_bar_for_fa_rows():
    ref = torch.linspace(-2.0, 2.0, 512).reshape(1, 1, 8, 64)
    assert sweep.gate("fa opt", ref.clone(), ref) == "ok"
    # within 2e-3 + 1e-2 |ref| everywhere
    assert sweep.gate("fa opt", ref + 1.9e-3 + 0.009 * ref.abs(), ref) == "ok"
    # 3e-3 off where ref = 0: over the bar for fa rows, well within 2e-2 for the others
    bad = ref.clone()
    bad[0, 0, 4, 0] = 3e-3
    zero_ref = ref.clone()
    zero_ref[0, 0, 4, 0] = 0.0
    assert sweep.gate("fa opt", bad, zero_ref).startswith("mismatch")
    assert sweep.gate("sdpa flash", bad, zero_ref) == "ok"
    assert sweep.gate("naive fp16", ref + 0.03, ref).startswith("mismatch")
    nan = ref.clone()
    nan[0, 0, 0, 0] = float("nan")
    assert sweep.gate("sdpa flash", nan, ref) == "mismatch non-finite"


def test_reference_slice_is_the_last_head_in_fp32():
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(2, 3, 40, 64, generator=g).half() for _ in range(3))
    ref, sl = sweep.reference_slice(q, k, v, causal=True)
    assert ref.dtype == torch.float32 and ref.shape == (1, 1, 40, 64)
    assert q[sl].shape == (1, 1, 40, 64)
    # causal row 0 sees only key 0
    torch.testing.assert_close(ref[0, 0, 0], v[1, 2, 0].float())


def _rows():
    rows = []
    for impl, tf, status in (("fa opt", 1200.4, "ok"), ("sdpa flash", 700.6, "ok")):
        rows.append({"gpu": "MI355X", "impl": impl, "B": 1, "H": 16, "N": 16384, "d": 128,
                     "causal": 0, "ms": 1.8, "tflops": tf, "status": status})
    rows.append({"gpu": "MI355X", "impl": "fa opt", "B": 4, "H": 16, "N": 4096, "d": 128,
                 "causal": 1, "ms": float("nan"), "tflops": float("nan"),
                 "status": "mismatch 3.1e-03"})
    return rows


def test_markdown_table():
    md = sweep.markdown_table(_rows(), ["fa opt", "sdpa flash"])
    assert md.splitlines() == [
        "| d | causal | N | B×H | fa opt | sdpa flash |",
        "|---|---|---|---|---|---|",
        "| 128 | 0 | 16384 | 1×16 | 1200 | 701 |",
        "| 128 | 1 | 4096 | 4×16 | mismatch 3.1 |  |",
    ]


def test_csv_round_trip(tmp_path):
    path = tmp_path / "sub" / "sweep.csv"
    sweep.write_csv(_rows(), path)
    with path.open() as f:
        got = list(csv.DictReader(f))
    assert [r["impl"] for r in got] == ["fa opt", "sdpa flash", "fa opt"]
    assert float(got[0]["tflops"]) == 1200.4 and got[2]["status"] == "mismatch 3.1e-03"


@pytest.mark.gpu
def test_sweep_runs_and_fa_rows_pass_the_gate(tmp_path):
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    out_csv, out_md = tmp_path / "s.csv", tmp_path / "s.md"
    print("case sweep d=64,128 N=1024 causal 0,1", flush=True)
    res = subprocess.run(
        [sys.executable, "-m", "fa.sweep", "--n", "1024", "--d", "64", "128", "--causal", "0", "1",
         "--impls", "fa opt", "fa splitkv", "sdpa flash", "--budget-ms", "100",
         "--csv", str(out_csv), "--md", str(out_md)],
        cwd=str(PKG), capture_output=True, text=True, timeout=240)
    assert res.returncode == 0, res.stdout + res.stderr
    with out_csv.open() as f:
        rows = list(csv.DictReader(f))
    assert len(rows) == 12
    for r in rows:
        assert (int(r["B"]), int(r["H"])) == sweep.paper_shape(1024, int(r["d"]))
        if r["impl"].startswith("fa "):
            assert r["status"] == "ok" and float(r["tflops"]) > 0, r
    assert "| 128 | 1 | 1024 | 16×16 |" in out_md.read_text()


@pytest.mark.gpu
def test_sweep_explicit_shapes_with_the_single_launch(tmp_path):
    """--shapes runs the given BxHxN shapes; 'fa single' (the C-ABI launch without routing)
    passes the same gate as fa.forward."""
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    out_csv = tmp_path / "s.csv"
    print("case sweep shapes 1x17x4096 2x3x700 d=128 non-causal", flush=True)
    res = subprocess.run(
        [sys.executable, "-m", "fa.sweep", "--shapes", "1x17x4096", "2x3x700", "--d", "128",
         "--causal", "0", "--impls", "fa opt", "fa single", "--budget-ms", "100",
         "--csv", str(out_csv)],
        cwd=str(PKG), capture_output=True, text=True, timeout=240)
    assert res.returncode == 0, res.stdout + res.stderr
    with out_csv.open() as f:
        rows = list(csv.DictReader(f))
    assert sorted((int(r["B"]), int(r["H"]), int(r["N"]), r["impl"]) for r in rows) == [
        (1, 17, 4096, "fa opt"), (1, 17, 4096, "fa single"),
        (2, 3, 700, "fa opt"), (2, 3, 700, "fa single")]
    assert all(r["status"] == "ok" and float(r["tflops"]) > 0 for r in rows), rows
