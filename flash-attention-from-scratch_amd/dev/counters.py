"""Summarise a dev/counters.sh run (rocprofv3 CSV output) as a short markdown report.

    python3 dev/counters.py OUT --shape B H N D causal [--variant opt] [--command TEXT]

Averages every counter over the attention kernel's dispatches except the first (the driver's
checked launch, which runs on a cold cache and clock), and derives:
  * MFMA utilisation: SQ_VALU_MFMA_BUSY_CYCLES per SIMD over GRBM_GUI_ACTIVE per XCD;
  * matrix FLOPs from SQ_INSTS_MFMA (32768 FLOPs per v_mfma_f32_32x32x16_f16, 16384 per
    v_mfma_f32_16x16x32_f16 in flash_fwd_pingpong16 and flash_fwd_simple16) against the
    algorithmic 4*B*H*N^2*d (halved for causal): a ratio above 1 is wasted matrix work;
  * LDS bank-conflict rate, MFMA/VALU co-execution, waits on LDS;
  * HBM bytes = FETCH_SIZE * fetch_scale + WRITE_SIZE * write_scale (KiB), against the
    algorithmic 4*B*H*N*d*2 bytes (Q, K, V read once, O written once). The scales convert the
    counters to bytes as measured with a copy kernel of known size on MI355X (a 256 MiB copy
    reads 131085 KiB of FETCH_SIZE and writes 262144 KiB of WRITE_SIZE: 1.9998 and 1.0).
Machine constants default to MI355X: 256 CUs (1024 SIMDs) in 8 XCDs, 2516.6 TFLOPS dense fp16.
"""

from __future__ import annotations

import argparse
import csv
import statistics
import sys
from collections import defaultdict
from pathlib import Path

def flops_per_mfma(kernel_name: str) -> int:
    """flash_fwd_pingpong16 and flash_fwd_simple16 issue v_mfma_f32_16x16x32_f16; the other
    kernels v_mfma_f32_32x32x16_f16."""
    m16 = "pingpong16" in kernel_name or "simple16" in kernel_name
    return 2 * 16 * 16 * 32 if m16 else 2 * 32 * 32 * 16


def _counters(path: Path, kernel: str) -> dict[str, float]:
    per_dispatch: dict[int, dict[str, float]] = defaultdict(dict)
    for f in sorted(path.glob("**/*counter_collection.csv")):
        with f.open() as fh:
            for row in csv.DictReader(fh):
                if kernel in row["Kernel_Name"]:
                    d = per_dispatch[int(row["Dispatch_Id"])]
                    name = row["Counter_Name"]
                    d[name] = d.get(name, 0.0) + float(row["Counter_Value"])
    ids = sorted(per_dispatch)[1:] or sorted(per_dispatch)
    out: dict[str, float] = {}
    for name in {n for i in ids for n in per_dispatch[i]}:
        out[name] = statistics.fmean(per_dispatch[i][name] for i in ids if name in per_dispatch[i])
    return out


def _durations(path: Path, kernel: str) -> tuple[str, list[float]]:
    names, durs = set(), []
    for f in sorted(path.glob("**/*kernel_trace.csv")):
        with f.open() as fh:
            rows = [r for r in csv.DictReader(fh) if kernel in r["Kernel_Name"]]
        for r in rows[1:]:
            names.add(r["Kernel_Name"])
            durs.append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9)
    return ", ".join(sorted(names)), durs


def main(argv: list[str]) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("out", type=Path)
    ap.add_argument("--shape", type=int, nargs=5, required=True, metavar=("B", "H", "N", "D", "C"))
    ap.add_argument("--variant", default="opt")
    ap.add_argument("--command", default="")
    ap.add_argument("--kernel", default="flash_fwd")
    ap.add_argument("--simds", type=int, default=1024)
    ap.add_argument("--xcds", type=int, default=8)
    ap.add_argument("--peak-tflops", type=float, default=2516.6)
    ap.add_argument("--fetch-scale", type=float, default=1.9998)
    ap.add_argument("--write-scale", type=float, default=1.0)
    a = ap.parse_args(argv)
    b, h, n, d, causal = a.shape
    flops = 4.0 * b * h * n * n * d / (2 if causal else 1)
    alg_bytes = 4.0 * b * h * n * d * 2

    name, durs = _durations(a.out / "trace", a.kernel)
    c = {}
    for p in ("pmcA", "pmcB", "fetch", "write"):
        c.update(_counters(a.out / p, a.kernel))

    lines = [f"# {a.kernel} counters: B={b} H={h} N={n} d={d} causal={causal} variant={a.variant}",
             "", f"Command: `{a.command}` (then `dev/counters.py` on its output).", "",
             f"Kernel: `{name}`", "", "| Quantity | Value |", "|---|---|"]

    def row(k: str, v: str) -> None:
        lines.append(f"| {k} | {v} |")

    if durs:
        avg = statistics.fmean(durs)
        row("launches timed (kernel trace, first dropped)", str(len(durs)))
        row("average duration", f"{avg * 1e3:.4f} ms (min {min(durs) * 1e3:.4f})")
        row("TFLOPS (algorithmic / average)",
            f"{flops / avg / 1e12:.1f} ({100 * flops / avg / 1e12 / a.peak_tflops:.1f} % of peak)")
    fpm = flops_per_mfma(name)
    shape = "16x16x32" if fpm == 16384 else "32x32x16"
    if "SQ_INSTS_MFMA" in c:
        row("MFMA FLOPs / algorithmic FLOPs", f"{c['SQ_INSTS_MFMA'] * fpm / flops:.4f}")
    if "SQ_VALU_MFMA_BUSY_CYCLES" in c and "GRBM_GUI_ACTIVE" in c:
        busy = c["SQ_VALU_MFMA_BUSY_CYCLES"] / a.simds
        active = c["GRBM_GUI_ACTIVE"] / a.xcds
        row("MFMA busy per SIMD / GPU active cycles", f"{busy:,.0f} / {active:,.0f} = "
            f"{100 * busy / active:.1f} %")
    if "SQ_INSTS_VALU" in c and "SQ_INSTS_MFMA" in c:
        row(f"non-MFMA VALU instructions per MFMA ({shape})",
            f"{(c['SQ_INSTS_VALU'] - c['SQ_INSTS_MFMA']) / c['SQ_INSTS_MFMA']:.2f}")
    if "SQ_INSTS_VALU_TRANS_F32" in c and "SQ_INSTS_MFMA" in c:
        row(f"transcendental (v_exp_f32 ...) per MFMA ({shape})",
            f"{c['SQ_INSTS_VALU_TRANS_F32'] / c['SQ_INSTS_MFMA']:.2f}")
    if "SQ_LDS_BANK_CONFLICT" in c and "SQ_LDS_IDX_ACTIVE" in c and c["SQ_LDS_IDX_ACTIVE"]:
        row("LDS bank-conflict cycles / LDS active cycles",
            f"{c['SQ_LDS_BANK_CONFLICT']:,.0f} / {c['SQ_LDS_IDX_ACTIVE']:,.0f}")
    if "SQ_VALU_MFMA_COEXEC_CYCLES" in c and "SQ_VALU_MFMA_BUSY_CYCLES" in c:
        row("MFMA/VALU co-execution cycles / MFMA busy cycles",
            f"{100 * c['SQ_VALU_MFMA_COEXEC_CYCLES'] / c['SQ_VALU_MFMA_BUSY_CYCLES']:.1f} %")
    if "SQ_WAIT_INST_LDS" in c and "SQ_WAVE_CYCLES" in c:
        row("wave cycles waiting on LDS / wave cycles",
            f"{100 * c['SQ_WAIT_INST_LDS'] / c['SQ_WAVE_CYCLES']:.1f} %")
    if "SQ_WAIT_ANY" in c and "SQ_WAVE_CYCLES" in c:
        row("wave cycles waiting on anything / wave cycles",
            f"{100 * c['SQ_WAIT_ANY'] / c['SQ_WAVE_CYCLES']:.1f} %")
    if "FETCH_SIZE" in c and "WRITE_SIZE" in c:
        hbm = 1024 * (c["FETCH_SIZE"] * a.fetch_scale + c["WRITE_SIZE"] * a.write_scale)
        row("HBM bytes per launch (scaled FETCH_SIZE + WRITE_SIZE)",
            f"{hbm:,.0f} = {hbm / alg_bytes:.2f} x algorithmic {alg_bytes:,.0f}")
        if durs:
            row("HBM bandwidth (bytes / average duration)",
                f"{hbm / statistics.fmean(durs) / 1e9:,.0f} GB/s of 8000")
    lines += ["", "Raw per-dispatch averages:", "", "| Counter | Value |", "|---|---|"]
    lines += [f"| {k} | {v:,.0f} |" for k, v in sorted(c.items())]
    print("\n".join(lines))
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
