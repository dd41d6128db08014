#!/usr/bin/env python3
"""Benchmark of the FlashAttention-2 forward on one MI355X; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg4] [--no-cpu]

Workload (the headline roofline shape): cfg4, B=1 H=16 N=16384 d=128 fp16, q/k/v ~ N(0,1).
One step = one non-causal forward followed by one causal forward on the same resident inputs.
value = algorithmic TFLOPS of the step, 4*B*H*N^2*d per non-causal pass plus half that per
causal pass (bench/benchmark.py:142 of the reference), divided by the measured step time.

Timing: untimed steps for at least --ramp-ms (300 ms; the clock settles from idle over a few
hundred milliseconds under this load, longer than a short warmup), then W untimed warmup steps,
then exactly K steps between two synchronizations; every
launch is bracketed by HIP events recorded on the stream the kernel runs on (torch's current
stream, which fa.forward launches on), so per-kernel averages come from the same run.
roofline: the non-causal kernel (the larger share of the step) against the dense fp16 MFMA
peak of MI355X (2516.6 TFLOPS = 256 CU x 2.4 GHz x 4096 FLOP/clk); the causal kernel is
reported beside it. cpu_baseline: the fp32 oracle (oracle/attention.py, a restatement of the
reference's fa/reference.py) timed on this host's cores on whole (b, h) slices of the same
inputs, for a bounded time; it performs the full N^2 work even when causal.
other_configs: after the headline measurement (outside its timed region, not part of value),
the other compute-bound configurations (cfg2 in both modes, cfg5 with its boosted keys) timed
the same way, 30 launches per mode after --ramp-ms of untimed ones, with the tile each one
runs; skip with --no-others.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
PKG = REPO / "flash-attention-from-scratch_amd"
sys.path.insert(0, str(PKG))
sys.path.insert(0, str(REPO))

PEAK_TFLOPS = 2516.6  # MI355X dense fp16 MFMA: 256 CU * 2.4 GHz * 4096 FLOP/clk/CU
HBM_GBPS = 8000.0


def _ensure_built() -> None:
    have = (PKG / "fa" / "libfa_hip.so").exists() and any((PKG / "fa").glob("_C*.so"))
    if not have:
        import fa_build

        fa_build.build_lib()
        fa_build.build_ext()


def cpu_baseline(cfg, q, k, v, budget_s: float) -> dict:
    """Times the fp32 oracle on whole (b, h) slices, alternating non-causal and causal, until
    `budget_s` seconds of CPU work (at least one slice per mode)."""
    import torch

    from oracle.attention import attention_fp32

    qc, kc, vc = (t.detach().cpu() for t in (q, k, v))
    b, h, n, d = qc.shape
    flops = 0.0
    secs = 0.0
    slices = 0
    modes = list(cfg.causal)
    attention_fp32(qc[:1, :1, :256], kc[:1, :1, :256], vc[:1, :1, :256])  # warm up BLAS
    i = 0
    while i < b * h * len(modes) and (secs < budget_s or i < len(modes)):
        causal = modes[i % len(modes)]
        bh = (i // len(modes)) % (b * h)
        bi, hi = divmod(bh, h)
        sl = (slice(bi, bi + 1), slice(hi, hi + 1))
        t0 = time.perf_counter()
        attention_fp32(qc[sl], kc[sl], vc[sl], causal=causal)
        secs += time.perf_counter() - t0
        flops += 4.0 * n * n * d / (2 if causal else 1)
        slices += 1
        i += 1
    return {
        "value": flops / secs / 1e12,
        "unit": "TFLOPS",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{slices} whole (b,h) slices of {cfg.name} (N={n}, d={d}), alternating "
                   f"{'/'.join('causal' if c else 'non-causal' for c in modes)}, "
                   f"{secs:.1f} s; fp32 torch oracle on the host CPU; full N^2 work also for "
                   f"causal, TFLOPS by the same algorithmic formula"),
        "host_cpu_count": os.cpu_count(),
    }


def copy_calibration(nbytes: int, steps: int) -> int:
    """Copies nbytes device-to-device `steps` times (torch copy_ kernel): each launch reads and
    writes exactly nbytes, which calibrates the HBM byte counters of rocprofv3."""
    import torch

    src = torch.empty(nbytes // 2, dtype=torch.float16, device="cuda").normal_()
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "device copy", "bytes_read": nbytes,
                      "bytes_written": nbytes, "launches": steps}), flush=True)
    return 0


def traffic_from_profiles(cfg_name: str, causal: bool):
    """HBM bytes per launch measured with rocprofv3 PMC counters, if a summary was committed."""
    f = REPO / "profiles" / f"traffic_{cfg_name}.json"
    if not f.exists():
        return None
    try:
        data = json.loads(f.read_text())
        return data["causal" if causal else "non_causal"]["hbm_bytes_per_launch"]
    except (KeyError, ValueError):
        return None


def other_configs(headline: str, variant: str, ramp_ms: float, launches: int = 30) -> dict:
    """cfg2 and cfg5 (the other compute-bound configurations; cfg1 and cfg3 are launch-latency
    bound, and their Python dispatch would be timed with them): per mode, the mean launch time of
    `launches` back-to-back calls, from HIP events on the current stream, and the tile the
    launcher picks. Before each mode, untimed calls for at least `ramp_ms`: the GPU idles while
    the host draws a configuration's inputs, and its clock takes a few hundred milliseconds to
    settle again."""
    import torch

    import fa
    from fa import native
    from fa.configs import CONFIGS, make_inputs

    out = {}
    for name in ("cfg2", "cfg5"):
        if name == headline:
            continue
        c = CONFIGS[name]
        q, k, v = make_inputs(c)
        for causal in c.causal:
            ramp0 = time.perf_counter()
            while (time.perf_counter() - ramp0) * 1e3 < ramp_ms:
                for _ in range(4):
                    fa.forward_variant(q, k, v, causal=causal, variant=variant)
                torch.cuda.synchronize()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(launches):
                o = fa.forward_variant(q, k, v, causal=causal, variant=variant)
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / launches
            tf = c.flops(causal) / (ms * 1e-3) / 1e12
            t = native.tile_config(c.head_dim, causal, variant, c.seqlen, c.batch, c.heads)
            out[f"{name}_{'causal' if causal else 'non_causal'}"] = {
                "shape": f"B={c.batch} H={c.heads} N={c.seqlen} d={c.head_dim}",
                "launch_ms": round(ms, 4), "tflops": round(tf, 2),
                "frac_of_peak": round(tf / PEAK_TFLOPS, 4),
                "finite": bool(torch.isfinite(o).all()), "schedule": t["schedule"],
            }
        del q, k, v
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    # The GPU takes tens of milliseconds to ramp its clock from idle: warm up past that.
    ap.add_argument("--warmup", type=int, default=20)
    # ... and, before those W steps, untimed steps for at least this long (whatever W is): the
    # clock takes a few hundred milliseconds to settle from idle under this load.
    ap.add_argument("--ramp-ms", type=float, default=300.0)
    ap.add_argument("--config", default="cfg4")
    ap.add_argument("--variant", default="opt", choices=["baseline", "opt", "fp16acc"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-others", action="store_true",
                    help="skip the timing of the other compute-bound configurations")
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU baseline work")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="calibration only: time a plain device copy of this many bytes (the "
                         "reference workload for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the attention forward has no "
              "multi-GPU path; each GPU would run an independent [B', H', N, d] slice). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    _ensure_built()
    import torch

    import fa
    from fa import native
    from fa.configs import CONFIGS, make_inputs

    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1
    if args.copy_bytes:
        return copy_calibration(args.copy_bytes, args.steps)
    cfg = CONFIGS[args.config]
    modes = list(cfg.causal)
    q, k, v = make_inputs(cfg)
    torch.cuda.synchronize()

    def step(record=None):
        for m, causal in enumerate(modes):
            if record is not None:
                record[m][0].record()
            o = fa.forward_variant(q, k, v, causal=causal, variant=args.variant)
            if record is not None:
                record[m][1].record()
        return o

    # Output check and event creation come before the warmup: the first isfinite/all call
    # loads torch's kernels (about 0.2 s with the GPU idle), and an idle gap between warmup
    # and timing lets the clock fall back, so the first timed launches would run cold.
    out = step()
    if not torch.isfinite(out).all():
        print("bench.py: non-finite output", file=sys.stderr)
        return 1
    ev = [[[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in modes]
          for _ in range(args.steps)]
    t_start = torch.cuda.Event(enable_timing=True)
    t_stop = torch.cuda.Event(enable_timing=True)
    for e in [t_start, t_stop] + [x for s_ev in ev for m_ev in s_ev for x in m_ev]:
        e.record()  # first use of each event outside the timed region

    ramp_steps = 0
    ramp0 = time.perf_counter()
    while (time.perf_counter() - ramp0) * 1e3 < args.ramp_ms:
        for _ in range(4):
            out = step()
        ramp_steps += 4
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        out = step()
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_start.record()
    for s in range(args.steps):
        out = step(ev[s])
    t_stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0

    if not torch.isfinite(out).all():
        print("bench.py: non-finite output", file=sys.stderr)
        return 1

    total_ms = t_start.elapsed_time(t_stop)
    ms_per_step = total_ms / args.steps
    step_flops = sum(cfg.flops(c) for c in modes)
    value = step_flops / (ms_per_step * 1e-3) / 1e12

    per_mode = {}
    for m, causal in enumerate(modes):
        times = [ev[s][m][0].elapsed_time(ev[s][m][1]) for s in range(args.steps)]
        avg = statistics.mean(times)
        tf = cfg.flops(causal) / (avg * 1e-3) / 1e12
        per_mode["causal" if causal else "non_causal"] = {
            "avg_launch_ms": round(avg, 4),
            "median_launch_ms": round(statistics.median(times), 4),
            "tflops": round(tf, 2),
            "frac_of_peak": round(tf / PEAK_TFLOPS, 4),
        }

    def roof(causal):
        pm = per_mode["causal" if causal else "non_causal"]
        return {"bound": "mfma", "achieved": pm["tflops"], "peak": PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": pm["frac_of_peak"],
                "traffic": traffic_from_profiles(cfg.name, causal),
                "algorithmic_bytes": cfg.bytes(),
                "launch_ms": pm["avg_launch_ms"]}

    tile = {("causal" if c else "non_causal"): native.tile_config(
        cfg.head_dim, c, args.variant, cfg.seqlen, cfg.batch, cfg.heads) for c in modes}
    result = {
        "metric": "attention fwd TFLOPS (4BHN^2d, /2 causal) and % of MI355X fp16 MFMA peak",
        "value": round(value, 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": f"{cfg.name}: B={cfg.batch} H={cfg.heads} N={cfg.seqlen} d={cfg.head_dim} "
                        f"fp16 q/k/v~N(0,1); step = "
                        + " + ".join("causal" if c else "non-causal" for c in modes)
                        + " forward",
            "batch": cfg.batch, "heads": cfg.heads, "seqlen": cfg.seqlen,
            "head_dim": cfg.head_dim, "variant": args.variant, "tiles": tile,
        },
        "frac_of_peak": round(value / PEAK_TFLOPS, 4),
        "per_mode": per_mode,
        "roofline": roof(False) if False in modes else roof(True),
        "roofline_causal": roof(True) if True in modes and False in modes else None,
        "wall_s_timed": round(wall, 3),
        "untimed_ramp": {"ms": round(args.ramp_ms, 1), "steps": ramp_steps},
        "device": torch.cuda.get_device_name(0),
    }
    if not args.no_others:
        result["other_configs"] = other_configs(args.config, args.variant, args.ramp_ms)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(cfg, q, k, v, args.cpu_budget)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
