"""fa.forward against the attention implementations PyTorch-ROCm ships, on MI355X.

    PYTHONPATH=flash-attention-from-scratch_amd python3 -m fa.sweep [--n ...] [--d ...] \
        [--causal ...] [--csv PATH] [--md PATH]

Counterpart of the reference's bench/benchmark.py (same shapes, timing and FLOP count):
shapes follow the FlashAttention-2 paper, B*N = 16k tokens and H*d = 2048, so B = 16384 / N
and H = 2048 / d (bench/benchmark.py:5-9, 155-156); FLOPs = 4*B*H*N^2*d, halved for causal
(:142); each call timed with HIP events after a warmup (10 calls as in :108-111, then at
least 200 ms of calls), median of 20 to 200 calls within a 1.5 s budget (:112-120); every
implementation's output is checked against fa's baseline kernel on the same inputs first
(max |diff| < 2e-2, :128-132).

Implementations: fa "opt", "fp16acc" and "baseline", fa's split-KV forward; torch SDPA with the FLASH_ATTENTION and
EFFICIENT_ATTENTION backends (the fused kernels of PyTorch-ROCm); and the naive fp16 matmul /
softmax / matmul. The SDPA math backend is left out: its batched GEMMs take transposed views,
which this GPU pool has seen fault. Inputs come from a seeded CPU generator.
"""

from __future__ import annotations

import argparse
import csv
import math
import statistics
import sys
from pathlib import Path


def _impls():
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    import fa

    def ours(variant):
        return lambda q, k, v, causal: fa.forward_variant(q, k, v, causal=causal, variant=variant)

    def sdpa(backend):
        def run(q, k, v, causal):
            with sdpa_kernel(backend):
                return F.scaled_dot_product_attention(q, k, v, is_causal=causal)

        return run

    return {
        "fa opt": ours("opt"),
        "fa splitkv": lambda q, k, v, causal: fa.forward_splitkv(q, k, v, causal=causal)[0],
        "fa fp16acc": ours("fp16acc"),
        "fa baseline": ours("baseline"),
        "sdpa flash": sdpa(SDPBackend.FLASH_ATTENTION),
        "sdpa efficient": sdpa(SDPBackend.EFFICIENT_ATTENTION),
        "naive fp16": lambda q, k, v, causal: fa.attention_naive_fp16(q, k, v, causal),
    }


def time_ms(fn, warmup: int = 10, min_iters: int = 20, max_iters: int = 200,
            budget_ms: float = 1500.0, warm_ms: float = 200.0) -> float:
    """Median event time of fn(). The warmup runs at least `warmup` calls and at least
    `warm_ms` of GPU time, so that every implementation starts at a settled clock whatever
    ran before it (at N = 512 ten calls last about a millisecond)."""
    import time

    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < warm_ms:
        fn()
        torch.cuda.synchronize()
    times = []
    while len(times) < max_iters and (len(times) < min_iters or sum(times) < budget_ms):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b))
    return statistics.median(times)


def main(argv: list[str]) -> int:
    import torch

    import fa

    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--n", type=int, nargs="*", default=[512, 1024, 2048, 4096, 8192, 16384])
    ap.add_argument("--d", type=int, nargs="*", default=[64, 128])
    ap.add_argument("--causal", type=int, nargs="*", default=[0, 1])
    ap.add_argument("--tokens", type=int, default=16384, help="B * N")
    ap.add_argument("--hidden", type=int, default=2048, help="H * d")
    ap.add_argument("--bh", type=int, nargs=2, default=None, metavar=("B", "H"),
                    help="fixed batch and heads instead of the FA2-paper shapes")
    ap.add_argument("--impls", nargs="*", default=None, help="subset of implementations")
    ap.add_argument("--csv", type=Path, default=Path("gpurun_out/sweep.csv"))
    ap.add_argument("--md", type=Path, default=None, help="also write a markdown table")
    args = ap.parse_args(argv)

    impls = _impls()
    if args.impls:
        impls = {k: v for k, v in impls.items() if k in args.impls}
    gpu = torch.cuda.get_device_name(0)
    print(f"GPU: {gpu}  torch {torch.__version__}  HIP {torch.version.hip}", flush=True)
    rows = []
    for d in args.d:
        for causal in map(bool, args.causal):
            for n in args.n:
                b, h = args.bh if args.bh else (max(1, args.tokens // n), args.hidden // d)
                g = torch.Generator().manual_seed(0)
                q, k, v = (torch.randn(b, h, n, d, generator=g).half().cuda() for _ in range(3))
                ref = fa.forward_variant(q, k, v, causal=causal, variant="baseline")
                flops = 4.0 * b * h * n * n * d / (2 if causal else 1)
                line = [f"d={d:3d} causal={int(causal)} N={n:5d} B={b:2d} H={h:2d} |"]
                for name, fn in impls.items():
                    try:
                        out = fn(q, k, v, causal)
                        err = (out.float() - ref.float()).abs().max().item()
                        del out
                        if not err < 2e-2:
                            status, ms = f"mismatch {err:.1e}", math.nan
                        else:
                            status, ms = "ok", time_ms(lambda: fn(q, k, v, causal))
                    except torch.OutOfMemoryError:
                        status, ms = "OOM", math.nan
                    except RuntimeError as e:  # backend not available for this GPU or shape
                        status, ms = f"unsupported: {str(e).splitlines()[0][:60]}", math.nan
                    torch.cuda.empty_cache()
                    tf = flops / (ms * 1e-3) / 1e12 if status == "ok" else math.nan
                    rows.append({"gpu": gpu, "impl": name, "B": b, "H": h, "N": n, "d": d,
                                 "causal": int(causal), "ms": ms, "tflops": tf,
                                 "status": status})
                    line.append(f"{name}: {tf:6.1f}" if status == "ok" else f"{name}: {status[:10]}")
                del q, k, v, ref
                torch.cuda.empty_cache()
                print("  ".join(line), flush=True)
    args.csv.parent.mkdir(parents=True, exist_ok=True)
    with args.csv.open("w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    print(f"wrote {args.csv}", flush=True)
    if args.md:
        names = list(impls)
        lines = ["| d | causal | N | B×H | " + " | ".join(names) + " |",
                 "|---|---|---|---|" + "---|" * len(names)]
        keys = sorted({(r["d"], r["causal"], r["N"], r["B"], r["H"]) for r in rows})
        for d, c, n, b, h in keys:
            cells = []
            for name in names:
                r = next(x for x in rows if (x["d"], x["causal"], x["N"], x["impl"]) == (d, c, n, name))
                cells.append(f"{r['tflops']:.0f}" if r["status"] == "ok" else r["status"][:12])
            lines.append(f"| {d} | {c} | {n} | {b}×{h} | " + " | ".join(cells) + " |")
        args.md.parent.mkdir(parents=True, exist_ok=True)
        args.md.write_text("\n".join(lines) + "\n")
        print(f"wrote {args.md}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
