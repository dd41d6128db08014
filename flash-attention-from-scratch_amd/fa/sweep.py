"""fa.forward against the attention implementations PyTorch-ROCm ships, on MI355X.

    PYTHONPATH=flash-attention-from-scratch_amd python3 -m fa.sweep [--n ...] [--d ...] \
        [--causal ...] [--csv PATH] [--md PATH]

Counterpart of the reference's bench/benchmark.py (same shapes, timing and FLOP count):
shapes follow the FlashAttention-2 paper, B*N = 16k tokens and H*d = 2048, so B = 16384 / N
and H = 2048 / d (bench/benchmark.py:5-9, 155-156, 165); FLOPs = 4*B*H*N^2*d, halved for
causal (:142); each call timed with HIP events after a warmup (10 calls as in :108-111, then
at least 200 ms of calls), median of 20 to 200 calls within a 1.5 s budget (:112-120).

Correctness gate before timing (the reference gates every implementation against its own
baseline kernel at max |diff| < 2e-2, :128-133, 172): here every implementation's output is
compared on one (b, h) slice, the last, with fa.attention_reference evaluated in fp32 on the
CPU (an fp32 restatement of the reference's fa/reference.py, independent of every HIP kernel
of this package). fa's own rows must meet the library's bar |out - ref| <= 2e-3 + 1e-2 |ref|;
the other implementations keep the reference benchmark's max |diff| < 2e-2.

Implementations: fa "opt", "fp16acc" and "baseline", fa's split-KV forward; torch SDPA with
the FLASH_ATTENTION and EFFICIENT_ATTENTION backends (the fused kernels of PyTorch-ROCm); and
the naive fp16 matmul / softmax / matmul. The SDPA math backend is left out: its batched GEMMs
take transposed views, which this GPU pool has seen fault. Inputs come from a seeded CPU
generator.
"""

from __future__ import annotations

import argparse
import csv
import math
import statistics
import sys
from pathlib import Path

# The library's accuracy bar (elementwise |out - ref| <= ATOL + RTOL |ref|) and the reference
# benchmark's cross-check bound for other implementations (bench/benchmark.py:131).
FA_ATOL, FA_RTOL = 2e-3, 1e-2
OTHER_MAX_ABS = 2e-2


def paper_shape(n: int, d: int, tokens: int = 16384, hidden: int = 2048) -> tuple[int, int]:
    """(B, H) of the FlashAttention-2 paper sweep: B * N = tokens, H * d = hidden
    (bench/benchmark.py:165: batch = 16384 // seqlen, nheads = 2048 // headdim)."""
    return max(1, tokens // n), hidden // d


def attention_flops(b: int, h: int, n: int, d: int, causal: bool) -> float:
    """4 * B * H * N^2 * d (two matmuls of 2 * N^2 * d per head), halved when causal
    (bench/benchmark.py:142)."""
    f = 4.0 * b * h * n * n * d
    return f / 2 if causal else f


def gate(impl: str, out_slice, ref_slice) -> str:
    """'ok' or 'mismatch <err>' for one implementation's output slice against the fp32
    reference slice (both CPU tensors of the same shape)."""
    out = out_slice.float()
    ref = ref_slice.float()
    if not bool(out.isfinite().all()):
        return "mismatch non-finite"
    diff = (out - ref).abs()
    if impl.startswith("fa "):
        excess = (diff - (FA_ATOL + FA_RTOL * ref.abs())).max().item()
        return "ok" if excess <= 0.0 else f"mismatch {diff.max().item():.1e}"
    err = diff.max().item()
    return "ok" if err < OTHER_MAX_ABS else f"mismatch {err:.1e}"


def reference_slice(q, k, v, causal: bool):
    """fa.attention_reference (fp32) of the last (b, h) slice, computed on the CPU."""
    from fa.reference import attention_reference

    sl = (slice(q.shape[0] - 1, q.shape[0]), slice(q.shape[1] - 1, q.shape[1]))
    return attention_reference(q[sl].cpu(), k[sl].cpu(), v[sl].cpu(), causal=causal), sl


def write_csv(rows: list[dict], path: Path) -> None:
    path.parent.mkdir(parents=True, exist_ok=True)
    with path.open("w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)


def markdown_table(rows: list[dict], names: list[str]) -> str:
    """One line per (d, causal, N) shape, one column of TFLOPS (or status) per implementation."""
    lines = ["| d | causal | N | B×H | " + " | ".join(names) + " |",
             "|---|---|---|---|" + "---|" * len(names)]
    keys = sorted({(r["d"], r["causal"], r["N"], r["B"], r["H"]) for r in rows})
    for d, c, n, b, h in keys:
        cells = []
        for name in names:
            r = next((x for x in rows
                      if (x["d"], x["causal"], x["N"], x["B"], x["H"], x["impl"]) ==
                      (d, c, n, b, h, name)), None)
            if r is None:
                cells.append("")
            else:
                cells.append(f"{r['tflops']:.0f}" if r["status"] == "ok" else r["status"][:12])
        lines.append(f"| {d} | {c} | {n} | {b}×{h} | " + " | ".join(cells) + " |")
    return "\n".join(lines) + "\n"


def _impls():
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    import fa

    def ours(variant):
        return lambda q, k, v, causal: fa.forward_variant(q, k, v, causal=causal, variant=variant)

    def single(q, k, v, causal):
        # one fa_flash_fwd launch through the C ABI, without the binding's split-KV routing
        # and head split
        from fa import native

        o = torch.empty_like(q)
        b, h, n, d = q.shape
        p = native.make_params(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), b, h, n, d,
                               d ** -0.5, causal, "opt")
        rc, msg = native.flash_fwd(p, torch.cuda.current_stream().cuda_stream)
        if rc != native.FA_OK:
            raise RuntimeError(msg)
        return o

    def sdpa(backend):
        def run(q, k, v, causal):
            with sdpa_kernel(backend):
                return F.scaled_dot_product_attention(q, k, v, is_causal=causal)

        return run

    return {
        "fa opt": ours("opt"),
        "fa single": single,
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

    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--n", type=int, nargs="*", default=[512, 1024, 2048, 4096, 8192, 16384])
    ap.add_argument("--d", type=int, nargs="*", default=[64, 128])
    ap.add_argument("--causal", type=int, nargs="*", default=[0, 1])
    ap.add_argument("--tokens", type=int, default=16384, help="B * N")
    ap.add_argument("--hidden", type=int, default=2048, help="H * d")
    ap.add_argument("--bh", type=int, nargs=2, default=None, metavar=("B", "H"),
                    help="fixed batch and heads instead of the FA2-paper shapes")
    ap.add_argument("--shapes", nargs="*", default=None, metavar="BxHxN",
                    help="explicit shapes (with --d and --causal) instead of --n")
    ap.add_argument("--impls", nargs="*", default=None, help="subset of implementations")
    ap.add_argument("--csv", type=Path, default=Path("out/sweep.csv"))
    ap.add_argument("--md", type=Path, default=None, help="also write a markdown table")
    ap.add_argument("--budget-ms", type=float, default=1500.0, help="timing budget per cell")
    args = ap.parse_args(argv)

    impls = _impls()
    if args.impls:
        impls = {k: v for k, v in impls.items() if k in args.impls}
    gpu = torch.cuda.get_device_name(0)
    print(f"GPU: {gpu}  torch {torch.__version__}  HIP {torch.version.hip}", flush=True)
    rows = []
    for d in args.d:
        for causal in map(bool, args.causal):
            shapes = ([tuple(int(x) for x in s.split("x")) for s in args.shapes] if args.shapes
                      else [(*(tuple(args.bh) if args.bh else
                               paper_shape(n, d, args.tokens, args.hidden)), n) for n in args.n])
            for b, h, n in shapes:
                g = torch.Generator().manual_seed(0)
                q, k, v = (torch.randn(b, h, n, d, generator=g).half().cuda() for _ in range(3))
                ref, sl = reference_slice(q, k, v, causal)
                flops = attention_flops(b, h, n, d, causal)
                line = [f"d={d:3d} causal={int(causal)} N={n:5d} B={b:2d} H={h:2d} |"]
                for name, fn in impls.items():
                    try:
                        out = fn(q, k, v, causal)
                        status = gate(name, out[sl].cpu(), ref)
                        del out
                        ms = (time_ms(lambda: fn(q, k, v, causal), budget_ms=args.budget_ms)
                              if status == "ok" else math.nan)
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
    write_csv(rows, args.csv)
    print(f"wrote {args.csv}", flush=True)
    if args.md:
        args.md.parent.mkdir(parents=True, exist_ok=True)
        args.md.write_text(markdown_table(rows, list(impls)))
        print(f"wrote {args.md}", flush=True)
    bad = [r for r in rows if r["impl"].startswith("fa ") and r["status"] != "ok"]
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
