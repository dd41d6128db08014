"""Tile tuning sweep: build the kernel library with other tile tables, time each with fa_dev.

    # on the build machine (hipcc; no GPU needed):
    python3 flash-attention-from-scratch_amd/dev/tune.py build <slot> [cand ...] [-j 4]
    # on the GPU machine:
    python3 flash-attention-from-scratch_amd/dev/tune.py run <slot> [--n 512 1024 4096 16384]
            [--reps 3] [--csv PATH] [--bh B H] [--dev-args "--std 0.5 --boost-keys 0.01:8"]

slot: one row of the tile table in csrc/flash_fwd.hip, named after its macro (see SLOTS):
      opt_d64[_causal]_small, opt_d128[_causal]_small, opt_d64[_causal]_tiny,
      opt_d128[_causal]_tiny, opt_d64, opt_d64_causal_short, opt_d64_causal,
      opt_d128[_causal]_vshort, opt_d128[_causal]_short, opt_d128[_causal], base_d64, base_d128
cand: "BC,NW,LAZY,SCHED" -- keys per tile, query waves per workgroup (BR = 32 * NW), lazy
      rescale (true/false) and schedule (SIMPLE on 32x32x16 MFMAs; SIMPLE16, the same schedule
      on 16x16x32 MFMAs; KSPLIT / KSPLIT4, which run two / four waves per query wave; or
      PINGPONG16, the ping-pong on 16x16x32 MFMAs: 8 waves; the 16x16x32 schedules take BC=32
      at D=128 and BC=64 at D=64), e.g. 32,8,true,PINGPONG16. Without candidates a default list
      for the slot is used.

`build` compiles csrc/flash_fwd.hip once per candidate with the slot's macro overridden, into
dev/_tune/<slot>/<cand>.so (candidates the tile checks reject fail to compile and are reported
as such), with the size thresholds of the table pinned so that the slot's row runs at every N
and B*H. `run` times every built library with dev/fa_dev on the
FlashAttention-2 paper shapes (B = 16384 / N, H = 2048 / d; --bh fixes B and H instead),
which also checks a sample of output rows; --dev-args passes input options to fa_dev. Each
cell is the best of `reps` medians (TFLOPS), and the table is printed and written as CSV. A
candidate whose output check fails (fa_dev exit 1) is recorded as FAIL and the sweep goes on;
a child killed by a signal or exiting 2 (a HIP runtime error, e.g. a memory fault) stops the
whole sweep with a non-zero status, so no further kernel is launched after a possible GPU
fault. The library in fa/ is never touched: copy a winning candidate into the tile table by
hand.
Counterpart of the reference's bench/tune.sh:49-71 (which rewrites the `using` line of its
tile table, rebuilds fa_dev and runs it on the same shapes).
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import csv
import json
import shlex
import subprocess
import sys
from pathlib import Path

DEV = Path(__file__).resolve().parent
PKG = DEV.parent
TUNE = DEV / "_tune"

# slot -> (macro, variant, head_dim, causal, extra defines). The extra defines pin the
# library's size thresholds so that the slot's row runs at every N and B*H of the sweep.
_ALL, _NONE = "2147483647", "0"
_BIG = [f"-DFA_SMALL_GRID_WGS={_NONE}"]
_SMALL = [f"-DFA_SMALL_GRID_WGS={_ALL}", f"-DFA_TINY_GRID_WGS={_NONE}"]
_TINY = [f"-DFA_SMALL_GRID_WGS={_ALL}", f"-DFA_TINY_GRID_WGS={_ALL}",
         f"-DFA_TINY_MIN_TILES={_NONE}"]
SLOTS = {
    "opt_d64_small": ("FA_OPT_D64_SMALL", "opt", 64, 0, _SMALL),
    "opt_d64_causal_small": ("FA_OPT_D64_SMALL", "opt", 64, 1, _SMALL),
    "opt_d128_small": ("FA_OPT_D128_SMALL", "opt", 128, 0, _SMALL),
    "opt_d128_causal_small": ("FA_OPT_D128_SMALL", "opt", 128, 1, _SMALL),
    "opt_d64_tiny": ("FA_OPT_D64_TINY", "opt", 64, 0, _TINY),
    "opt_d64_causal_tiny": ("FA_OPT_D64_TINY", "opt", 64, 1, _TINY),
    "opt_d128_tiny": ("FA_OPT_D128_TINY", "opt", 128, 0, _TINY),
    "opt_d128_causal_tiny": ("FA_OPT_D128_TINY", "opt", 128, 1, _TINY),
    "opt_d64": ("FA_OPT_D64", "opt", 64, 0, [*_BIG, f"-DFA_D64_ONE_ROUND_MIN_N={_ALL}"]),
    "opt_d64_causal_short": ("FA_OPT_D64_CAUSAL_SHORT", "opt", 64, 1,
                             [*_BIG, f"-DFA_D64_CAUSAL_SHORT_MAX_N={_ALL}",
                              f"-DFA_D64_CAUSAL_ROUND_MAX_WGS={_NONE}"]),
    "opt_d64_causal": ("FA_OPT_D64_CAUSAL", "opt", 64, 1,
                       [*_BIG, f"-DFA_D64_CAUSAL_SHORT_MAX_N={_NONE}",
                        f"-DFA_D64_CAUSAL_ROUND_MAX_WGS={_NONE}"]),
    "opt_d64_causal_round": ("FA_OPT_D64_CAUSAL_ROUND", "opt", 64, 1,
                             [*_BIG, f"-DFA_D64_CAUSAL_ROUND_MIN_N={_NONE}",
                              f"-DFA_D64_CAUSAL_ROUND_MAX_WGS={_ALL}"]),
    "opt_d128_vshort": ("FA_OPT_D128_VSHORT", "opt", 128, 0,
                        [*_BIG, f"-DFA_D128_VSHORT_MAX_N={_ALL}"]),
    "opt_d128_short": ("FA_OPT_D128_SHORT", "opt", 128, 0,
                       [*_BIG, f"-DFA_D128_VSHORT_MAX_N={_NONE}",
                        f"-DFA_D128_SHORT_MAX_N={_ALL}"]),
    "opt_d128": ("FA_OPT_D128", "opt", 128, 0,
                 [*_BIG, f"-DFA_D128_VSHORT_MAX_N={_NONE}", f"-DFA_D128_SHORT_MAX_N={_NONE}"]),
    "opt_d128_causal_vshort": ("FA_OPT_D128_CAUSAL_VSHORT", "opt", 128, 1,
                               [*_BIG, f"-DFA_D128_CAUSAL_VSHORT_MAX_N={_ALL}"]),
    "opt_d128_causal_short": ("FA_OPT_D128_CAUSAL_SHORT", "opt", 128, 1,
                              [*_BIG, f"-DFA_D128_CAUSAL_VSHORT_MAX_N={_NONE}",
                               f"-DFA_D128_CAUSAL_SHORT_MAX_N={_ALL}"]),
    "opt_d128_causal": ("FA_OPT_D128_CAUSAL", "opt", 128, 1,
                        [*_BIG, f"-DFA_D128_CAUSAL_VSHORT_MAX_N={_NONE}",
                         f"-DFA_D128_CAUSAL_SHORT_MAX_N={_NONE}"]),
    "base_d64": ("FA_BASE_D64", "base", 64, 0, []),
    "base_d128": ("FA_BASE_D128", "base", 128, 0, []),
}
DEFAULT_CANDS = {
    64: ["64,8,true,PINGPONG16", "64,8,true,SIMPLE16", "64,4,true,SIMPLE16", "32,4,true,SIMPLE",
         "64,4,true,SIMPLE", "64,8,true,SIMPLE", "64,4,false,SIMPLE", "64,2,true,KSPLIT",
         "32,2,true,KSPLIT", "64,2,true,KSPLIT4"],
    128: ["32,8,true,PINGPONG16", "32,4,true,SIMPLE16", "32,8,true,SIMPLE16", "32,4,true,SIMPLE",
          "64,4,true,SIMPLE", "64,8,true,SIMPLE", "64,4,false,SIMPLE", "32,2,true,KSPLIT",
          "32,4,true,KSPLIT", "32,2,true,KSPLIT4"],
}


def _lib_path(slot: str, cand: str) -> Path:
    return TUNE / slot / (cand.replace(",", "_") + ".so")


def _build_one(slot: str, cand: str) -> tuple[str, str]:
    sys.path.insert(0, str(PKG))
    import fa_build

    macro, _, _, _, extra = SLOTS[slot]
    parts = cand.split(",")
    if len(parts) != 4:
        return cand, "bad candidate (want BC,NW,LAZY,SCHED)"
    out = _lib_path(slot, cand)
    out.parent.mkdir(parents=True, exist_ok=True)
    cmd = [fa_build._hipcc(), *fa_build.HIP_FLAGS, "-shared", f"-I{fa_build.INCLUDE}",
           f"-I{fa_build.CSRC}", f"-D{macro}={', '.join(parts)}", *extra,
           str(fa_build.CSRC / "flash_fwd.hip"), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        out.unlink(missing_ok=True)
        first = next((ln for ln in res.stderr.splitlines() if "error" in ln), "compile error")
        return cand, "build failed: " + first.strip()[:160]
    return cand, "ok"


def build(slot: str, cands: list[str], jobs: int) -> int:
    d = SLOTS[slot][2]
    cands = cands or DEFAULT_CANDS[d]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for cand, status in ex.map(lambda c: _build_one(slot, c), cands):
            print(f"{slot} {cand:22s} {status}", flush=True)
    return 0


def run(slot: str, ns: list[int], reps: int, csv_path: Path | None,
        bh: list[int] | None = None, dev_args: str = "") -> int:
    _, variant, d, causal, _ = SLOTS[slot]
    libs = sorted((TUNE / slot).glob("*.so"))
    if not libs:
        print(f"nothing built for {slot}: run `tune.py build {slot}` first", file=sys.stderr)
        return 2
    fa_dev = DEV / "fa_dev"
    print(f"{slot:22s}" + "".join(f" N={n:<7d}" for n in ns) + "  (TFLOPS, best of "
          f"{reps} medians)", flush=True)
    rows = []
    for lib in libs:
        cand = lib.stem.replace("_", ",")
        cells = []
        for n in ns:
            best = None
            for _ in range(reps):
                b, h = bh if bh else (max(1, 16384 // n), 2048 // d)
                args = [str(fa_dev), str(b), str(h), str(n), str(d), str(causal), "30", variant,
                        "--lib", str(lib), "--json", *shlex.split(dev_args)]
                res = subprocess.run(args, capture_output=True, text=True, timeout=300)
                if res.returncode < 0 or res.returncode == 2:
                    # killed by a signal (e.g. a memory-fault abort) or a HIP runtime error:
                    # the GPU may be in a bad state, launch nothing more
                    print(f"  {cand} N={n}: fa_dev ended with rc={res.returncode}; stopping the "
                          f"sweep\n{res.stderr.strip()[-2000:]}", file=sys.stderr, flush=True)
                    return 3
                line = res.stdout.strip().splitlines()[0] if res.stdout.strip() else ""
                if res.returncode != 0 or not line.startswith("{"):
                    best = "FAIL"
                    print(f"  {cand} N={n}: rc={res.returncode} {res.stdout.strip()} "
                          f"{res.stderr.strip()[:200]}", flush=True)
                    break
                rec = json.loads(line)
                best = rec["tflops"] if best is None else max(best, rec["tflops"])
            cells.append(best)
            rows.append({"slot": slot, "candidate": cand, "N": n, "d": d, "causal": causal,
                         "tflops": best})
        print(f"{cand:22s}" + "".join(f" {c if isinstance(c, str) else f'{c:.1f}':<9s}"
                                      for c in cells), flush=True)
    if csv_path:
        csv_path.parent.mkdir(parents=True, exist_ok=True)
        with csv_path.open("w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=list(rows[0]))
            w.writeheader()
            w.writerows(rows)
        print(f"wrote {csv_path}", flush=True)
    return 0


def main(argv: list[str]) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    b = sub.add_parser("build")
    b.add_argument("slot", choices=sorted(SLOTS))
    b.add_argument("cands", nargs="*")
    b.add_argument("-j", "--jobs", type=int, default=4)
    r = sub.add_parser("run")
    r.add_argument("slot", choices=sorted(SLOTS))
    r.add_argument("--n", type=int, nargs="+", default=[512, 1024, 4096, 16384])
    r.add_argument("--reps", type=int, default=3)
    r.add_argument("--csv", type=Path, default=None)
    r.add_argument("--bh", type=int, nargs=2, default=None, metavar=("B", "H"))
    r.add_argument("--dev-args", default="")
    a = ap.parse_args(argv)
    if a.cmd == "build":
        return build(a.slot, a.cands, a.jobs)
    return run(a.slot, a.n, a.reps, a.csv, a.bh, a.dev_args)


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
