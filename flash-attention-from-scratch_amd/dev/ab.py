"""A/B timing of kernel-library builds that differ in their FA_* build options, with fa_dev.

    # on the build machine (hipcc; no GPU needed):
    python3 flash-attention-from-scratch_amd/dev/ab.py build NAME [--define FA_X=V ...]
    # on the GPU machine:
    python3 flash-attention-from-scratch_amd/dev/ab.py run NAME [NAME ...]
            --shape "B H N D causal" [--shape ...] [--rounds 3] [--iters 30]
            [--input "--sink 13"] [--csv PATH]

`build` compiles csrc/flash_fwd.hip with the given macros into dev/_ab/NAME.so (NAME "default"
takes no defines; the library in fa/ is never touched). `run` times the named libraries with
dev/fa_dev, interleaved: every round runs every shape with every library in turn, so a clock
drift or a slow box weighs on all of them alike (on this pool one build's speed differs by up
to 8 % between boxes, more than most changes). Each cell is the median of the round medians,
printed with its change against the first library. `--input` passes fa_dev's input options
(--std, --boost-keys, --sink). fa_dev also checks sampled output rows against an fp64 row
formula: a library whose check fails is reported FAIL for that shape (its time is not used);
a child killed by a signal or exiting 2 (a HIP runtime error, e.g. a memory fault) stops the
run with a non-zero status, so no further kernel is launched after a possible GPU fault.
Counterpart of the reference's ablation runs (docs/fa3_fa4_techniques.md:43-50, which flip a
template flag and re-run the benchmark).
"""

from __future__ import annotations

import argparse
import csv
import json
import shlex
import statistics
import subprocess
import sys
from pathlib import Path

DEV = Path(__file__).resolve().parent
PKG = DEV.parent
OUT = DEV / "_ab"
FA_DEV = DEV / "fa_dev"


def lib_path(name: str) -> Path:
    return OUT / f"{name}.so"


def build(name: str, defines: list[str]) -> Path:
    sys.path.insert(0, str(PKG))
    import fa_build

    for d in defines:
        if not d.split("=", 1)[0].startswith("FA_"):
            raise SystemExit(f"--define takes the library's FA_* options, got {d}")
    OUT.mkdir(exist_ok=True)
    out = lib_path(name)
    cmd = [fa_build._hipcc(), *fa_build.HIP_FLAGS, "-shared", f"-I{fa_build.INCLUDE}",
           f"-I{fa_build.CSRC}", "-Rpass-analysis=kernel-resource-usage",
           *(f"-D{d}" for d in defines), str(fa_build.CSRC / "flash_fwd.hip"), "-o", str(out)]
    print("+", " ".join(shlex.quote(c) for c in cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        err = "\n".join(ln for ln in res.stderr.splitlines() if "remark:" not in ln)
        raise SystemExit(f"build failed ({res.returncode})\n{err}")
    spills = {k: v["scratch"] for k, v in fa_build._kernel_resources(res.stderr).items()
              if v.get("scratch", 0)}
    if spills:
        print(f"warning: kernels with scratch (register spills): {spills}", flush=True)
    print(f"built {out}", flush=True)
    return out


def run(names: list[str], shapes: list[str], rounds: int, iters: int, inputs: str,
        csv_path: str | None) -> int:
    libs = [lib_path(n) for n in names]
    for lib in libs:
        if not lib.exists():
            raise SystemExit(f"{lib} is not built (dev/ab.py build {lib.stem})")
    times: dict[tuple[str, str], list[float]] = {}
    failed: set[tuple[str, str]] = set()
    for r in range(rounds):
        for shape in shapes:
            for name, lib in zip(names, libs):
                cmd = [str(FA_DEV), *shape.split(), str(iters), "opt", "--lib", str(lib),
                       "--json", "--warmup-ms", "300", *shlex.split(inputs)]
                p = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
                if p.returncode < 0 or p.returncode == 2:
                    print(f"stop: {name} {shape} exited {p.returncode}\n{p.stderr[-2000:]}",
                          flush=True)
                    return 3
                rec = json.loads(p.stdout.strip().splitlines()[0])
                if p.returncode != 0:
                    failed.add((shape, name))
                    print(f"round {r} {shape:22s} {name:16s}     FAIL (max |err| "
                          f"{rec.get('max_abs_err')})", flush=True)
                    continue
                times.setdefault((shape, name), []).append(rec["tflops"])
                print(f"round {r} {shape:22s} {name:16s} {rec['tflops']:8.1f}", flush=True)
    rows = []
    print("== median of round medians, TFLOPS (change against the first library)")
    for shape in shapes:
        base = None
        for name in names:
            v = times.get((shape, name))
            if not v:
                print(f"{shape:22s} {name:16s}     FAIL", flush=True)
                rows.append([shape, name, "FAIL", ""])
                continue
            m = statistics.median(v)
            base = base or m
            print(f"{shape:22s} {name:16s} {m:8.1f} {100 * (m / base - 1):+6.1f} %  "
                  f"rounds={[round(x) for x in v]}", flush=True)
            rows.append([shape, name, f"{m:.1f}", f"{100 * (m / base - 1):+.1f}"])
    if csv_path:
        with open(csv_path, "w", newline="") as f:
            w = csv.writer(f)
            w.writerow(["shape", "library", "tflops", "change_pct"])
            w.writerows(rows)
    return 1 if failed else 0


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    b = sub.add_parser("build")
    b.add_argument("name")
    b.add_argument("--define", action="append", default=[], metavar="FA_NAME=VALUE")
    r = sub.add_parser("run")
    r.add_argument("names", nargs="+")
    r.add_argument("--shape", action="append", required=True, help='"B H N D causal"')
    r.add_argument("--rounds", type=int, default=3)
    r.add_argument("--iters", type=int, default=30)
    r.add_argument("--input", default="", help="fa_dev input options, e.g. '--sink 13'")
    r.add_argument("--csv")
    a = ap.parse_args()
    if a.cmd == "build":
        build(a.name, a.define)
    else:
        sys.exit(run(a.names, a.shape, a.rounds, a.iters, a.input, a.csv))


if __name__ == "__main__":
    main()
