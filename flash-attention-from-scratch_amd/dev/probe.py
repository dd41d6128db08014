"""Summary of a ping-pong timeline dump (dev/fa_dev --probe PATH, library built with FA_PROBE=1).

    python3 flash-attention-from-scratch_amd/dev/probe.py PATH [--json]

Per workgroup the dump holds 32 uint64 values: the 100 MHz constant clock (s_memrealtime) at
slot 0 (kernel entry) and, for item i of the workgroup (0, or 1 for the second item of a causal
pair), slots 1 + 5i .. 5 + 5i (its first pass starts, its prologue's loads have landed, its
steady tiles are done, its last tile is done, its O stores are issued); slot 12 when a second
pass starts; slots 11 and 13 the shader clock's cycle count (s_memtime) at the workgroup's
entry and end; the HW_ID (14) and XCC_ID (15) hardware registers; and slots 16 + 5i .. 20 + 5i
inside item i's phases (its prologue's loads are issued, they have landed before the barrier,
the first tile's S is computed, the first steady tile is done, the final test has passed its
barrier). Printed: medians over the workgroups of each phase of each item, of the steps inside
them (`detail`, when those stamps are present), and of the gap between a pair's items; the idle time
between one workgroup's last stamp and the next workgroup's entry on the same CU; when the
CUs and the XCDs finish, from the first workgroup's entry; and each XCD's median clock (cycles
over 100 MHz ticks from entry to the last O store). Only the stamps of wave 0 are
recorded, so the phases are that wave's view (the barriers make them the workgroup's).
"""

from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

import numpy as np

SLOTS = 32
TICKS_PER_US = 100.0  # s_memrealtime counts at 100 MHz
PHASES = ("prologue", "steady", "last_tile", "final_and_store")
# Steps inside an item, as (name, from slot, to slot) for item 0 (item 1: + 5 on every slot).
DETAIL = (("issue_loads", 1, 16), ("load_wait", 16, 17), ("barrier_wait", 17, 2),
          ("first_s", 2, 18), ("first_tile", 18, 19), ("steady_rest", 19, 3),
          ("last_tile", 3, 4), ("final_test", 4, 20), ("store_issue", 20, 5))


def load(path: Path) -> np.ndarray:
    """The stamps as an int64 array [workgroups, 32] (workgroups that stamped nothing dropped)."""
    raw = np.fromfile(path, dtype=np.uint64)
    if raw.size % SLOTS:
        raise ValueError(f"{path}: {raw.size} values, not a multiple of {SLOTS}")
    a = raw.reshape(-1, SLOTS).astype(np.int64)
    return a[a[:, 0] != 0]


def cu_key(hw_id: np.ndarray, xcc_id: np.ndarray) -> np.ndarray:
    """One integer per CU: XCC, shader engine, shader array and CU fields of HW_ID (gfx9 layout:
    cu_id bits 8-11, sh_id bit 12, se_id bits 13-15) and XCC_ID bits 0-3."""
    cu = (hw_id >> 8) & 0xF
    sh = (hw_id >> 12) & 0x1
    se = (hw_id >> 13) & 0x7
    return (((xcc_id & 0xF) * 8 + se) * 2 + sh) * 16 + cu


def summarize(a: np.ndarray) -> dict:
    if a.size == 0:
        raise ValueError("no workgroup stamped (a library built without FA_PROBE=1?)")
    t0 = a[:, 0].min()
    us = lambda x: (x - t0) / TICKS_PER_US  # noqa: E731
    pairs = bool((a[:, 6] != 0).any())
    n_items = 2 if pairs else 1
    out: dict = {"workgroups": int(a.shape[0]), "pairs": pairs, "items": {}}
    ends = np.zeros(a.shape[0], dtype=np.float64)
    for i in range(n_items):
        base = 1 + 5 * i
        have = a[:, base] != 0
        t = [us(a[have, base + k]) for k in range(5)]
        out["items"][i] = {name: float(np.median(t[k + 1] - t[k]))
                           for k, name in enumerate(PHASES)}
        full = have & np.all(a[:, [lo + 5 * i for _, lo, _ in DETAIL]
                               + [hi + 5 * i for _, _, hi in DETAIL]] != 0, axis=1)
        if full.any():
            out.setdefault("detail", {})[i] = {
                name: float(np.median(us(a[full, hi + 5 * i]) - us(a[full, lo + 5 * i])))
                for name, lo, hi in DETAIL}
        ends[have] = np.maximum(ends[have], t[4])
    out["entry_to_item"] = float(np.median(us(a[:, 1]) - us(a[:, 0])))
    if pairs:
        have = a[:, 6] != 0
        out["gap_between_items"] = float(np.median(us(a[have, 6]) - us(a[have, 5])))
    out["second_passes"] = int((a[:, 12] != 0).sum())
    key = cu_key(a[:, 14], a[:, 15])
    start = us(a[:, 0])
    gaps, cu_end = [], []
    for k in np.unique(key):
        idx = np.where(key == k)[0]
        order = idx[np.argsort(start[idx])]
        gaps.extend(start[order[1:]] - ends[order[:-1]])
        cu_end.append(ends[order].max())
    xcc = a[:, 15] & 0xF
    xcd_end = [float(ends[xcc == x].max()) for x in np.unique(xcc)]
    last = np.where(a[:, 10] != 0, a[:, 10], a[:, 5])
    have = (a[:, 11] != 0) & (a[:, 13] != 0) & (last > a[:, 0])
    if have.any():
        ns = (last - a[:, 0]) * (1000.0 / TICKS_PER_US)
        ghz = (a[:, 13] - a[:, 11]) / np.where(ns > 0, ns, 1.0)  # cycles per ns
        out["xcd_clock_ghz"] = [float(np.median(ghz[have & (xcc == x)]))
                                for x in np.unique(xcc)]
    out["cus"] = int(len(cu_end))
    out["gap_between_workgroups_on_a_cu"] = float(np.median(gaps)) if gaps else None
    out["cu_end"] = {"min": float(np.min(cu_end)), "median": float(np.median(cu_end)),
                     "max": float(np.max(cu_end))}
    out["xcd_end"] = xcd_end
    out["launch_us"] = float(ends.max())
    return out


def report(s: dict) -> str:
    lines = [f"{s['workgroups']} workgroups on {s['cus']} CUs, "
             f"{'causal pairs' if s['pairs'] else 'one item each'}; launch {s['launch_us']:.1f} us "
             f"(from the first entry to the last O store); second passes: {s['second_passes']}",
             f"entry to first item: {s['entry_to_item']:.2f} us"]
    for i, ph in s["items"].items():
        lines.append(f"item {i}: " + ", ".join(f"{k} {v:.2f} us" for k, v in ph.items()))
        if i in s.get("detail", {}):
            lines.append("  steps: " + ", ".join(f"{k} {v:.2f}" for k, v in
                                                  s["detail"][i].items()) + " us")
    if s["pairs"]:
        lines.append(f"between a pair's items: {s['gap_between_items']:.2f} us")
    if s["gap_between_workgroups_on_a_cu"] is not None:
        lines.append(f"idle between consecutive workgroups on a CU: "
                     f"{s['gap_between_workgroups_on_a_cu']:.2f} us")
    c = s["cu_end"]
    lines.append(f"CUs finish at {c['min']:.1f} / {c['median']:.1f} / {c['max']:.1f} us "
                 f"(min / median / max)")
    lines.append("XCDs finish at " + ", ".join(f"{x:.1f}" for x in s["xcd_end"]) + " us")
    if "xcd_clock_ghz" in s:
        lines.append("XCD clocks (median over their workgroups) "
                     + ", ".join(f"{x:.3f}" for x in s["xcd_clock_ghz"]) + " GHz")
    return "\n".join(lines)


def main(argv: list[str]) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("path", type=Path)
    ap.add_argument("--json", action="store_true")
    args = ap.parse_args(argv)
    s = summarize(load(args.path))
    print(json.dumps(s, indent=1) if args.json else report(s))
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
