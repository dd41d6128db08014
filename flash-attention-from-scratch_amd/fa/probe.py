"""Power and clock measurements on MI355X (not part of the attention API).

    PYTHONPATH=flash-attention-from-scratch_amd python3 -m fa.probe [ceiling] [clock] [busy] [phase]
                                                                  [lds] [timeline]

ceiling: TFLOPS and measured clock of pure v_mfma_f32_32x32x16_f16 streams on random fp16
         operands (8 waves per CU), alone and with the per-tile VALU work and LDS fragment reads
         of attention added, and of a v_mfma_f32_16x16x32_f16 stream of the same FLOPs
         (fa/libfa_probe.so, csrc/fa_probe.hip).
clock:   the clock the attention kernels themselves run at, and their shader cycles per
         workgroup, on the benchmark shapes (fa/libfa_hip_clock.so: the library built with
         per-workgroup s_memtime / s_memrealtime recording).
busy:    the same for cfg4's non-causal kernel with 16, 8, 4, 2 and 1 heads: with fewer busy CUs
         the clock rises at unchanged cycles per workgroup when chip power is the limit.
phase:   the ping-pong kernel's steady state on cfg4, per wave group: shader cycles per tile spent
         issuing the softmax phase and the matrix phase, and waiting at each phase's end
         (s_memtime stamps at the phase-end waits of the clock-probe build).
timeline: for the cfg4 and cfg2 kernels, the fraction of the launch's span each CU spends
         inside a workgroup, each chiplet's finish time and clock, and the spread of workgroup
         durations (start stamps on the chip-wide 100 MHz counter, HW_ID / XCC_ID per workgroup).
Prints one JSON line per measurement. Build first: fa_build.py --only probe.
"""

from __future__ import annotations

import ctypes
import json
import math
import statistics
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
PEAK_TFLOPS = 2516.6


def _emit(rec: dict) -> None:
    print(json.dumps(rec), flush=True)


def ceiling(blocks: int = 1024, iters: int = 2000) -> None:
    so = ctypes.CDLL(str(HERE / "libfa_probe.so"))
    so.fa_probe_ceiling.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_int,
                                    ctypes.POINTER(ctypes.c_float),
                                    ctypes.POINTER(ctypes.c_double),
                                    ctypes.POINTER(ctypes.c_double)]
    for shape, valu, lds in ((s, v, l) for s in (0, 1) for v, l in ((0, 0), (1, 0), (0, 1), (1, 1))):
        ms, ghz, cyc = ctypes.c_float(), ctypes.c_double(), ctypes.c_double()
        rc = so.fa_probe_ceiling(valu, lds, shape, blocks, iters, ctypes.byref(ms),
                                 ctypes.byref(ghz), ctypes.byref(cyc))
        if rc != 0:
            raise RuntimeError(f"fa_probe_ceiling failed with HIP status {rc}")
        flops = blocks * 8 * iters * 16 * 32768.0
        tf = flops / (ms.value * 1e-3) / 1e12
        _emit({"probe": "mfma_ceiling",
               "mfma": "16x16x32" if shape else "32x32x16",
               "softmax_valu": bool(valu), "lds_fragments": bool(lds),
               "tflops": round(tf, 1), "frac_of_peak": round(tf / PEAK_TFLOPS, 4),
               "clock_ghz": round(ghz.value, 3),
               "cycles_per_iteration_per_workgroup": round(cyc.value / iters, 1)})


def lds(blocks: int = 256, iters: int = 4000) -> None:
    """LDS read throughput per CU for the two fragment-read instructions, alone."""
    so = ctypes.CDLL(str(HERE / "libfa_probe.so"))
    so.fa_probe_lds.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_double),
                                ctypes.POINTER(ctypes.c_double)]
    for mode, name, bytes_per_read in ((0, "ds_read_b128", 16), (1, "ds_read_b64_tr_b16", 8),
                                       (2, "ds_read_b128 (16x16x32 K)", 16),
                                       (3, "ds_read_b64_tr_b16 (16x16x32 V^T)", 8),
                                       (4, "ds_read_b64_tr_b16 (16x16x32 V^T, unswizzled)", 8),
                                       (5, "ds_read_b128 (16x16x32 K, split key blocks)", 16),
                                       (6, "ds_read_b64_tr_b16 (16x16x32 V^T, split key blocks)",
                                        8)):
        ms, ghz, cyc = ctypes.c_float(), ctypes.c_double(), ctypes.c_double()
        rc = so.fa_probe_lds(mode, blocks, iters, ctypes.byref(ms), ctypes.byref(ghz),
                             ctypes.byref(cyc))
        if rc != 0:
            raise RuntimeError(f"fa_probe_lds failed with HIP status {rc}")
        per_wg = 8 * 64 * 8 * bytes_per_read * iters  # waves x lanes x reads x bytes x rounds
        # 256 workgroups of 8 waves: about one per CU, so this is bytes per CU cycle
        _emit({"probe": "lds_read", "instruction": name,
               "bytes_per_cycle_per_workgroup": round(per_wg / cyc.value, 1),
               "clock_ghz": round(ghz.value, 3), "ms": round(ms.value, 3)})


def _clock_lib():
    from fa import native

    import os

    # FA_CLOCK_LIB: another clock-probe build of the library (e.g. with -D switches) to measure
    so = ctypes.CDLL(os.environ.get("FA_CLOCK_LIB", str(HERE / "libfa_hip_clock.so")))
    so.fa_flash_fwd.argtypes = [ctypes.POINTER(native.FaParams), ctypes.c_void_p]
    so.fa_flash_fwd.restype = ctypes.c_int
    so.fa_last_error.restype = ctypes.c_char_p
    so.fa_probe_clock_fetch.argtypes = [ctypes.POINTER(ctypes.c_ulonglong)]
    so.fa_probe_phase_fetch.argtypes = [ctypes.POINTER(ctypes.c_ulonglong)]
    return so


def _run_clock(so, q, k, v, causal: bool, reps: int = 20, full: bool = False):
    import numpy as np
    import torch

    from fa import native

    b, h, n, d = q.shape
    o = torch.empty_like(q)
    p = native.make_params(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), b, h, n, d,
                           1.0 / math.sqrt(d), causal, "opt")
    stream = torch.cuda.current_stream().cuda_stream
    for _ in range(reps):
        rc = so.fa_flash_fwd(ctypes.byref(p), ctypes.c_void_p(stream))
        if rc != 0:
            raise RuntimeError(so.fa_last_error().decode())
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        so.fa_flash_fwd(ctypes.byref(p), ctypes.c_void_p(stream))
        e1.record()
        e1.synchronize()
        times.append(e0.elapsed_time(e1))
    buf = (ctypes.c_ulonglong * (65536 * 4))()
    so.fa_probe_clock_fetch(buf)
    tile = native.tile_config(d, causal, "opt", n, b, h)
    n_wg = b * h * ((n + tile["block_q"] - 1) // tile["block_q"])
    raw = np.frombuffer(buf, dtype=np.uint64).reshape(65536, 4)[:n_wg]
    raw = raw[raw[:, 1] > 0]  # workgroups that recorded (e.g. not the empty split-KV ones)
    arr = raw[:, :2].astype(np.float64)
    ghz = arr[:, 0] / (arr[:, 1] * 10.0)
    if full:
        return statistics.median(times), raw
    return statistics.median(times), float(np.median(ghz)), float(np.median(arr[:, 0])), n_wg


def clock() -> None:
    import torch

    from fa.configs import CONFIGS, make_inputs

    so = _clock_lib()
    for name in ("cfg4", "cfg2", "cfg5"):
        cfg = CONFIGS[name]
        q, k, v = make_inputs(cfg)
        for causal in cfg.causal:
            ms, ghz, cyc, n_wg = _run_clock(so, q, k, v, causal)
            tf = cfg.flops(causal) / (ms * 1e-3) / 1e12
            _emit({"probe": "kernel_clock", "config": name, "causal": causal, "workgroups": n_wg,
                   "median_ms": round(ms, 4), "tflops": round(tf, 1),
                   "clock_ghz_median": round(ghz, 3),
                   "cycles_per_workgroup_median": round(cyc)})
        del q, k, v
        torch.cuda.empty_cache()


def busy() -> None:
    import torch

    so = _clock_lib()
    n, d = 16384, 128
    for heads in (16, 8, 4, 2, 1):
        g = torch.Generator().manual_seed(0)
        q, k, v = (torch.randn(1, heads, n, d, generator=g).half().cuda() for _ in range(3))
        ms, ghz, cyc, n_wg = _run_clock(so, q, k, v, False, reps=10)
        tf = 4.0 * heads * n * n * d / (ms * 1e-3) / 1e12
        _emit({"probe": "busy_cus", "heads": heads, "workgroups": n_wg, "median_ms": round(ms, 4),
               "tflops": round(tf, 1), "clock_ghz_median": round(ghz, 3),
               "cycles_per_workgroup_median": round(cyc)})


def phase() -> None:
    import numpy as np

    from fa.configs import CONFIGS, make_inputs

    so = _clock_lib()
    cfg = CONFIGS["cfg4"]
    q, k, v = make_inputs(cfg)
    for causal in (False, True):
        ms, ghz, _, n_wg = _run_clock(so, q, k, v, causal)
        buf = (ctypes.c_ulonglong * (8192 * 8 * 6))()
        so.fa_probe_phase_fetch(buf)
        a = np.frombuffer(buf, dtype=np.uint64).reshape(8192, 8, 6)[:n_wg].astype(np.float64)
        rec = {"probe": "pingpong_phases", "config": "cfg4", "causal": causal,
               "median_ms": round(ms, 4), "clock_ghz_median": round(ghz, 3),
               "tflops": round(cfg.flops(causal) / (ms * 1e-3) / 1e12, 1)}
        for grp in (0, 1):
            g = a[:, 4 * grp:4 * grp + 4]
            tiles = g[:, :, 4]
            for i, name in enumerate(("softmax_issue", "softmax_wait", "matrix_issue",
                                      "matrix_wait")):
                rec[f"group{grp}_{name}"] = round(float(np.mean(g[:, :, i][tiles > 0] /
                                                                tiles[tiles > 0])), 1)
        rec["mfma_cycles_per_tile_per_wave"] = 16 * 32
        _emit(rec)


def timeline() -> None:
    """Per-CU occupancy of the last launch: how much of the kernel's span each CU spent inside a
    workgroup, when each chiplet (XCC) finished, and the spread of workgroup durations."""
    import numpy as np
    import torch

    from fa.configs import CONFIGS, make_inputs

    so = _clock_lib()
    for name in ("cfg4", "cfg2"):
        cfg = CONFIGS[name]
        q, k, v = make_inputs(cfg)
        for causal in cfg.causal:
            ms, raw = _run_clock(so, q, k, v, causal, reps=10, full=True)
            ticks = raw[:, 1].astype(np.int64)
            start = raw[:, 2].astype(np.int64)
            start = start - start.min()
            end = start + ticks
            span = int(end.max())
            xcc = (raw[:, 3] >> np.uint64(32)).astype(np.int64) & 0xF
            hw = (raw[:, 3] & np.uint64(0xFFFFFFFF)).astype(np.int64)
            cu = xcc * 4096 + ((hw >> 8) & 0xFF)  # cu_id, sh_id, se_id (HW_ID bits 15:8)
            ghz = raw[:, 0].astype(np.float64) / (ticks * 10.0)
            busy_frac = []
            for c in np.unique(cu):
                sel = np.argsort(start[cu == c])
                s_c, e_c = start[cu == c][sel], end[cu == c][sel]
                covered, cur_s, cur_e = 0, s_c[0], e_c[0]
                for a, b in zip(s_c[1:], e_c[1:]):  # union of the CU's busy intervals
                    if a > cur_e:
                        covered += cur_e - cur_s
                        cur_s, cur_e = a, b
                    else:
                        cur_e = max(cur_e, b)
                covered += cur_e - cur_s
                busy_frac.append(covered / span)
            xcc_end = [round(float(end[xcc == x].max()) / 100.0, 1) for x in np.unique(xcc)]
            xcc_ghz = [round(float(np.median(ghz[xcc == x])), 3) for x in np.unique(xcc)]
            _emit({"probe": "timeline", "config": name, "causal": causal, "event_ms": round(ms, 4),
                   "span_us": round(span / 100.0, 1), "workgroups": int(len(raw)),
                   "cus": int(len(np.unique(cu))),
                   "cu_busy_frac_mean": round(float(np.mean(busy_frac)), 4),
                   "cu_busy_frac_min": round(float(np.min(busy_frac)), 4),
                   "wg_us_min_median_max": [round(float(x) / 100.0, 1) for x in
                                            (ticks.min(), np.median(ticks), ticks.max())],
                   "xcc_end_us": xcc_end, "xcc_clock_ghz": xcc_ghz})
        del q, k, v
        torch.cuda.empty_cache()


def main(argv: list[str]) -> int:
    what = argv or ["ceiling", "clock", "busy", "phase"]
    for w in what:
        {"ceiling": ceiling, "clock": clock, "busy": busy, "phase": phase, "lds": lds,
         "timeline": timeline}[w]()
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
