"""TEST INFRASTRUCTURE ONLY: a CPU model of the ping-pong kernels' softmax arithmetic, per row.

`flash_fwd_pingpong16` (csrc/flash_fwd.hip) takes P against a reference max per row and never
re-tests most tiles. This module restates the arithmetic each key tile of one query row goes
through, so that a CPU test can ask what that arithmetic loses on a given input:

* the item's first tile (exact): m = tile max + margin, p = fp16(exp2(s - m));
* unchecked tiles: p = fp16(exp2(s - m)) with no test, in steps of three after the first tile
  (non-causal: up to the steady tiles' end; causal: the leading tiles that no row of the 256-row
  block masks);
* checked tiles (the one or two steady tiles left over, the causal band): the same p, and if
  one overflows fp16 the tile is redone with the lazy rescale (raise m to the tile max only
  when it grew by more than 8, as in the reference's LAZY softmax,
  csrc/kernels/flash_fwd.cu:365-395);
* the last tile (general_tiles16): exact with the lazy rescale, margin 0;
* the row sum l is the sum of the fp16 p; an infinite l sends the row to the second pass, in
  which every steady tile is checked (the kernel may also leave the first pass early; that
  changes only its cost);
* an item whose first tile votes "wide" (`wide_rows`: some row's four lanes all see a score
  range above FA_PP16_SPREAD) runs every steady tile checked from the start
  (`checked_from_start`), as the second pass does;
* O = sum p v (fp16 p times fp16 v, accumulated in fp64 here) / l, rounded to fp16.

Rounding: fp16 conversion is numpy's round-to-nearest-even with subnormals, as the kernel's
v_cvt_pk_f16_f32; exp2 is numpy's, within an ulp of v_exp_f32. The model is not bitwise; it
reproduces which keys become subnormal or zero, which is what decides accuracy here. It
models the kernel, it is not the oracle: tests compare it with oracle/attention_fp64.c rows.
"""

from __future__ import annotations

import numpy as np

BR = 256  # query rows per ping-pong workgroup (8 waves of 32)


def _f16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float64)


def m16_key(kb: int, i: int) -> int:
    """Tile row of M index i of score block kb on the 16x16x32 path (fa::geom::m16_key,
    csrc/fa_geometry.h): two 16-key blocks per 32 keys, interleaved by 8 rows."""
    return 32 * (kb // 2) + 8 * (kb % 2) + (i % 8) + 16 * ((i // 8) % 2)


def wide_rows(s_first: np.ndarray, spread: float) -> np.ndarray:
    """The first tile's wide-spread vote of flash_fwd_pingpong16 (softmax16_wide), per row.

    s_first: [rows, >= 32] scores of the item's first key tile, times scale*log2(e). Lane group
    g (lanes 16 g .. 16 g + 15) holds keys m16_key(kb, 4 g + r), r = 0..3, of score block kb (the
    MFMA's C layout: row 4 (lane / 16) + r); the vote looks at blocks 0 and 1, the tile's first
    32 keys, and a row is wide if each group's range (max - min) exceeds `spread`."""
    s_first = np.asarray(s_first, np.float32)
    groups = [s_first[:, [m16_key(kb, 4 * g + r) for kb in (0, 1) for r in range(4)]]
              for g in range(4)]
    ranges = np.stack([x.max(axis=1) - x.min(axis=1) for x in groups], axis=1)
    return ranges.min(axis=1) > spread


def _tile_classes(n: int, r: int, bc: int, causal: bool, second_pass: bool) -> list[str]:
    """Per key tile of row r's item: 'exact' (first, with margin), 'unchecked', 'checked',
    'last' (general, lazy) or 'idle' (not computed by r's wave)."""
    q0 = BR * (r // BR)
    qw = q0 + 32 * ((r - q0) // 32)
    kv_end = min(n, q0 + BR) if causal else n
    n_tiles = -(-kv_end // bc)
    n_act = min((qw + 31) // bc + 1, n_tiles) if causal else n_tiles
    n_steady = max(0, n_tiles - 1)
    n_busy = min(n_steady, n_act) if causal else n_steady
    cls = ["idle"] * n_tiles
    if n_busy > 0:
        cls[0] = "exact"
        if second_pass:
            n_free = 0
        else:
            n_free = min(n_busy, max(0, min(q0 + 1, n)) // bc) if causal else n_busy
        jj = 1
        while jj + 3 <= n_free:
            cls[jj:jj + 3] = ["unchecked"] * 3
            jj += 3
        for t in range(jj, n_busy):
            cls[t] = "checked"
    if n_steady < n_act:
        cls[n_steady] = "last"
    return cls


def pp16_row(s: np.ndarray, v: np.ndarray, r: int, n: int, *, causal: bool, margin: float,
             bc: int = 32, checked_from_start: bool = False) -> tuple[np.ndarray, dict]:
    """Output row r (fp16 values as float64, [d]) of the ping-pong arithmetic.

    s: row r's scores times scale*log2(e) over all n keys (float32; the model masks keys > r
    when causal); v: [n, d] values (fp16 values); checked_from_start: the item's first tile voted
    wide (`wide_rows` over its rows). Returns (o, info) with info["l"] the row sum in units of
    the final reference max, info["m"] that max, info["second_pass"]."""
    s = np.asarray(s, np.float32).copy()
    if causal:
        s[r + 1:] = -np.inf
    v64 = np.asarray(v, np.float64)

    def run(m: float, second: bool):
        cls = _tile_classes(n, r, bc, causal, second)
        o = np.zeros(v64.shape[1])
        l = 0.0

        def exp_p(st, m_):
            with np.errstate(over="ignore"):
                return _f16(np.exp2((st - np.float32(m_)).astype(np.float32)))

        for t, c in enumerate(cls):
            if c == "idle":
                continue
            sl = slice(t * bc, min(n, (t + 1) * bc))
            st = s[sl]
            mx = float(st.max())
            grow = False
            if c == "exact":
                grow = m == -np.inf or mx > m + 8.0
                m_new = max(m, mx + margin) if grow else m
            elif c == "last":
                grow = mx > m + 8.0 if m != -np.inf else mx != -np.inf
                m_new = max(m, mx) if grow else m
            else:
                m_new = m
            if c == "checked" and not np.all(np.isfinite(exp_p(st, m))):
                if mx > m + 8.0:
                    grow, m_new = True, max(m, mx)
            if grow and m_new != m:
                a = 0.0 if m == -np.inf else 2.0 ** (m - m_new)
                o *= a
                l *= a
                m = m_new
            m_use = 0.0 if m == -np.inf else m
            p = exp_p(st, m_use)
            with np.errstate(invalid="ignore"):  # inf * 0 of an overflowing first pass
                l += float(p.sum())
                o += p @ v64[sl]
        return o, l, m

    o, l, m = run(-np.inf, checked_from_start)
    second = not np.isfinite(l)
    if second:
        o, l, m = run(-np.inf, True)
    out = _f16(o / l) if l > 0 else np.zeros_like(o)
    return out, {"l": l, "m": m, "second_pass": second}
