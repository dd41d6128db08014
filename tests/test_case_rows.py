"""CPU: the GPU tests' shape lists reach the tile rows they are meant to cover.

fa_tile_config runs on the host, so the row each GPU case selects is checked here, before any
GPU run: every expected tile of the row and switch tests, the ping-pong cases, the large-grid
edge lengths, and full coverage of the opt rows by the NaN-prefilled-O shapes and the row
tests (each (head_dim, causal, tile) combination the table can pick).
"""

from __future__ import annotations

import pytest

from fa import native

import test_forward_routing as routing
import test_lse_splitkv as lse_cases
import test_tile_rows as rows


def _tile(b, h, n, d, causal, variant="opt"):
    t = native.tile_config(d, causal, variant, n, b, h)
    return t["block_q"], t["block_k"], t["waves"], t["lds_bytes"], t["schedule"]


# Every (head_dim, causal, tile) the opt table can pick: the key split for small grids, the
# simple schedule on 32x32x16 MFMAs (d=64 causal up to 2048 keys, d=128 up to 256 keys, causal
# 512; 128-key tiles for causal d=64 grids of at most 512 items) or on 16x16x32 MFMAs, and the ping-pong (d=128 long sequences, d=64 non-causal grids of
# one round).
OPT_ROWS = {
    (64, False, rows.SMALL64), (64, True, rows.SMALL64),
    (64, True, rows.SIMPLE64X8), (64, True, rows.ROUND64),
    (64, False, rows.S16_64X8), (64, True, rows.S16_64X8), (64, False, rows.PP64),
    (128, False, rows.SMALL128), (128, True, rows.SMALL128),
    (128, False, rows.SIMPLE128X4), (128, True, rows.SIMPLE128X4),
    (128, False, rows.S16_128X4), (128, True, rows.S16_128X4),
    (128, False, rows.PP128), (128, True, rows.PP128),
    (64, False, rows.TINY64), (64, True, rows.TINY64),
    (128, False, rows.TINY128), (128, True, rows.TINY128),
}


@pytest.mark.parametrize("b,h,n,d,causal,want", rows.ROWS + rows.SWITCHES)
def test_row_cases_select_their_tile(b, h, n, d, causal, want):
    assert _tile(b, h, n, d, causal) == want


def test_row_cases_cover_every_opt_row():
    assert {(d, c, w) for _, _, _, d, c, w in rows.ROWS} == OPT_ROWS


def test_simple16_cases_select_simple16():
    for b, h, n, d, causal in rows.S16_CASES:
        assert _tile(b, h, n, d, causal)[4] == "simple16"


def test_m16_scale_cases_select_their_rows():
    for b, h, n, d, causal, want in rows.M16_SCALE_CASES:
        assert _tile(b, h, n, d, causal) == want
        assert want[4] in ("pingpong16", "simple16")


@pytest.mark.parametrize("n", [1, 17, 65, 257, 1000])
def test_edge_lengths_stay_off_the_small_grid_row(n):
    for d in (64, 128):
        for causal in (False, True):
            assert _tile(16, 16, n, d, causal)[0] in (128, 256)


def test_tail_shapes_cover_every_opt_row():
    got = {(d, c, _tile(b, h, n, d, c)) for b, h, n, d, c, var in routing.TAIL_SHAPES
           if var == "opt"}
    assert got == OPT_ROWS


def test_lse_cases_cover_every_kind_of_tile():
    got = {_tile(b, h, n, d, c) for b, h, n, d, c in lse_cases.LSE_CASES}
    want = {w for _, _, w in OPT_ROWS}
    assert got == want
