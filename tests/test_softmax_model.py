"""CPU: the ping-pong kernels' softmax arithmetic (tests/pp16_softmax_model.py) on inputs with an
attention sink, against the fp64 oracle rows, at the north-star tolerance.

An attention sink is one early key that every query weighs far above the rest (key 0 here,
+10..14 nats over scores ~N(0, 1)). The ping-pong takes p against its first key tile's max plus
FA_PP16_UNCHECKED_MARGIN and never re-tests the later tiles, so with a margin the sink lowers
every other key's p by 2^margin. With 8, the 16k-key tail falls into fp16's flush range and
its ~6 % of the row's weight vanishes from O and l alike, with no overflow to trigger a second
pass. The reference's lazy softmax (csrc/kernels/flash_fwd.cu:365-395) takes p against a key's
own score and cannot lose it. The test pins that a margin of 8 fails on this input (the model
and input catch the flaw) and that the margin the library is built with passes.
"""

from __future__ import annotations

import math
import re

import numpy as np
import pytest
import torch

from conftest import ATOL, RTOL
from oracle import attention as orc
from pp16_softmax_model import pp16_row, wide_rows

N = 16384
D = 128
ROWS = [0, 1, 31, 32, 255, 256, 300, 4095, 8191, 12000, N - 2, N - 1]


def sink_qkv(h: int, n: int, d: int, boost: float, seed: int):
    """q, k, v ~ N(0, 1) fp16, with a constant feature 0 in every query (q[..., 0] = 4) and key 0
    aligned with it, so that key 0's score is `boost` nats above a typical key's for every
    query (k[0, 0] = boost * sqrt(d) / 4 adds boost to q . k / sqrt(d))."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, h, n, d, generator=g)
    k = torch.randn(1, h, n, d, generator=g)
    v = torch.randn(1, h, n, d, generator=g)
    q[..., 0] = 4.0
    k[:, :, 0, 0] = boost * math.sqrt(d) / 4.0
    return q.half(), k.half(), v.half()


def built_margin() -> float:
    from fa import native

    m = re.search(r"pp16_margin=(\d+)", native.version())
    assert m, native.version()
    return float(m.group(1))


def built_spread() -> float:
    from fa import native

    m = re.search(r"pp16_spread=(\d+)", native.version())
    assert m, native.version()
    return float(m.group(1))


def _worst(q, k, v, causal: bool, margin: float, rows=ROWS,
           checked_from_start: bool = False) -> tuple[float, list[dict]]:
    """Largest |model - oracle| / (ATOL + RTOL |oracle|) over `rows` of head 0, and the infos."""
    n, d = q.shape[2], q.shape[3]
    c = np.float32(d ** -0.5 * math.log2(math.e))
    ref = orc.attention_fp64_rows(q, k, v, causal, 0, rows)
    q32, k32 = q[0, 0].float(), k[0, 0].float()
    s = (q32[rows] @ k32.t()).numpy() * c
    v32 = v[0, 0].float().numpy()
    worst, infos = 0.0, []
    for i, r in enumerate(rows):
        out, info = pp16_row(s[i], v32, r, n, causal=causal, margin=margin,
                             checked_from_start=checked_from_start)
        worst = max(worst, float((np.abs(out - ref[i]) / (ATOL + RTOL * np.abs(ref[i]))).max()))
        infos.append(info)
    return worst, infos


@pytest.mark.parametrize("boost", [12.0, 14.0])
def test_margin_8_loses_the_tail_behind_a_sink(boost):
    """The flaw a positive margin had: red at margin 8 (a planted mutant of the kernel's
    arithmetic, which the checks below must catch), with no second pass to repair it."""
    q, k, v = sink_qkv(1, N, D, boost, seed=int(boost))
    worst, infos = _worst(q, k, v, False, 8.0)
    assert worst > 1.5, worst
    assert not any(i["second_pass"] for i in infos)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("boost", [10.0, 12.0, 13.0, 14.0])
def test_built_margin_keeps_the_tail_behind_a_sink(boost, causal):
    q, k, v = sink_qkv(1, N, D, boost, seed=int(boost))
    margin = built_margin()
    worst, infos = _worst(q, k, v, causal, margin)
    assert worst <= 1.0, (margin, worst)
    if margin == 0.0:
        # the reference max is a key's score: the row sum holds that key's p = 1
        assert all(i["l"] >= 1.0 for i in infos)


@pytest.mark.parametrize("margin", [0.0, 8.0])
def test_model_matches_oracle_on_benchmark_inputs(margin):
    """q, k, v ~ N(0, 1) (the BASELINE configs' inputs): the model is within tolerance with
    either margin, so the sink test above isolates the flush, not a flaw of the model."""
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(1, 1, N, D, generator=g).half() for _ in range(3))
    for causal in (False, True):
        worst, infos = _worst(q, k, v, causal, margin)
        assert worst <= 0.5, (causal, worst)
        assert not any(i["second_pass"] for i in infos)


def test_model_second_pass_on_overflow():
    """A score rising ~40 exp2 units after the first tile overflows fp16 against the first
    tile's max: the row takes the second pass and still matches the oracle (the kernel's
    recompute, tests/test_flash_fwd.py::test_overflow_recompute on the GPU)."""
    g = torch.Generator().manual_seed(21)
    n = 2048
    q = torch.randn(1, 1, n, D, generator=g)
    k = torch.randn(1, 1, n, D, generator=g)
    k[:, :, :64] *= 0.1
    k[:, :, 64:] *= 8.0
    v = torch.randn(1, 1, n, D, generator=g)
    q, k, v = q.half(), k.half(), v.half()
    rows = [0, 100, 255, 256, 1000, n - 1]
    for causal in (False, True):
        worst, infos = _worst(q, k, v, causal, built_margin(), rows)
        assert worst <= 1.0, (causal, worst)
        assert any(i["second_pass"] for i in infos)


def _first_tiles(d: int, bc: int, std: float, seed: int, sink: float = 0.0,
                 outliers: int = 0, chunks: int = 64, rows: int = 1024) -> np.ndarray:
    """First key tiles' scores (times scale*log2(e)) of `chunks` items of `rows` query rows each:
    q, k ~ N(0, std^2) in fp16; `sink` nats added to key 0's score; `outliers` keys of each
    tile (at random positions) scaled x8."""
    g = torch.Generator().manual_seed(seed)
    c = d ** -0.5 * math.log2(math.e)
    out = []
    for _ in range(chunks):
        q = (torch.randn(rows, d, generator=g) * std).half().float()
        k = torch.randn(bc, d, generator=g) * std
        if outliers:
            k[torch.randperm(bc, generator=g)[:outliers]] *= 8.0
        s = q @ k.half().float().t() * c
        s[:, 0] += sink * math.log2(math.e)
        out.append(s.numpy())
    return np.concatenate(out)


@pytest.mark.parametrize("d, bc", [(128, 32), (64, 64)])
def test_spread_vote_separates_input_classes(d, bc):
    """The ping-pong's first-tile vote (softmax16_wide, restated by `wide_rows`) at the built
    threshold, on 2^16 query rows per class: q, k ~ N(0, 1) (the BASELINE configs' inputs), the
    same with an attention sink of 13 nats or with one or two keys x8 in the tile, leave every
    row unflagged, so those items keep the unchecked tiles; q, k ~ N(0, 1.6^2) flags over a
    tenth of the rows, so every 256-row item runs checked. Taking the largest lane range instead
    of the smallest would flag the sink and outlier rows; a threshold near the benchmark rows'
    largest range (about 7 exp2 units) would flag benchmark items. The layout (which lanes
    hold which keys) is pinned in tests/test_geometry.py."""
    spread = built_spread()
    assert spread > 0
    for name, kw in [("N(0,1)", {}), ("sink", {"sink": 13.0}), ("one outlier", {"outliers": 1}),
                     ("two outliers", {"outliers": 2})]:
        s = _first_tiles(d, bc, 1.0, seed=5, **kw)
        assert not wide_rows(s, spread).any(), name
        # margin below the threshold on the benchmark rows
        assert not wide_rows(s, spread - 1.0).any() or name != "N(0,1)", name
    wide = wide_rows(_first_tiles(d, bc, 1.6, seed=6), spread)
    assert wide.mean() > 0.1, wide.mean()
    assert wide.reshape(-1, 256).any(axis=1).all()


@pytest.mark.parametrize("causal", [False, True])
def test_wide_items_run_checked_from_the_start(causal):
    """q, k ~ N(0, 1.6^2) at 16k keys: rows of an item that voted wide run every steady tile
    checked (no second pass) and match the fp64 oracle at the north-star tolerance."""
    g = torch.Generator().manual_seed(8)
    q, k, v = (torch.randn(1, 1, N, D, generator=g) * sc for sc in (1.6, 1.6, 1.0))
    q, k, v = q.half(), k.half(), v.half()
    worst, infos = _worst(q, k, v, causal, built_margin(), checked_from_start=True)
    assert worst <= 1.0, worst
    assert not any(i["second_pass"] for i in infos)
