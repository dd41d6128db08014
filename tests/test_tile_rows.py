"""GPU: every row of the tile table against the CPU oracle, and both sides of every switch.

The launcher picks a tile from (variant, head_dim, causal, N, B*H) (csrc/flash_fwd.hip, tile
table). Each case here first checks, through fa_tile_config, that its shape selects the row it
is meant to cover, then compares fa.forward with the fp32 oracle on a few (b, h) slices (the
first, the last and one in between) with the north-star tolerance. Sequence lengths are
ragged (not multiples of the tile) wherever a row allows it.
"""

from __future__ import annotations

import pytest
import torch

from conftest import ATOL, RTOL
from oracle import attention as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")


def _check(b, h, n, d, causal, want, seed=11):
    import fa
    from fa import native

    tile = native.tile_config(d, causal, "opt", n, b, h)
    got = (tile["block_q"], tile["block_k"], tile["waves"], tile["lds_bytes"], tile["schedule"])
    print(f"case B={b} H={h} N={n} d={d} causal={causal} tile={got}", flush=True)
    assert got == want, (got, want)
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(b, h, n, d, generator=g).half() for _ in range(3))
    out = fa.forward(q.cuda(), k.cuda(), v.cuda(), causal=causal).cpu()
    for bi, hi in {(0, 0), (b // 2, h // 2), (b - 1, h - 1)}:
        sl = (slice(bi, bi + 1), slice(hi, hi + 1))
        ref = orc.attention_fp32(q[sl], k[sl], v[sl], causal=causal)
        torch.testing.assert_close(out[sl].float(), ref, atol=ATOL, rtol=RTOL)


# (block_q, block_k, waves, lds_bytes, schedule)
PP128 = (256, 32, 8, 49152, "pingpong16")      # ping-pong, d=128
PP64 = (256, 64, 8, 49152, "pingpong16")       # ping-pong, d=64 (one round of 256 items)
SIMPLE64X8 = (256, 64, 8, 32768, "simple")     # 32x32x16 MFMAs
ROUND64 = (256, 128, 8, 65536, "simple")       # causal d=64 grids of at most 512 items
S16_64X8 = (256, 64, 8, 32768, "simple16")     # the simple schedule on 16x16x32 MFMAs
SIMPLE128X4 = (128, 32, 4, 32768, "simple")
S16_128X4 = (128, 32, 4, 32768, "simple16")
SMALL64 = (64, 64, 4, 65536, "ksplit")         # key split: 64 rows, 2 x 2 waves, BC=64
SMALL128 = (64, 32, 4, 65536, "ksplit")        # key split: 64 rows, 2 x 2 waves, BC=32
TINY64 = (64, 64, 8, 131072, "ksplit4")        # four-way key split: 64 rows, 4 x 2 waves, BC=64
TINY128 = (64, 32, 8, 131072, "ksplit4")       # four-way key split: 64 rows, 4 x 2 waves, BC=32

ROWS = [
    # (B, H, N, d, causal, expected tile)
    (1, 3, 900, 64, False, SMALL64),          # 15 key tiles: two-way split
    (2, 8, 900, 64, True, SMALL64),
    (1, 3, 1000, 64, False, TINY64),          # 48 query blocks of 64, 16 key tiles
    (2, 8, 1000, 64, True, TINY64),           # the benchmark's ragged config
    (1, 12, 1500, 128, False, SMALL128),      # 288 query blocks of 64: two-way split
    (1, 12, 1500, 128, True, SMALL128),
    (1, 2, 1500, 128, False, TINY128),
    (1, 2, 1500, 128, True, TINY128),
    (4, 16, 1000, 64, False, S16_64X8),
    (1, 32, 2500, 64, False, S16_64X8),
    (1, 8, 8000, 64, False, PP64),            # 256 items: one round of one workgroup per CU
    (1, 9, 8000, 64, False, S16_64X8),
    (4, 16, 1000, 64, True, SIMPLE64X8),
    (3, 32, 2500, 64, True, S16_64X8),
    (2, 8, 8500, 64, True, S16_64X8),
    (2, 16, 2000, 64, True, ROUND64),
    (16, 16, 250, 128, False, SIMPLE128X4),
    (8, 16, 700, 128, False, S16_128X4),
    (2, 16, 2500, 128, False, PP128),
    (16, 16, 500, 128, True, SIMPLE128X4),
    (4, 16, 1000, 128, True, S16_128X4),
    (1, 16, 4000, 128, True, PP128),
]


@pytest.mark.parametrize("b,h,n,d,causal,want", ROWS)
def test_row(b, h, n, d, causal, want):
    _check(b, h, n, d, causal, want)


SWITCHES = [
    (8, 32, 256, 128, False, SIMPLE128X4), (8, 32, 257, 128, False, S16_128X4),
    (4, 32, 1536, 128, False, S16_128X4), (4, 32, 1537, 128, False, PP128),
    (4, 32, 512, 128, True, SIMPLE128X4), (4, 32, 513, 128, True, S16_128X4),
    (1, 32, 3072, 128, True, S16_128X4), (1, 32, 3073, 128, True, PP128),
    # grids in head groups (256 heads or more) keep the 16x16x32 simple tile up to 4096 keys
    (8, 32, 4096, 128, True, S16_128X4), (8, 32, 4097, 128, True, PP128),
    (4, 16, 1535, 64, True, SIMPLE64X8), (4, 16, 1536, 64, True, ROUND64),
    (2, 16, 4096, 64, True, ROUND64), (2, 17, 4096, 64, True, S16_64X8),
    (8, 16, 2048, 64, True, SIMPLE64X8), (8, 16, 2049, 64, True, S16_64X8),
    # d=64 ping-pong for one round of 256 items from 4096 keys
    (1, 16, 4095, 64, False, S16_64X8), (1, 16, 4096, 64, False, PP64),
    (1, 17, 4096, 64, False, S16_64X8), (1, 4, 16384, 64, False, PP64),
    # small-grid boundary: B*H*ceil(N/256) = 255 and 256 workgroups of 8 waves
    (1, 17, 3840, 128, False, SMALL128), (1, 16, 4096, 128, False, PP128),
    (1, 17, 3840, 64, True, SMALL64), (1, 16, 4096, 64, True, ROUND64),
    # four-way split: at most 256 query blocks of 64 rows and at least 16 key tiles
    (1, 16, 1024, 64, False, TINY64), (1, 17, 1024, 64, False, SMALL64),
    (1, 16, 960, 64, True, SMALL64), (1, 16, 961, 64, True, TINY64),
    (1, 16, 1024, 128, True, TINY128), (1, 17, 1024, 128, True, SMALL128),
    (1, 16, 480, 128, False, SMALL128), (1, 16, 481, 128, False, TINY128),
]


@pytest.mark.parametrize("b,h,n,d,causal,want", SWITCHES)
def test_switch(b, h, n, d, causal, want):
    _check(b, h, n, d, causal, want, seed=12)


@pytest.mark.parametrize("n", [1, 17, 65, 257, 1000])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_edge_lengths_large_grid(n, d, causal):
    """The reference's edge lengths (tests/test_flash_fwd.py:27) on a grid large enough for the
    main rows (B*H = 256, so never the small-grid row)."""
    import fa
    from fa import native

    b, h = 16, 16
    tile = native.tile_config(d, causal, "opt", n, b, h)
    print(f"case B={b} H={h} N={n} d={d} causal={causal} tile={tile}", flush=True)
    assert tile["block_q"] in (128, 256)  # a main row, not the 64-row key split
    g = torch.Generator().manual_seed(n + d)
    q, k, v = (torch.randn(b, h, n, d, generator=g).half() for _ in range(3))
    out = fa.forward(q.cuda(), k.cuda(), v.cuda(), causal=causal).cpu()
    for bi, hi in {(0, 0), (7, 9), (15, 15)}:
        sl = (slice(bi, bi + 1), slice(hi, hi + 1))
        ref = orc.attention_fp32(q[sl], k[sl], v[sl], causal=causal)
        torch.testing.assert_close(out[sl].float(), ref, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("d,causal", [(64, False), (128, True)])
def test_more_heads_than_the_reference_grid_limit(d, causal):
    """B*H = 70000 > 65535, which the reference rejects (its grid.y is B*H,
    csrc/kernels/flash_fwd.cu:571-572, 629-631); the 1-D grid here takes it."""
    import fa

    b, h, n = 70000, 1, 16
    g = torch.Generator().manual_seed(70000 + d)
    q, k, v = (torch.randn(b, h, n, d, generator=g).half() for _ in range(3))
    out = fa.forward(q.cuda(), k.cuda(), v.cuda(), causal=causal).cpu()
    for bi in (0, 35000, b - 1):
        sl = (slice(bi, bi + 1), slice(0, 1))
        ref = orc.attention_fp32(q[sl], k[sl], v[sl], causal=causal)
        torch.testing.assert_close(out[sl].float(), ref, atol=ATOL, rtol=RTOL)


PP_SCALE_CASES = [(4, 16, 1700, False), (2, 16, 3300, True)]
# (B, H, N, d, causal, tile): the rows on 16x16x32 MFMAs
M16_SCALE_CASES = [(b, h, n, 128, c, PP128) for b, h, n, c in PP_SCALE_CASES] + [
    (4, 16, 1100, 64, False, S16_64X8), (3, 16, 3100, 64, True, S16_64X8),
    (8, 16, 700, 128, False, S16_128X4), (4, 16, 1500, 128, True, S16_128X4),
]


@pytest.mark.parametrize("b,h,n,d,causal,want", M16_SCALE_CASES)
@pytest.mark.parametrize("scale", [0.3, -0.2, 0.0, 1.5])
def test_m16_rows_scales_and_lse(b, h, n, d, causal, want, scale):
    """The rows on 16x16x32 MFMAs (the d=128 ping-pong, the simple schedule's SIMPLE16 rows)
    with custom, negative (Q negated), zero and large softmax scales, O and the row LSE,
    against the oracle."""
    import fa
    from fa import native

    tile = native.tile_config(d, causal, "opt", n, b, h)
    got = (tile["block_q"], tile["block_k"], tile["waves"], tile["lds_bytes"], tile["schedule"])
    print(f"case B={b} H={h} N={n} d={d} causal={causal} scale={scale} tile={got}", flush=True)
    assert got == want
    g = torch.Generator().manual_seed(int(1000 * scale) + n)
    q, k, v = (torch.randn(b, h, n, d, generator=g).half() for _ in range(3))
    out, lse = fa.forward_lse(q.cuda(), k.cuda(), v.cuda(), causal=causal, softmax_scale=scale)
    out, lse = out.cpu(), lse.cpu()
    for bi, hi in {(0, 0), (b - 1, h - 1)}:
        sl = (slice(bi, bi + 1), slice(hi, hi + 1))
        ref = orc.attention_fp32(q[sl], k[sl], v[sl], causal=causal, scale=scale)
        torch.testing.assert_close(out[sl].float(), ref, atol=ATOL, rtol=RTOL)
        ref_lse = orc.lse_fp32(q[sl], k[sl], causal=causal, scale=scale)
        torch.testing.assert_close(lse[sl], ref_lse, atol=2e-3, rtol=0)


# (B, H, N, d, causal): the simple schedule on 16x16x32 MFMAs, one shape per kind of its rows
S16_CASES = [(4, 16, 1100, 64, False), (4, 16, 2600, 64, True), (8, 16, 700, 128, False),
             (4, 16, 1500, 128, True)]


@pytest.mark.parametrize("b,h,n,d,causal", S16_CASES)
@pytest.mark.parametrize("kind", ["jump", "spread", "sink"])
def test_simple16_rescale_paths(b, h, n, d, causal, kind):
    """Inputs that take the 16x16x32 simple tile off its optimistic softmax: scores that jump by
    far more than 2^16 after 512 keys (the optimistic pass overflows, the tile is redone exactly
    and O rescaled), q, k ~ N(0, 1.9^2) (row maxima that keep rising, in every other head), and
    a key 0 about 13 nats above the rest (an attention sink: the first tile's max is the row's,
    and the rest of the row lies 17-20 exp2 units below it). Three (b, h) slices against the
    fp32 oracle."""
    import fa
    from fa import native

    tile = native.tile_config(d, causal, "opt", n, b, h)
    print(f"case s16 {kind} B={b} H={h} N={n} d={d} causal={causal} tile={tile}", flush=True)
    assert tile["schedule"] == "simple16"
    g = torch.Generator().manual_seed(n + d + len(kind))
    q, k, v = (torch.randn(b, h, n, d, generator=g) for _ in range(3))
    if kind == "jump":
        k[:, :, :512] *= 0.05
        k[:, :, 512:] *= 3.0
    elif kind == "spread":
        q[:, 0::2] *= 1.9
        k[:, 0::2] *= 1.9
    else:
        q[..., 0] = 4.0
        k[:, :, 0, 0] = 13.0 * d ** 0.5 / 4.0
    q, k, v = q.half(), k.half(), v.half()
    out = fa.forward(q.cuda(), k.cuda(), v.cuda(), causal=causal).cpu()
    assert torch.isfinite(out).all()
    for bi, hi in {(0, 0), (b // 2, h // 2), (b - 1, h - 1)}:
        sl = (slice(bi, bi + 1), slice(hi, hi + 1))
        ref = orc.attention_fp32(q[sl], k[sl], v[sl], causal=causal)
        torch.testing.assert_close(out[sl].float(), ref, atol=ATOL, rtol=RTOL)


# (B, H, N) causal d=128 grids of the simple schedules with 256 heads or more: the launcher runs
# them in groups of 64 heads (fa::geom::causal_group_heads). 3x100x1500: four full groups and a
# last one of 44 heads.
GROUP_CASES = [(16, 16, 1024, "simple16"), (32, 16, 512, "simple"), (3, 100, 1500, "simple16"),
               (2, 128, 2000, "simple16")]


@pytest.mark.parametrize("b,h,n,sched", GROUP_CASES)
def test_causal_head_groups(b, h, n, sched):
    """fa.forward and fa.forward_lse on grouped causal grids against the oracle, on heads at
    the edges of the groups (the first and last of the first two groups, the first of the last
    group, the last head)."""
    import fa
    from fa import native

    d = 128
    tile = native.tile_config(d, True, "opt", n, b, h)
    print(f"case groups B={b} H={h} N={n} tile={tile}", flush=True)
    assert tile["schedule"] == sched
    g = torch.Generator().manual_seed(n + h)
    q, k, v = (torch.randn(b, h, n, d, generator=g).half() for _ in range(3))
    out, lse = fa.forward_lse(q.cuda(), k.cuda(), v.cuda(), causal=True)
    out, lse = out.cpu(), lse.cpu()
    bh = b * h
    o1 = fa.forward(q.cuda(), k.cuda(), v.cuda(), causal=True).cpu()
    assert torch.equal(o1, out)
    for f in sorted({0, 63, 64, 127, (bh - 1) // 64 * 64, bh - 1}):
        bi, hi = divmod(f, h)
        sl = (slice(bi, bi + 1), slice(hi, hi + 1))
        ref = orc.attention_fp32(q[sl], k[sl], v[sl], causal=True)
        torch.testing.assert_close(out[sl].float(), ref, atol=ATOL, rtol=RTOL)
        torch.testing.assert_close(lse[sl], orc.lse_fp32(q[sl], k[sl], causal=True), atol=2e-3,
                                   rtol=0)
