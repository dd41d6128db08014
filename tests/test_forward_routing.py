"""GPU: how fa.forward serves grids too small to fill the GPU, and which rows it writes.

* Routing. For few-head long-sequence shapes the library's split-KV plan reports
  `preferred` (csrc/flash_fwd.hip, splitkv_preferred), and the binding's forward and
  forward_lse then run the split-KV pair instead of the single launch (the reference lists a
  scheduler for such grids as open work: docs/fa3_fa4_techniques.md:29-30). Each routed shape
  is checked three ways: fa.forward is bitwise fa.forward_splitkv (the same plan), forward_lse's
  O is bitwise forward's, and every (b, h) slice matches the fp32 oracle. Each shape on the
  other side of a routing boundary must be bitwise the single launch fa_flash_fwd.
* Output coverage. O is pre-filled with NaN (and a sentinel guard follows it) before a call
  of each C entry point on ragged shapes of every tile row: afterwards every element of O
  must be finite and within tolerance of the oracle (so every row < N and every feature was
  written), and the guard must be untouched (nothing written past O).
* Degenerate shapes at the binding: N = 0 returns an empty output without a launch
  (csrc/bindings.cpp:60-62 of the reference); B, H or D = 0 with N > 0 reach the launcher and
  raise ValueError, as in the reference (csrc/kernels/flash_fwd.cu:626-628, 635-638).
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


def _qkv(b, h, n, d, seed):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(b, h, n, d, generator=g).half() for _ in range(3))


def _params(q, k, v, o, causal, variant="opt", scale=None):
    from fa import native

    b, h, n, d = q.shape
    sc = d ** -0.5 if scale is None else scale
    return native.make_params(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), b, h, n, d,
                              sc, causal, variant)


def _single_launch(q, k, v, causal):
    from fa import native

    o = torch.empty_like(q)
    rc, msg = native.flash_fwd(_params(q, k, v, o, causal),
                               torch.cuda.current_stream().cuda_stream)
    assert rc == native.FA_OK, msg
    torch.cuda.synchronize()
    return o


def _preferred(b, h, n, d, causal, variant="opt"):
    from fa import native

    p = native.make_params(0x1000, 0x1000, 0x1000, 0x1000, b, h, n, d, d ** -0.5, causal, variant)
    return native.splitkv_plan(p, 0)["preferred"] == 1


ROUTED = [
    # (B, H, N, d, causal): one GPU's share of the headline shape split by heads, and kin
    (1, 1, 16384, 128, False), (1, 1, 16384, 128, True),
    (1, 2, 16384, 128, False), (1, 2, 16384, 128, True),
    (1, 1, 32768, 128, False), (1, 1, 32768, 128, True),
    (1, 2, 4096, 128, True), (1, 4, 8192, 64, False),
    (1, 1, 16384, 64, True),     # causal d = 64 from 16384 keys
    (1, 8, 8192, 128, True),     # causal, one round of 256 query blocks from 8192 keys
    (1, 8, 8192, 64, True),
]


@pytest.mark.parametrize("b,h,n,d,causal", ROUTED)
def test_routed_shapes(b, h, n, d, causal):
    import fa

    print(f"case routed B={b} H={h} N={n} d={d} causal={causal}", flush=True)
    assert _preferred(b, h, n, d, causal)
    q, k, v = _qkv(b, h, n, d, seed=n + h + d)
    qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
    out = fa.forward(qc, kc, vc, causal=causal)
    o_split, lse_split = fa.forward_splitkv(qc, kc, vc, causal=causal)
    assert torch.equal(out, o_split)
    o_lse, lse = fa.forward_lse(qc, kc, vc, causal=causal)
    assert torch.equal(o_lse, out) and torch.equal(lse, lse_split)
    assert torch.equal(fa.forward(qc, kc, vc, causal=causal, fp16_accum=True), out)
    out = out.cpu()
    for bi in range(b):
        for hi in range(h):
            sl = (slice(bi, bi + 1), slice(hi, hi + 1))
            ref = orc.attention_fp32(q[sl], k[sl], v[sl], causal=causal)
            torch.testing.assert_close(out[sl].float(), ref, atol=ATOL, rtol=RTOL)


NOT_ROUTED = [
    # each is one step over a boundary of the routing rule
    (1, 2, 4095, 128, True),     # N below 4096
    (1, 4, 8192, 64, True),      # causal d = 64 below 16384 keys keeps the single launch
    (1, 10, 8192, 128, True),    # causal, 320 query blocks: more than one round
    (1, 16, 4096, 128, True),    # causal, one round below 8192 keys
    (1, 3, 16383, 64, True),     # (a small grid)
    (1, 16, 4096, 128, False),   # 16 x 16 = 256 workgroups of 8 waves: fills the GPU
    (2, 8, 1000, 64, True),      # the benchmark's ragged config: short
]


@pytest.mark.parametrize("b,h,n,d,causal", NOT_ROUTED)
def test_shapes_past_the_routing_boundaries_take_the_single_launch(b, h, n, d, causal):
    import fa

    print(f"case not routed B={b} H={h} N={n} d={d} causal={causal}", flush=True)
    assert not _preferred(b, h, n, d, causal)
    q, k, v = (t.cuda() for t in _qkv(b, h, n, d, seed=n + h + d))
    assert torch.equal(fa.forward(q, k, v, causal=causal), _single_launch(q, k, v, causal))


@pytest.mark.parametrize("b,h,n,d", [(1, 17, 8192, 128), (1, 20, 10000, 128), (1, 17, 8192, 64)])
def test_head_split_of_a_mostly_empty_last_round(b, h, n, d):
    """fa_tail_plan splits the heads: the first run as one single launch, the rest through
    split-KV. forward must be bitwise those two calls on the two head ranges, forward_lse's O
    bitwise forward's, and rows of the first, a boundary and the last head match fp64."""
    import fa
    from fa import native

    p = native.make_params(0x1000, 0x1000, 0x1000, 0x1000, b, h, n, d, d ** -0.5, False, "opt")
    heads = native.tail_plan(p)
    print(f"case head split B={b} H={h} N={n} d={d} heads={heads}", flush=True)
    assert 0 < heads < b * h
    q, k, v = (t.cuda() for t in _qkv(b, h, n, d, seed=n + h))
    out = fa.forward(q, k, v)
    flat = [t.view(1, b * h, n, d) for t in (q, k, v)]
    first = _single_launch(*(t[:, :heads] for t in flat), False)
    rest, _ = fa.forward_splitkv(*(t[:, heads:] for t in flat))
    assert torch.equal(out.view(1, b * h, n, d)[:, :heads], first)
    assert torch.equal(out.view(1, b * h, n, d)[:, heads:], rest)
    o_lse, lse = fa.forward_lse(q, k, v)
    assert torch.equal(o_lse, out)
    rows = [0, 255, 256, n // 2, n - 1]
    outc = out.float().cpu().view(b * h, n, d)
    for bh in (0, heads - 1, heads, b * h - 1):
        ref = torch.from_numpy(orc.attention_fp64_rows(q, k, v, False, bh, rows)).float()
        torch.testing.assert_close(outc[bh, rows], ref, atol=ATOL, rtol=RTOL)
        lse_ref = torch.from_numpy(orc.lse_fp64_rows(q, k, False, bh, rows)).float()
        torch.testing.assert_close(lse.view(b * h, n)[bh, rows].cpu(), lse_ref, atol=2e-3,
                                   rtol=0)


def test_baseline_variant_is_never_routed():
    import fa

    assert _preferred(1, 2, 16384, 128, False)
    assert not _preferred(1, 2, 16384, 128, False, variant="baseline")
    q, k, v = (t.cuda() for t in _qkv(1, 1, 4096, 128, seed=5))
    from fa import native

    o = torch.empty_like(q)
    rc, msg = native.flash_fwd(_params(q, k, v, o, False, variant="baseline"),
                               torch.cuda.current_stream().cuda_stream)
    assert rc == native.FA_OK, msg
    assert torch.equal(fa.forward_variant(q, k, v, variant="baseline"), o)


# ---- every row written: NaN-prefilled O through the C ABI ------------------------------------
# Ragged shapes (N not a multiple of any tile) reaching every row of the tile table.
TAIL_SHAPES = [
    # (B, H, N, d, causal, variant)
    (1, 3, 1000, 64, False, "opt"), (2, 3, 777, 64, True, "opt"),          # small grid, d=64
    (1, 3, 700, 64, False, "opt"), (2, 3, 1001, 64, True, "opt"),          # (two/four-way)
    (1, 2, 1500, 128, False, "opt"), (1, 2, 1499, 128, True, "opt"),       # small grid, d=128
    (1, 2, 450, 128, False, "opt"), (1, 2, 449, 128, True, "opt"),         # (four/two-way)
    (4, 16, 1001, 64, False, "opt"), (4, 16, 999, 64, True, "opt"),        # simple 8 waves
    (1, 32, 2501, 64, False, "opt"),                                        # (16x16x32 and
    (1, 8, 8000, 64, False, "opt"), (2, 8, 8500, 64, True, "opt"),         # 32x32x16 MFMAs)
    (3, 16, 1699, 64, True, "opt"),                                         # 128-key causal
    (8, 16, 703, 128, False, "opt"), (4, 16, 1003, 128, True, "opt"),      # simple 4 waves
    (16, 16, 251, 128, False, "opt"), (16, 16, 509, 128, True, "opt"),
    (2, 16, 2501, 128, False, "opt"), (1, 16, 4001, 128, True, "opt"),     # ping-pong d=128
    (2, 3, 333, 64, True, "baseline"), (2, 3, 333, 128, False, "baseline"),
]
GUARD = 4096


def _nan_filled_o(q):
    buf = torch.full((q.numel() + GUARD,), float("nan"), dtype=torch.float16, device="cuda")
    buf[q.numel():] = 7.0
    return buf, buf[:q.numel()].view(q.shape)


def _check_written(q, k, v, o, buf, causal, scale=None):
    assert torch.all(buf[q.numel():] == 7.0), "write past the end of O"
    assert torch.isfinite(o).all(), "O element left unwritten (still NaN)"
    b, h, _, _ = q.shape
    oc, qc, kc, vc = (t.cpu() for t in (o, q, k, v))
    for bi, hi in {(0, 0), (b - 1, h - 1)}:
        sl = (slice(bi, bi + 1), slice(hi, hi + 1))
        ref = orc.attention_fp32(qc[sl], kc[sl], vc[sl], causal=causal, scale=scale)
        torch.testing.assert_close(oc[sl].float(), ref, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("b,h,n,d,causal,variant", TAIL_SHAPES)
def test_nan_prefilled_output_fully_written(b, h, n, d, causal, variant):
    from fa import native

    print(f"case nan-fill B={b} H={h} N={n} d={d} causal={causal} {variant}", flush=True)
    q, k, v = (t.cuda() for t in _qkv(b, h, n, d, seed=3 * n + d))
    stream = torch.cuda.current_stream().cuda_stream
    # fa_flash_fwd
    buf, o = _nan_filled_o(q)
    rc, msg = native.flash_fwd(_params(q, k, v, o, causal, variant), stream)
    assert rc == native.FA_OK, msg
    torch.cuda.synchronize()
    _check_written(q, k, v, o, buf, causal)
    # fa_flash_fwd_lse: O and every LSE entry written
    buf, o = _nan_filled_o(q)
    lse_v = torch.full((b, h, n), float("nan"), device="cuda")
    rc, msg = native.flash_fwd_lse(_params(q, k, v, o, causal, variant), lse_v.data_ptr(), stream)
    assert rc == native.FA_OK, msg
    torch.cuda.synchronize()
    _check_written(q, k, v, o, buf, causal)
    assert torch.isfinite(lse_v).all()


@pytest.mark.parametrize("b,h,n,d,causal,splits", [(1, 2, 3001, 128, True, 0),
                                                   (1, 3, 2049, 64, False, 3),
                                                   (2, 2, 1999, 64, True, 0),
                                                   (1, 1, 9001, 128, False, 0)])
def test_nan_prefilled_output_splitkv(b, h, n, d, causal, splits):
    """fa_flash_fwd_splitkv, with the workspace pre-filled with NaN too: the combine kernel
    must read only the partial results the partial pass wrote."""
    from fa import native

    print(f"case nan-fill splitkv B={b} H={h} N={n} d={d} causal={causal}", flush=True)
    q, k, v = (t.cuda() for t in _qkv(b, h, n, d, seed=5 * n + d))
    buf, o = _nan_filled_o(q)
    p = _params(q, k, v, o, causal)
    plan = native.splitkv_plan(p, splits)
    ws = torch.full((plan["workspace_bytes"] // 4,), float("nan"), device="cuda")
    lse = torch.full((b, h, n), float("nan"), device="cuda")
    rc, msg = native.flash_fwd_splitkv(p, lse.data_ptr(), splits, ws.data_ptr(),
                                       plan["workspace_bytes"],
                                       torch.cuda.current_stream().cuda_stream)
    assert rc == native.FA_OK, msg
    torch.cuda.synchronize()
    _check_written(q, k, v, o, buf, causal)
    assert torch.isfinite(lse).all()


# ---- degenerate shapes at the binding --------------------------------------------------------
@pytest.mark.parametrize("shape, words", [
    ((0, 2, 64, 64), "batch, heads and seqlen must be positive"),
    ((1, 0, 64, 128), "batch, heads and seqlen must be positive"),
    ((1, 2, 64, 0), "head_dim must be 64 or 128, got 0"),
    ((1, 2, 64, 96), "head_dim must be 64 or 128, got 96"),
])
def test_empty_dims_raise_like_the_reference(shape, words):
    import fa

    q = torch.zeros(shape, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError, match=words):
        fa.forward(q, q, q)
    with pytest.raises(ValueError, match=words):
        fa.forward_variant(q, q, q, causal=True, variant="baseline")
    with pytest.raises(ValueError, match=words):
        fa.forward_lse(q, q, q)
    with pytest.raises(ValueError, match=words):
        fa.forward_splitkv(q, q, q)


@pytest.mark.parametrize("shape", [(1, 2, 0, 64), (0, 2, 0, 128), (2, 3, 0, 96)])
def test_zero_seqlen_returns_empty(shape):
    import fa

    q = torch.zeros(shape, dtype=torch.float16, device="cuda")
    for out in (fa.forward(q, q, q), fa.forward(q, q, q, causal=True), fa.forward_lse(q, q, q)[0],
                fa.forward_splitkv(q, q, q)[0]):
        assert out.shape == q.shape and out.dtype == torch.float16
    o, lse = fa.forward_lse(q, q, q)
    assert lse.shape == shape[:3] and lse.dtype == torch.float32
