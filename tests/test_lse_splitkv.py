"""GPU: the LSE output (fa.forward_lse, fa_flash_fwd_lse) and the split-KV forward
(fa.forward_splitkv, fa_flash_fwd_splitkv) against the CPU oracle.

Neither exists in the reference; the oracle's LSE is pinned by closed forms
(tests/test_oracle_lse.py). Bars: O within the north-star tolerance |d| <= 2e-3 + 1e-2 |ref|;
LSE within 2e-3 absolute (the row sum is taken over the fp16 P values the kernel multiplies
with V, so LSE carries up to ~5e-4 of fp16 rounding); O of forward_lse bitwise equal to
forward's; split-KV deterministic run to run.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import ATOL, RTOL
from oracle import attention as orc

pytestmark = pytest.mark.gpu
LSE_ATOL = 2e-3


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")


def _qkv(b, h, n, d, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return tuple((torch.randn(b, h, n, d, generator=g) * scale).half() for _ in range(3))


def _slices(b, h):
    return [(slice(bi, bi + 1), slice(hi, hi + 1)) for bi, hi in {(0, 0), (b - 1, h - 1)}]


# Shapes that reach every kind of tile row (small grid, simple, ping-pong).
LSE_CASES = [
    (2, 3, 257, 64, False), (2, 3, 1000, 128, True),      # small grids
    (1, 4, 1100, 64, True), (1, 2, 450, 128, False),      # (four-way d=64, two-way d=128)
    (4, 16, 1000, 64, True), (8, 16, 700, 128, False),    # simple 8 and 4 waves, large grid
    (16, 16, 250, 128, False),                            # (on 32x32x16 and 16x16x32 MFMAs)
    (2, 16, 5000, 64, True), (2, 16, 2500, 128, False),   # simple d=64 long / ping-pong d=128
    (3, 16, 1700, 64, True),                              # 128-key tiles, causal d=64
    (1, 16, 4000, 128, True),                             # ping-pong causal
    (1, 8, 8000, 64, False),                              # ping-pong d=64, one round
]


@pytest.mark.parametrize("b,h,n,d,causal", LSE_CASES)
@pytest.mark.parametrize("variant", ["opt", "baseline"])
def test_forward_lse(b, h, n, d, causal, variant):
    import fa

    print(f"case lse B={b} H={h} N={n} d={d} causal={causal} {variant}", flush=True)
    q, k, v = _qkv(b, h, n, d, seed=n + d)
    qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
    o, lse = fa.forward_lse(qc, kc, vc, causal=causal, variant=variant)
    assert lse.dtype == torch.float32 and lse.shape == (b, h, n)
    assert torch.equal(o, fa.forward_variant(qc, kc, vc, causal=causal, variant=variant))
    o, lse = o.cpu(), lse.cpu()
    for sl in _slices(b, h):
        torch.testing.assert_close(o[sl].float(), orc.attention_fp32(q[sl], k[sl], v[sl], causal),
                                   atol=ATOL, rtol=RTOL)
        torch.testing.assert_close(lse[sl], orc.lse_fp32(q[sl], k[sl], causal), atol=LSE_ATOL,
                                   rtol=0)


@pytest.mark.parametrize("scale", [0.3, -0.2, 0.0])
def test_forward_lse_custom_scale(scale):
    import fa

    q, k, v = _qkv(1, 2, 300, 128, seed=4)
    for causal in (False, True):
        _, lse = fa.forward_lse(q.cuda(), k.cuda(), v.cuda(), causal=causal, softmax_scale=scale)
        torch.testing.assert_close(lse.cpu(), orc.lse_fp32(q, k, causal, scale), atol=LSE_ATOL,
                                   rtol=0)


def test_forward_lse_fp64_rows_long():
    import fa

    q, k, v = _qkv(1, 2, 9000, 128, seed=5)
    _, lse = fa.forward_lse(q.cuda(), k.cuda(), v.cuda(), causal=True)
    rows = [0, 1, 255, 256, 4500, 8999]
    for bh in range(2):
        want = orc.lse_fp64_rows(q, k, True, bh, rows)
        np.testing.assert_allclose(lse[0, bh, rows].cpu().double().numpy(), want, atol=LSE_ATOL)


SPLIT_CASES = [
    # (B, H, N, d, causal, num_splits)
    (2, 8, 1000, 64, True, 0), (2, 8, 1000, 64, False, 3),
    (1, 2, 3001, 128, True, 0), (1, 2, 3001, 128, True, 5), (1, 2, 3001, 128, False, 1),
    (1, 3, 2048, 128, False, 7), (1, 1, 17, 64, True, 0), (1, 1, 1, 128, False, 4),
    (1, 2, 700, 64, True, 1000),
    # automatic plans with several ranges per query block (steady ping-pong state per range)
    (1, 4, 4097, 64, True, 0), (1, 1, 5000, 128, False, 0), (1, 1, 6000, 128, True, 0),
]


@pytest.mark.parametrize("b,h,n,d,causal,splits", SPLIT_CASES)
def test_forward_splitkv(b, h, n, d, causal, splits):
    import fa

    print(f"case splitkv B={b} H={h} N={n} d={d} causal={causal} splits={splits}", flush=True)
    q, k, v = _qkv(b, h, n, d, seed=3 * n + d)
    qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
    o, lse = fa.forward_splitkv(qc, kc, vc, causal=causal, num_splits=splits)
    o2, lse2 = fa.forward_splitkv(qc, kc, vc, causal=causal, num_splits=splits)
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    o, lse = o.cpu(), lse.cpu()
    for sl in _slices(b, h):
        torch.testing.assert_close(o[sl].float(), orc.attention_fp32(q[sl], k[sl], v[sl], causal),
                                   atol=ATOL, rtol=RTOL)
        torch.testing.assert_close(lse[sl], orc.lse_fp32(q[sl], k[sl], causal), atol=LSE_ATOL,
                                   rtol=0)


def test_splitkv_long_rows_fp64():
    """B*H = 2 at N = 16384, d = 128 (one GPU's share of the headline shape split 8 ways by
    heads): selected rows against the fp64 oracle, causal and not."""
    import fa

    q, k, v = _qkv(1, 2, 16384, 128, seed=6)
    rows = [0, 1, 127, 128, 8191, 16383]
    for causal in (False, True):
        o, lse = fa.forward_splitkv(q.cuda(), k.cuda(), v.cuda(), causal=causal)
        for bh in range(2):
            want = orc.attention_fp64_rows(q, k, v, causal, bh, rows)
            got = o[0, bh, rows].cpu().double().numpy()
            np.testing.assert_allclose(got, want, atol=ATOL, rtol=RTOL)
            np.testing.assert_allclose(lse[0, bh, rows].cpu().double().numpy(),
                                       orc.lse_fp64_rows(q, k, causal, bh, rows), atol=LSE_ATOL)


def test_splitkv_c_abi_matches_binding():
    """The raw C entry point with a caller workspace gives the binding's bits."""
    import fa
    from fa import native

    q, k, v = (t.cuda() for t in _qkv(1, 2, 1500, 64, seed=7))
    o_ref, lse_ref = fa.forward_splitkv(q, k, v, causal=True, num_splits=0)
    o = torch.empty_like(q)
    lse = torch.empty(1, 2, 1500, device="cuda")
    p = native.make_params(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), 1, 2, 1500, 64,
                           0.125, True, "opt")
    plan = native.splitkv_plan(p, 0)
    ws = torch.empty(plan["workspace_bytes"] // 4, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    rc, msg = native.flash_fwd_splitkv(p, lse.data_ptr(), 0, ws.data_ptr(),
                                       plan["workspace_bytes"], stream)
    assert rc == native.FA_OK, msg
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref) and torch.equal(lse, lse_ref)
