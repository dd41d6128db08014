"""GPU: seeded random shapes and arguments against the CPU oracle.

Forty draws (fixed seed, so the case list is the same on every run) of batch, heads, sequence
length, head dim, causal, variant and softmax scale, with B*H*N small enough for the oracle but
spread so that every tile row (small grid key split, simple, ping-pong) and both
sides of the size thresholds come up. Each case checks fa.forward_variant against the fp32
oracle on two (b, h) slices with the north-star tolerance, and fa.forward_lse's LSE against the
oracle's LSE (2e-3 absolute). Further seeded draws take the head split, and ping-pong shapes
under the input classes that steer its softmax (wide spreads, outlier keys, a sink, scores
that widen late).
"""

from __future__ import annotations

import math
import random

import pytest
import torch

from conftest import ATOL, RTOL
from oracle import attention as orc

pytestmark = pytest.mark.gpu


def _cases(count=40, seed=20261201):
    rnd = random.Random(seed)
    out = []
    for i in range(count):
        d = rnd.choice([64, 128])
        n = rnd.choice([1, 7, 31, 64, 100, 255, 256, 257, 1000, 2047, 2049, 3073, 4097, 5000, 8193])
        # half the draws on grids of at least 256 eight-wave workgroups (the large-grid rows),
        # half below; at most 8M elements per tensor
        blocks = (n + 255) // 256
        bh_large = -(-256 // blocks)
        if rnd.random() < 0.5 and bh_large * n * d <= 8 << 20:
            bh = rnd.randint(bh_large, max(bh_large, min(2 * bh_large, (8 << 20) // (n * d))))
        else:
            bh = rnd.randint(1, max(1, min(bh_large - 1, (1 << 20) // (n * d) + 1)))
        b = rnd.choice([x for x in (1, 2, 4) if bh % x == 0])
        h = bh // b
        causal = rnd.random() < 0.5
        variant = rnd.choice(["opt", "opt", "fp16acc", "baseline"])
        scale = rnd.choice([None, None, 0.05, 0.3, -0.2])
        out.append((i, b, h, n, d, causal, variant, scale))
    return out


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")


@pytest.mark.parametrize("i,b,h,n,d,causal,variant,scale", _cases())
def test_random_case(i, b, h, n, d, causal, variant, scale):
    import fa
    from fa import native

    tile = native.tile_config(d, causal, variant, n, b, h)
    print(f"case {i}: B={b} H={h} N={n} d={d} causal={causal} {variant} scale={scale} "
          f"tile={tile}", flush=True)
    g = torch.Generator().manual_seed(1000 + i)
    q, k, v = (torch.randn(b, h, n, d, generator=g).half() for _ in range(3))
    qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
    if scale is None:
        out = fa.forward_variant(qc, kc, vc, causal=causal, variant=variant)
    else:
        out = fa._C.forward(qc, kc, vc, causal, scale, variant)
    _, lse = fa.forward_lse(qc, kc, vc, causal=causal, softmax_scale=scale, variant=variant)
    out, lse = out.cpu(), lse.cpu()
    for bi, hi in {(0, 0), (b - 1, h - 1)}:
        sl = (slice(bi, bi + 1), slice(hi, hi + 1))
        ref = orc.attention_fp32(q[sl], k[sl], v[sl], causal=causal, scale=scale)
        torch.testing.assert_close(out[sl].float(), ref, atol=ATOL, rtol=RTOL)
        ref_lse = orc.lse_fp32(q[sl], k[sl], causal, scale)
        torch.testing.assert_close(lse[sl], ref_lse, atol=2e-3, rtol=0)
    assert math.isfinite(float(out.float().abs().max()))


def _head_split_heads(bh, n):
    """The head split rule restated (non-causal, N >= 4096, ping-pong grids of 256-row items
    at one workgroup per CU): the heads whose items fill the whole rounds of 256, when the last
    round is at most a third full and those heads still make 256 items or more; else 0."""
    nqb = -(-n // 256)
    items = bh * nqb
    full, last = divmod(items, 256)
    if full < 1 or last == 0 or 3 * last > 256:
        return 0
    heads = full * 256 // nqb
    return heads if heads * nqb >= 256 and heads < bh else 0


def _head_split_cases(count=6, seed=20261202):
    rnd = random.Random(seed)
    out = []
    while len(out) < count:
        d = rnd.choice([64, 128])
        n = rnd.choice([4096, 4500, 5000, 6000, 8192, 9000, 10000])
        bh = rnd.randint(2, max(2, (12 << 20) // (n * d)))
        heads = _head_split_heads(bh, n)
        if heads:
            b = rnd.choice([x for x in (1, 2, 3) if bh % x == 0])
            out.append((len(out), b, bh // b, n, d, heads))
    return out


@pytest.mark.parametrize("i,b,h,n,d,heads", _head_split_cases())
def test_random_head_split_case(i, b, h, n, d, heads):
    """Seeded shapes that take fa_tail_plan's head split: the library's plan equals the rule
    restated above, and fa.forward / fa.forward_lse match the oracle on the first head, the
    last head of the single launch, the first split head and the last head."""
    import fa
    from fa import native

    p = native.make_params(0x1000, 0x1000, 0x1000, 0x1000, b, h, n, d, d ** -0.5, False, "opt")
    print(f"case split {i}: B={b} H={h} N={n} d={d} heads={heads}", flush=True)
    assert native.tail_plan(p) == heads
    g = torch.Generator().manual_seed(2000 + i)
    q, k, v = (torch.randn(b, h, n, d, generator=g).half() for _ in range(3))
    qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
    out = fa.forward(qc, kc, vc).cpu()
    _, lse = fa.forward_lse(qc, kc, vc)
    lse = lse.cpu()
    for f in sorted({0, heads - 1, heads, b * h - 1}):
        bi, hi = divmod(f, h)
        sl = (slice(bi, bi + 1), slice(hi, hi + 1))
        ref = orc.attention_fp32(q[sl], k[sl], v[sl])
        torch.testing.assert_close(out[sl].float(), ref, atol=ATOL, rtol=RTOL)
        torch.testing.assert_close(lse[sl], orc.lse_fp32(q[sl], k[sl], False), atol=2e-3, rtol=0)


# Ping-pong shapes (d=128 large grids in both modes, d=64 one-round grids) for the input-class
# draws below: (b, h, n, d, causal).
PP_SHAPES = [(4, 16, 4096, 128, False), (2, 16, 5000, 128, False), (1, 16, 8193, 128, False),
             (8, 8, 2049, 128, False), (4, 16, 4096, 128, True), (2, 16, 5000, 128, True),
             (1, 16, 8193, 128, True), (4, 8, 3300, 128, True), (1, 16, 4096, 64, False),
             (1, 4, 16384, 64, False), (1, 8, 8000, 64, False)]
KINDS = ["spread 1.3", "spread 1.6", "spread 2.0", "outliers", "sink", "late"]


def _class_cases(count=14, seed=20261203):
    rnd = random.Random(seed)
    cases = [(i,) + PP_SHAPES[i % len(PP_SHAPES)] + (KINDS[i % len(KINDS)],)
             for i in range(len(PP_SHAPES))]
    while len(cases) < count:
        cases.append((len(cases),) + rnd.choice(PP_SHAPES) + (rnd.choice(KINDS),))
    return cases


def _class_inputs(b, h, n, d, kind, seed):
    """q, k, v fp16 on the CPU: ~N(0, 1), then per kind: q and k x s ("spread s": the first
    tile's vote runs the ping-pong items checked from the start); 1 % of the key rows x8
    ("outliers": items overflow their unchecked run and are redone, later workgroups start
    checked); key 0 about 13 nats above the rest ("sink": neither); keys from n/3 on x2.5
    ("late": scores that widen after the first tile, which the vote cannot see: redone)."""
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(b, h, n, d, generator=g) for _ in range(3))
    if kind.startswith("spread"):
        s = float(kind.split()[1])
        q, k = q * s, k * s
    elif kind == "outliers":
        k = k * ((torch.rand(b, h, n, 1, generator=g) < 0.01).float() * 7.0 + 1.0)
    elif kind == "sink":
        q[..., 0] = 4.0
        k[:, :, 0, 0] = 13.0 * d ** 0.5 / 4.0
    else:
        k[:, :, n // 3:] *= 2.5
    return q.half(), k.half(), v.half()


@pytest.mark.parametrize("i,b,h,n,d,causal,kind", _class_cases())
def test_random_input_class_case(i, b, h, n, d, causal, kind):
    """Seeded ping-pong shapes under the input classes that steer its softmax (the first tile's
    wide-spread vote, the redo of an overflowing item, the launch's switch to checked starts,
    or none of them): fa.forward against the fp32 oracle on the first and last (b, h) slices."""
    import fa
    from fa import native

    tile = native.tile_config(d, causal, "opt", n, b, h)
    print(f"case class {i}: B={b} H={h} N={n} d={d} causal={causal} {kind} tile={tile}",
          flush=True)
    assert tile["schedule"] == "pingpong16", tile
    q, k, v = _class_inputs(b, h, n, d, kind, seed=3000 + i)
    out = fa.forward(q.cuda(), k.cuda(), v.cuda(), causal=causal).cpu()
    assert torch.isfinite(out).all()
    for bi, hi in {(0, 0), (b - 1, h - 1)}:
        sl = (slice(bi, bi + 1), slice(hi, hi + 1))
        ref = orc.attention_fp32(q[sl], k[sl], v[sl], causal=causal)
        torch.testing.assert_close(out[sl].float(), ref, atol=ATOL, rtol=RTOL)
