"""CPU: pins the LSE oracle (oracle.attention.lse_fp32 and lse_fp64_rows) before it is trusted.

The reference has no LSE output, so nothing of its own pins these; the mathematics does.
For scores s_j = scale * q_i . k_j over the visible keys j of row i, LSE_i = log sum_j exp(s_j):
  * q = 0 (or scale = 0): every s_j = 0, LSE_i = log(number of visible keys) = log(n), or
    log(i + 1) when causal;
  * causal row 0 sees only key 0: LSE_0 = scale * q_0 . k_0;
  * duplicating every key (non-causal, [K; K]) doubles every term: LSE + log 2;
  * adding a constant c to every score adds c: with q_i = e_0 * a and k_j = e_0 * a + w_j for
    w_j orthogonal to e_0, s_j = scale * a^2 for all j -- a closed form of the shift;
  * the fp32 (torch) and fp64 (C) restatements agree on random inputs;
  * planted mistakes (base-2 log, no max shift in fp16, the causal mask off by one, the scale
    left out) each fail at least one check.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as orc


def _qk(b, h, n, d, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return tuple((torch.randn(b, h, n, d, generator=g) * scale).half() for _ in range(2))


def _fp32(q, k, causal, scale):
    return orc.lse_fp32(q, k, causal, scale).double().numpy()


def _fp64(q, k, causal, scale):
    b, h, n, _ = q.shape
    return np.stack([orc.lse_fp64_rows(q, k, causal, bh, range(n), scale)
                     for bh in range(b * h)]).reshape(b, h, n)


IMPLS = {"fp32": _fp32, "fp64": _fp64}


def check_zero_query(impl):
    _, k = _qk(1, 2, 37, 64, seed=1)
    q = torch.zeros_like(k)
    n = 37
    np.testing.assert_allclose(impl(q, k, False, None), np.full((1, 2, n), math.log(n)),
                               rtol=1e-6)
    np.testing.assert_allclose(impl(q, k, True, None),
                               np.broadcast_to(np.log(np.arange(1, n + 1)), (1, 2, n)),
                               rtol=1e-6, atol=1e-7)


def check_zero_scale(impl):
    q, k = _qk(1, 1, 20, 128, seed=2)
    np.testing.assert_allclose(impl(q, k, False, 0.0), np.full((1, 1, 20), math.log(20)),
                               rtol=1e-6)


def check_causal_row0(impl):
    q, k = _qk(2, 2, 9, 64, seed=3)
    got = impl(q, k, True, 0.3)[:, :, 0]
    want = (q[:, :, 0].double() * k[:, :, 0].double()).sum(-1).numpy() * 0.3
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def check_duplicated_keys(impl):
    q, k = _qk(1, 2, 24, 64, seed=4)
    q2 = torch.cat([q, q], dim=2)            # same rows twice; keys [K; K]
    k2 = torch.cat([k, k], dim=2)
    base = impl(q, k, False, None)
    dup = impl(q2, k2, False, None)[:, :, :24]
    np.testing.assert_allclose(dup, base + math.log(2.0), rtol=1e-5, atol=1e-5)


def check_constant_shift(impl):
    n, d, a = 16, 64, 1.5
    g = torch.Generator().manual_seed(5)
    w = torch.randn(1, 1, n, d, generator=g)
    w[..., 0] = 0.0
    q = torch.zeros(1, 1, n, d)
    q[..., 0] = a
    k = w.clone()
    k[..., 0] = a
    q, k = q.half(), k.half()
    a16 = float(torch.tensor(a).half())
    c = 0.25 * a16 * a16                     # every score is scale * a^2 with scale 0.25
    np.testing.assert_allclose(impl(q, k, False, 0.25), np.full((1, 1, n), c + math.log(n)),
                               rtol=1e-6)


CHECKS = [check_zero_query, check_zero_scale, check_causal_row0, check_duplicated_keys,
          check_constant_shift]


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
@pytest.mark.parametrize("impl", list(IMPLS))
def test_lse_oracle_pinning(impl, check):
    check(IMPLS[impl])


def test_lse_fp32_and_fp64_agree():
    for causal in (False, True):
        q, k = _qk(2, 3, 129, 128, seed=6)
        np.testing.assert_allclose(_fp32(q, k, causal, None), _fp64(q, k, causal, None),
                                   atol=2e-6, rtol=1e-6)


def _mutant(kind):
    def impl(q, k, causal, scale):
        d, n = q.shape[-1], q.shape[-2]
        sc = 1.0 / math.sqrt(d) if scale is None else scale
        if kind == "no_scale":
            sc = 1.0
        s = q.double() @ k.double().transpose(-2, -1) * sc
        if causal:
            diag = 0 if kind == "diag_masked" else 1
            s = s.masked_fill(torch.ones(n, n, dtype=torch.bool).triu(diag), float("-inf"))
        if kind == "log2":
            return (torch.logsumexp(s, -1) / math.log(2.0)).numpy()
        if kind == "no_max_shift_fp16":
            return torch.log(torch.exp(s).half().double().sum(-1)).numpy()
        return torch.logsumexp(s, -1).numpy()

    return impl


@pytest.mark.parametrize("kind", ["no_scale", "diag_masked", "log2", "no_max_shift_fp16"])
def test_planted_lse_mistakes_are_caught(kind):
    caught = []
    for check in CHECKS:
        try:
            with np.errstate(all="ignore"):
                check(_mutant(kind))
        except AssertionError:
            caught.append(check.__name__)
    assert caught, f"mutant {kind} passed every LSE pinning check"


def test_correct_lse_mutant_passes():
    for check in CHECKS:
        check(_mutant("none"))
