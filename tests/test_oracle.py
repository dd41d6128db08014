"""CPU: pins the oracle (oracle/attention.py, oracle/attention_fp64.c) before it is trusted.

The reference ships no golden vectors for this path (its tests draw seeded random inputs and
compare with an fp32 / fp64 recomputation, tests/test_flash_fwd.py:18-36,
tests/cpp/test_flash_fwd.cu:115-187), so the oracle is pinned by what the mathematics fixes:
  * the binary16 decoder against numpy for all 65536 bit patterns;
  * a hand-computed 2-row example, causal and not;
  * closed forms used by the reference's own tests: q = 0 gives mean(V) (prefix means when
    causal, tests/test_flash_fwd.py:60-70), causal row 0 equals V[0] (:106-110), and the
    custom-scale equivalence (:97-103);
  * a one-hot closed form (one key dominates by a known margin), key/value permutation
    invariance (non-causal) and query permutation equivariance;
  * agreement of the two independent restatements (torch fp32 and C fp64), and with torch's
    scaled_dot_product_attention in float64 (a library routine);
  * planted mistakes: each plausible oracle bug below must fail at least one of these checks.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as orc

import fa.reference as fref  # the package's user-facing torch reference (not the oracle)


def _qkv(b, h, n, d, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return tuple((torch.randn(b, h, n, d, generator=g) * scale).half() for _ in range(3))


def test_half_decoder_all_bit_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float64)
    got = np.array([orc.half_to_double(int(b)) for b in bits])
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])


def _hand_example():
    # d = 1: q = [1, 2], k = [0, 1], v = [1, 3], scale 1.
    q = torch.tensor([1.0, 2.0]).half().view(1, 1, 2, 1)
    k = torch.tensor([0.0, 1.0]).half().view(1, 1, 2, 1)
    v = torch.tensor([1.0, 3.0]).half().view(1, 1, 2, 1)
    e = math.e
    full = np.array([(1 + 3 * e) / (1 + e), (1 + 3 * e**2) / (1 + e**2)])
    causal = np.array([1.0, (1 + 3 * e**2) / (1 + e**2)])
    return q, k, v, full, causal


@pytest.mark.parametrize("impl", ["fp64", "fp32"])
def test_hand_computed_example(impl):
    q, k, v, full, causal = _hand_example()
    for c, want in ((False, full), (True, causal)):
        if impl == "fp64":
            got = orc.attention_fp64(q, k, v, causal=c, scale=1.0).reshape(-1)
            np.testing.assert_allclose(got, want, rtol=1e-14, atol=0)
        else:
            got = orc.attention_fp32(q, k, v, causal=c, scale=1.0).reshape(-1).double().numpy()
            np.testing.assert_allclose(got, want, rtol=1e-6, atol=0)


# ---- the pinning checks, as functions of an attention implementation -------------------------
# impl(q, k, v, causal, scale) -> float64 numpy [B, H, N, D]


def _check_zero_query_is_mean(impl):
    _, k, v = _qkv(1, 2, 96, 64, seed=11)
    q = torch.zeros_like(k)
    vv = v.double().numpy()
    np.testing.assert_allclose(impl(q, k, v, False, None), np.broadcast_to(
        vv.mean(axis=2, keepdims=True), vv.shape), atol=1e-6, rtol=1e-6)
    prefix = np.cumsum(vv, axis=2) / np.arange(1, vv.shape[2] + 1)[None, None, :, None]
    np.testing.assert_allclose(impl(q, k, v, True, None), prefix, atol=1e-6, rtol=1e-6)


def _check_causal_row0(impl):
    q, k, v = _qkv(1, 2, 40, 64, seed=12)
    out = impl(q, k, v, True, None)
    np.testing.assert_allclose(out[:, :, 0], v[:, :, 0].double().numpy(), atol=1e-6, rtol=0)


def _check_one_hot(impl):
    # q_i = e_0 for all i; k_j = 0 except key 7 = 12 * e_0, scale 1: row scores are 12 at key 7
    # and 0 elsewhere (for the visible keys).
    n, d = 32, 64
    q = torch.zeros(1, 1, n, d)
    q[..., 0] = 1.0
    k = torch.zeros(1, 1, n, d)
    k[0, 0, 7, 0] = 12.0
    g = torch.Generator().manual_seed(13)
    v = torch.randn(1, 1, n, d, generator=g)
    q, k, v = q.half(), k.half(), v.half()
    vv = v.double().numpy()[0, 0]
    for causal in (False, True):
        want = np.empty((n, d))
        for i in range(n):
            vis = range(i + 1) if causal else range(n)
            w = np.array([math.exp(12.0) if j == 7 else 1.0 for j in vis])
            want[i] = (w[:, None] * vv[list(vis)]).sum(0) / w.sum()
        np.testing.assert_allclose(impl(q, k, v, causal, 1.0)[0, 0], want, atol=1e-6, rtol=1e-6)


def _check_scale_equivalence(impl):
    q, k, v = _qkv(1, 1, 50, 64, seed=14)
    # scale 2/sqrt(d) on q equals the default scale on 2q (doubling is exact in fp16).
    a = impl(q, k, v, False, 2.0 / math.sqrt(64))
    b = impl((q.float() * 2).half(), k, v, False, None)
    np.testing.assert_allclose(a, b, atol=1e-6, rtol=1e-6)


def _check_permutations(impl):
    q, k, v = _qkv(1, 1, 48, 64, seed=15)
    base = impl(q, k, v, False, None)
    perm = torch.randperm(48, generator=torch.Generator().manual_seed(16))
    kp, vp = k[:, :, perm].contiguous(), v[:, :, perm].contiguous()
    np.testing.assert_allclose(impl(q, kp, vp, False, None), base, atol=1e-6, rtol=1e-6)
    qp = q[:, :, perm].contiguous()
    np.testing.assert_allclose(impl(qp, k, v, False, None), base[:, :, perm.numpy()], atol=1e-6,
                               rtol=1e-6)


def _check_sdpa(impl):
    for causal in (False, True):
        q, k, v = _qkv(2, 2, 70, 64, seed=17)
        want = torch.nn.functional.scaled_dot_product_attention(
            q.double(), k.double(), v.double(), is_causal=causal).numpy()
        np.testing.assert_allclose(impl(q, k, v, causal, None), want, atol=1e-6, rtol=1e-6)


CHECKS = [_check_zero_query_is_mean, _check_causal_row0, _check_one_hot,
          _check_scale_equivalence, _check_permutations, _check_sdpa]


def _fp64(q, k, v, causal, scale):
    return orc.attention_fp64(q, k, v, causal=causal, scale=scale)


def _fp32(q, k, v, causal, scale):
    return orc.attention_fp32(q, k, v, causal=causal, scale=scale).double().numpy()


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__[7:])
@pytest.mark.parametrize("impl", [_fp64, _fp32], ids=["fp64", "fp32"])
def test_oracle_pinning(impl, check):
    check(impl)


def test_fp32_and_fp64_oracles_agree():
    for causal in (False, True):
        q, k, v = _qkv(2, 3, 129, 128, seed=18)
        np.testing.assert_allclose(_fp32(q, k, v, causal, None), _fp64(q, k, v, causal, None),
                                   atol=2e-6, rtol=1e-5)


def test_fp64_rows_match_full():
    q, k, v = _qkv(2, 2, 77, 64, seed=19)
    full = _fp64(q, k, v, True, None).reshape(4, 77, 64)
    rows = [0, 5, 76]
    np.testing.assert_array_equal(orc.attention_fp64_rows(q, k, v, True, 3, rows), full[3, rows])


def test_package_attention_reference_matches_oracle():
    """fa.attention_reference is public API (fa/reference.py:8-18 of the reference)."""
    for causal in (False, True):
        q, k, v = _qkv(2, 2, 65, 64, seed=20)
        got = fref.attention_reference(q, k, v, causal=causal)
        assert got.dtype == torch.float32
        np.testing.assert_allclose(got.double().numpy(), _fp64(q, k, v, causal, None),
                                   atol=2e-6, rtol=1e-5)


# ---- planted mistakes: each must be caught ----------------------------------------------------
def _mutant(kind):
    def impl(q, k, v, causal, scale):
        q32, k32, v32 = q.double(), k.double(), v.double()
        d, n = q.shape[-1], q.shape[-2]
        sc = 1.0 / math.sqrt(d) if scale is None else scale
        if kind == "no_sqrt":
            sc = 1.0 / d if scale is None else scale
        s = q32 @ k32.transpose(-2, -1) * sc
        if kind == "keys_as_queries":
            s = s.transpose(-2, -1)
        if causal:
            diag = 0 if kind == "diag_masked" else 1
            mask = torch.ones(n, n, dtype=torch.bool).triu(diag)
            if kind == "future_visible":
                mask = torch.ones(n, n, dtype=torch.bool).tril(-1)
            s = s.masked_fill(mask, float("-inf"))
        dim = -2 if kind == "softmax_wrong_dim" else -1
        p = torch.softmax(s, dim=dim)
        if kind == "no_max_shift_fp16":
            p = torch.exp(s.half().double())
            p = p / p.sum(-1, keepdim=True)
        return (p @ v32).numpy()

    return impl


@pytest.mark.parametrize("kind", ["no_sqrt", "keys_as_queries", "diag_masked", "future_visible",
                                  "softmax_wrong_dim"])
def test_planted_mistakes_are_caught(kind):
    impl = _mutant(kind)
    caught = []
    for check in CHECKS:
        try:
            with np.errstate(all="ignore"):
                check(impl)
        except AssertionError:
            caught.append(check.__name__)
    assert caught, f"mutant {kind} passed every pinning check"


def test_correct_mutant_baseline_passes():
    """The mutant harness itself, with no mistake planted, passes every check."""
    impl = _mutant("none")
    for check in CHECKS:
        check(impl)
