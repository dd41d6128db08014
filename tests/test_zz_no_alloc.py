"""fa_flash_fwd_splitkv_static: the split-KV forward with the library's static scratch as its
workspace, for callers that cannot allocate device memory.

GPU: two calls in a row through the C ABI, the second on a smaller input (the scratch still
holds the first call's partial results), each bitwise equal to fa_flash_fwd_splitkv with a
caller workspace on the same input and plan (O and LSE); then the first shape again.
CPU: a plan larger than the scratch, and bad arguments, are rejected before any HIP call.
"""

from __future__ import annotations

import pytest
import torch

from fa import native

GOOD = dict(q=0x1000, k=0x2000, v=0x3000, o=0x4000, batch=1, heads=2, seqlen=16384,
            head_dim=128, softmax_scale=0.125, causal=False, variant="opt")


def test_oversized_plan_is_rejected_before_any_launch():
    p = native.make_params(**{**GOOD, "causal": True})
    need = native.splitkv_plan(p, 0)["workspace_bytes"]
    assert need > native.STATIC_SCRATCH_BYTES      # 8 ranges x 2 heads x 16k rows x 129 x 4 B
    rc, msg = native.flash_fwd_splitkv_static(p, None, 0)
    assert rc == native.FA_EINVAL
    assert f"needs {need} bytes" in msg and str(native.STATIC_SCRATCH_BYTES) in msg
    # the same shape with fewer ranges fits
    assert native.splitkv_plan(p, 3)["workspace_bytes"] <= native.STATIC_SCRATCH_BYTES


@pytest.mark.parametrize("over, words", [
    (dict(batch=0), "batch, heads and seqlen must be positive"),
    (dict(head_dim=96), "head_dim must be 64 or 128, got 96"),
    (dict(q=0), "non-null"),
])
def test_bad_arguments_are_rejected(over, words):
    rc, msg = native.flash_fwd_splitkv_static(native.make_params(**{**GOOD, **over}), None, 0)
    assert rc == native.FA_EINVAL and words in msg
    rc, msg = native.flash_fwd_splitkv_static(native.make_params(**GOOD), None, -1)
    assert rc == native.FA_EINVAL and "num_splits" in msg
    rc, msg = native.flash_fwd_splitkv_static(native.make_params(**GOOD), 0x1001, 0)
    assert rc == native.FA_EINVAL and "4-byte aligned" in msg


def _run_both(b, h, n, d, causal, splits, seed):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(b, h, n, d, generator=g).half().cuda() for _ in range(3))
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for static in (False, True):
        o = torch.full_like(q, float("nan"))
        lse = torch.full((b, h, n), float("nan"), device="cuda")
        p = native.make_params(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), b, h, n,
                               d, d ** -0.5, causal, "opt")
        if static:
            rc, msg = native.flash_fwd_splitkv_static(p, lse.data_ptr(), splits, stream)
        else:
            plan = native.splitkv_plan(p, splits)
            assert plan["workspace_bytes"] <= native.STATIC_SCRATCH_BYTES
            ws = torch.empty(plan["workspace_bytes"] // 4, device="cuda")
            rc, msg = native.flash_fwd_splitkv(p, lse.data_ptr(), splits, ws.data_ptr(),
                                               plan["workspace_bytes"], stream)
        assert rc == native.FA_OK, msg
        torch.cuda.synchronize()
        outs.append((o, lse))
    (o_ws, lse_ws), (o_st, lse_st) = outs
    assert torch.isfinite(o_st).all() and torch.isfinite(lse_st).all()
    assert torch.equal(o_st, o_ws) and torch.equal(lse_st, lse_ws)


@pytest.mark.gpu
def test_static_scratch_matches_caller_workspace_on_consecutive_calls():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    # 1) one GPU's share of the headline shape split 8 ways by heads: 2 ranges, 32 MiB
    print("case static 1x2x16384 d128 non-causal", flush=True)
    _run_both(1, 2, 16384, 128, False, 0, seed=1)
    # 2) a smaller input right after it: the scratch still holds call 1's partial results
    print("case static 1x1x3001 d128 causal", flush=True)
    _run_both(1, 1, 3001, 128, True, 0, seed=2)
    print("case static 2x3x1000 d64 causal, 3 ranges", flush=True)
    _run_both(2, 3, 1000, 64, True, 3, seed=3)
    # 3) the first shape again, causal with a plan that fits
    print("case static 1x2x16384 d128 causal, 3 ranges", flush=True)
    _run_both(1, 2, 16384, 128, True, 3, seed=4)
