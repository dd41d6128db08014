"""FlashAttention-2 forward for AMD MI355X (gfx950), written from scratch in HIP.

    import fa
    o = fa.forward(q, k, v, causal=False)     # q, k, v: [B, H, N, D] fp16 on a ROCm GPU, D in {64, 128}
    o = fa.forward(q, k, v, fp16_accum=True)  # accepted; same kernel on CDNA4 (see forward)

Same Python surface as the reference package (fa/__init__.py:14-38 of
aligoldenhat/flash-attention-from-scratch): `forward`, `forward_variant` and
`attention_reference`. The work is done by hand-written HIP kernels in libfa_hip.so, reached
through the PyTorch-ROCm extension `fa._C` and the C ABI of include/fa_hip.h. There is no
fallback path: importing this package fails if the native extension is not built.
"""

from __future__ import annotations

import torch

try:
    from fa import _C
except ImportError as exc:  # pragma: no cover - exercised only on a broken install
    raise ImportError(
        "fa: the native extension fa._C (and libfa_hip.so) is not built; run "
        "`python flash-attention-from-scratch_amd/fa_build.py` (or __graft_entry__.build())"
    ) from exc

from fa.reference import attention_naive_fp16, attention_reference


def forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    softmax_scale: float | None = None,
    fp16_accum: bool = False,
) -> torch.Tensor:
    """O = softmax(Q K^T * scale) V, scale defaulting to 1/sqrt(D).

    Follows fa/__init__.py:14-28 of the reference. fp16_accum selects the "fp16acc" kernel
    build, as in the reference. On CDNA4 the fp16 MFMA accumulates in fp32 and has no faster
    fp16-accumulate form, so that build is the fp32-accumulate kernel: it gives no speed-up
    and its output is bitwise identical to the default.
    """
    variant = "fp16acc" if fp16_accum else "opt"
    return _C.forward(q, k, v, causal, softmax_scale, variant)


def forward_variant(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False, variant: str = "opt"
) -> torch.Tensor:
    """Run a specific kernel build: 'baseline', 'opt' or 'fp16acc' (fa/__init__.py:31-35)."""
    return _C.forward(q, k, v, causal, None, variant)


def forward_lse(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    softmax_scale: float | None = None,
    variant: str = "opt",
) -> tuple[torch.Tensor, torch.Tensor]:
    """(O, LSE): O as `forward`, bitwise, and LSE[b, h, i] = log(sum_j exp(scale * q_i . k_j))
    over the keys row i sees, fp32 [B, H, N]. Not in the reference package; the LSE is what
    merging partial attention results (split-KV, context parallelism) needs."""
    return _C.forward_lse(q, k, v, causal, softmax_scale, variant)


def forward_splitkv(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    softmax_scale: float | None = None,
    num_splits: int = 0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(O, LSE) computed split-KV: every query block's keys are cut into ranges processed by
    separate workgroups and merged by their LSEs. For grids too small to fill the GPU (few
    heads, long sequences). num_splits = 0 picks the ranges automatically. Matches `forward`
    within fp32 rounding of the merge. Not in the reference package."""
    return _C.forward_splitkv(q, k, v, causal, softmax_scale, num_splits)


__all__ = ["forward", "forward_variant", "forward_lse", "forward_splitkv", "attention_reference",
           "attention_naive_fp16"]
