"""Plain-PyTorch attention that the package exports for users (fa.attention_reference).

Same names and semantics as the reference package's fa/reference.py:8-30. These are part of
the public surface, not the kernel's test oracle (that lives in oracle/ and is only used by
tests and the benchmark's CPU baseline); fa.forward never calls them.
"""

from __future__ import annotations

import math

import torch


def _scores(q: torch.Tensor, k: torch.Tensor, causal: bool) -> torch.Tensor:
    n_q, n_k = q.shape[-2], k.shape[-2]
    s = torch.matmul(q, k.transpose(-2, -1).contiguous()) / math.sqrt(q.shape[-1])
    if causal:
        keep = torch.ones(n_q, n_k, dtype=torch.bool, device=q.device).tril()
        s = s.masked_fill(~keep, float("-inf"))
    return s


def attention_reference(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False
) -> torch.Tensor:
    """Exact attention in float32: softmax(q k^T / sqrt(D)) v, returned as float32.

    Key j is visible to query i iff j <= i when causal (fa/reference.py:8-18).
    """
    p = torch.softmax(_scores(q.float(), k.float(), causal), dim=-1)
    return torch.matmul(p, v.float())


def attention_naive_fp16(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False
) -> torch.Tensor:
    """What a straightforward user writes: the N x N matrix materialized in the input dtype
    (fa/reference.py:21-30); a benchmark baseline only."""
    return torch.matmul(torch.softmax(_scores(q, k, causal), dim=-1), v)
