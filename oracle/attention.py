"""TEST INFRASTRUCTURE ONLY -- the checker, never the product.

Only tests/, the smoke check of __graft_entry__.py and the CPU-baseline leg of bench.py may
import this module. The product path (fa.forward -> fa._C -> libfa_hip.so) never does.

Two CPU restatements of the reference's attention:

* attention_fp32: float32 exact attention, following fa/reference.py:8-18 of the reference
  (upcast to fp32, scores = q k^T * scale, strict upper triangle -> -inf when causal, softmax
  over the last dim, times v), computed one (batch, head) slice at a time so the N x N score
  matrix of the long configurations fits in host memory (the arithmetic per slice is
  unchanged). `scale` defaults to 1/sqrt(d) like the reference; a custom scale is the
  reference's own equivalence (tests/test_flash_fwd.py:97-103) made explicit.
* attention_fp64_rows: double precision per-row brute force in C (attention_fp64.c), following
  tests/cpp/test_flash_fwd.cu:115-152 and csrc/dev/main.cu:31-63, for selected rows of any size.
* lse_fp32 / lse_fp64_rows: the rows' log-sum-exp, log(sum_j exp(scale * q_i . k_j)) over the
  visible keys, which the library's forward_lse / split-KV paths return. The reference has no
  LSE output; these are pinned by closed forms in tests/test_oracle.py (q = 0 gives log of the
  visible-key count, causal row 0 gives its own score, duplicating every key adds log 2, a
  shift of all scores by c adds c) and by fp32/fp64 agreement.

Inputs are taken exactly as given (fp16 tensors are read bit-for-bit), on the CPU.
"""

from __future__ import annotations

import ctypes
import math
from functools import lru_cache
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
FP64_LIB = HERE / "liboracle_fp64.so"


def attention_fp32(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
                   scale: float | None = None) -> torch.Tensor:
    """Exact fp32 attention of [B, H, N, D] tensors, on the CPU; returns float32 [B, H, N, D]."""
    q, k, v = (t.detach().to("cpu") for t in (q, k, v))
    b, h, n, d = q.shape
    sc = (1.0 / math.sqrt(d)) if scale is None else float(scale)
    out = torch.empty(b, h, n, d, dtype=torch.float32)
    mask = torch.ones(n, n, dtype=torch.bool).triu(1) if causal else None
    for bi in range(b):
        for hi in range(h):
            q32, k32, v32 = q[bi, hi].float(), k[bi, hi].float(), v[bi, hi].float()
            s = (q32 @ k32.t()) * sc
            if mask is not None:
                s.masked_fill_(mask, float("-inf"))
            out[bi, hi] = torch.softmax(s, dim=-1) @ v32
    return out


def lse_fp32(q: torch.Tensor, k: torch.Tensor, causal: bool = False,
             scale: float | None = None) -> torch.Tensor:
    """Row log-sum-exp of the scaled scores of [B, H, N, D] tensors, fp32 [B, H, N], on the CPU,
    one (batch, head) slice at a time (same scores and mask as attention_fp32)."""
    q, k = (t.detach().to("cpu") for t in (q, k))
    b, h, n, d = q.shape
    sc = (1.0 / math.sqrt(d)) if scale is None else float(scale)
    out = torch.empty(b, h, n, dtype=torch.float32)
    mask = torch.ones(n, n, dtype=torch.bool).triu(1) if causal else None
    for bi in range(b):
        for hi in range(h):
            s = (q[bi, hi].float() @ k[bi, hi].float().t()) * sc
            if mask is not None:
                s.masked_fill_(mask, float("-inf"))
            out[bi, hi] = torch.logsumexp(s, dim=-1)
    return out


@lru_cache(maxsize=1)
def _fp64_lib() -> ctypes.CDLL:
    if not FP64_LIB.exists():
        raise ImportError(f"oracle: {FP64_LIB} is not built (flash-attention-from-scratch_amd/fa_build.py)")
    so = ctypes.CDLL(str(FP64_LIB))
    so.oracle_attention_rows.argtypes = [
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
        ctypes.c_int64, ctypes.c_double, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
        ctypes.c_void_p,
    ]
    so.oracle_attention_rows.restype = ctypes.c_int
    so.oracle_lse_rows.argtypes = [
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
        ctypes.c_double, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
    ]
    so.oracle_lse_rows.restype = ctypes.c_int
    so.oracle_half_to_double.argtypes = [ctypes.c_uint16]
    so.oracle_half_to_double.restype = ctypes.c_double
    return so


def half_to_double(bits: int) -> float:
    return _fp64_lib().oracle_half_to_double(bits)


def attention_fp64_rows(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool,
                        bh: int, rows, scale: float | None = None) -> np.ndarray:
    """fp64 attention rows `rows` of flattened head `bh` of fp16 [B, H, N, D] tensors.

    Returns a float64 array [len(rows), D].
    """
    if q.dtype != torch.float16:
        raise TypeError("attention_fp64_rows takes the fp16 tensors the kernel sees")
    b, h, n, d = q.shape
    sc = (1.0 / math.sqrt(d)) if scale is None else float(scale)
    qn, kn, vn = (np.ascontiguousarray(t.detach().cpu().reshape(b * h, n, d).numpy().view(np.uint16))
                  for t in (q, k, v))
    rows_a = np.ascontiguousarray(np.asarray(rows, dtype=np.int64))
    out = np.empty((len(rows_a), d), dtype=np.float64)
    rc = _fp64_lib().oracle_attention_rows(
        qn.ctypes.data, kn.ctypes.data, vn.ctypes.data, int(bh), n, d, sc, int(bool(causal)),
        rows_a.ctypes.data, len(rows_a), out.ctypes.data)
    if rc != 0:
        raise ValueError("oracle_attention_rows: bad arguments")
    return out


def attention_fp64(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = False,
                   scale: float | None = None) -> np.ndarray:
    """fp64 attention of every row (small shapes): float64 [B, H, N, D]."""
    b, h, n, d = q.shape
    out = np.empty((b * h, n, d), dtype=np.float64)
    for bh in range(b * h):
        out[bh] = attention_fp64_rows(q, k, v, causal, bh, range(n), scale)
    return out.reshape(b, h, n, d)


def lse_fp64_rows(q: torch.Tensor, k: torch.Tensor, causal: bool, bh: int, rows,
                  scale: float | None = None) -> np.ndarray:
    """fp64 log-sum-exp of rows `rows` of flattened head `bh` of fp16 [B, H, N, D] tensors."""
    if q.dtype != torch.float16:
        raise TypeError("lse_fp64_rows takes the fp16 tensors the kernel sees")
    b, h, n, d = q.shape
    sc = (1.0 / math.sqrt(d)) if scale is None else float(scale)
    qn, kn = (np.ascontiguousarray(t.detach().cpu().reshape(b * h, n, d).numpy().view(np.uint16))
              for t in (q, k))
    rows_a = np.ascontiguousarray(np.asarray(rows, dtype=np.int64))
    out = np.empty(len(rows_a), dtype=np.float64)
    rc = _fp64_lib().oracle_lse_rows(qn.ctypes.data, kn.ctypes.data, int(bh), n, d, sc,
                                     int(bool(causal)), rows_a.ctypes.data, len(rows_a),
                                     out.ctypes.data)
    if rc != 0:
        raise ValueError("oracle_lse_rows: bad arguments")
    return out
