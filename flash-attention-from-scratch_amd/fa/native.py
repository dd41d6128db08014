"""ctypes view of the C ABI in include/fa_hip.h (libfa_hip.so next to this file).

Used by the tests and the benchmark to call the launcher without PyTorch types in between,
and by any caller that wants the raw entry points. Loading the library touches no GPU.
"""

from __future__ import annotations

import ctypes
from functools import lru_cache
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libfa_hip.so"

FA_OK, FA_EINVAL, FA_EHIP = 0, 1, 2
VARIANTS = {"baseline": 0, "opt": 1, "fp16acc": 2}


class FaParams(ctypes.Structure):
    """struct fa_params (include/fa_hip.h)."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("seqlen", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("causal", ctypes.c_uint8),
        ("variant", ctypes.c_uint8),
        ("reserved", ctypes.c_uint8 * 2),
    ]


class FaTileInfo(ctypes.Structure):
    """struct fa_tile_info (include/fa_hip.h)."""

    _fields_ = [
        ("block_q", ctypes.c_int32),
        ("block_k", ctypes.c_int32),
        ("waves", ctypes.c_int32),
        ("lds_bytes", ctypes.c_int32),
        ("schedule", ctypes.c_int32),
    ]


# fa_schedule (include/fa_hip.h): the main-loop schedule of a tile, by name.
SCHEDULES = {0: "simple", 3: "ksplit", 4: "pingpong16", 5: "ksplit4", 6: "simple16"}


class FaSplitKvInfo(ctypes.Structure):
    """struct fa_splitkv_info (include/fa_hip.h)."""

    _fields_ = [
        ("num_splits", ctypes.c_int32),
        ("tiles_per_split", ctypes.c_int32),
        ("block_q", ctypes.c_int32),
        ("block_k", ctypes.c_int32),
        ("workspace_bytes", ctypes.c_uint64),
        ("preferred", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


@lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(f"fa: {LIB_PATH} is not built (run flash-attention-from-scratch_amd/fa_build.py)")
    so = ctypes.CDLL(str(LIB_PATH))
    so.fa_flash_fwd.argtypes = [ctypes.POINTER(FaParams), ctypes.c_void_p]
    so.fa_flash_fwd.restype = ctypes.c_int
    so.fa_flash_fwd_lse.argtypes = [ctypes.POINTER(FaParams), ctypes.c_void_p, ctypes.c_void_p]
    so.fa_flash_fwd_lse.restype = ctypes.c_int
    so.fa_splitkv_plan.argtypes = [ctypes.POINTER(FaParams), ctypes.c_int32,
                                   ctypes.POINTER(FaSplitKvInfo)]
    so.fa_splitkv_plan.restype = ctypes.c_int
    so.fa_tail_plan.argtypes = [ctypes.POINTER(FaParams), ctypes.POINTER(ctypes.c_int64)]
    so.fa_tail_plan.restype = ctypes.c_int
    so.fa_flash_fwd_splitkv.argtypes = [ctypes.POINTER(FaParams), ctypes.c_void_p,
                                        ctypes.c_int32, ctypes.c_void_p, ctypes.c_uint64,
                                        ctypes.c_void_p]
    so.fa_flash_fwd_splitkv.restype = ctypes.c_int
    so.fa_flash_fwd_splitkv_static.argtypes = [ctypes.POINTER(FaParams), ctypes.c_void_p,
                                               ctypes.c_int32, ctypes.c_void_p]
    so.fa_flash_fwd_splitkv_static.restype = ctypes.c_int
    so.fa_last_error.argtypes = []
    so.fa_last_error.restype = ctypes.c_char_p
    so.fa_tile_config.argtypes = [ctypes.POINTER(FaParams), ctypes.POINTER(FaTileInfo)]
    so.fa_tile_config.restype = ctypes.c_int
    so.fa_version.argtypes = []
    so.fa_version.restype = ctypes.c_char_p
    return so


def make_params(q: int, k: int, v: int, o: int, batch: int, heads: int, seqlen: int,
                head_dim: int, softmax_scale: float, causal: bool, variant: str | int = "opt"
                ) -> FaParams:
    p = FaParams()
    p.q, p.k, p.v, p.o = q, k, v, o
    p.batch, p.heads, p.seqlen, p.head_dim = batch, heads, seqlen, head_dim
    p.softmax_scale = softmax_scale
    p.causal = 1 if causal else 0
    p.variant = VARIANTS[variant] if isinstance(variant, str) else int(variant)
    return p


def flash_fwd(params: FaParams, stream: int | None = None) -> tuple[int, str]:
    """Calls fa_flash_fwd; returns (status, fa_last_error())."""
    so = lib()
    rc = so.fa_flash_fwd(ctypes.byref(params), ctypes.c_void_p(stream or 0))
    return rc, so.fa_last_error().decode()


def flash_fwd_lse(params: FaParams, lse: int, stream: int | None = None) -> tuple[int, str]:
    """Calls fa_flash_fwd_lse (lse: device address of a [B, H, N] fp32 buffer)."""
    so = lib()
    rc = so.fa_flash_fwd_lse(ctypes.byref(params), ctypes.c_void_p(lse),
                             ctypes.c_void_p(stream or 0))
    return rc, so.fa_last_error().decode()


def splitkv_plan(params: FaParams, num_splits: int = 0) -> dict:
    """fa_splitkv_plan: key ranges and workspace size of a split-KV call."""
    so = lib()
    info = FaSplitKvInfo()
    rc = so.fa_splitkv_plan(ctypes.byref(params), num_splits, ctypes.byref(info))
    if rc != FA_OK:
        raise ValueError(so.fa_last_error().decode())
    return {f: getattr(info, f) for f, _ in FaSplitKvInfo._fields_}


def tail_plan(params: FaParams) -> int:
    """fa_tail_plan: heads of the single launch in a head split (0: no split)."""
    so = lib()
    heads = ctypes.c_int64()
    rc = so.fa_tail_plan(ctypes.byref(params), ctypes.byref(heads))
    if rc != FA_OK:
        raise ValueError(so.fa_last_error().decode())
    return heads.value


def flash_fwd_splitkv(params: FaParams, lse: int | None, num_splits: int, workspace: int,
                      workspace_bytes: int, stream: int | None = None) -> tuple[int, str]:
    """Calls fa_flash_fwd_splitkv; returns (status, fa_last_error())."""
    so = lib()
    rc = so.fa_flash_fwd_splitkv(ctypes.byref(params), ctypes.c_void_p(lse or 0), num_splits,
                                 ctypes.c_void_p(workspace), workspace_bytes,
                                 ctypes.c_void_p(stream or 0))
    return rc, so.fa_last_error().decode()


STATIC_SCRATCH_BYTES = 64 << 20  # FA_STATIC_SCRATCH_BYTES of include/fa_hip.h


def flash_fwd_splitkv_static(params: FaParams, lse: int | None, num_splits: int,
                             stream: int | None = None) -> tuple[int, str]:
    """Calls fa_flash_fwd_splitkv_static (the library's own static scratch as workspace)."""
    so = lib()
    rc = so.fa_flash_fwd_splitkv_static(ctypes.byref(params), ctypes.c_void_p(lse or 0),
                                        num_splits, ctypes.c_void_p(stream or 0))
    return rc, so.fa_last_error().decode()


def tile_config(head_dim: int, causal: bool, variant: str | int = "opt",
                seqlen: int = 16384, batch: int = 1, heads: int = 16) -> dict:
    """Tile fa_flash_fwd launches for these arguments (fa_tile_config)."""
    so = lib()
    info = FaTileInfo()
    p = make_params(0, 0, 0, 0, batch, heads, seqlen, head_dim, 1.0, causal, variant)
    rc = so.fa_tile_config(ctypes.byref(p), ctypes.byref(info))
    if rc != FA_OK:
        raise ValueError(so.fa_last_error().decode())
    return {"block_q": info.block_q, "block_k": info.block_k, "waves": info.waves,
            "lds_bytes": info.lds_bytes, "schedule": SCHEDULES[info.schedule]}


def version() -> str:
    return lib().fa_version().decode()
