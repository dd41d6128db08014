"""GPU: one-wave checks of the gfx950 instructions the kernel is built from
(tests/blocks/fa_blocks.hip). Counterpart of the reference's tests/cpp/test_ptx.cu
(mma layout :93-167 with exact integer-valued products, ldmatrix :173-250, cp.async :318-352,
exp2 accuracy :357-424). Products of small integers are exact in fp32, so layouts are checked
bit for bit.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent / "blocks" / "libfa_blocks.so"


@pytest.fixture(scope="module")
def blk():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    torch.cuda.init()
    return ctypes.CDLL(str(LIB))


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def _ok(rc):
    assert rc == 0, f"hip error {rc}"


def test_tr16_lane_mapping(blk):
    """ds_read_b64_tr_b16 transposes 4 x 16 blocks within each 16-lane group."""
    out = np.zeros(256, dtype=np.uint16)
    _ok(blk.fab_tr16_probe(_ptr(out)))
    got = out.view(np.float16).astype(np.int64).reshape(64, 4)
    want = np.array([[64 * (l // 16) + 16 * i + (l % 16) for i in range(4)] for l in range(64)])
    print("tr16 mapping (lane: elements):", {l: got[l].tolist() for l in range(0, 64, 5)})
    np.testing.assert_array_equal(got, want)


def test_tr16_block_addressing(blk):
    """The kernel's addressing (fa::geom::tr16_row/col) delivers column l%16 of a 4-row block."""
    tile = (np.arange(16 * 64) % 2039).astype(np.float16)
    out = np.zeros(256, dtype=np.uint16)
    _ok(blk.fab_tr16_block(_ptr(tile.view(np.uint16)), _ptr(out)))
    got = out.view(np.float16).reshape(64, 4)
    t = tile.reshape(16, 64)
    want = np.array([[t[4 * (l // 16) + e, 16 * (l // 16) + l % 16] for e in range(4)]
                     for l in range(64)])
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("shape", [(32, 16, 32), (16, 32, 16)])
def test_mfma_layout_exact(blk, shape):
    m, kdim, n = shape
    rng = np.random.default_rng(3)
    a = rng.integers(-8, 9, size=(m, kdim)).astype(np.float16)
    b = rng.integers(-8, 9, size=(kdim, n)).astype(np.float16)
    c = np.zeros((m, n), dtype=np.float32)
    fn = blk.fab_mfma32 if m == 32 else blk.fab_mfma16
    _ok(fn(_ptr(a.view(np.uint16)), _ptr(b.view(np.uint16)), _ptr(c)))
    np.testing.assert_array_equal(c, a.astype(np.float32) @ b.astype(np.float32))


@pytest.mark.parametrize("dist", [32, 16])
def test_permlane_pair_reductions(blk, dist):
    """max/sum with lane ^ 32 (v_permlane32_swap) and lane ^ 16 (v_permlane16_swap)."""
    x = np.random.default_rng(4).standard_normal(64).astype(np.float32)
    mx = np.zeros(64, np.float32)
    sm = np.zeros(64, np.float32)
    fn = blk.fab_xor32 if dist == 32 else blk.fab_xor16
    _ok(fn(_ptr(x), _ptr(mx), _ptr(sm)))
    partner = x[np.arange(64) ^ dist]
    np.testing.assert_array_equal(mx, np.maximum(x, partner))
    np.testing.assert_array_equal(sm, x + partner)


def test_exp2_accuracy_and_specials(blk):
    x = np.concatenate([np.linspace(-30, 0, 4000), np.linspace(0, 10, 1000),
                        np.arange(-20, 11)]).astype(np.float32)
    y = np.zeros_like(x)
    _ok(blk.fab_exp2(_ptr(x), _ptr(y), ctypes.c_int(x.size)))
    want = np.exp2(x.astype(np.float64))
    rel = np.abs(y - want) / want
    assert rel.max() < 4e-7, rel.max()  # a few ulp of fp32
    ints = x[-31:]
    np.testing.assert_array_equal(y[-31:], np.exp2(ints))  # powers of two are exact
    sp = np.array([-np.inf, 0.0, -200.0, -126.0], dtype=np.float32)
    ys = np.zeros_like(sp)
    _ok(blk.fab_exp2(_ptr(sp), _ptr(ys), ctypes.c_int(sp.size)))
    assert ys[0] == 0.0  # masked scores (-inf) contribute exactly nothing
    assert ys[1] == 1.0
    assert 0.0 <= ys[2] < 1e-38
    assert abs(ys[3] - 2.0**-126) <= 2.0**-149 * 4


def test_pack8_rounds_to_nearest_even(blk):
    rng = np.random.default_rng(5)
    x = np.concatenate([
        rng.standard_normal(4096) * 4,
        rng.uniform(0, 1, 4096),
        # exact halfway points between adjacent fp16 values in [1, 2): ties to even
        1.0 + (np.arange(512) * 2 + 1) * 2.0**-11,
        [65504.0, 65519.0, 65520.0, 1e6, -1e6, 6e-8, 0.0, -0.0],
    ]).astype(np.float32)
    x = x[: (x.size // 8) * 8]
    y = np.zeros(x.size, dtype=np.uint16)
    _ok(blk.fab_pack8(_ptr(x), _ptr(y), ctypes.c_int(x.size)))
    np.testing.assert_array_equal(y, x.astype(np.float16).view(np.uint16))


def test_lds_dma_slot_per_lane(blk):
    src = np.arange(512, dtype=np.uint16)
    perm = np.random.default_rng(6).permutation(64).astype(np.int32)
    out = np.zeros(512, dtype=np.uint16)
    _ok(blk.fab_lds_dma(_ptr(src), _ptr(perm), _ptr(out)))
    want = src.reshape(64, 8)[perm].reshape(-1)
    np.testing.assert_array_equal(out, want)


def test_buffer_lds_dma_zero_fills_out_of_range(blk):
    """Lanes whose 16-byte chunk lies at or past the resource size write zeros to LDS (the
    kernel relies on this for K/V rows >= N); in-range lanes copy their chunk. Offsets up to
    2 KiB past a 1 KiB source stay inside the range check, so nothing is read out of bounds."""
    src = (np.arange(512) + 1).astype(np.uint16)
    perm = np.random.default_rng(7).permutation(64).astype(np.int32)
    chunks = np.where(np.arange(64) % 3 == 0, perm + 64, perm).astype(np.int32)  # some >= 64
    for nbytes in (1024, 512, 0):
        out = np.zeros(512, dtype=np.uint16)
        _ok(blk.fab_lds_dma_buf(_ptr(src), _ptr(chunks), ctypes.c_int(nbytes), _ptr(out)))
        got = out.reshape(64, 8)
        for lane in range(64):
            c = chunks[lane]
            want = src.reshape(64, 8)[c] if 16 * c + 16 <= nbytes else np.zeros(8, np.uint16)
            np.testing.assert_array_equal(got[lane], want, err_msg=f"lane {lane} bytes {nbytes}")


def test_sum8_f16_accumulates_in_fp32(blk):
    rng = np.random.default_rng(8)
    x = rng.uniform(0, 256, size=(1000, 8)).astype(np.float16)
    y = np.zeros(1000, dtype=np.float32)
    _ok(blk.fab_sum8(_ptr(x.view(np.uint16)), _ptr(y), ctypes.c_int(1000)))
    want = x.astype(np.float64).sum(axis=1)
    np.testing.assert_allclose(y, want, rtol=2e-7 * 8, atol=0)


@pytest.mark.parametrize("dist", [16, 32])
def test_pair_swap_lane_layout(blk, dist):
    """pair_swap16 / pair_swap32: lane l of the lower row of each pair (l % (2 dist) < dist)
    gets {a[l], a[l + dist]}, lane l of the upper row {b[l - dist], b[l]} -- the exchange that
    lets each lane of a pair store 8 consecutive output features with one 16-byte store."""
    vals = np.arange(512, dtype=np.float16)          # lane l: a = 8l .. 8l+3, b = 8l+4 .. 8l+7
    out = np.zeros(512, dtype=np.uint16)
    _ok(blk.fab_pair_swap(_ptr(vals.view(np.uint16)), _ptr(out), dist))
    got = out.view(np.float16).astype(np.int64).reshape(64, 8)
    a = np.arange(512).reshape(64, 8)[:, :4]
    b = np.arange(512).reshape(64, 8)[:, 4:]
    want = np.zeros((64, 8), dtype=np.int64)
    for lane in range(64):
        p = lane ^ dist
        if lane % (2 * dist) < dist:
            want[lane] = np.concatenate([a[lane], a[p]])
        else:
            want[lane] = np.concatenate([b[p], b[lane]])
    np.testing.assert_array_equal(got, want)
