"""CPU: the kernel's integer tile geometry (csrc/fa_geometry.h), through a g++ build of the
same header. Counterpart of the reference's host-side swizzle checks
(tests/cpp/test_ptx.cu:256-313: permutation and bank-conflict freedom), re-targeted to the
gfx950 access patterns, plus the tile-count, mask and work-map arithmetic
(csrc/kernels/flash_fwd.cu:183-194, 502-505).

LDS bank model used here, measured on MI355X with a saturating microbenchmark of
ds_read_b128 / ds_read_b64_tr_b16 over fixed lane-offset patterns (the patterns and their
measured outcome are the table MEASURED below): 64 banks of 4 bytes (bank = byte_offset / 4
mod 64); a ds_read_b128 is served 16 lanes at a time, a ds_read_b64_tr_b16 32 lanes at a time;
a group is conflict-free when no bank is hit at two different addresses.
"""

from __future__ import annotations

import ctypes
import itertools
from pathlib import Path

import pytest

LIB = Path(__file__).resolve().parent / "geometry" / "libfa_geom.so"


@pytest.fixture(scope="module")
def geo():
    so = ctypes.CDLL(str(LIB))
    so.geom_work_of.argtypes = [ctypes.c_int] * 4 + [ctypes.POINTER(ctypes.c_int)] * 2
    so.geom_work_of_xcd.argtypes = [ctypes.c_int] * 4 + [ctypes.POINTER(ctypes.c_int)] * 2
    so.geom_work_of_xcd_grouped.argtypes = [ctypes.c_int] * 4 + [ctypes.POINTER(ctypes.c_int)] * 2
    so.geom_causal_group_heads.argtypes = [ctypes.c_int, ctypes.c_longlong]
    so.geom_split_range.argtypes = [ctypes.c_int] * 3 + [ctypes.POINTER(ctypes.c_int)] * 2
    so.geom_causal_pair.argtypes = [ctypes.c_int] * 3 + [ctypes.POINTER(ctypes.c_int)] * 3
    so.geom_causal_pairs_pay.argtypes = [ctypes.c_longlong, ctypes.c_int, ctypes.c_int]
    so.geom_causal_singles_makespan.argtypes = [ctypes.c_longlong, ctypes.c_int, ctypes.c_int]
    so.geom_causal_singles_makespan.restype = ctypes.c_longlong
    return so


def _banks(byte_off, nbytes):
    return [((byte_off + 4 * w) // 4) % 64 for w in range(nbytes // 4)]


def _conflict_free(offsets, nbytes, group):
    """True when every `group`-lane group hits each bank at no more than one address."""
    for g0 in range(0, len(offsets), group):
        seen = {}
        for o in offsets[g0:g0 + group]:
            for w in range(nbytes // 4):
                addr = o + 4 * w
                bank = (addr // 4) % 64
                if seen.setdefault(bank, addr) != addr:
                    return False
    return True


def _k_offsets(geo, d, nb=0, kk=0):
    rb = 2 * d
    return [geo.geom_tile_offset(32 * nb + (l % 32), 2 * kk + l // 32, rb) for l in range(64)]


# Patterns timed on MI355X (16 waves of one workgroup, 8 reads in flight each): True = ran at
# the conflict-free rate (same time as a contiguous read), False = measurably slower.
MEASURED_B128 = {
    "contiguous": ([16 * l for l in range(64)], True),
    "broadcast": ([0] * 64, True),
    "stride256": ([256 * l for l in range(32)] * 2, False),
    "16x16B per 256B row": ([16 * (l % 16) + 256 * (l // 16) for l in range(64)], True),
    "8x16B per 256B row": ([16 * (l % 8) + 256 * (l // 8) for l in range(64)], False),
    "8x16B per 128B row": ([16 * (l % 8) + 128 * (l // 8) for l in range(64)], True),
    "d128 rows, no swizzle": ([256 * (l % 32) + 16 * (l // 32) for l in range(64)], False),
    "d128 rows, 3-bit row xor": ([256 * (l % 32) + 16 * ((l // 32) ^ (((l % 32) & 3) << 1 | ((l % 32) >> 2) & 1)) for l in range(64)], False),
    "d64 rows, no swizzle": ([128 * (l % 32) + 16 * (l // 32) for l in range(64)], False),
}
MEASURED_TR = {
    "contiguous": ([8 * l for l in range(64)], True),
    "32x8B per 256B": ([8 * (l % 32) + 512 * (l // 32) for l in range(64)], True),
    "16x8B per 256B row": ([8 * (l % 16) + 256 * (l // 16) for l in range(64)], False),
}


@pytest.mark.parametrize("name", sorted(MEASURED_B128))
def test_bank_model_matches_measured_b128(name):
    offs, free = MEASURED_B128[name]
    assert _conflict_free(offs, 16, 16) == free


@pytest.mark.parametrize("name", sorted(MEASURED_TR))
def test_bank_model_matches_measured_tr(name):
    offs, free = MEASURED_TR[name]
    assert _conflict_free(offs, 8, 32) == free


@pytest.mark.parametrize("d", [64, 128])
def test_swizzle_is_a_permutation_of_each_row(geo, d):
    cpr = d // 8
    for row in range(256):
        phys = [geo.geom_swizzle_chunk(row, c, 2 * d) for c in range(cpr)]
        assert sorted(phys) == list(range(cpr))
        assert all(geo.geom_swizzle_chunk(row, p, 2 * d) == c for c, p in enumerate(phys))


@pytest.mark.parametrize("d", [64, 128])
def test_k_fragment_reads_are_conflict_free(geo, d):
    """ds_read_b128 of the S^T A operand: lane l reads row 32*nb + l%32, chunk 2*kk + l//32."""
    for nb, kk in itertools.product(range(4), range(d // 16)):
        offs = _k_offsets(geo, d, nb, kk)
        assert _conflict_free(offs, 16, 16), (nb, kk)
        for g0 in range(0, 64, 16):  # and each group spreads over all 64 banks
            banks = sum((_banks(o, 16) for o in offs[g0:g0 + 16]), [])
            assert sorted(banks) == list(range(64)), (nb, kk, g0)


def _v_read_offsets(geo, d, nb, h, db, e):
    """Byte offsets the kernel's V^T transposed reads use (flash_fwd.hip, O^T += V^T P^T)."""
    rb = 2 * d
    out = []
    for l in range(64):
        hi = l >> 5
        row = 32 * nb + 16 * h + 8 * e + 4 * hi + geo.geom_tr16_row(l)
        colh = 32 * db + 16 * ((l >> 4) & 1) + geo.geom_tr16_col(l)
        out.append(geo.geom_tile_offset(row, colh // 8, rb) + 2 * (colh % 8))
        # the kernel adds the 16-row multiples as immediates to an offset computed at row % 16
        local = geo.geom_tile_offset(row % 16, colh // 8, rb) + 2 * (colh % 8)
        assert out[-1] == local + (row - row % 16) * rb
    return out


def _tr16_received(offs, g0):
    """Byte addresses whose halves lane g0 + j receives (element i = 0..3) from one
    ds_read_b64_tr_b16 of the 16-lane group g0..g0+15, lane m having addressed the 4 halves at
    offs[m]: element i of lane j is half j % 4 of lane 4i + j // 4's address. This is the
    instruction's lane semantic as measured on MI355X (tests/test_blocks.py::
    test_tr16_lane_mapping: with lane m addressing halves 4m..4m+3 of a counting tile, lane j
    receives 16i + j)."""
    return [[offs[g0 + 4 * i + j // 4] + 2 * (j % 4) for i in range(4)] for j in range(16)]


def test_tr16_model_reproduces_the_gpu_probe():
    """_tr16_received on the probe's addressing (lane m of the wave: halves 4m..4m+3 of a
    counting tile) gives what tests/test_blocks.py::test_tr16_lane_mapping measures on the GPU:
    lane l receives 64 (l // 16) + 16 i + l % 16."""
    offs = [8 * m for m in range(64)]
    for g0 in range(0, 64, 16):
        for j, addrs in enumerate(_tr16_received(offs, g0)):
            l = g0 + j
            assert [a // 2 for a in addrs] == [64 * (l // 16) + 16 * i + l % 16 for i in range(4)]


def _logical(geo, addr, rb, m16=False, d=None):
    """(row, half column) of the logical tile element stored at byte `addr`."""
    row, phys = addr // rb, (addr % rb) // 16
    chunk = geo.geom_swizzle_chunk_m16(row, phys, d) if m16 else geo.geom_swizzle_chunk(row, phys, rb)
    return row, 8 * chunk + (addr % 16) // 2


@pytest.mark.parametrize("d", [64, 128])
def test_v_transposed_reads_are_conflict_free(geo, d):
    for nb, h, db, e in itertools.product(range(2), range(2), range(d // 32), range(2)):
        offs = _v_read_offsets(geo, d, nb, h, db, e)
        assert _conflict_free(offs, 8, 32), (nb, h, db, e)
        for g0 in range(0, 64, 32):
            banks = sum((_banks(o, 8) for o in offs[g0:g0 + 32]), [])
            assert sorted(banks) == list(range(64)), (nb, h, db, e, g0)


@pytest.mark.parametrize("d", [64, 128])
def test_v_transposed_reads_deliver_the_pv_keys(geo, d):
    """Each 16-lane group addresses a 4-row x 16-column block whose transpose gives lane l the
    keys pv_key(l, 4e + i) (i = 0..3) of feature column 32*db + l%32."""
    rb = 2 * d
    for nb, h, db, e in itertools.product(range(2), range(2), range(d // 32), range(2)):
        offs = _v_read_offsets(geo, d, nb, h, db, e)
        for g0 in range(0, 64, 16):
            # logical (row, col) of what each lane of the group addresses
            cells = []
            for l in range(g0, g0 + 16):
                row = offs[l] // rb
                phys_chunk = (offs[l] % rb) // 16
                colh = 8 * geo.geom_swizzle_chunk(row, phys_chunk, rb) + (offs[l] % 16) // 2
                cells.append((row, colh))
            rows = sorted({r for r, _ in cells})
            assert len(rows) == 4 and rows == list(range(rows[0], rows[0] + 4))
            cols = sorted({c + j for _, c in cells for j in range(4)})
            assert cols == list(range(cols[0], cols[0] + 16))
            # what each lane receives, through the instruction's lane semantic
            for j, addrs in enumerate(_tr16_received(offs, g0)):
                lane = g0 + j
                for i, addr in enumerate(addrs):
                    assert _logical(geo, addr, rb) == (
                        32 * nb + 16 * h + geo.geom_pv_key(lane, 4 * e + i), 32 * db + lane % 32)


@pytest.mark.parametrize("d", [64, 128])
def test_k_fragment_immediates(geo, d):
    """The kernel reads K fragment (nb, kk) at koff[kk] + 32*nb*row_bytes."""
    rb = 2 * d
    for nb, kk, l in itertools.product(range(4), range(d // 16), range(64)):
        assert geo.geom_tile_offset(32 * nb + l % 32, 2 * kk + l // 32, rb) == \
            geo.geom_tile_offset(l % 32, 2 * kk + l // 32, rb) + 32 * nb * rb


def test_p_operand_slots_are_the_score_accumulators(geo):
    for lane, nb, h, i in itertools.product(range(64), range(4), range(2), range(8)):
        assert geo.geom_st_key(lane, nb, 8 * h + i) == 32 * nb + 16 * h + geo.geom_pv_key(lane, i)


# ---- the 16x16x32 layout (flash_fwd_pingpong16: d = 128 with 32-key tiles, d = 64 with 64) --

M16 = {128: dict(bc=32, kb=2, dc=4, db=8, ks=1), 64: dict(bc=64, kb=4, dc=2, db=4, ks=2)}


def test_m16_key_blocks_split_the_tile(geo):
    """Key block kb holds rows 32(kb/2) + 8(kb%2) + {0..7, 16..23}: its 16 rows lie in both
    16-row halves of its 32-key group."""
    for kb in range(4):
        base = 32 * (kb // 2) + 8 * (kb % 2)
        rows = [geo.geom_m16_key(kb, i) for i in range(16)]
        assert rows == [base + r for r in range(8)] + [base + 16 + r for r in range(8)]
    for d, c in M16.items():
        assert sorted(geo.geom_m16_key(kb, i) for kb in range(c["kb"]) for i in range(16)) == \
            list(range(c["bc"]))


@pytest.mark.parametrize("d", [64, 128])
def test_m16_swizzle_is_a_permutation_of_each_row(geo, d):
    cpr = d // 8
    for row in range(256):
        phys = [geo.geom_swizzle_chunk_m16(row, c, d) for c in range(cpr)]
        assert sorted(phys) == list(range(cpr))
        assert all(geo.geom_swizzle_chunk_m16(row, p, d) == c for c, p in enumerate(phys))
        # +8 rows inside a key block's half, and +32 rows (next key group), keep the xor
        assert geo.geom_row_xor_m16(row + 32, d) == geo.geom_row_xor_m16(row, d)
        if row % 16 < 8:
            assert geo.geom_row_xor_m16(row + 8, d) == geo.geom_row_xor_m16(row, d)


@pytest.mark.parametrize("d", [64, 128])
def test_m16_k_tile_layout_is_a_permutation(geo, d):
    bc, cpr = M16[d]["bc"], d // 8
    cells = [(geo.geom_m16_kslot_row(s, d), geo.geom_m16_kslot_chunk(s, d)) for s in range(bc * cpr)]
    assert sorted(cells) == [(r, c) for r in range(bc) for c in range(cpr)]


@pytest.mark.parametrize("d", [64, 128])
def test_m16_k_reads_use_the_32x32_addresses_and_get_the_operand(geo, d):
    """The K operand of MFMA step (kb, dc) is read at the 32x32x16 path's fragment addresses
    (nb = kb/2, kk = (kb%2)*DC + dc; conflict-free, test_k_fragment_reads_are_conflict_free),
    and lane l gets key row m16_key(kb, l%16), chunk m16_kchunk(dc, l//16)."""
    c = M16[d]
    for kb, dc in itertools.product(range(c["kb"]), range(c["dc"])):
        offs = _k_offsets(geo, d, kb // 2, (kb % 2) * c["dc"] + dc)
        for l, o in enumerate(offs):
            assert o % 16 == 0
            slot = o // 16
            assert geo.geom_m16_kslot_row(slot, d) == geo.geom_m16_key(kb, l % 16), (kb, dc, l)
            assert geo.geom_m16_kslot_chunk(slot, d) == geo.geom_m16_kchunk(dc, l // 16, d)
    # the Q^T operand order: features 8*m16_kchunk(dc, g) .. +7 cover D once per lane
    assert sorted(geo.geom_m16_kchunk(dc, g, d) for dc in range(c["dc"]) for g in range(4)) == \
        list(range(d // 8))


@pytest.mark.parametrize("d", [64, 128])
def test_m16_k_tile_dma_reads_whole_64_byte_pieces(geo, d):
    """Each DMA request (64 consecutive LDS slots) reads its global chunks as aligned runs of
    four (64 bytes), so the permuted layout costs no extra global sectors."""
    rb, n = 2 * d, M16[d]["bc"] * d // 8
    for s0 in range(0, n, 64):
        src = sorted(rb * geo.geom_m16_kslot_row(s, d) + 16 * geo.geom_m16_kslot_chunk(s, d)
                     for s in range(s0, s0 + 64))
        pieces = {a // 64 for a in src}
        assert len(pieces) == 16, s0
        assert all(sum(1 for a in src if a // 64 == p) == 4 for p in pieces)


def _v16_read_offsets(geo, d, t, db, e):
    """V^T transposed read e (0, 1) of k step t, fragment db: lane l addresses row
    pv16_key(l, t, 4e) + tr16_row(l), feature column 16*db + tr16_col(l)."""
    out = []
    for l in range(64):
        row = geo.geom_pv16_key(l, t, 4 * e) + geo.geom_tr16_row(l)
        colh = 16 * db + geo.geom_tr16_col(l)
        out.append(geo.geom_tile_offset_m16(row, colh // 8, d) + 2 * (colh % 8))
    base = [geo.geom_tile_offset_m16(geo.geom_pv16_key(l, 0, 0) + geo.geom_tr16_row(l),
                                     (16 * db + geo.geom_tr16_col(l)) // 8, d)
            + 2 * ((16 * db + geo.geom_tr16_col(l)) % 8) for l in range(64)]
    # the kernel reads it at the (t, e) = (0, 0) offset plus 32t + 8e rows (immediates)
    assert all(o == b + (32 * t + 8 * e) * 2 * d for o, b in zip(out, base))
    return out


@pytest.mark.parametrize("d", [64, 128])
def test_m16_v_transposed_reads_are_conflict_free(geo, d):
    c = M16[d]
    for t, db, e in itertools.product(range(c["ks"]), range(c["db"]), range(2)):
        offs = _v16_read_offsets(geo, d, t, db, e)
        assert _conflict_free(offs, 8, 32), (t, db, e)
        for g0 in range(0, 64, 32):
            banks = sum((_banks(o, 8) for o in offs[g0:g0 + 32]), [])
            assert sorted(banks) == list(range(64)), (t, db, e, g0)


@pytest.mark.parametrize("d", [64, 128])
def test_m16_v_transposed_reads_deliver_the_pv16_keys(geo, d):
    """Each 16-lane group reads a 4-row x 16-column block whose transpose hands lane l feature
    16*db + l%16 at keys pv16_key(l, t, 4e + i), i = 0..3."""
    c, rb = M16[d], 2 * d
    for t, db, e in itertools.product(range(c["ks"]), range(c["db"]), range(2)):
        offs = _v16_read_offsets(geo, d, t, db, e)
        for g0 in range(0, 64, 16):
            cells = []
            for l in range(g0, g0 + 16):
                row = offs[l] // rb
                phys_chunk = (offs[l] % rb) // 16
                colh = 8 * geo.geom_swizzle_chunk_m16(row, phys_chunk, d) + (offs[l] % 16) // 2
                cells.append((row, colh))
            rows = sorted({r for r, _ in cells})
            assert len(rows) == 4 and rows == list(range(rows[0], rows[0] + 4))
            cols = sorted({col + j for _, col in cells for j in range(4)})
            assert cols == list(range(cols[0], cols[0] + 16))
            for j, addrs in enumerate(_tr16_received(offs, g0)):
                lane = g0 + j
                for i, addr in enumerate(addrs):
                    assert _logical(geo, addr, rb, True, d) == (
                        geo.geom_pv16_key(lane, t, 4 * e + i), 16 * db + lane % 16)


@pytest.mark.parametrize("d", [64, 128])
def test_m16_p_operand_slots_are_the_score_accumulators(geo, d):
    """Slot 4*(kb%2) + r of k step kb//2 of the P^T operand is score accumulator r of block kb,
    and the key of a slot depends only on lane // 16 (the MFMA pairs A and B slots by k index,
    8*(lane//16) + i); the 32 k indices of a step cover its 32 keys once."""
    c = M16[d]
    for lane, kb, r in itertools.product(range(64), range(c["kb"]), range(4)):
        assert geo.geom_st16_key(lane, kb, r) == geo.geom_pv16_key(lane, kb // 2, 4 * (kb % 2) + r)
    for lane, t, i in itertools.product(range(64), range(c["ks"]), range(8)):
        assert geo.geom_pv16_key(lane, t, i) == geo.geom_pv16_key(16 * (lane // 16), t, i)
    for t in range(c["ks"]):
        keys = {geo.geom_pv16_key(16 * g, t, i) for g in range(4) for i in range(8)}
        assert keys == set(range(32 * t, 32 * t + 32))


@pytest.mark.parametrize("d", [64, 128])
def test_m16_score_blocks_cover_the_tile_once(geo, d):
    c = M16[d]
    cells = {(geo.geom_st16_key(l, kb, r), geo.geom_st16_query(l, qb))
             for l in range(64) for kb in range(c["kb"]) for qb in range(2) for r in range(4)}
    assert cells == {(k, q) for k in range(c["bc"]) for q in range(32)}
    for lane, kb, r in itertools.product(range(64), range(c["kb"]), range(4)):
        assert geo.geom_st16_key(lane, kb, r) == geo.geom_m16_key(kb, geo.geom_mfma16_c_row(lane, r))


def test_spread_vote_model_uses_the_kernels_lane_groups(geo):
    """The CPU model of the ping-pong's first-tile vote (tests/pp16_softmax_model.py) groups a
    row's first 32 keys as the kernel's lanes hold them: lanes 16 g .. 16 g + 15 hold keys
    st16_key(lane, kb, r) of blocks kb = 0, 1 (the same for all 16 lanes of a group), and the
    four groups split the 32 keys."""
    from pp16_softmax_model import m16_key

    for kb, i in itertools.product(range(4), range(16)):
        assert m16_key(kb, i) == geo.geom_m16_key(kb, i)
    groups = []
    for g in range(4):
        keys = {geo.geom_st16_key(16 * g + x, kb, r) for x in range(16) for kb in (0, 1)
                for r in range(4)}
        assert keys == {m16_key(kb, 4 * g + r) for kb in (0, 1) for r in range(4)}, g
        groups.append(keys)
    assert sorted(k for grp in groups for k in grp) == list(range(32))


def test_mfma_c_layouts_cover_each_cell_once(geo):
    cells = {(geo.geom_mfma32_c_row(l, r), geo.geom_mfma32_c_col(l))
             for l in range(64) for r in range(16)}
    assert cells == {(m, n) for m in range(32) for n in range(32)}
    cells = {(geo.geom_mfma16_c_row(l, r), geo.geom_mfma16_c_col(l))
             for l in range(64) for r in range(4)}
    assert cells == {(m, n) for m in range(16) for n in range(16)}


@pytest.mark.parametrize("causal", [0, 1])
def test_num_kv_tiles(geo, causal):
    for n, bq, bk in itertools.product([1, 17, 63, 64, 65, 100, 128, 257, 1000, 2048],
                                       [64, 128, 256], [32, 64, 128]):
        for q0 in range(0, n, bq):
            last_q = min(n, q0 + bq) - 1
            last_key = last_q if causal else n - 1
            assert geo.geom_num_kv_tiles(n, q0, bq, bk, causal) == last_key // bk + 1


@pytest.mark.parametrize("causal", [0, 1])
def test_mask_predicates(geo, causal):
    rows = 32
    for n, bk in itertools.product([1, 31, 64, 65, 100, 200], [32, 64]):
        for qw in range(0, n, rows):
            for kt in range(0, n + bk, bk):
                masked = [[(key >= n) or (causal and key > q) for key in range(kt, kt + bk)]
                          for q in range(qw, qw + rows)]
                anym = any(any(r) for r in masked)
                allm_causal = all(all(key > q for key in range(kt, kt + bk))
                                  for q in range(qw, qw + rows))
                if anym:
                    assert geo.geom_tile_needs_mask(n, kt, bk, qw, causal)
                assert geo.geom_tile_fully_masked(kt, qw, rows, causal) == int(
                    bool(causal) and allm_causal)


def test_st_key_splits_into_lane_and_accumulator_parts(geo):
    for lane, nb, r in itertools.product(range(64), range(4), range(16)):
        assert geo.geom_st_key(lane, nb, r) == geo.geom_st_key(0, nb, r) + geo.geom_st_key_lane(lane)


@pytest.mark.parametrize("causal", [0, 1])
def test_score_mask_threshold(geo, causal):
    """The simple and key-split tiles mask accumulator (nb, r) of `lane` iff
    st_key(0, nb, r) > st_mask_limit(...): that must be exactly "key >= n, or (causal) key right
    of the lane's query" for every lane, accumulator, tile and query of a tile that is masked."""
    k0 = {(nb, r): geo.geom_st_key(0, nb, r) for nb in range(2) for r in range(16)}
    lane_key = {(lane, nb, r): geo.geom_st_key(lane, nb, r)
                for lane in range(64) for nb in range(2) for r in range(16)}
    for n, bk in itertools.product([1, 31, 64, 65, 100, 200], [32, 64]):
        for qw in range(0, n + 32, 32):
            for kt in range(0, n + bk, bk):
                for lane in range(64):
                    qrow = qw + (lane & 31)
                    lim = geo.geom_st_mask_limit(n, kt, qrow, lane, causal)
                    for nb in range(bk // 32):
                        for r in range(16):
                            key = kt + lane_key[(lane, nb, r)]
                            want = key >= n or (causal and key > qrow)
                            assert (k0[(nb, r)] > lim) == want, (n, bk, qw, kt, lane, nb, r)


def test_score_mask_threshold_catches_a_dropped_bound(geo):
    """Planted on the CPU: a threshold that forgets n (causal rows past the end) or the query
    must disagree with the direct predicate somewhere."""
    def lim_without_n(n, kt, qrow, lane):
        return qrow - kt - geo.geom_st_key_lane(lane)

    def lim_without_q(n, kt, qrow, lane):
        return n - 1 - kt - geo.geom_st_key_lane(lane)

    for bad in (lim_without_n, lim_without_q):
        found = False
        for n, kt, lane, nb, r in itertools.product([40, 100], [0, 32, 64], range(64), range(2),
                                                   range(16)):
            qrow = 64 + (lane & 31)
            key = kt + geo.geom_st_key(lane, nb, r)
            want = key >= n or key > qrow
            if (geo.geom_st_key(0, nb, r) > bad(n, kt, qrow, lane)) != want:
                found = True
                break
        assert found, bad.__name__


def test_st16_key_splits_into_lane_and_accumulator_parts(geo):
    for lane, kb, r in itertools.product(range(64), range(4), range(4)):
        assert geo.geom_st16_key(lane, kb, r) == (geo.geom_st16_key(0, kb, r)
                                                   + geo.geom_st16_key_lane(lane))


@pytest.mark.parametrize("causal", [0, 1])
def test_score_mask_threshold_16x16(geo, causal):
    """The simple schedule on 16x16x32 MFMAs masks accumulator r of block (kb, qb) of `lane` iff
    st16_key(0, kb, r) > st16_mask_limit(...): exactly "key >= n, or (causal) key right of the
    query" for every lane, block, accumulator, tile and wave of a tile that is masked (64-key
    tiles at d=64, 32-key tiles at d=128)."""
    k0 = {(kb, r): geo.geom_st16_key(0, kb, r) for kb in range(4) for r in range(4)}
    lane_key = {(lane, kb, r): geo.geom_st16_key(lane, kb, r)
                for lane in range(64) for kb in range(4) for r in range(4)}
    for n, bk in itertools.product([1, 17, 64, 65, 100, 200], [32, 64]):
        for qw in range(0, n + 32, 32):
            for kt in range(0, n + bk, bk):
                for lane, qb in itertools.product(range(64), range(2)):
                    query = qw + geo.geom_st16_query(lane, qb)
                    lim = geo.geom_st16_mask_limit(n, kt, qw, lane, qb, causal)
                    for kb, r in itertools.product(range(bk // 16), range(4)):
                        key = kt + lane_key[(lane, kb, r)]
                        want = key >= n or (causal and key > query)
                        assert (k0[(kb, r)] > lim) == want, (n, bk, qw, kt, lane, qb, kb, r)


def test_score_mask_threshold_16x16_catches_a_wrong_query(geo):
    """Planted on the CPU: a threshold that takes the query of block 0 for block 1 (or the
    32x32 layout's lane part) must disagree with the direct predicate somewhere."""
    def lim_block0(n, kt, qw, lane, qb):
        return geo.geom_st16_mask_limit(n, kt, qw, lane, 0, 1)

    def lim_lane32(n, kt, qw, lane, qb):
        return (geo.geom_st16_mask_limit(n, kt, qw, lane, qb, 1) + geo.geom_st16_key_lane(lane)
                - geo.geom_st_key_lane(lane))

    for bad in (lim_block0, lim_lane32):
        found = False
        for kt, lane, qb, kb, r in itertools.product([0, 32], range(64), range(2), range(4),
                                                     range(4)):
            n, qw = 200, 32
            query = qw + geo.geom_st16_query(lane, qb)
            key = kt + geo.geom_st16_key(lane, kb, r)
            want = key >= n or key > query
            if (geo.geom_st16_key(0, kb, r) > bad(n, kt, qw, lane, qb)) != want:
                found = True
                break
        assert found, bad.__name__


@pytest.mark.parametrize("causal", [0, 1])
def test_work_map_is_a_bijection(geo, causal):
    for bhc, nqb in [(1, 1), (6, 9), (16, 128), (512, 16)]:
        seen = set()
        prev = None
        bh, qb = ctypes.c_int(), ctypes.c_int()
        for bid in range(bhc * nqb):
            geo.geom_work_of(bid, bhc, nqb, causal, ctypes.byref(bh), ctypes.byref(qb))
            assert 0 <= bh.value < bhc and 0 <= qb.value < nqb
            seen.add((bh.value, qb.value))
            if causal and prev is not None:
                assert qb.value <= prev  # longest (highest) query blocks launch first
            prev = qb.value
        assert len(seen) == bhc * nqb


def _xcd_map(geo, bhc, nqb, causal):
    bh, qb = ctypes.c_int(), ctypes.c_int()
    out = []
    for bid in range(bhc * nqb):
        geo.geom_work_of_xcd(bid, bhc, nqb, causal, ctypes.byref(bh), ctypes.byref(qb))
        out.append((bh.value, qb.value))
    return out


XCD_SHAPES = [(1, 1), (1, 7), (3, 5), (8, 8), (12, 64), (16, 64), (16, 128), (64, 16),
              (512, 8), (24, 3), (40, 17), (7, 9)]


@pytest.mark.parametrize("causal", [0, 1])
def test_xcd_work_map_is_a_bijection(geo, causal):
    for bhc, nqb in XCD_SHAPES:
        items = _xcd_map(geo, bhc, nqb, causal)
        assert all(0 <= h < bhc and 0 <= q < nqb for h, q in items)
        assert len(set(items)) == bhc * nqb, (bhc, nqb)


def test_xcd_work_map_keeps_heads_together(geo):
    """Workgroup id b runs on XCD b % 8. Non-causal: each XCD holds one contiguous run of the
    head-major items, so a head spans one XCD when B*H is a multiple of 8 and otherwise only as
    many as its query blocks need (two when it has fewer than an eighth of the items), and the
    XCDs get item counts within one of each other. Causal: work_of's global longest-first
    order."""
    for bhc, nqb in XCD_SHAPES:
        for causal in (0, 1):
            items = _xcd_map(geo, bhc, nqb, causal)
            if causal:
                bh, qb = ctypes.c_int(), ctypes.c_int()
                for bid, item in enumerate(items):
                    geo.geom_work_of(bid, bhc, nqb, causal, ctypes.byref(bh), ctypes.byref(qb))
                    assert item == (bh.value, qb.value)
                continue
            xcds_of_head = {}
            per_xcd = [[] for _ in range(8)]
            for bid, (h, q) in enumerate(items):
                xcds_of_head.setdefault(h, set()).add(bid % 8)
                per_xcd[bid % 8].append((h, q))
            counts = [len(x) for x in per_xcd]
            assert max(counts) - min(counts) <= 1
            per = max(1, bhc * nqb // 8)
            span = 1 if bhc % 8 == 0 else -(-nqb // per) + 1
            assert max(len(v) for v in xcds_of_head.values()) <= span
            for lst in per_xcd:  # contiguous head-major runs, in order
                flat = [h * nqb + q for h, q in lst]
                assert flat == list(range(flat[0], flat[0] + len(flat))) if flat else True


def test_split_ranges_partition_each_query_block(geo):
    """Split-KV: the ranges of a query block with n_all key tiles are exactly the
    ceil(n_all / tps) ranges the combine kernel reads, non-empty, at most tps tiles each,
    within one tile of each other in length, and together cover [0, n_all) once, in order."""
    b, c = ctypes.c_int(), ctypes.c_int()
    for n_all in (1, 2, 3, 7, 8, 9, 33, 64, 65, 100, 512, 4097):
        for tps in (1, 2, 3, 4, 16, 32, 33, 65, 128, 600):
            ranges = -(-n_all // tps)
            got = []
            for split in range(ranges + 3):
                geo.geom_split_range(n_all, tps, split, ctypes.byref(b), ctypes.byref(c))
                if split >= ranges:
                    assert c.value == 0
                    continue
                got.append((b.value, c.value))
            assert [x[0] for x in got] == [sum(x[1] for x in got[:i]) for i in range(len(got))]
            assert sum(x[1] for x in got) == n_all
            lens = [x[1] for x in got]
            assert min(lens) >= 1 and max(lens) <= tps and max(lens) - min(lens) <= 1


PAIR_SHAPES = [(1, 1), (1, 2), (1, 3), (16, 64), (64, 16), (3, 9), (7, 5), (1, 65), (40, 12)]


def _pairs(geo, bhc, nqb):
    bh, lo_, hi_ = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    out = []
    for bid in range(bhc * ((nqb + 1) // 2)):
        geo.geom_causal_pair(bid, bhc, nqb, ctypes.byref(bh), ctypes.byref(hi_), ctypes.byref(lo_))
        out.append((bh.value, hi_.value, lo_.value))
    return out


def test_causal_pairs_cover_every_query_block_once(geo):
    for bhc, nqb in PAIR_SHAPES:
        seen = []
        for h, hi, lo in _pairs(geo, bhc, nqb):
            assert 0 <= h < bhc and hi == nqb - 1 - lo if lo >= 0 else hi == (nqb - 1) // 2
            seen.append((h, hi))
            if lo >= 0:
                assert lo < hi
                seen.append((h, lo))
        assert sorted(seen) == [(h, q) for h in range(bhc) for q in range(nqb)], (bhc, nqb)


def test_causal_pairs_are_equal_work(geo):
    """A causal query block qb visits qb + 1 key blocks: every pair visits n_qblocks + 1 (the
    middle block of an odd count, alone, about half)."""
    for bhc, nqb in PAIR_SHAPES:
        for h, hi, lo in _pairs(geo, bhc, nqb):
            work = (hi + 1) + (lo + 1 if lo >= 0 else 0)
            assert work == nqb + 1 or (lo < 0 and nqb % 2 == 1 and work == (nqb + 1) // 2)


def test_causal_pairs_keep_heads_on_one_xcd(geo):
    """The (head, pair) items follow work_of_xcd's non-causal order."""
    bh, qb = ctypes.c_int(), ctypes.c_int()
    for bhc, nqb in PAIR_SHAPES:
        pairs = (nqb + 1) // 2
        for bid, (h, hi, lo) in enumerate(_pairs(geo, bhc, nqb)):
            geo.geom_work_of_xcd(bid, bhc, pairs, 0, ctypes.byref(bh), ctypes.byref(qb))
            assert (h, nqb - 1 - hi) == (bh.value, qb.value)


# (B*H, query blocks of 256 rows): measured on MI355X, d=128 causal, pairs against singles
PAIRS_WIN = [(16, 64), (64, 16), (128, 12), (16, 32)]   # cfg4, cfg2, 8x16x3000, 1x16x8192
SINGLES_WIN = [(16, 48), (48, 24), (32, 24), (32, 40)]  # 1x16x12288, 3x16x6144, 2x16x6144, 1x32x10240


def test_causal_pairs_choice_follows_the_measurements(geo):
    for bhc, nqb in PAIRS_WIN:
        assert geo.geom_causal_pairs_pay(bhc, nqb, 256) == 1, (bhc, nqb)
    for bhc, nqb in SINGLES_WIN:
        assert geo.geom_causal_pairs_pay(bhc, nqb, 256) == 0, (bhc, nqb)


def test_causal_pairs_taken_whenever_rounds_are_full(geo):
    """An even number of query blocks and a pair count that fills whole rounds: the pairs'
    time is total / slots exactly, which no schedule beats."""
    for nqb in range(2, 130, 2):
        for rounds in (1, 2, 3, 7):
            slots = 256
            pairs = rounds * slots
            if pairs % (nqb // 2):
                continue
            assert geo.geom_causal_pairs_pay(pairs // (nqb // 2), nqb, slots) == 1, (nqb, rounds)


def _lpt(bhc, nqb, slots):
    """Longest-first list schedule of the single query blocks, one heap entry per CU."""
    import heapq

    loads = [0] * slots
    for qb in range(nqb - 1, -1, -1):
        for _ in range(bhc):
            heapq.heapreplace(loads, loads[0] + qb + 1)
    return max(loads)


def test_causal_singles_makespan_estimates_a_list_schedule(geo):
    """Within one key block or 3 % of a one-item-at-a-time list schedule from 9 query blocks
    up (the causal ping-pong's range), exact where every CU gets the same count of each
    length."""
    for bhc in (1, 3, 8, 12, 16, 24, 40, 48, 64, 200, 300, 1000):
        for nqb in range(9, 80, 4):
            est, ref = geo.geom_causal_singles_makespan(bhc, nqb, 256), _lpt(bhc, nqb, 256)
            assert abs(est - ref) <= max(1, 0.03 * ref), (bhc, nqb, est, ref)
    for nqb in (1, 2, 9, 33):
        assert geo.geom_causal_singles_makespan(512, nqb, 256) == _lpt(512, nqb, 256)


def test_causal_pairs_choice_against_a_list_schedule(geo):
    """Pairs are given up only where the singles' list schedule ends at least 1 % before the
    pairs' rounds, and kept wherever it ends less than 5 % before them."""
    for bhc in (1, 3, 8, 16, 24, 40, 64, 100):
        for nqb in (9, 12, 16, 24, 33, 48, 64):
            pairs = -(-bhc * ((nqb + 1) // 2) // 256) * (nqb + 1)
            singles = _lpt(bhc, nqb, 256)
            if geo.geom_causal_pairs_pay(bhc, nqb, 256) == 0:
                assert singles <= 0.99 * pairs, (bhc, nqb, pairs, singles)
            elif singles < 0.95 * pairs:
                pytest.fail(f"pairs kept at {(bhc, nqb)}: {pairs} vs {singles}")


# ---- mutation check of the layout tests above ---------------------------------------------------
# Counterpart of the reference's planted-bug check of its building-block tests
# (docs/testing.md:64-74: removing the swizzle XOR and a wrong ldmatrix lane map each failed a
# unit test). Here the same two mistakes are planted in a stand-in for the geometry library --
# the real functions, except the mutated ones, which are written out below -- and fed through
# the conflict and lane-map checks of this file, each of which must then fail.


class _Mutant:
    def __init__(self, geo, **over):
        self._geo, self._over = geo, over

    def __getattr__(self, name):
        return self._over.get(name, getattr(self._geo, name))


def _unswizzled(geo):
    """No row XOR in either layout: chunk c of row r at byte r * row_bytes + 16 c."""
    return _Mutant(
        geo,
        geom_row_xor=lambda row, rb: 0,
        geom_swizzle_chunk=lambda row, chunk, rb: chunk,
        geom_tile_offset=lambda row, chunk, rb: row * rb + 16 * chunk,
        geom_row_xor_m16=lambda row, d: 0,
        geom_swizzle_chunk_m16=lambda row, chunk, d: chunk,
        geom_tile_offset_m16=lambda row, chunk, d: row * 2 * d + 16 * chunk,
    )


def _tr16_transposed(geo):
    """The transposing read's lane map with row and column roles swapped: lane l addresses row
    l % 4 and column 4 * ((l % 16) // 4) instead of row (l % 16) // 4 and column 4 (l % 4)."""
    return _Mutant(geo, geom_tr16_row=lambda lane: lane & 3,
                   geom_tr16_col=lambda lane: 4 * ((lane & 15) >> 2))


@pytest.mark.parametrize("check", [test_k_fragment_reads_are_conflict_free,
                                   test_v_transposed_reads_are_conflict_free,
                                   test_m16_v_transposed_reads_are_conflict_free])
def test_unswizzled_layout_is_caught(geo, check):
    with pytest.raises(AssertionError):
        check(_unswizzled(geo), 128)


@pytest.mark.parametrize("check", [test_v_transposed_reads_deliver_the_pv_keys,
                                   test_m16_v_transposed_reads_deliver_the_pv16_keys])
def test_wrong_tr16_lane_map_is_caught(geo, check):
    for d in (64, 128):
        with pytest.raises(AssertionError):
            check(_tr16_transposed(geo), d)


def test_mutants_leave_the_checks_green_on_the_real_layout(geo):
    """The checks above pass through the stand-in when nothing is mutated, so a failure under
    a mutant is the mutant's doing."""
    same = _Mutant(geo)
    for d in (64, 128):
        test_k_fragment_reads_are_conflict_free(same, d)
        test_v_transposed_reads_are_conflict_free(same, d)
        test_m16_v_transposed_reads_are_conflict_free(same, d)
        test_v_transposed_reads_deliver_the_pv_keys(same, d)
        test_m16_v_transposed_reads_deliver_the_pv16_keys(same, d)


def _grouped(geo, bid, bhc, nqb, group):
    bh, qb = ctypes.c_int(), ctypes.c_int()
    geo.geom_work_of_xcd_grouped(bid, bhc, nqb, group, ctypes.byref(bh), ctypes.byref(qb))
    return bh.value, qb.value


@pytest.mark.parametrize("bhc,nqb", [(256, 16), (336, 6), (512, 4), (300, 7), (64, 8), (65, 3)])
def test_causal_head_groups(geo, bhc, nqb):
    """work_of_xcd with head groups (causal simple-schedule grids at d=128 from 256 heads): a
    bijection onto (head, query block); heads run in groups of 64 in order, longest query block
    first within a group (the last group may be smaller); every query block of a head lands on
    one XCD (id % 8); and 64 or fewer heads keep the global longest-first order."""
    g = 64
    items = [_grouped(geo, bid, bhc, nqb, g) for bid in range(bhc * nqb)]
    assert sorted(items) == [(h, q) for h in range(bhc) for q in range(nqb)]
    if bhc <= g:
        assert items == [(bid % bhc, nqb - 1 - bid // bhc) for bid in range(bhc * nqb)]
        return
    pos = 0
    for first in range(0, bhc, g):
        heads = min(g, bhc - first)
        chunk = items[pos:pos + heads * nqb]
        assert {h for h, _ in chunk} == set(range(first, first + heads))
        assert [q for _, q in chunk] == sorted((q for _, q in chunk), reverse=True)
        pos += heads * nqb
    xcd = {}
    for bid, (h, _) in enumerate(items):
        xcd.setdefault(h, set()).add(bid % 8)
    if bhc % 8 == 0:
        assert all(len(x) == 1 for x in xcd.values())


def test_causal_group_heads_rule(geo):
    """Head groups of 64 at head dim 128 from 256 heads (four groups) on, none at d=64 or with
    fewer heads."""
    assert geo.geom_causal_group_heads(128, 256) == 64
    assert geo.geom_causal_group_heads(128, 512) == 64
    assert geo.geom_causal_group_heads(128, 255) == 0
    assert geo.geom_causal_group_heads(64, 1024) == 0
