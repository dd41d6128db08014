// Integer tile geometry of the gfx950 FlashAttention-2 forward: LDS swizzle, MFMA register
// layouts, transpose-read addressing, tile counts and the workgroup -> (head, query block) map.
//
// Plain constexpr C++ with no HIP types: clang compiles constexpr functions for both host and
// device, so the kernel and the host-side unit tests (built with g++) use this one definition.
#pragma once

#include <cstdint>

namespace fa::geom {

// ---- LDS layout of a K or V tile ------------------------------------------------------------
// A tile is [rows][D] fp16, row-major, row_bytes = 2*D (128 B for D=64, 256 B for D=128). The
// 16-byte chunks of a row are permuted by an XOR with a function of the row.
//
// gfx950 LDS, as measured on MI355X: 64 banks x 4 bytes (256 bytes per cycle); a
// ds_read_b128 is served 16 lanes at a time and a ds_read_b64_tr_b16 32 lanes at a time, and
// a group is conflict-free when its lanes hit distinct 4-byte banks (or the same address).
// The two read patterns of the kernel are:
//   * K fragments (ds_read_b128): lanes l..l+15 read the same logical chunk of 16 consecutive
//     rows;
//   * V^T fragments (ds_read_b64_tr_b16): 32 lanes read logical chunks 4a..4a+3 of 4
//     consecutive rows starting at a multiple of 4 (8 bytes per lane).
// D=128 (one row spans all 64 banks): row_xor = 4*(row%4) + (row/4)%4 is a bijection on
// row%16 (K groups conflict-free) and gives 4 consecutive rows distinct high bits (V groups
// conflict-free). D=64 (two rows per bank line): row_xor = 4*((row/2)%2) + (row/4)%4 is a
// bijection on the rows of one parity among 16 (K), and differs in bit 2 between rows r and
// r+2 (V). Replaces the reference's 8-row XOR for ldmatrix (csrc/common.cuh:38-42), which
// targets a different bank geometry and access pattern.
constexpr int row_xor(int row, int row_bytes) {
    return row_bytes >= 256 ? (((row & 3) << 2) | ((row >> 2) & 3))
                            : ((((row >> 1) & 1) << 2) | ((row >> 2) & 3));
}

// Physical chunk slot of logical 16-byte chunk `chunk` of `row`. For a fixed row this is an
// involution (XOR), so the same function maps physical slots back to logical chunks.
constexpr int swizzle_chunk(int row, int chunk, int row_bytes) {
    return chunk ^ row_xor(row, row_bytes);
}

// Byte offset of (row, logical chunk) inside a tile with `row_bytes` bytes per row.
constexpr int tile_offset(int row, int chunk, int row_bytes) {
    return row * row_bytes + 16 * swizzle_chunk(row, chunk, row_bytes);
}

// ---- v_mfma_f32_32x32x16_f16 register layouts (wave64) --------------------------------------
// A (32x16): lane l holds A[l % 32][8*(l/32) + i], i = 0..7.
// B (16x32): lane l holds B[8*(l/32) + i][l % 32], i = 0..7.
// C (32x32): lane l, accumulator r (0..15) holds C[mfma32_c_row(l, r)][l % 32].
// Only the C mapping and the m/n indices matter for correctness: the k index of A and B is
// paired lane-by-lane, so any consistent k order gives the same product.
constexpr int mfma32_c_row(int lane, int r) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }
constexpr int mfma32_c_col(int lane) { return lane & 31; }

// v_mfma_f32_16x16x32_f16: A (16x32) lane l holds A[l % 16][8*(l/16) + i]; B likewise;
// C (16x16): lane l, accumulator r (0..3) holds C[4*(l/16) + r][l % 16].
constexpr int mfma16_c_row(int lane, int r) { return 4 * (lane >> 4) + r; }
constexpr int mfma16_c_col(int lane) { return lane & 15; }

// ---- The 16x16x32 MFMA path (flash_fwd_pingpong16; D = 128 with 32-key tiles, D = 64 with
// 64-key tiles; d is the head dim, rows are 2d bytes) ------------------------------------------
// Key blocks: the 16 keys of score block kb (the M rows of its MFMAs) are tile rows
// 32*(kb/2) + 8*(kb%2) + {0..7, 16..23}, i.e. row m16_key(kb, i) for M index i: each 32-key
// group of the tile holds two key blocks interleaved by 8 rows. A 16-lane group of a K operand
// then spans both 4 KiB halves of a D = 128 tile, and so does each half-wave of a V^T read.
// Measured on MI355X (8 waves per CU, conflict-free patterns): ds_read_b128 at 256 B per CU
// cycle with this split against 128 B with contiguous 16-row blocks (all lanes in one 4 KiB
// half); ds_read_b64_tr_b16 at 160 B against 132 B (and 64 B for the 32x32x16 V^T pattern,
// four lanes groups on the same four rows).
constexpr int m16_key(int kb, int i) {
    return 32 * (kb >> 1) + 8 * (kb & 1) + (i & 7) + 16 * ((i >> 3) & 1);
}

// LDS swizzle of the V tiles of this path. D = 128: row_xor_m16 = 2*(row%8) + (row/16)%2. A V^T
// read (32 lanes: 8 rows aligned to 8, logical chunks 2c and 2c+1, 32 bytes per row) sees the 8
// even or the 8 odd values, which put the 8 row pieces on 16 distinct chunks. D = 64 (two rows
// per 256-byte bank line): row_xor_m16 = 2*((row/2)%4) moves the 32-byte piece of each of the 4
// even rows (banks 0-31) and of the 4 odd rows (banks 32-63) to its own quarter. In both, rows
// 8 apart within a key block's half and rows 32 apart share the value, so the second read of a
// fragment and the next 32-key group are immediate offsets.
constexpr int row_xor_m16(int row, int d) {
    return d >= 128 ? (((row & 7) << 1) | ((row >> 4) & 1)) : (((row >> 1) & 3) << 1);
}
constexpr int swizzle_chunk_m16(int row, int chunk, int d) { return chunk ^ row_xor_m16(row, d); }
constexpr int tile_offset_m16(int row, int chunk, int d) {
    return row * 2 * d + 16 * swizzle_chunk_m16(row, chunk, d);
}

// K tiles of this path use their own LDS layout: the K operand of MFMA step (kb, dc) is read
// with exactly the lane addresses of the 32x32x16 path's K fragment (nb, kk) with nb = kb / 2,
// kk = (kb % 2) * DC + dc (DC = d / 32), tile_offset(32 nb + lane % 32, 2kk + lane / 32, 2d),
// whose ds_read_b128 pattern measures conflict-free (the direct 16x16x32 pattern, four lane
// groups on four chunks of the same 16 rows, costs 4 conflict cycles per read on MI355X). Lane
// l must receive key row m16_key(kb, l % 16), 16-byte chunk m16_kchunk(dc, l / 16, d): the
// MFMA's k slots 8g..8g+7 of lane group g are features 8 * m16_kchunk(dc, g, d) .. +7, and the
// Q^T operand uses the same order. m16_kslot_row / m16_kslot_chunk give the element that
// 16-byte LDS slot `slot` holds.
// (For d = 64 the two lane groups a DMA request covers, g and g + 2, get adjacent chunk pairs,
// so that each request reads whole 64-byte pieces of a K row.)
constexpr int m16_kchunk(int dc, int grp, int d) {
    return d >= 128 ? 4 * grp + dc : 4 * (grp & 1) + 2 * (grp >> 1) + dc;
}
constexpr int m16_kslot_t(int slot, int d) {
    return (slot % (d / 8)) ^ row_xor(slot / (d / 8), 2 * d);
}
constexpr int m16_kslot_kb(int slot, int d) {  // 2 nb + kk / DC
    return 2 * ((slot / (d / 8)) >> 5) + (m16_kslot_t(slot, d) >> 1) / (d / 32);
}
constexpr int m16_kslot_row(int slot, int d) {
    return m16_key(m16_kslot_kb(slot, d), (slot / (d / 8)) & 15);
}
constexpr int m16_kslot_chunk(int slot, int d) {
    return m16_kchunk((m16_kslot_t(slot, d) >> 1) % (d / 32),
                      (((slot / (d / 8)) >> 4) & 1) + 2 * (m16_kslot_t(slot, d) & 1), d);
}

// S^T = K Q^T of a wave (32 queries) and a key tile in 16x16 blocks (kb, qb): accumulator r
// of block (kb, qb) in `lane` is key st16_key(lane, kb, r) of the tile and query
// st16_query(lane, qb) of the wave. Each lane thus holds 4 keys of 2 queries per key block.
constexpr int st16_key(int lane, int kb, int r) { return m16_key(kb, mfma16_c_row(lane, r)); }
constexpr int st16_query(int lane, int qb) { return 16 * qb + (lane & 15); }

// st16_key splits into a lane part and a compile-time accumulator part, as st_key does:
// st16_key(lane, kb, r) = st16_key(0, kb, r) + st16_key_lane(lane) (lane / 16 = 2h + a selects
// the 8-row half a and the 16-row half h of the key block).
constexpr int st16_key_lane(int lane) { return 4 * ((lane >> 4) & 1) + 16 * (lane >> 5); }

// Mask threshold of query block qb of a 16x16 score tile (as st_mask_limit): key
// kt + st16_key(lane, kb, r) is masked for query qw + st16_query(lane, qb) iff it is >= n or
// (causal) right of that query, i.e. iff st16_key(0, kb, r) > st16_mask_limit(...).
constexpr int st16_mask_limit(int n, int kt, int qw, int lane, int qb, bool causal) {
    const int qrow = qw + st16_query(lane, qb);
    return (causal && qrow < n - 1 ? qrow : n - 1) - kt - st16_key_lane(lane);
}

// Key carried by operand slot i (0..7) of k step t (32 keys) of the O^T += V^T P^T MFMA in
// `lane`: slots 0..3 are the lane's scores of key block 2t, slots 4..7 those of block 2t + 1,
// so P^T of query block qb is the lane's own 8 exponentials in order (no shuffle), and the
// V^T operand reads these keys. The key depends on lane / 16, t and i only, as the MFMA's
// shared k index requires.
constexpr int pv16_key(int lane, int t, int i) { return st16_key(lane, 2 * t + (i >> 2), i & 3); }

// ---- Transposed operand reads (ds_read_b64_tr_b16) ------------------------------------------
// Within each group of 16 lanes, the instruction loads a 4 x 16 block of 16-bit values
// (4 rows, 16 consecutive columns) and returns it transposed: lane j of the group receives
// column j, rows 0..3, as its four halves. tr16_row / tr16_col give the (row, column) that
// lane j must address (8 bytes = 4 columns starting there) for that result.
constexpr int tr16_row(int lane) { return (lane & 15) >> 2; }
constexpr int tr16_col(int lane) { return 4 * (lane & 3); }

// ---- Score-tile index maps (S^T = K Q^T in 32x32 MFMA blocks) --------------------------------
// Key offset within a tile of accumulator r of 32-key block nb held by `lane`; that lane's
// query is always lane % 32 of the wave's 32 queries.
constexpr int st_key(int lane, int nb, int r) { return 32 * nb + mfma32_c_row(lane, r); }

// st_key splits into a lane part and a compile-time accumulator part:
// st_key(lane, nb, r) = st_key(0, nb, r) + st_key_lane(lane).
constexpr int st_key_lane(int lane) { return 4 * (lane >> 5); }

// Masking of a score tile: key kt + st_key(lane, nb, r) is masked iff it is >= n or (causal)
// right of the lane's query qrow, i.e. iff it exceeds min(n - 1, qrow). With the split above,
// that is st_key(0, nb, r) > st_mask_limit(n, kt, qrow, lane, causal): one threshold per lane and
// tile, then one compare and one select per score.
constexpr int st_mask_limit(int n, int kt, int qrow, int lane, bool causal) {
    return (causal && qrow < n - 1 ? qrow : n - 1) - kt - st_key_lane(lane);
}

// Key offset (within a 16-key MFMA step) of operand slot i (0..7) of the P.V product. Equal to
// the score accumulator that feeds it: slot i of step h is accumulator 8*h + i of its block.
constexpr int pv_key(int lane, int i) { return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3); }

// ---- Work decomposition ---------------------------------------------------------------------
// ceil(a / b) for a >= 0, b > 0, without forming a + b - 1 (which overflows for a near
// INT32_MAX).
constexpr int ceil_div(int a, int b) { return a / b + (a % b > 0 ? 1 : 0); }

// Number of K/V tiles a workgroup whose first query row is q0 visits. Causal workgroups stop
// at the tile holding their last query's diagonal (tiles above it are fully masked);
// follows csrc/kernels/flash_fwd.cu:193-194 (kv_end = min(n, q0 + BR)).
constexpr int num_kv_tiles(int n, int q0, int block_q, int block_k, bool causal) {
    const int kv_end = causal ? (n < q0 + block_q ? n : q0 + block_q) : n;
    return ceil_div(kv_end, block_k);
}

// Whether a tile [kt, kt+block_k) needs any masking for queries [qw, qw+rows): keys past the
// end of the sequence, or (causal) keys right of the diagonal of the first query.
// Follows the needs_mask test of csrc/kernels/flash_fwd.cu:502-505.
constexpr bool tile_needs_mask(int n, int kt, int block_k, int qw, bool causal) {
    return (kt + block_k > n) || (causal && kt + block_k - 1 > qw);
}

// Whether every key of the tile is masked for all queries [qw, qw+rows) (causal only).
constexpr bool tile_fully_masked(int kt, int qw, int rows, bool causal) {
    return causal && kt > qw + rows - 1;
}

// Number of leading tiles a wave whose queries are [qw, qw+rows) computes: all of them when
// not causal; when causal, those with a key <= its last query (the rest are fully masked and
// the wave only takes part in their barriers). 0 for a wave entirely past the sequence.
constexpr int wave_active_tiles(int n, int qw, int rows, int block_k, int n_tiles, bool causal) {
    if (qw >= n) return 0;
    if (!causal) return n_tiles;
    const int t = (qw + rows - 1) / block_k + 1;
    return t < n_tiles ? t : n_tiles;
}

// Length of the leading run of tiles that need no mask for a wave starting at query qw
// (tile_needs_mask is false exactly for j < this), capped at n_act.
constexpr int wave_unmasked_tiles(int n, int qw, int block_k, int n_act, bool causal) {
    int t = n / block_k;
    if (causal && (qw + 1) / block_k < t) t = (qw + 1) / block_k;
    return t < n_act ? t : n_act;
}

// Split-KV: the key tiles [begin, begin + count) of range `split` of a query block that visits
// n_all tiles. The block is cut into ceil(n_all / tps) ranges (the count the combine kernel
// reads for its rows) of near-equal length (floor or ceil of n_all / ranges, at most tps), so
// that no range is a short remainder; count = 0 for a range the block does not have.
struct KeyRange {
    int begin;
    int count;
};
constexpr KeyRange split_range(int n_all, int tps, int split) {
    const int ranges = ceil_div(n_all, tps);
    if (split >= ranges) return KeyRange{0, 0};
    const long long b = static_cast<long long>(split) * n_all / ranges;
    const long long e = static_cast<long long>(split + 1) * n_all / ranges;
    return KeyRange{static_cast<int>(b), static_cast<int>(e - b)};
}

// Workgroup id -> (batch*head index, query block). Consecutive ids share the query block and
// walk the heads; causal runs the longest query blocks first (as
// csrc/kernels/flash_fwd.cu:183-185). Used by the split-KV partial passes (within one key
// range) and by work_of_xcd for causal grids.
struct Work {
    int bh;
    int qb;
};
constexpr Work work_of(int block_id, int bh_count, int n_qblocks, bool causal) {
    const int qi = block_id / bh_count;
    return Work{block_id % bh_count, causal ? n_qblocks - 1 - qi : qi};
}

// Workgroup id -> (batch*head index, query block), XCD-aware for non-causal grids. MI355X
// deals workgroup ids round-robin to its kXcds XCDs (id % 8), and each XCD has its own L2. The
// non-causal (head, query block) items are laid out head-major and XCD x receives one
// contiguous eighth of them (slot s = id / 8 is the s-th item of that eighth), so the query
// blocks of a head run on one XCD at about the same time and share its K/V in that XCD's L2,
// whatever B*H is; all items are equal, so the XCDs stay balanced. (work_of walks the heads with
// consecutive ids, which scatters a head's query blocks in time: on many short heads, e.g.
// 512 heads of 2048 keys, their K/V are then re-read from HBM by every query block.)
// Causal grids keep work_of's global longest-first order (its tail, the shortest query blocks
// last everywhere at once, is worth more than L2 locality on most shapes), unless group_heads
// > 0 (the launcher's choice, causal_group_heads): then the heads run in groups of group_heads,
// longest query blocks first within each group, so that the query blocks of a head run close in
// time and share its K/V in L2 and the last-level cache. With group_heads a multiple of 8 the
// blocks of a head also stay on one XCD (id % 8 = head % 8 within a group).
constexpr int kXcds = 8;
constexpr Work work_of_xcd(int block_id, int bh_count, int n_qblocks, bool causal,
                           int group_heads = 0) {
    if (causal) {
        const int G = group_heads;
        if (G > 0 && bh_count > G) {
            const int grp = block_id / (G * n_qblocks);
            const int first = grp * G;
            const int heads = bh_count - first < G ? bh_count - first : G;  // last group: rest
            const int r = block_id - grp * G * n_qblocks;
            return Work{first + r % heads, n_qblocks - 1 - r / heads};
        }
        return work_of(block_id, bh_count, n_qblocks, causal);
    }
    const int x = block_id % kXcds;
    const int slot = block_id / kXcds;
    const long long total = static_cast<long long>(bh_count) * n_qblocks;
    const long long per = total / kXcds;
    const long long extra = total % kXcds;
    const long long t = x * per + (x < extra ? x : extra) + slot;
    return Work{static_cast<int>(t / n_qblocks), static_cast<int>(t % n_qblocks)};
}

// Causal grids of paired query blocks: workgroup id -> (batch*head index, long query block
// n_qblocks - 1 - p, short query block p, or -1 when p is the middle block of an odd count).
// A causal query block qb visits qb + 1 key blocks, so every pair visits n_qblocks + 1 and all
// workgroups are equal. The (head, pair) items run in work_of_xcd's order (a head's pairs
// together on one XCD). Equal workgroups also let the dispatcher start the next workgroup on a
// CU as soon as one ends: with the longest-first order of unequal workgroups, MI355X left CUs
// idle for 5-7 us (median) between workgroups on cfg4 causal, against 1-1.3 us when all
// workgroups are equal.
struct PairWork {
    int bh;
    int qb_long;
    int qb_short;
};
constexpr PairWork causal_pair(int block_id, int bh_count, int n_qblocks) {
    const int pairs = (n_qblocks + 1) / 2;
    const Work w = work_of_xcd(block_id, bh_count, pairs, false);
    const int lo = w.qb;
    const int hi = n_qblocks - 1 - lo;
    return PairWork{w.bh, hi, hi != lo ? lo : -1};
}

// Makespan estimate, in key blocks, of the causal ping-pong grid of single query blocks: bh_count
// copies of the lengths n_qblocks, ..., 1 (query block qb visits qb + 1 key blocks) dealt in
// work_of's longest-first order to `slots` CUs, each taking the next workgroup when it frees (a
// longest-first list schedule). Level by level: the bh_count blocks of one length give every CU
// bh_count / slots of them and one more to each of the bh_count % slots least loaded CUs (the
// list schedule can give two to one CU whose load trails by more than the length; the estimate
// stays within one key block or 3 % of it from 9 query blocks up). Loads are kept as
// ascending (load, count) groups, so a level costs O(groups). Returns -1 past kMaxGroups
// groups. Host-side.
constexpr int kMaxGroups = 256;
inline long long causal_singles_makespan(long long bh_count, int n_qblocks, int slots) {
    long long load[kMaxGroups + 1];
    long long cnt[kMaxGroups + 1];
    long long up_l[kMaxGroups + 1];
    long long up_c[kMaxGroups + 1];
    long long out_l[2 * kMaxGroups + 2];
    long long out_c[2 * kMaxGroups + 2];
    int ng = 1;
    load[0] = 0;
    cnt[0] = slots;
    for (int len = n_qblocks; len >= 1; --len) {
        const long long full = bh_count / slots;
        long long r = bh_count % slots;
        for (int i = 0; i < ng; ++i) load[i] += full * len;
        // the r least loaded machines take one more block of this length
        int nu = 0;
        int i = 0;
        while (r > 0) {
            const long long take = cnt[i] < r ? cnt[i] : r;
            up_l[nu] = load[i] + len;
            up_c[nu] = take;
            ++nu;
            r -= take;
            cnt[i] -= take;
            if (cnt[i] == 0) ++i;
        }
        // merge the raised groups (ascending) with the rest (ascending, from group i)
        int no = 0;
        int a = 0;
        int b = i;
        while (a < nu || b < ng) {
            const bool from_up = b >= ng || (a < nu && up_l[a] <= load[b]);
            const long long l = from_up ? up_l[a] : load[b];
            const long long c = from_up ? up_c[a++] : cnt[b++];
            if (c == 0) continue;
            if (no > 0 && out_l[no - 1] == l) {
                out_c[no - 1] += c;
            } else {
                out_l[no] = l;
                out_c[no] = c;
                ++no;
            }
        }
        if (no > kMaxGroups) return -1;
        for (int k = 0; k < no; ++k) {
            load[k] = out_l[k];
            cnt[k] = out_c[k];
        }
        ng = no;
    }
    return load[ng - 1];
}

// Whether a causal ping-pong grid runs (long, short) pairs (causal_pair) or one query block per
// workgroup in work_of's longest-first order. The ping-pong holds one workgroup per CU, so W
// equal pair workgroups run in ceil(W / slots) rounds of n_qblocks + 1 key blocks each
// (slots = CUs), while the single blocks end at causal_singles_makespan plus about 3 % on MI355X
// (dispatch gaps between unequal workgroups: pairs measured 1.4-2.3 % faster where the two
// schedules end together). Pairs are kept unless their last round is empty enough for the
// singles to end first: 1x16x12288 d=128 (384 pairs, 1.5 rounds) ran 9.4 % and 3x16x6144
// 18.6 % faster as singles. Host-side (launch grid choice).
constexpr int kCus = 256;  // MI355X compute units: 8 XCDs of 32
inline bool causal_pairs_pay(long long bh_count, int n_qblocks, int slots) {
    const long long w = bh_count * ((n_qblocks + 1) / 2);
    // 64 rounds or more: a partly empty last round costs under 2 %; more than 1024 query
    // blocks: pairs too (the estimate's cost grows with the block count), which also keeps
    // every product below in range
    if (w >= 64LL * slots || n_qblocks > 1024) return true;
    const long long pairs = (w + slots - 1) / slots * (n_qblocks + 1);
    const long long singles = causal_singles_makespan(bh_count, n_qblocks, slots);
    return singles < 0 || 100 * pairs <= 103 * singles;
}

// Head groups of a causal simple-schedule grid (work_of_xcd's group_heads): 64 at head dim 128
// from 256 heads on (four groups or more), else 0. At d = 128 the global longest-first order
// re-reads a head's K/V from HBM for each of its query blocks, which run far apart in time.
// Measured on MI355X (interleaved A/B, causal, the simple and 16x16x32 simple tiles):
// 32x16x512 +16.6 %, 32x16x1024 +15 %, 16x16x1024 +7.7 %, 16x16x2048 +9.4 %, 21x16x768 +5.1 %.
// With fewer groups the last one leaves CUs idle (10x16x1536, 2.5 groups: -7.8 %; 5x16x3072,
// 1.25: -14 %), and at d = 64 the gains and losses were mixed (-6 to +7 % across shapes), so
// those keep the global order. Host-side (launch argument). Build option
// FA_CAUSAL_GROUP_HEADS: the group size (a multiple of 8), 0 for the global order everywhere.
#ifndef FA_CAUSAL_GROUP_HEADS
#define FA_CAUSAL_GROUP_HEADS 64
#endif
constexpr int kCausalGroupHeads = FA_CAUSAL_GROUP_HEADS;
static_assert(kCausalGroupHeads >= 0 && kCausalGroupHeads % 8 == 0,
              "head groups are whole multiples of the 8 XCDs");
inline int causal_group_heads(int head_dim, long long bh_count) {
    return kCausalGroupHeads > 0 && head_dim == 128 && bh_count >= 4LL * kCausalGroupHeads
               ? kCausalGroupHeads
               : 0;
}

}  // namespace fa::geom
