// Host-side C wrappers around the kernel's integer tile geometry (fa_geometry.h), built with
// g++ so the CPU tests (tests/test_geometry.py) check the very functions the kernel inlines.
#include "fa_geometry.h"

namespace g = fa::geom;

extern "C" {
int geom_row_xor(int row, int row_bytes) { return g::row_xor(row, row_bytes); }
int geom_swizzle_chunk(int row, int chunk, int row_bytes) {
    return g::swizzle_chunk(row, chunk, row_bytes);
}
int geom_tile_offset(int row, int chunk, int row_bytes) { return g::tile_offset(row, chunk, row_bytes); }
int geom_mfma32_c_row(int lane, int r) { return g::mfma32_c_row(lane, r); }
int geom_mfma32_c_col(int lane) { return g::mfma32_c_col(lane); }
int geom_mfma16_c_row(int lane, int r) { return g::mfma16_c_row(lane, r); }
int geom_mfma16_c_col(int lane) { return g::mfma16_c_col(lane); }
int geom_tr16_row(int lane) { return g::tr16_row(lane); }
int geom_tr16_col(int lane) { return g::tr16_col(lane); }
int geom_st_key(int lane, int nb, int r) { return g::st_key(lane, nb, r); }
int geom_st_key_lane(int lane) { return g::st_key_lane(lane); }
int geom_st_mask_limit(int n, int kt, int qrow, int lane, int causal) {
    return g::st_mask_limit(n, kt, qrow, lane, causal != 0);
}
int geom_m16_key(int kb, int i) { return g::m16_key(kb, i); }
int geom_m16_kchunk(int dc, int grp, int d) { return g::m16_kchunk(dc, grp, d); }
int geom_m16_kslot_row(int slot, int d) { return g::m16_kslot_row(slot, d); }
int geom_m16_kslot_chunk(int slot, int d) { return g::m16_kslot_chunk(slot, d); }
int geom_row_xor_m16(int row, int d) { return g::row_xor_m16(row, d); }
int geom_swizzle_chunk_m16(int row, int chunk, int d) { return g::swizzle_chunk_m16(row, chunk, d); }
int geom_tile_offset_m16(int row, int chunk, int d) { return g::tile_offset_m16(row, chunk, d); }
int geom_st16_key(int lane, int kb, int r) { return g::st16_key(lane, kb, r); }
int geom_st16_query(int lane, int qb) { return g::st16_query(lane, qb); }
int geom_st16_key_lane(int lane) { return g::st16_key_lane(lane); }
int geom_st16_mask_limit(int n, int kt, int qw, int lane, int qb, int causal) {
    return g::st16_mask_limit(n, kt, qw, lane, qb, causal != 0);
}
int geom_pv16_key(int lane, int t, int i) { return g::pv16_key(lane, t, i); }
int geom_pv_key(int lane, int i) { return g::pv_key(lane, i); }
int geom_num_kv_tiles(int n, int q0, int block_q, int block_k, int causal) {
    return g::num_kv_tiles(n, q0, block_q, block_k, causal != 0);
}
int geom_tile_needs_mask(int n, int kt, int block_k, int qw, int causal) {
    return g::tile_needs_mask(n, kt, block_k, qw, causal != 0) ? 1 : 0;
}
int geom_tile_fully_masked(int kt, int qw, int rows, int causal) {
    return g::tile_fully_masked(kt, qw, rows, causal != 0) ? 1 : 0;
}
int geom_wave_active_tiles(int n, int qw, int rows, int block_k, int n_tiles, int causal) {
    return g::wave_active_tiles(n, qw, rows, block_k, n_tiles, causal != 0);
}
int geom_wave_unmasked_tiles(int n, int qw, int block_k, int n_act, int causal) {
    return g::wave_unmasked_tiles(n, qw, block_k, n_act, causal != 0);
}
void geom_split_range(int n_all, int tps, int split, int* begin, int* count) {
    const g::KeyRange r = g::split_range(n_all, tps, split);
    *begin = r.begin;
    *count = r.count;
}
void geom_work_of_xcd(int block_id, int bh_count, int n_qblocks, int causal, int* bh, int* qb) {
    const g::Work w = g::work_of_xcd(block_id, bh_count, n_qblocks, causal != 0);
    *bh = w.bh;
    *qb = w.qb;
}
void geom_work_of_xcd_grouped(int block_id, int bh_count, int n_qblocks, int group_heads,
                              int* bh, int* qb) {
    const g::Work w = g::work_of_xcd(block_id, bh_count, n_qblocks, true, group_heads);
    *bh = w.bh;
    *qb = w.qb;
}
int geom_causal_group_heads(int head_dim, long long bh_count) {
    return g::causal_group_heads(head_dim, bh_count);
}
long long geom_causal_singles_makespan(long long bh_count, int n_qblocks, int slots) {
    return g::causal_singles_makespan(bh_count, n_qblocks, slots);
}
int geom_causal_pairs_pay(long long bh_count, int n_qblocks, int slots) {
    return g::causal_pairs_pay(bh_count, n_qblocks, slots) ? 1 : 0;
}
void geom_causal_pair(int block_id, int bh_count, int n_qblocks, int* bh, int* qb_long,
                      int* qb_short) {
    const g::PairWork w = g::causal_pair(block_id, bh_count, n_qblocks);
    *bh = w.bh;
    *qb_long = w.qb_long;
    *qb_short = w.qb_short;
}
void geom_work_of(int block_id, int bh_count, int n_qblocks, int causal, int* bh, int* qb) {
    const g::Work w = g::work_of(block_id, bh_count, n_qblocks, causal != 0);
    *bh = w.bh;
    *qb = w.qb;
}
}
