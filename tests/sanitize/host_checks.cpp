// Host-side checks run under AddressSanitizer and UndefinedBehaviorSanitizer
// (tests/test_host_sanitizers.py builds this file with -fsanitize=address,undefined; the
// counterpart of the reference's host ASan/UBSan preset, cmake/Sanitizers.cmake:10-24).
//
//   geom    every function of csrc/fa_geometry.h over its lane / row / slot domain, and the
//           tile-count, mask and work-map arithmetic over sequence lengths up to 2^30, with
//           the invariants the kernels rely on;
//   oracle  oracle/attention_fp64.c on small seeded fp16 inputs, edge arguments included
//           (row 0 of a causal head, the last row, out-of-range rows, empty row lists);
//   abi     (only when built with -DWITH_ABI and linked to a sanitized libfa_hip) the host
//           paths of the C ABI: argument validation, tile choice and split-KV planning over a
//           grid of shapes, none of which touches the GPU.
//
// Exit status 0 when every check holds; a sanitizer report aborts with a non-zero status.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "fa_geometry.h"

#ifdef WITH_ABI
#include "fa_hip.h"
#endif

extern "C" {
double oracle_half_to_double(uint16_t h);
int oracle_attention_rows(const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t bh,
                          int64_t n, int64_t d, double scale, int causal, const int64_t* rows,
                          int64_t n_rows, double* out);
int oracle_lse_rows(const uint16_t* q, const uint16_t* k, int64_t bh, int64_t n, int64_t d,
                    double scale, int causal, const int64_t* rows, int64_t n_rows, double* out);
}

namespace g = fa::geom;

static int g_failures = 0;
#define CHECK(cond)                                                         \
    do {                                                                    \
        if (!(cond)) {                                                      \
            std::fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #cond); \
            ++g_failures;                                                   \
        }                                                                   \
    } while (0)

static void check_geometry() {
    for (int d : {64, 128}) {
        const int row_bytes = 2 * d, cpr = d / 8;
        // swizzles are permutations of the chunks of a row
        for (int row = 0; row < 64; ++row) {
            std::vector<int> seen(cpr, 0), seen16(cpr, 0);
            for (int c = 0; c < cpr; ++c) {
                const int p = g::swizzle_chunk(row, c, row_bytes);
                const int p16 = g::swizzle_chunk_m16(row, c, d);
                CHECK(p >= 0 && p < cpr && p16 >= 0 && p16 < cpr);
                if (p >= 0 && p < cpr) ++seen[p];
                if (p16 >= 0 && p16 < cpr) ++seen16[p16];
                CHECK(g::tile_offset(row, c, row_bytes) == row * row_bytes + 16 * p);
            }
            for (int c = 0; c < cpr; ++c) CHECK(seen[c] == 1 && seen16[c] == 1);
        }
        // the permuted K tile of the 16x16x32 path: every (row, chunk) of a tile exactly once
        const int bc = d == 128 ? 32 : 64;
        std::vector<int> hit(bc * cpr, 0);
        for (int slot = 0; slot < bc * cpr; ++slot) {
            const int r = g::m16_kslot_row(slot, d), c = g::m16_kslot_chunk(slot, d);
            CHECK(r >= 0 && r < bc && c >= 0 && c < cpr);
            if (r >= 0 && r < bc && c >= 0 && c < cpr) ++hit[r * cpr + c];
        }
        for (int x : hit) CHECK(x == 1);
    }
    for (int lane = 0; lane < 64; ++lane) {
        for (int r = 0; r < 16; ++r) CHECK(g::mfma32_c_row(lane, r) >= 0 && g::mfma32_c_row(lane, r) < 32);
        for (int r = 0; r < 4; ++r) CHECK(g::mfma16_c_row(lane, r) >= 0 && g::mfma16_c_row(lane, r) < 16);
        CHECK(g::tr16_row(lane) < 4 && g::tr16_col(lane) < 16);
        for (int kb = 0; kb < 4; ++kb)
            for (int r = 0; r < 4; ++r) CHECK(g::st16_key(lane, kb, r) >= 0 && g::st16_key(lane, kb, r) < 64);
        for (int t = 0; t < 2; ++t)
            for (int i = 0; i < 8; ++i) CHECK(g::pv16_key(lane, t, i) >= 0 && g::pv16_key(lane, t, i) < 64);
    }
    // tile counts, masks and the work map up to N = 2^30 (no signed overflow anywhere)
    const int ns[] = {1, 2, 31, 32, 33, 255, 256, 257, 1000, 4096, 16383, 16384, 65537,
                      1 << 20, (1 << 30) - 1, 1 << 30};
    for (int n : ns) {
        for (int causal = 0; causal < 2; ++causal) {
            for (int bq : {64, 128, 256}) {
                for (int bk : {32, 64}) {
                    const int nqb = g::ceil_div(n, bq);
                    for (int qb : {0, 1, nqb / 2, nqb - 1}) {
                        if (qb < 0 || qb >= nqb) continue;
                        const int q0 = qb * bq;
                        const int nt = g::num_kv_tiles(n, q0, bq, bk, causal != 0);
                        CHECK(nt >= 1 && nt <= g::ceil_div(n, bk));
                        for (int w = 0; w < bq / 32; ++w) {
                            const int qw = q0 + 32 * w;
                            const int act = g::wave_active_tiles(n, qw, 32, bk, nt, causal != 0);
                            CHECK(act >= 0 && act <= nt);
                            const int um = g::wave_unmasked_tiles(n, qw, bk, act, causal != 0);
                            CHECK(um >= 0 && um <= act);
                            for (int j = 0; j < um; ++j) {
                                CHECK(!g::tile_needs_mask(n, j * bk, bk, qw, causal != 0));
                            }
                        }
                        // split ranges partition the tiles, near-equal, in order
                        for (int tps : {1, 3, 16, 65, 1 << 20}) {
                            if (g::ceil_div(nt, tps) > 4096) continue;  // bound the loop
                            int next = 0;
                            for (int s = 0; s < g::ceil_div(nt, tps) + 2; ++s) {
                                const g::KeyRange r = g::split_range(nt, tps, s);
                                if (r.count == 0) continue;
                                CHECK(r.begin == next && r.count <= tps);
                                next = r.begin + r.count;
                            }
                            CHECK(next == nt);
                        }
                    }
                    // the work map is a bijection onto (bh, qb)
                    if (nqb <= 64) {
                        for (int bh_count : {1, 3, 16}) {
                            std::vector<int> seen(static_cast<size_t>(bh_count) * nqb, 0);
                            for (int id = 0; id < bh_count * nqb; ++id) {
                                const g::Work w = g::work_of(id, bh_count, nqb, causal != 0);
                                CHECK(w.bh >= 0 && w.bh < bh_count && w.qb >= 0 && w.qb < nqb);
                                if (w.bh >= 0 && w.bh < bh_count && w.qb >= 0 && w.qb < nqb)
                                    ++seen[static_cast<size_t>(w.bh) * nqb + w.qb];
                            }
                            for (int x : seen) CHECK(x == 1);
                        }
                    }
                }
            }
        }
    }
}

// float -> binary16 bits, round to nearest even, for the finite normal range used here
// (|x| in [2^-14, 65504]) and zero; smaller magnitudes flush to signed zero.
static uint16_t to_half_bits(float x) {
    uint32_t f;
    std::memcpy(&f, &x, 4);
    const uint32_t sign = (f >> 16) & 0x8000U;
    const int exp = static_cast<int>((f >> 23) & 0xFF) - 127 + 15;
    if (exp <= 0) return static_cast<uint16_t>(sign);
    uint32_t mant = f & 0x7FFFFFU;
    uint32_t h = (static_cast<uint32_t>(exp) << 10) | (mant >> 13);
    const uint32_t rest = mant & 0x1FFFU;
    if (rest > 0x1000U || (rest == 0x1000U && (h & 1U))) ++h;  // carries into the exponent
    return static_cast<uint16_t>(sign | h);
}

static void check_oracle() {
    // every binary16 pattern decodes without UB
    for (uint32_t h = 0; h < 65536; ++h) {
        const double x = oracle_half_to_double(static_cast<uint16_t>(h));
        const uint32_t e = (h >> 10) & 31;
        CHECK(e == 31 || std::isfinite(x));
    }
    uint64_t state = 12345;
    auto rnd = [&]() {
        state = state * 6364136223846793005ULL + 1442695040888963407ULL;
        return static_cast<float>((state >> 40) & 0xFFFF) / 32768.0F - 1.0F;
    };
    for (int d : {64, 128}) {
        for (int n : {1, 2, 17, 65}) {
            const int bhs = 3;
            const size_t elems = static_cast<size_t>(bhs) * n * d;
            std::vector<uint16_t> q(elems), k(elems), v(elems);
            for (size_t i = 0; i < elems; ++i) {
                q[i] = to_half_bits(rnd());
                k[i] = to_half_bits(rnd());
                v[i] = to_half_bits(rnd());
            }
            for (int causal = 0; causal < 2; ++causal) {
                for (int bh = 0; bh < bhs; ++bh) {
                    std::vector<int64_t> rows;
                    for (int i = 0; i < n; ++i) rows.push_back(i);
                    std::vector<double> out(rows.size() * d), lse(rows.size());
                    CHECK(oracle_attention_rows(q.data(), k.data(), v.data(), bh, n, d,
                                                1.0 / std::sqrt(d), causal, rows.data(),
                                                static_cast<int64_t>(rows.size()), out.data()) == 0);
                    CHECK(oracle_lse_rows(q.data(), k.data(), bh, n, d, 1.0 / std::sqrt(d), causal,
                                          rows.data(), static_cast<int64_t>(rows.size()),
                                          lse.data()) == 0);
                    if (causal) {  // row 0 sees key 0 only: O = V[0]
                        for (int c = 0; c < d; ++c) {
                            CHECK(out[c] == oracle_half_to_double(
                                                v[static_cast<size_t>(bh) * n * d + c]));
                        }
                    }
                    for (double x : out) CHECK(std::isfinite(x));
                    for (double x : lse) CHECK(std::isfinite(x));
                }
                // out-of-range rows are rejected, an empty row list is fine
                const int64_t bad[] = {n};
                const int64_t neg[] = {-1};
                double sink[128];
                CHECK(oracle_attention_rows(q.data(), k.data(), v.data(), 0, n, d, 0.1, causal,
                                            bad, 1, sink) == -1);
                CHECK(oracle_lse_rows(q.data(), k.data(), 0, n, d, 0.1, causal, neg, 1, sink) == -1);
                CHECK(oracle_attention_rows(q.data(), k.data(), v.data(), 0, n, d, 0.1, causal,
                                            bad, 0, sink) == 0);
                CHECK(oracle_attention_rows(q.data(), k.data(), v.data(), 0, 0, d, 0.1, causal,
                                            bad, 0, sink) == -1);
            }
        }
    }
}

#ifdef WITH_ABI
static void check_abi() {
    fa_params p{};
    p.q = p.k = p.v = reinterpret_cast<const void*>(0x1000);
    p.o = reinterpret_cast<void*>(0x2000);
    p.softmax_scale = 0.125F;
    CHECK(fa_flash_fwd(nullptr, nullptr) == FA_EINVAL && std::strlen(fa_last_error()) > 0);
    const int64_t dims[] = {-1, 0, 1, 2, 3, 16, 255, 256, 1000, 4095, 4096, 16384, 65535, 70000,
                            1 << 20, INT32_MAX};
    fa_tile_info tile{};
    fa_splitkv_info info{};
    int checked = 0;
    for (int64_t b : {int64_t(-1), int64_t(0), int64_t(1), int64_t(4), int64_t(70000)}) {
        for (int64_t h : {int64_t(0), int64_t(1), int64_t(16), int64_t(1) << 12}) {
            for (int64_t n : dims) {
                for (int d : {0, 64, 96, 128}) {
                    for (int causal = 0; causal < 3; ++causal) {
                        for (int var = 0; var < 4; ++var) {
                            p.batch = static_cast<int32_t>(b);
                            p.heads = static_cast<int32_t>(h);
                            p.seqlen = static_cast<int32_t>(n);
                            p.head_dim = d;
                            p.causal = static_cast<uint8_t>(causal);
                            p.variant = static_cast<uint8_t>(var);
                            const bool valid_dims = b > 0 && h > 0 && n > 0 &&
                                                    (d == 64 || d == 128) && n * d <= INT32_MAX;
                            const int rt = fa_tile_config(&p, &tile);
                            CHECK(rt == FA_OK || rt == FA_EINVAL);
                            if (rt == FA_OK) CHECK(tile.block_q > 0 && tile.block_k > 0);
                            const int rp = fa_splitkv_plan(&p, var == 3 ? 5 : 0, &info);
                            CHECK(rp == (valid_dims ? FA_OK : FA_EINVAL));
                            if (rp == FA_OK) {
                                CHECK(info.num_splits >= 1 && info.tiles_per_split >= 1);
                                CHECK(info.preferred == 0 || info.preferred == 1);
                            }
                            // invalid parameter sets are rejected before any HIP call; valid
                            // ones are never launched here (no GPU in this process)
                            const bool would_launch = valid_dims && causal < 2 && var < 3 &&
                                                      b * h * ((n + 63) / 64) <= INT32_MAX;
                            if (!would_launch) {
                                CHECK(fa_flash_fwd(&p, nullptr) == FA_EINVAL);
                                CHECK(fa_flash_fwd_lse(&p, reinterpret_cast<float*>(0x3000),
                                                       nullptr) == FA_EINVAL);
                                CHECK(fa_flash_fwd_splitkv(&p, nullptr, 0,
                                                           reinterpret_cast<void*>(0x4000),
                                                           ~0ULL, nullptr) == FA_EINVAL);
                                CHECK(fa_flash_fwd_splitkv_static(&p, nullptr, 0, nullptr) ==
                                      FA_EINVAL);
                                CHECK(std::strlen(fa_last_error()) > 0);
                                ++checked;
                            }
                        }
                    }
                }
            }
        }
    }
    CHECK(checked > 1000);
    CHECK(std::strstr(fa_version(), "gfx950") != nullptr);
}
#endif

int main(int argc, char** argv) {
    // parts to run: "geom", "oracle", "abi" (default: every part built in)
    auto want = [&](const char* part) {
        if (argc < 2) return true;
        for (int a = 1; a < argc; ++a)
            if (std::strcmp(argv[a], part) == 0) return true;
        return false;
    };
    if (want("geom")) check_geometry();
    if (want("oracle")) check_oracle();
#ifdef WITH_ABI
    if (want("abi")) check_abi();
#endif
    std::printf("host checks: %d failures\n", g_failures);
    return g_failures == 0 ? 0 : 1;
}
