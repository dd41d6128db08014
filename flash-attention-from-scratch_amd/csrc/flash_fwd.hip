// FlashAttention-2 forward for AMD MI355X (gfx950, CDNA4), written for the hardware:
//
//   O = softmax(Q K^T * scale) V        Q, K, V, O: [B, H, N, D] fp16, fp32 accumulation
//
// Work decomposition
//   * A workgroup of NW wave64s owns BR = 32*NW consecutive query rows of one (batch, head);
//     each wave owns 32 of them for the whole kernel, so a row's softmax statistics never leave
//     the wave (the FA2 split-Q scheme of csrc/kernels/flash_fwd.cu:7-12).
//   * The workgroup streams over keys in tiles of BC rows, double-buffered in LDS and filled by
//     buffer_load_dwordx4 ... lds (direct HBM/L2 -> LDS, no VGPR staging): the next tiles are
//     in flight while tile j is computed, with one workgroup barrier per tile.
//
// Per tile and wave, on CDNA4 matrix cores:
//   * S^T = K Q^T with v_mfma_f32_32x32x16_f16: A = K rows (read from swizzled LDS with
//     ds_read_b128), B = Q^T (held in VGPRs for the whole kernel, loaded once). Computing the
//     transpose puts one query column in each lane: lane l holds query l%32 and 16 keys per
//     32-key block, so the row max is an in-lane max plus one v_permlane32_swap.
//   * Online softmax in base 2 in fp32 (v_exp_f32), with conditional ("lazy") rescaling of O.
//   * O^T += V^T P^T with the same MFMA: the S^T accumulator of a lane is already in the B
//     operand layout of this product (same query column, 8 keys per 16-key step), so P is
//     converted to fp16 in place and never moves. V^T comes from LDS through the gfx950
//     transposing read ds_read_b64_tr_b16, which hands each lane 4 consecutive keys of one
//     feature column.
//   * The long-sequence rows (flash_fwd_pingpong16) do the same work on v_mfma_f32_16x16x32_f16,
//     two MFMAs per 32x32x16 one: at MI355X's power limit that shape sustains about 20 % more
//     FLOPS. Each lane then holds 4 keys of two queries per 16-key block; row statistics span the
//     four lanes of a query (v_permlane16_swap and v_permlane32_swap).
//   * Causal: tiles right of the diagonal are never loaded; masking runs only on diagonal and
//     tail tiles; longest query blocks launch first.
//   * Ragged N: the buffer resource of a K/V tile ends at row N, so rows >= N arrive as zeros
//     (their scores are masked to -inf and contribute exactly 0); Q row indices are clamped to
//     N-1 and the clamped rows are never stored.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>
#include <utility>

#include "fa_device.h"
#include "fa_geometry.h"
#include "fa_hip.h"

// Workspace of fa_flash_fwd_splitkv_static (see static_scratch below): FA_STATIC_SCRATCH_BYTES
// (fa_hip.h) per GPU.
static __device__ __align__(256) float scratch[FA_STATIC_SCRATCH_BYTES / sizeof(float)];

// Overflow record of the ping-pong's unchecked softmax, per GPU: the id of a launch (high 32
// bits; every launch gets a new one, never 0) and the number of its workgroups that had to redo
// an item with the checked softmax (low 32). A workgroup of the same launch that starts after
// FA_PP16_ADAPT_WGS of them runs its items checked from the start. Best effort: workgroups of
// the first round start before any overflow is known, and counts of launches that run at once
// on other streams can be dropped.
static __device__ unsigned long long pp_overflow_record;

// Timeline probe, a development build option (off in the library): with FA_PROBE 1 wave 0 of
// every ping-pong workgroup writes the 100 MHz constant clock (s_memrealtime) at fixed points
// of its items, and its CU and XCC ids, into probe_stamps[blockIdx.x * 32 + slot];
// fa_probe_clear / fa_probe_read (exported only by such a build) hand the array to the host
// (dev/fa_dev --probe, summarized by dev/probe.py). Slots: 0 kernel entry; per item i (0, 1),
// 1 + 5i its first pass starts, 2 + 5i the prologue's loads have landed (after its barrier),
// 3 + 5i the steady tiles are done, 4 + 5i the last tile is done, 5 + 5i the O stores are
// issued; 12 a second pass starts; 11 and 13 the shader clock's cycle count (s_memtime) at the
// workgroup's entry and end; 14 HW_ID; 15 XCC_ID; and within item i's phases, 16 + 5i the
// prologue's loads are issued, 17 + 5i they have landed (the wave's own wait, before the
// barrier), 18 + 5i the first tile's S is computed, 19 + 5i the first steady tile is done,
// 20 + 5i the item's final test has passed its barrier.
#ifndef FA_PROBE
#define FA_PROBE 0
#endif
#if FA_PROBE
constexpr int kProbeSlots = 32;
constexpr unsigned kProbeWorkgroups = 1U << 16;
static __device__ unsigned long long probe_stamps[kProbeWorkgroups * kProbeSlots];
#endif

namespace fa {
namespace {

constexpr float kLn2 = 0.693147180559945309F;  // converts base-2 LSEs to natural log

using namespace fa::dev;
namespace g = fa::geom;

// Compile-time tile shape and options. Counterpart of the reference's Config/Opt pair
// (csrc/kernels/flash_fwd.cu:70-100), re-derived for 64-wide waves and 32x32 MFMA blocks.
// FA_OPTIMISTIC 1: the simple and key-split tiles with lazy rescale first take p against the
// running max, without the tile's row max, and fall back to the exact softmax of the tile only
// if some p overflows fp16 (softmax_any); 0: the exact softmax in every tile.
#ifndef FA_OPTIMISTIC
#define FA_OPTIMISTIC 1
#endif

// Causal ping-pong grids of workgroups that each run a (long, short) pair of query blocks of
// one head (fa::geom::causal_pair; not in split-KV passes), where fa::geom::causal_pairs_pay
// finds that they end no later than single query blocks; 0 runs single blocks always.
#ifndef FA_CAUSAL_PAIRS
#define FA_CAUSAL_PAIRS 1
#endif

// Main-loop schedules: SIMPLE (flash_fwd_kernel: each wave runs QK, softmax and PV of a tile in
// turn, on 32x32x16 MFMAs), SIMPLE16 (flash_fwd_simple16: the same schedule with the ping-pong's
// 16x16x32 tile math), KSPLIT / KSPLIT4 (flash_fwd_ksplit: two or four waves per 32 query rows,
// each on every second or fourth key tile), PINGPONG16 (flash_fwd_pingpong16: two groups of
// waves alternate between an MFMA-only phase and a softmax phase, on 16x16x32 MFMAs; the table's
// long d = 128 rows). The values are fa_tile_info's `schedule` (fa_schedule) and the names the
// -D tile overrides use.
enum Sched {
    SIMPLE = FA_SCHED_SIMPLE,
    KSPLIT = FA_SCHED_KSPLIT,
    PINGPONG16 = FA_SCHED_PINGPONG16,
    KSPLIT4 = FA_SCHED_KSPLIT4,
    SIMPLE16 = FA_SCHED_SIMPLE16
};

// K/V buffers of the simple schedule: 2 (refill one tile ahead, wait for all DMA at each tile)
// or 3 (two tiles ahead; a tile waits only for its own DMA, the next tile's stays in flight).
#ifndef FA_SIMPLE_NBUF
#define FA_SIMPLE_NBUF 2
#endif
static_assert(FA_SIMPLE_NBUF == 2 || FA_SIMPLE_NBUF == 3, "two or three K/V buffers");
// Wave priority of the simple tile's matrix work, per head size: bit 0 raises it (s_setprio 1)
// while a wave issues its S = QK^T MFMAs, bit 1 while it issues its O += PV MFMAs; 0 leaves
// every wave at priority 0. Bit 0 measured +1 to +2 % on the d=128 tiles; at d=64 no setting
// changed the many-heads causal shape by more than 0.3 %.
#ifndef FA_SIMPLE_PRIO_D64
#define FA_SIMPLE_PRIO_D64 0
#endif
#ifndef FA_SIMPLE_PRIO_D128
#define FA_SIMPLE_PRIO_D128 1
#endif

template <int D_, int BC_, int NW_, bool LAZY_, int SCHED_>
struct Tile {
    static constexpr int D = D_;            // head dim (64 or 128)
    static constexpr int BC = BC_;          // keys per K/V tile
    static constexpr int NW = NW_;          // wave64s per workgroup
    static constexpr bool LAZY = LAZY_;     // rescale O only when a row max grows by > 2^8
    static constexpr int SCHED = SCHED_;    // main-loop schedule (Sched)
    static constexpr int BR = 32 * NW;      // query rows per workgroup
    static constexpr int KS =  // waves per 32 query rows (key parts)
        SCHED == KSPLIT ? 2 : (SCHED == KSPLIT4 ? 4 : 1);
    static constexpr int THREADS = 64 * NW * KS;
    static constexpr int ROW_BYTES = 2 * D;
    static constexpr int CPR = D / 8;                  // 16-byte chunks per row
    static constexpr int TILE_BYTES = BC * ROW_BYTES;  // one K or V tile
    static constexpr bool M16 = SCHED == PINGPONG16 || SCHED == SIMPLE16;  // 16x16x32 layouts
    static constexpr int NBUF =  // per K, V (the simple schedule's third only within 64 KiB)
        SCHED == PINGPONG16 ? 3
                            : ((SCHED == SIMPLE || SCHED == SIMPLE16) && 6 * TILE_BYTES <= 64 * 1024
                                   ? FA_SIMPLE_NBUF
                                   : 2);
    static constexpr int LDS_BYTES = 2 * NBUF * TILE_BYTES * KS;
    static constexpr int NB = BC / 32;                 // 32-key MFMA blocks per tile
    static constexpr int KK = D / 16;                  // 16-deep MFMA steps over D
    static constexpr int DB = D / 32;                  // 32-wide output blocks over D
    static constexpr int DMA_ITERS = (BC * CPR) / (64 * NW);
    static_assert(D == 64 || D == 128, "head dim must be 64 or 128");
    static_assert(BC % 32 == 0, "BC must be a multiple of the 32-key MFMA block");
    static_assert((BC * CPR) % (64 * NW) == 0, "tile must split evenly over the waves");
    static_assert(LDS_BYTES <= (KS == 4 ? 160 : 64) * 1024, "static LDS budget");
};

// DMA plan of one wave for a K or V tile: DMA_ITERS 16-byte-per-lane buffer->LDS copies, each
// filling 64 consecutive physical chunk slots of the swizzled tile; the lane reads the global
// chunk whose swizzled home is its slot. Offsets are relative to the tile's first row.
// KLAYOUT: the K-tile layout of the 16x16x32 path (fa::geom::m16_kslot_row / _chunk).
template <class T, bool KLAYOUT = false>
struct TileDma {
    int voff[T::DMA_ITERS];  // byte offset of the lane's source chunk
    int lds0[T::DMA_ITERS];  // wave-uniform LDS byte offset of the wave's 64 slots
    __device__ __forceinline__ TileDma(int wave, int lane) {
#pragma unroll
        for (int it = 0; it < T::DMA_ITERS; ++it) {
            const int slot0 = (it * T::NW + wave) * 64;
            const int slot = slot0 + lane;
            int row = slot / T::CPR;
            int chunk;
            if (KLAYOUT) {
                row = g::m16_kslot_row(slot, T::D);
                chunk = g::m16_kslot_chunk(slot, T::D);
            } else {
                chunk = T::M16 ? g::swizzle_chunk_m16(row, slot % T::CPR, T::D)
                               : g::swizzle_chunk(row, slot % T::CPR, T::ROW_BYTES);
            }
            voff[it] = row * T::ROW_BYTES + 16 * chunk;
            lds0[it] = slot0 * 16;
        }
    }
};

// Copies K or V rows [kt, kt + BC) of one head into a swizzled LDS tile. The buffer resource
// covers rows [kt, n) only, so rows >= n are zero-filled by the hardware range check (their
// scores are masked, and zero V rows keep 0 * garbage from ever forming a NaN); the per-tile
// offset lives in the scalar resource, so a refill costs no VALU work.
template <class T, bool KL = false>
__device__ __forceinline__ void load_tile(const f16* head, int kt, int n, char* lds,
                                          const TileDma<T, KL>& dma) {
    const char* base = reinterpret_cast<const char*>(head) + static_cast<size_t>(kt) * T::ROW_BYTES;
    const auto rsrc = make_rsrc(base, static_cast<unsigned>(max(0, n - kt)) * T::ROW_BYTES);
#pragma unroll
    for (int it = 0; it < T::DMA_ITERS; ++it) lds_dma16_buf(rsrc, dma.voff[it], lds + dma.lds0[it]);
}

// ---- per-wave building blocks -----------------------------------------------------------------
// Lane-dependent LDS offsets of the MFMA operands. The row XOR depends on row % 16 only and
// every row offset added later (32-key blocks, 16-key steps) is a multiple of 16 rows, so those
// become immediate offsets of the ds_read instructions.
template <class T>
struct Frag {
    int koff[T::KK];     // K fragment kk: row lane%32, logical chunk 2*kk + lane/32
    int voff[T::DB][2];  // V^T fragment (db, e): rows 8e + 4*(lane/32) + tr16_row, 16 columns
    __device__ __forceinline__ explicit Frag(int lane) {
        const int col = lane & 31;
        const int hi = lane >> 5;
#pragma unroll
        for (int kk = 0; kk < T::KK; ++kk) koff[kk] = g::tile_offset(col, 2 * kk + hi, T::ROW_BYTES);
#pragma unroll
        for (int db = 0; db < T::DB; ++db)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int row = 8 * e + 4 * hi + g::tr16_row(lane);
                const int c = 32 * db + 16 * ((lane >> 4) & 1) + g::tr16_col(lane);  // halves
                voff[db][e] = g::tile_offset(row, c >> 3, T::ROW_BYTES) + 2 * (c & 7);
            }
    }
};

// Q^T operand: lane holds Q[qrow][16*kk + 8*(lane/32) .. +7] for every kk (32 VGPRs at D=128).
template <class T>
__device__ __forceinline__ void load_q(const f16* qh, int qrow, int n, int lane, int negate_q,
                                       f16x8 (&qf)[T::KK]) {
    const f16* src = qh + static_cast<size_t>(min(qrow, n - 1)) * T::D + 8 * (lane >> 5);
#pragma unroll
    for (int kk = 0; kk < T::KK; ++kk) qf[kk] = *reinterpret_cast<const f16x8*>(src + 16 * kk);
    if (negate_q) {
#pragma unroll
        for (int kk = 0; kk < T::KK; ++kk) qf[kk] = -qf[kk];
    }
}

// S^T = K Q^T for one tile: NB x KK MFMAs, K fragments from LDS.
template <class T>
__device__ __forceinline__ void qk_tile(const char* kl, const Frag<T>& fr,
                                        const f16x8 (&qf)[T::KK], f32x16 (&s)[T::NB]) {
#pragma unroll
    for (int nb = 0; nb < T::NB; ++nb) {
        s[nb] = f32x16{};
#pragma unroll
        for (int kk = 0; kk < T::KK; ++kk) {
            const f16x8 a =
                *reinterpret_cast<const f16x8*>(kl + fr.koff[kk] + nb * 32 * T::ROW_BYTES);
            s[nb] = mfma32(a, qf[kk], s[nb]);
        }
    }
}

// Keys >= n, and (causal) keys right of the lane's query, get -inf: one lane threshold, then a
// compare against each accumulator's compile-time key offset and a select per score.
template <class T, bool CAUSAL>
__device__ __forceinline__ void mask_tile(f32x16 (&s)[T::NB], int kt, int n, int qrow, int lane) {
    const int lim = g::st_mask_limit(n, kt, qrow, lane, CAUSAL);
#pragma unroll
    for (int nb = 0; nb < T::NB; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[nb][r] = g::st_key(0, nb, r) > lim ? -INFINITY : s[nb][r];
}

// Online softmax of one tile in base 2 (csrc/kernels/flash_fwd.cu:347-422 is the reference's).
// Updates the running max m and the lane's partial row sum l, and returns in `rescale`
// (wave-uniform) whether O must be multiplied by `alpha` before this tile's P.V is added.
// Without LAZY, O is rescaled whenever a row max grows; with LAZY only when one grows by more
// than 8 (log2 units), otherwise the stale max stays in use and p may reach 2^8 (exact: l and
// O see the same p). Selects instead of branches keep this straight-line code.
template <class T>
__device__ __forceinline__ void softmax_tile(const f32x16 (&s)[T::NB], float scale_log2,
                                             float& m_run, float& l_run, float& alpha,
                                             bool& rescale, f16x8 (&p)[T::NB][2]) {
    float mx = -INFINITY;
#pragma unroll
    for (int nb = 0; nb < T::NB; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[nb][r]);
    mx = max_xor32(mx) * scale_log2;  // both halves of the wave agree on the query's tile max
    rescale = wave_any(T::LAZY ? (mx > m_run + 8.0F) : (mx > m_run));
    const float m_new = rescale ? fmaxf(m_run, mx) : m_run;
    // m_new is -inf only for a row that has seen nothing but masked keys; use 0 there so that
    // -inf - -inf never forms a NaN (its p values are exp2(-inf) = 0).
    const float m_use = (m_new == -INFINITY) ? 0.0F : m_new;
    alpha = exp2_fast(m_run - m_use);
    m_run = m_new;
    // The row sum is taken over the fp16 P values the P.V MFMA consumes (v_dot2 with fp32
    // accumulation), so numerator and denominator of O see identical weights.
    float sum = 0.0F;
#pragma unroll
    for (int nb = 0; nb < T::NB; ++nb) {
        float e[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) e[r] = exp2_fast(fmaf(s[nb][r], scale_log2, -m_use));
        p[nb][0] = pack8(e[0], e[1], e[2], e[3], e[4], e[5], e[6], e[7]);
        p[nb][1] = pack8(e[8], e[9], e[10], e[11], e[12], e[13], e[14], e[15]);
        sum = sum8_f16(p[nb][1], sum8_f16(p[nb][0], sum));
    }
    l_run = (rescale ? l_run * alpha : l_run) + sum;
}

template <class T>
__device__ __forceinline__ void rescale_o(f32x16 (&oacc)[T::DB], float alpha) {
#pragma unroll
    for (int db = 0; db < T::DB; ++db) oacc[db] *= alpha;
}

// Optimistic softmax of one tile (LAZY tiles): p = exp2(s*c - m) against the running max m,
// without the tile's row max. If some p of the wave reaches 65520 (a score above m by 16 log2
// units or more; also the first tile, where m = -inf, and a row whose keys are all masked so
// far, where -inf - -inf is NaN), the fp16 pack gives inf or NaN and so does the lane's row sum:
// `overflow` is set (wave-uniform), l is left alone and the caller redoes the tile with
// softmax_tile. Otherwise every p lies in [0, 65504], held by fp16 at its usual precision and by
// the fp32 accumulators of O and l, so the result is the same softmax against a different valid
// reference point. Each group of 8 exponentials is packed at once, which keeps 8 temporaries
// live instead of 16 * NB (the simple d=64 tiles must stay within 128 VGPRs for four waves per
// SIMD, whose interleaving hides the exponentials' latency).
template <class T>
__device__ __forceinline__ void softmax_optimistic(const f32x16 (&s)[T::NB], float scale_log2,
                                                   float m_run, float& l_run, bool& overflow,
                                                   f16x8 (&p)[T::NB][2]) {
    float sum0 = 0.0F;
    float sum1 = 0.0F;
#pragma unroll
    for (int nb = 0; nb < T::NB; ++nb)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float e[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) e[r] = exp2_fast(fmaf(s[nb][8 * h + r], scale_log2, -m_run));
            p[nb][h] = pack8(e[0], e[1], e[2], e[3], e[4], e[5], e[6], e[7]);
            if (h == 0) {
                sum0 = sum8_f16(p[nb][h], sum0);
            } else {
                sum1 = sum8_f16(p[nb][h], sum1);
            }
        }
    const float sum = sum0 + sum1;
    overflow = wave_any(!(sum < INFINITY));
    l_run = overflow ? l_run : l_run + sum;
}

// Softmax of one tile for the simple and key-split schedules: optimistic first when the tile
// is LAZY (FA_OPTIMISTIC), exact (softmax_tile, with the rescale of O) when that overflows or
// the tile is not LAZY. FIRST marks the first tile of the item, which the callers peel off
// their loops: its running max is -inf, so the optimistic pass would always overflow, and O is
// still zero, so it needs no rescale; both are left out there. (A run-time flag instead costs
// the d=128 causal simple tile 68 VGPRs and a third of its occupancy.)
template <class T, bool FIRST>
__device__ __forceinline__ void softmax_any(const f32x16 (&s)[T::NB], float scale_log2,
                                            float& m_run, float& l_run, f32x16 (&oacc)[T::DB],
                                            f16x8 (&p)[T::NB][2]) {
    bool exact = true;
    if constexpr (T::LAZY && FA_OPTIMISTIC && !FIRST) {
        softmax_optimistic<T>(s, scale_log2, m_run, l_run, exact, p);
    }
    if (exact) {
        float alpha;
        bool rescale;
        softmax_tile<T>(s, scale_log2, m_run, l_run, alpha, rescale, p);
        if (!FIRST && rescale) rescale_o<T>(oacc, alpha);
    }
}

// O^T += V^T P^T for one tile: NB x 2 x DB MFMAs, V^T fragments by transposed LDS reads.
template <class T>
__device__ __forceinline__ void pv_tile(const char* vl, const Frag<T>& fr,
                                        const f16x8 (&p)[T::NB][2], f32x16 (&oacc)[T::DB]) {
#pragma unroll
    for (int nb = 0; nb < T::NB; ++nb)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int db = 0; db < T::DB; ++db) {
                const char* base = vl + (32 * nb + 16 * h) * T::ROW_BYTES;
                const f16x4 lo = lds_read_tr16(base + fr.voff[db][0]);
                const f16x4 up = lds_read_tr16(base + fr.voff[db][1]);
                const f16x8 a = {lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
                oacc[db] = mfma32(a, p[nb][h], oacc[db]);
            }
}

// Base-2 log-sum-exp of the row's scaled scores, m + log2(l): the lane's running max m (the
// reference its exponentials were taken against) and the row sum l of both wave halves. l >= 1
// whenever the row saw a key (the key that set m contributed exp2(0)); -inf for a row that saw
// none (a split whose keys are all masked for it).
__device__ __forceinline__ float row_lse2(float m_run, float l_tot) {
    return l_tot > 0.0F ? m_run + __builtin_amdgcn_logf(l_tot) : -INFINITY;
}

// O = acc / l as fp16 (RNE) for the lane's query row, if it is < n. The lane holds feature
// columns 32*db + 8*rq + 4*(lane/32) + 0..3; the two wave halves, which hold the same query,
// trade half of them (pair_swap32) so that each lane writes 8 consecutive features per 16-byte
// store. If lse_h is not null, the row's natural-log LSE (log of the sum of exp(scale * q.k)
// over its keys) goes to lse_h[qrow].
template <class T>
__device__ __forceinline__ void store_o_tot(f16* oh, float* lse_h, int qrow, int n, int lane,
                                            float m_run, float l_tot,
                                            const f32x16 (&oacc)[T::DB]) {
    const float inv = (l_tot > 0.0F) ? (1.0F / l_tot) : 0.0F;
    f16x8 out[T::DB][2];
#pragma unroll
    for (int db = 0; db < T::DB; ++db)
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const f32x16& a = oacc[db];
            out[db][r] = pair_swap32(
                pack4(a[8 * r] * inv, a[8 * r + 1] * inv, a[8 * r + 2] * inv, a[8 * r + 3] * inv),
                pack4(a[8 * r + 4] * inv, a[8 * r + 5] * inv, a[8 * r + 6] * inv,
                      a[8 * r + 7] * inv));
        }
    if (qrow >= n) return;
    if (lse_h != nullptr && lane < 32) lse_h[qrow] = row_lse2(m_run, l_tot) * kLn2;
    // lower half: features 32db + 16r + 0..7, upper half: 32db + 16r + 8..15
    f16* dst = oh + static_cast<size_t>(qrow) * T::D + 8 * (lane >> 5);
#pragma unroll
    for (int db = 0; db < T::DB; ++db)
#pragma unroll
        for (int r = 0; r < 2; ++r) *reinterpret_cast<f16x8*>(dst + 32 * db + 16 * r) = out[db][r];
}

// Same, from the lane's partial row sum (its keys of each 32-key block; the two wave halves
// hold the two halves of a row's keys).
template <class T>
__device__ __forceinline__ void store_o(f16* oh, float* lse_h, int qrow, int n, int lane,
                                        float m_run, float l_run, const f32x16 (&oacc)[T::DB]) {
    store_o_tot<T>(oh, lse_h, qrow, n, lane, m_run, sum_xor32(l_run), oacc);
}

// Split-KV partial result of the lane's query row, if it is < n: O_s = acc / l in fp32 (16-byte
// stores) and the base-2 LSE of the split's keys, for the combine kernel.
template <class T>
__device__ __forceinline__ void store_partial(float* op, float* lp, int qrow, int n, int lane,
                                              float m_run, float l_run,
                                              const f32x16 (&oacc)[T::DB]) {
    const float l_tot = sum_xor32(l_run);
    const float inv = (l_tot > 0.0F) ? (1.0F / l_tot) : 0.0F;
    if (qrow >= n) return;
    if (lane < 32) lp[qrow] = row_lse2(m_run, l_tot);
    float* dst = op + static_cast<size_t>(qrow) * T::D + 4 * (lane >> 5);
#pragma unroll
    for (int db = 0; db < T::DB; ++db)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
            const f32x16& a = oacc[db];
            *reinterpret_cast<f32x4*>(dst + 32 * db + 8 * rq) =
                f32x4{a[4 * rq] * inv, a[4 * rq + 1] * inv, a[4 * rq + 2] * inv,
                      a[4 * rq + 3] * inv};
        }
}

// ---- kernel, simple schedule (the "baseline" build) -----------------------------------------
// Per tile: barrier, prefetch tile j+1, then S = QK^T, softmax, O += PV in sequence.
// SPLIT (split-KV): block id = split * (B*H*query blocks) + work item; the workgroup runs key
// range `split` of its query block (geom::split_range) and writes the partial
// O and LSE of each row to o_part / lse_part (layout [split][b*h][n][d] and [split][b*h][n]);
// a workgroup whose range is empty exits at once (the combine kernel never reads it).
template <class T, bool CAUSAL, bool SPLIT = false>
__global__ __launch_bounds__(T::THREADS) void flash_fwd_kernel(
    const f16* __restrict__ q, const f16* __restrict__ k, const f16* __restrict__ v,
    f16* __restrict__ o, float* __restrict__ lse, int n, int bh_count, int n_qblocks,
    float scale_log2, int negate_q, int tiles_per_split, float* __restrict__ o_part,
    float* __restrict__ lse_part, unsigned /*launch_id*/, int group_heads) {
    // One LDS object per buffer, and the buffer of each tile fixed at compile time (the loop is
    // unrolled by the buffer count): the compiler then sees that the refill of one buffer cannot
    // alias the reads of another and waits for a tile's DMA only at the barrier that starts the
    // tile. With one array it would wait for the next tile's refill before this tile's P.V reads.
    constexpr int NBUF = T::NBUF;
    __shared__ __attribute__((aligned(1024))) char k_lds0[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char k_lds1[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char k_lds2[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char v_lds0[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char v_lds1[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char v_lds2[T::TILE_BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = wave_uniform(threadIdx.x >> 6);
    const int items = bh_count * n_qblocks;
    const int split = SPLIT ? static_cast<int>(blockIdx.x) / items : 0;
    // One (head, query block) item: the whole single-item kernel.
    auto run_item = [&](const g::Work w) {
    const size_t head = static_cast<size_t>(w.bh) * n * T::D;
    const f16* kh = k + head;
    const f16* vh = v + head;
    const int q0 = w.qb * T::BR;
    const int qw = q0 + wave * 32;       // first query of this wave
    const int qrow = qw + (lane & 31);   // this lane's query
    const int n_all = g::num_kv_tiles(n, q0, T::BR, T::BC, CAUSAL);
    const g::KeyRange range = SPLIT ? g::split_range(n_all, tiles_per_split, split)
                                    : g::KeyRange{0, n_all};
    const int j_begin = range.begin;
    const int n_tiles = range.begin + range.count;  // absolute: tiles [j_begin, n_tiles)
    // Workgroup-uniform exit of an empty split. Compiled only into the split-KV build: in the
    // plain one the extra exit costs the causal d=64 tile 30 VGPRs (and half its occupancy).
    if (SPLIT && range.count == 0) return;

    // Tile j lives in buffer (j - j_begin) % NBUF.
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    auto kbuf = [&](auto b) {
        constexpr int B = decltype(b)::value;
        return B == 0 ? k_lds0 : (B == 1 ? k_lds1 : k_lds2);
    };
    auto vbuf = [&](auto b) {
        constexpr int B = decltype(b)::value;
        return B == 0 ? v_lds0 : (B == 1 ? v_lds1 : v_lds2);
    };

    constexpr int PRIO = T::D == 128 ? FA_SIMPLE_PRIO_D128 : FA_SIMPLE_PRIO_D64;
    const TileDma<T> dma(wave, lane);
    load_tile<T>(kh, j_begin * T::BC, n, kbuf(I0{}), dma);
    load_tile<T>(vh, j_begin * T::BC, n, vbuf(I0{}), dma);
    if constexpr (NBUF == 3) {
        if (j_begin + 1 < n_tiles) {
            load_tile<T>(kh, (j_begin + 1) * T::BC, n, kbuf(I1{}), dma);
            load_tile<T>(vh, (j_begin + 1) * T::BC, n, vbuf(I1{}), dma);
        }
    }
    f16x8 qf[T::KK];
    load_q<T>(q + head, qrow, n, lane, negate_q, qf);
    const Frag<T> fr(lane);

    f32x16 oacc[T::DB];
#pragma unroll
    for (int db = 0; db < T::DB; ++db) oacc[db] = f32x16{};
    float m_run = -INFINITY;  // running max of this lane's query, log2 domain (scaled)
    float l_run = 0.0F;       // this lane's partial row sum (its 16 keys of each 32-key block)

    // Tile j in buffer B: its DMA landed (with three buffers the next tile's may still be in
    // flight: its 2 * DMA_ITERS requests are the newest), barrier, refill of the buffer read by
    // the previous tile with tile j + NBUF - 1, then S = QK^T, mask, softmax and O += PV.
    auto tile = [&](int j, auto b, auto first) {
        constexpr int B = decltype(b)::value;
        using Refill = std::integral_constant<int, (B + NBUF - 1) % NBUF>;
        if (NBUF == 3 && j > j_begin && j + 1 < n_tiles) {
            // vmcnt(2 * DMA_ITERS) lgkmcnt(0): only the next tile's requests stay in flight
            // (the first tile also waits for the Q loads issued after its DMA)
            __builtin_amdgcn_s_waitcnt(static_cast<short>(0x0070 | (2 * T::DMA_ITERS)));
        } else {
            wait_vmem();
        }
        __syncthreads();  // tile j is in LDS for every wave; tile j-1's buffers are free
        if (j + NBUF - 1 < n_tiles) {
            load_tile<T>(kh, (j + NBUF - 1) * T::BC, n, kbuf(Refill{}), dma);
            load_tile<T>(vh, (j + NBUF - 1) * T::BC, n, vbuf(Refill{}), dma);
        }
        const int kt = j * T::BC;
        if (qw >= n || g::tile_fully_masked(kt, qw, 32, CAUSAL)) return;  // wave-uniform
        f32x16 s[T::NB];
        if constexpr (PRIO & 1) __builtin_amdgcn_s_setprio(1);
        qk_tile<T>(kbuf(b), fr, qf, s);
        if constexpr (PRIO & 1) __builtin_amdgcn_s_setprio(0);
        if (g::tile_needs_mask(n, kt, T::BC, qw, CAUSAL)) mask_tile<T, CAUSAL>(s, kt, n, qrow, lane);
        f16x8 p[T::NB][2];
        softmax_any<T, decltype(first)::value>(s, scale_log2, m_run, l_run, oacc, p);
        if constexpr (PRIO & 2) __builtin_amdgcn_s_setprio(1);
        pv_tile<T>(vbuf(b), fr, p, oacc);
        if constexpr (PRIO & 2) __builtin_amdgcn_s_setprio(0);
    };
    // The item has at least one tile (an empty split returned above); the first is peeled off.
    using Later = std::false_type;
    tile(j_begin, I0{}, std::true_type{});
    int j = j_begin + 1;
    if constexpr (NBUF == 3) {
        for (; j + 3 <= n_tiles; j += 3) {
            tile(j, I1{}, Later{});
            tile(j + 1, I2{}, Later{});
            tile(j + 2, I0{}, Later{});
        }
        if (j < n_tiles) tile(j, I1{}, Later{});
        if (j + 1 < n_tiles) tile(j + 1, I2{}, Later{});
    } else {
        for (; j + 2 <= n_tiles; j += 2) {
            tile(j, I1{}, Later{});
            tile(j + 1, I0{}, Later{});
        }
        if (j < n_tiles) tile(j, I1{}, Later{});
    }
    if constexpr (SPLIT) {
        const size_t part = static_cast<size_t>(split) * bh_count + w.bh;
        store_partial<T>(o_part + part * n * T::D, lse_part + part * n, qrow, n, lane, m_run,
                         l_run, oacc);
    } else {
        store_o<T>(o + head, lse ? lse + static_cast<size_t>(w.bh) * n : nullptr, qrow, n, lane,
                   m_run, l_run, oacc);
    }
    };
    // (A causal grid of (long, short) query-block pairs, as the ping-pong runs, measured 2-9 %
    // slower for this schedule on most shapes: its two or more workgroups per CU already hide
    // the dispatch gaps that the pairs remove.)
    run_item(SPLIT ? g::work_of(static_cast<int>(blockIdx.x) - split * items, bh_count,
                                n_qblocks, CAUSAL)
                   : g::work_of_xcd(blockIdx.x, bh_count, n_qblocks, CAUSAL, group_heads));
}

// Split-KV combine: for each row, LSE = log2-sum-exp2 of the splits' base-2 LSEs, and
// O = sum_s 2^(lse_s - LSE) O_s. Splits past a causal row block's last key tile were never
// run and are not read. One thread per 8 features of a row (one 16-byte store).
template <int D>
struct CombineGeom {
    static constexpr int TPR = D / 8;          // threads per row
    static constexpr int ROWS = 256 / TPR;     // rows per 256-thread block
};
template <int D>
__global__ __launch_bounds__(256) void flash_fwd_combine(
    const float* __restrict__ o_part, const float* __restrict__ lse_part, f16* __restrict__ o,
    float* __restrict__ lse, int n, int bh_count, int n_splits, int tiles_per_split, int causal,
    int block_q, int block_k) {
    constexpr int TPR = CombineGeom<D>::TPR;
    const long long row = static_cast<long long>(blockIdx.x) * CombineGeom<D>::ROWS +
                          threadIdx.x / TPR;
    if (row >= static_cast<long long>(bh_count) * n) return;
    const int c = 8 * (threadIdx.x % TPR);
    const int i = static_cast<int>(row % n);
    int splits = n_splits;
    if (causal) {
        const int kv_end = min(n, (i / block_q + 1) * block_q);
        splits = min(n_splits, g::ceil_div(g::ceil_div(kv_end, block_k), tiles_per_split));
    }
    const size_t plane = static_cast<size_t>(bh_count) * n;  // rows per split
    float m = -INFINITY;
    for (int s = 0; s < splits; ++s) m = fmaxf(m, lse_part[s * plane + row]);
    float wsum = 0.0F;
    f32x4 acc0{}, acc1{};
    for (int s = 0; s < splits; ++s) {
        const float wgt = exp2_fast(lse_part[s * plane + row] - m);
        const float* src = o_part + (s * plane + row) * D + c;
        wsum += wgt;
        acc0 += wgt * *reinterpret_cast<const f32x4*>(src);
        acc1 += wgt * *reinterpret_cast<const f32x4*>(src + 4);
    }
    const float inv = 1.0F / wsum;  // >= 1: the split holding the row's max weighs 1
    *reinterpret_cast<f16x8*>(o + row * D + c) =
        pack8(acc0[0] * inv, acc0[1] * inv, acc0[2] * inv, acc0[3] * inv, acc1[0] * inv,
              acc1[1] * inv, acc1[2] * inv, acc1[3] * inv);
    if (lse != nullptr && c == 0) lse[row] = (m + __builtin_amdgcn_logf(wsum)) * kLn2;
}

// ---- kernel, key-split schedule (small grids) --------------------------------------------------
// KS waves per 32 query rows (KS = 2, or 4 for grids of one workgroup per CU): wave w takes key
// tiles part, part + KS, part + 2 KS, ... of the query block (part = w / NW), each with its own
// running max, row sum and O (simple schedule per tile). At the end the parts merge pairwise
// through LDS in log2(KS) rounds, part p + d handing (m, l, O) to part p (d = KS/2, ..., 1),
// which merges them (O = 2^(m_a - m) O_a + 2^(m_b - m) O_b, l likewise); part 0 stores. KS times
// the waves of the simple schedule on the same grid, for grids too small to fill the GPU, with
// no workspace.
template <class T, bool CAUSAL>
__global__ __launch_bounds__(T::THREADS) void flash_fwd_ksplit(
    const f16* __restrict__ q, const f16* __restrict__ k, const f16* __restrict__ v,
    f16* __restrict__ o, float* __restrict__ lse, int n, int bh_count, int n_qblocks,
    float scale_log2, int negate_q, int /*tiles_per_split*/, float* /*o_part*/,
    float* /*lse_part*/, unsigned /*launch_id*/, int group_heads) {
    constexpr int KS = T::KS;
    static_assert(KS == 2 || KS == 4, "two or four key parts");
    // One LDS object per (key part, buffer) for K and V, and the buffer of each step fixed at
    // compile time (the step loop is unrolled by two): the compiler then sees that a refill
    // cannot alias the reads of the other buffer and waits for DMA only at the step barrier.
    // (Parts 2 and 3 exist only with KS = 4.) The merge reuses buffer 0 of each part.
    __shared__ __attribute__((aligned(1024))) char k00[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char k01[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char k10[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char k11[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char k20[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char k21[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char k30[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char k31[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char v00[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char v01[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char v10[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char v11[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char v20[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char v21[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char v30[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char v31[T::TILE_BYTES];
    static_assert(T::NW * 64 * 8 <= T::TILE_BYTES && T::NW * 64 * 16 * 4 <= T::TILE_BYTES,
                  "the merge's (m, l) and O blocks fit in one tile buffer each");

    const int lane = threadIdx.x & 63;
    const int wave = wave_uniform(threadIdx.x >> 6);
    const int part = wave / T::NW;  // key tiles part, part + KS, ...
    const int wq = wave % T::NW;    // which 32 query rows
    const g::Work w = g::work_of_xcd(blockIdx.x, bh_count, n_qblocks, CAUSAL, group_heads);
    const size_t head = static_cast<size_t>(w.bh) * n * T::D;
    const f16* kh = k + head;
    const f16* vh = v + head;
    const int q0 = w.qb * T::BR;
    const int qw = q0 + wq * 32;
    const int qrow = qw + (lane & 31);
    const int n_tiles = g::num_kv_tiles(n, q0, T::BR, T::BC, CAUSAL);
    const int n_steps = (n_tiles + KS - 1) / KS;
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    // Buffer b of key part H (both compile-time).
    auto kbuf = [&](auto hc, auto b) {
        constexpr int H = decltype(hc)::value;
        constexpr int B = decltype(b)::value;
        if constexpr (H == 0) return B == 0 ? k00 : k01;
        else if constexpr (H == 1) return B == 0 ? k10 : k11;
        else if constexpr (H == 2) return B == 0 ? k20 : k21;
        else return B == 0 ? k30 : k31;
    };
    auto vbuf = [&](auto hc, auto b) {
        constexpr int H = decltype(hc)::value;
        constexpr int B = decltype(b)::value;
        if constexpr (H == 0) return B == 0 ? v00 : v01;
        else if constexpr (H == 1) return B == 0 ? v10 : v11;
        else if constexpr (H == 2) return B == 0 ? v20 : v21;
        else return B == 0 ? v30 : v31;
    };
    // Calls f with the wave's part as a compile-time constant (wave-uniform branch).
    auto with_part = [&](auto&& f) {
        if constexpr (KS == 4) {
            if (part == 3) return f(std::integral_constant<int, 3>{});
            if (part == 2) return f(std::integral_constant<int, 2>{});
        }
        if (part == 1) return f(I1{});
        return f(I0{});
    };

    const TileDma<T> dma(wq, lane);
    with_part([&](auto hc) {
        constexpr int H = decltype(hc)::value;
        if (H < n_tiles) {
            load_tile<T>(kh, H * T::BC, n, kbuf(hc, I0{}), dma);
            load_tile<T>(vh, H * T::BC, n, vbuf(hc, I0{}), dma);
        }
    });
    f16x8 qf[T::KK];
    load_q<T>(q + head, qrow, n, lane, negate_q, qf);
    const Frag<T> fr(lane);

    f32x16 oacc[T::DB];
#pragma unroll
    for (int db = 0; db < T::DB; ++db) oacc[db] = f32x16{};
    float m_run = -INFINITY;
    float l_run = 0.0F;

    // Step j in buffer B = j % 2: key part H's tile KS j + H.
    auto step = [&](int j, auto hc, auto b, auto first) {
        constexpr int H = decltype(hc)::value;
        using Other = std::integral_constant<int, 1 - decltype(b)::value>;
        wait_vmem();
        __syncthreads();  // step j's tiles are in LDS; step j-1's buffers are free
        const int tn = KS * (j + 1) + H;
        if (tn < n_tiles) {
            load_tile<T>(kh, tn * T::BC, n, kbuf(hc, Other{}), dma);
            load_tile<T>(vh, tn * T::BC, n, vbuf(hc, Other{}), dma);
        }
        const int t = KS * j + H;
        const int kt = t * T::BC;
        if (t >= n_tiles || qw >= n || g::tile_fully_masked(kt, qw, 32, CAUSAL)) return;
        f32x16 s[T::NB];
        qk_tile<T>(kbuf(hc, b), fr, qf, s);
        if (g::tile_needs_mask(n, kt, T::BC, qw, CAUSAL)) mask_tile<T, CAUSAL>(s, kt, n, qrow, lane);
        f16x8 p[T::NB][2];
        softmax_any<T, decltype(first)::value>(s, scale_log2, m_run, l_run, oacc, p);
        pv_tile<T>(vbuf(hc, b), fr, p, oacc);
    };
    // wave-uniform branch; every part passes the same number of barriers. n_steps >= 1; step 0
    // (each part's first tile) is peeled off.
    with_part([&](auto hc) {
        using Later = std::false_type;
        step(0, hc, I0{}, std::true_type{});
        int j = 1;
        for (; j + 2 <= n_steps; j += 2) {
            step(j, hc, I1{}, Later{});
            step(j + 1, hc, I0{}, Later{});
        }
        if (j < n_steps) step(j, hc, I1{}, Later{});
    });

    // Merge. In round d (d = KS/2, ..., 1), part p + d (p < d) writes (m, l) to its buffer k_0
    // and then O, one 32-column block at a time, to its buffer v_0; part p merges. Lanes write
    // 8 and 16 bytes at consecutive addresses (O as four 16-byte pieces per block, piece-major),
    // which keeps every access free of bank conflicts.
    float l_tot = sum_xor32(l_run);
    const int slot = wq * 64 + lane;
    wait_vmem();
    __syncthreads();  // every wave is done with the tile buffers
#pragma unroll
    for (int d = KS / 2; d >= 1; d /= 2) {
        const bool sender = part >= d && part < 2 * d;
        const bool receiver = part < d;
        // buffers k_0 and v_0 of part src (1, 2 or 3: a sender), read by its receiver too
        auto ml_of = [&](int src) -> float* {
            if constexpr (KS == 4) {
                if (src == 3) return reinterpret_cast<float*>(k30);
                if (src == 2) return reinterpret_cast<float*>(k20);
            }
            return reinterpret_cast<float*>(k10);
        };
        auto ob_of = [&](int src) -> float* {
            if constexpr (KS == 4) {
                if (src == 3) return reinterpret_cast<float*>(v30);
                if (src == 2) return reinterpret_cast<float*>(v20);
            }
            return reinterpret_cast<float*>(v10);
        };
        if (sender) {
            *reinterpret_cast<f32x2*>(ml_of(part) + 2 * slot) = f32x2{m_run, l_tot};
        }
        __syncthreads();
        float wa = 1.0F, wb = 0.0F;
        if (receiver) {
            const f32x2 mb_lb = *reinterpret_cast<const f32x2*>(ml_of(part + d) + 2 * slot);
            const float mb = mb_lb[0];
            const float m_new = fmaxf(m_run, mb);
            // a part that saw no key has m = -inf and weighs 0; both -inf only for rows >= n
            wa = m_run == -INFINITY ? 0.0F : exp2_fast(m_run - m_new);
            wb = mb == -INFINITY ? 0.0F : exp2_fast(mb - m_new);
            l_tot = l_tot * wa + mb_lb[1] * wb;
            m_run = m_new;
        }
#pragma unroll
        for (int db = 0; db < T::DB; ++db) {
            if (sender) {
                float* ob = ob_of(part);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    *reinterpret_cast<f32x4*>(ob + 4 * (r * T::NW * 64 + slot)) =
                        f32x4{oacc[db][4 * r], oacc[db][4 * r + 1], oacc[db][4 * r + 2],
                              oacc[db][4 * r + 3]};
                }
            }
            __syncthreads();
            if (receiver) {
                const float* ob = ob_of(part + d);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const f32x4 x = *reinterpret_cast<const f32x4*>(ob + 4 * (r * T::NW * 64 + slot));
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        oacc[db][4 * r + i] = oacc[db][4 * r + i] * wa + x[i] * wb;
                    }
                }
            }
            __syncthreads();
        }
    }
    if (part == 0) {
        store_o_tot<T>(o + head, lse ? lse + static_cast<size_t>(w.bh) * n : nullptr, qrow, n,
                       lane, m_run, l_tot, oacc);
    }
}

// ---- ping-pong schedule: phase protocol ---------------------------------------------------------
// Eight waves, two groups of four: the hardware deals the waves of a workgroup round-robin to
// the four SIMDs of the CU, so waves w and w+4 share a SIMD. Every wave alternates two phases
// per K/V tile, separated by workgroup barriers:
//   softmax phase S_j: fragment reads of K_{j+1} and V_j from LDS (for the next phase),
//                      interleaved with the softmax of tile j (P_j, row sums, rare exact
//                      rescale of O) on the VALU;
//   matrix phase  M_j: S_{j+1} = K_{j+1} Q^T and O += P_j V_j (32 MFMAs per wave) and the
//                      wave's share of the K/V refill.
// Group 1 runs one phase behind group 0 (group 0: S_j in global phase 2j, M_j in 2j+1), so in
// every phase one wave of each SIMD feeds the matrix pipe while the other works on the VALU and
// the LDS, and only four waves read LDS at a time, each a whole phase ahead of its use.
// K_t and V_t live in buffer t % 3. In M_j group 0 requests K_{j+3} and V_{j+2}, group 1
// requests K_{j+4} and V_{j+3} (its M_{-1} is an extra first phase); every request must land by
// the barrier that ends the next-but-one odd phase, so each wave waits with vmcnt(2) (its two
// newest requests stay in flight) at the end of its odd phases. Each tile is thus requested 3
// or 4 phases before its first read, and replaces a tile whose last read was in an earlier
// phase. Diagonal and tail tiles are masked inside the steady phases; only the last tile, which
// has no successor to prefetch, goes through general_tiles16 afterwards.
// Wave priorities (s_setprio) of the ping-pong's matrix phase and softmax phase.
#ifndef FA_PP_PRIO
#define FA_PP_PRIO 1
#endif
#ifndef FA_PP_SPRIO
#define FA_PP_SPRIO 0
#endif
// Scheduler pattern: F DS reads, then N times {R DS reads, V VALU instructions}
// (sched_group_barrier masks 0x100 DS read, 0x002 VALU | 0x400 transcendental).
template <int R, int V, int N, int F = 0>
__device__ __forceinline__ void sched_reads_valu() {
    if constexpr (F > 0) __builtin_amdgcn_sched_group_barrier(0x100, F, 0);
#pragma unroll
    for (int i = 0; i < N; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, R, 0);
        __builtin_amdgcn_sched_group_barrier(0x402, V, 0);
    }
}

// End of a phase: the wave's LDS reads have completed (and, with WAIT_DMA, all but its two
// newest DMA requests), then the workgroup barrier. The waits are s_waitcnt builtins rather
// than asm so that the compiler's own wait tracking sees them (it then adds no waits of its own
// for DMA that has already landed); the empty asm statements keep LDS accesses from moving
// across. s_waitcnt immediates (gfx9 layout): vmcnt in bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8.
constexpr short WAIT_VM2_LGKM0 = 0x0072;                  // vmcnt(2) lgkmcnt(0)
constexpr short WAIT_LGKM0 = static_cast<short>(0xC07F);  // lgkmcnt(0)
template <bool WAIT_DMA>
__device__ __forceinline__ void end_phase() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(WAIT_DMA ? WAIT_VM2_LGKM0 : WAIT_LGKM0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// ---- ping-pong on 16x16x32 MFMAs (D = 128 with 32-key tiles, D = 64 with 64-key tiles) --------
// The schedule and buffer protocol above, with the matrix work on v_mfma_f32_16x16x32_f16
// (two of half the FLOPs per 32x32x16). On MI355X, which runs this
// kernel at its power limit, a stream of 16x16x32 MFMAs on random fp16 data sustains about
// 20 % more FLOPS than the same FLOPs in 32x32x16 MFMAs: the chip holds a higher clock.
// Per wave (32 queries) and key tile: S^T in 16x16 blocks s[kb][qb] (key block kb =
// fa::geom::m16_key rows, queries 16qb..), so a lane holds 4 keys of each of two queries
// (lane % 16 and 16 + lane % 16) and keeps a running max and sum per query block. P^T of query
// block qb and 32-key step t is the lane's own 8 exponentials, in the key order
// fa::geom::pv16_key that the V^T operand reads. O^T in blocks oacc[db][qb] (features 16db..,
// queries 16qb..). V tiles use the swizzle fa::geom::row_xor_m16; K tiles are stored so that
// the K operand is read at the 32x32x16 path's conflict-free addresses (m16_kslot_row).
// Fragment reads and softmax VALU of the softmax phase, as "F, R, V": F of the 24 reads first,
// then groups of {R reads, V VALU instructions} (R divides 24 - F). Non-causal tiles ask for
// 16 reads before the first exponential and 8 per 24 VALU after; the compiler then issues all
// 24 reads (8 K, 16 V^T) ahead of the softmax arithmetic: at d=128 +0.7-1.0 % over {8 reads,
// 16 VALU} on three non-causal shapes, interleaved A/B, and +0.3-0.4 % on the d=64 split-KV
// pass. (Asking for all 24 reads in one group, with the VALU left unordered, measured -5 %.)
// With the unchecked softmax, 8 per 32 VALU after the first 16 measured +0.4 % more on cfg4
// and cfg2 (+0.3-0.6 % on the split-KV passes; 40 or 48 VALU, or 20 reads first and 4 per 32,
// the same; 16 then 4 per 16: -2 %).
// The causal kernel with the per-tile checked softmax in every tile (FA_PP16_UNCHECKED 0)
// measured 0 to -0.3 % with it (and -0.2 to -1.0 % with seven other groupings) and keeps
// {8, 16}; with the unchecked softmax up to the band it takes {16, 8, 24} in every tile (+3.1 %
// on cfg4 causal, against +2.1 % with {8, 16} in every tile; {16, 8, 32}: -0.1 %).
#ifndef FA_PP16_SCHED_NC
#define FA_PP16_SCHED_NC 16, 8, 32
#endif
#ifndef FA_PP16_SCHED_CU
#define FA_PP16_SCHED_CU 16, 8, 24
#endif
#ifndef FA_PP16_SCHED
#define FA_PP16_SCHED 0, 8, 16
#endif
template <int F_, int R_, int V_>
struct ReadSched {
    static constexpr int F = F_;
    static constexpr int R = R_;
    static constexpr int V = V_;
};
template <class T, bool CAUSAL, bool CHECKED>
using PP16ReadSched = std::conditional_t<
    !CAUSAL, ReadSched<FA_PP16_SCHED_NC>,
    std::conditional_t<CHECKED, ReadSched<FA_PP16_SCHED>, ReadSched<FA_PP16_SCHED_CU>>>;
// Matrix phase: the refill goes after MFMA pair FA_PP16_MID; FA_PP16_PV_FIRST puts each pair's
// P.V MFMA before its QK^T one.
#ifndef FA_PP16_MID
#define FA_PP16_MID 1
#endif
#ifndef FA_PP16_PV_FIRST
#define FA_PP16_PV_FIRST 0
#endif
// The unchecked run tests for an overflow at the boundaries of chunks of 1, 2, 4, ... steps of
// three tiles, at most FA_PP16_EXIT_STEPS steps long (outside its inner loop, which stays the
// plain three-tile body); 0 runs it as one chunk, i.e. without the early exit.
#ifndef FA_PP16_EXIT_STEPS
#define FA_PP16_EXIT_STEPS 32
#endif
// A ping-pong workgroup runs its items checked from the start once this many workgroups of the
// same launch have had to redo an item (pp_overflow_record); 0 never does.
#ifndef FA_PP16_ADAPT_WGS
#define FA_PP16_ADAPT_WGS 8
#endif

// Flags that the waves of a workgroup share in LDS, ordered by the workgroup's barriers. Relaxed
// workgroup-scope atomics compile to ds_read / ds_write; volatile accesses compile to flat
// instructions (a volatile access keeps its generic address), which also count as
// vector-memory operations. The compiler still puts an s_waitcnt vmcnt(0) before each of these
// ds accesses (the K/V tiles arrive by buffer-to-LDS DMA, which that counter tracks, and it
// cannot tell the flags from the DMA's destinations), so a chunk-boundary test drains the K/V
// prefetches in flight. Inline ds_read_b32 / ds_write_b32 avoid that wait but measured 0.1-1.1 %
// slower on five ping-pong shapes (the prefetches have mostly landed by a chunk boundary, and
// the register assignment moved), so the atomics stay.
__device__ __forceinline__ int flag_get(const int& f) {
    return __hip_atomic_load(&f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void flag_set(int& f, int v) {
    __hip_atomic_store(&f, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// FA_PROBE stamps (no code otherwise): the clock at `slot`, and the hardware ids.
__device__ __forceinline__ void probe_stamp(int wave, int lane, int slot) {
#if FA_PROBE
    // The clock is read by every wave (a uniform value) and fed to an empty volatile asm, which
    // the compiler keeps in order with the kernel's own volatile asm (its s_waitcnt waits), so
    // the read cannot sink below the next wait.
    const unsigned long long t = __builtin_amdgcn_s_memrealtime();
    asm volatile("" ::"s"(t));
    if (wave == 0 && lane == 0 && blockIdx.x < kProbeWorkgroups) {
        probe_stamps[blockIdx.x * kProbeSlots + slot] = t;
    }
#else
    (void)wave;
    (void)lane;
    (void)slot;
#endif
}
// The shader clock's cycle count at `slot` (with the clock stamps, the workgroup's mean clock).
__device__ __forceinline__ void probe_cycles(int wave, int lane, int slot) {
#if FA_PROBE
    // (at the workgroup's entry and end only: nothing to keep in order around it)
    if (wave == 0 && lane == 0 && blockIdx.x < kProbeWorkgroups) {
        probe_stamps[blockIdx.x * kProbeSlots + slot] = __builtin_amdgcn_s_memtime();
    }
#else
    (void)wave;
    (void)lane;
    (void)slot;
#endif
}
__device__ __forceinline__ void probe_ids(int wave, int lane) {
#if FA_PROBE
    // s_getreg operand: register id | offset << 6 | (bits - 1) << 11 (HW_ID 4, XCC_ID 20)
    constexpr int kHwId = 4 | (0 << 6) | (31 << 11);
    constexpr int kXccId = 20 | (0 << 6) | (31 << 11);
    if (wave == 0 && lane == 0 && blockIdx.x < kProbeWorkgroups) {
        probe_stamps[blockIdx.x * kProbeSlots + 14] = __builtin_amdgcn_s_getreg(kHwId);
        probe_stamps[blockIdx.x * kProbeSlots + 15] = __builtin_amdgcn_s_getreg(kXccId);
    }
#else
    (void)wave;
    (void)lane;
#endif
}

// Counts one more workgroup of launch `id` in pp_overflow_record that had to redo an item (one
// lane). The first count of a launch claims the record with one compare-and-swap; every other
// count is an atomic add, which cannot fail however many workgroups count at once (a retry loop
// of compare-and-swaps let about one of them through per round). If another launch holds the
// record (launches on other streams), the count is dropped: the switch is best effort.
__device__ __forceinline__ void note_overflow(unsigned id) {
    unsigned long long cur =
        __hip_atomic_load(&pp_overflow_record, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (static_cast<unsigned>(cur >> 32) != id) {
        if (__hip_atomic_compare_exchange_strong(
                &pp_overflow_record, &cur, (static_cast<unsigned long long>(id) << 32) | 1ULL,
                __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
            return;
        }
        if (static_cast<unsigned>(cur >> 32) != id) return;  // (cur: the value found)
    }
    __hip_atomic_fetch_add(&pp_overflow_record, 1ULL, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Unchecked softmax (non-causal ping-pong): the matrix phase adds the row sums of P after MFMA
// pairs FA_PP16_SUM_PAIR, +2, ... (pair 8 measured best of 1, 4, 8, 10, 12, 13; one v_dot2
// after each pair from 6, 8 or 10 instead lost 1-3 %). FA_PP16_UNCHECKED 0 keeps the per-tile
// checked softmax in every kernel.
#ifndef FA_PP16_SUM_PAIR
#define FA_PP16_SUM_PAIR 8
#endif
#ifndef FA_PP16_UNCHECKED
#define FA_PP16_UNCHECKED 1
#endif
// The first steady tile sets the reference max m of the unchecked tiles FA_PP16_UNCHECKED_MARGIN
// (exp2 units) above its own max; a later key overflows fp16 when it exceeds the first tile's
// max by 16 + MARGIN, and a key more than 25 - MARGIN below the first tile's max rounds to 0.
// With MARGIN 0 (the default) m is a key's score, so m <= the row's true max: no p is flushed
// unless it is below 2^-25 of the row's largest p, and the row sum is at least 1 (the key at m
// gives p = 1), which bounds the weight of all flushed and subnormal p together by
// N * 2^-25 of the row sum -- the guarantee of the reference's lazy softmax, whose stale max is
// also a key's score (csrc/kernels/flash_fwd.cu:365-395). A positive MARGIN trades that for
// fewer second passes on wide score spreads: with 8, a key that dominates the first tile (an
// attention sink) pushed the other keys' p into the flush range, and at 16k keys rows lost
// up to 2.7x the north-star tolerance with no second pass (tests/test_softmax_model.py).
#ifndef FA_PP16_UNCHECKED_MARGIN
#define FA_PP16_UNCHECKED_MARGIN 0
#endif
static_assert(FA_PP16_UNCHECKED_MARGIN >= 0 && FA_PP16_UNCHECKED_MARGIN <= 8,
              "the lazy rescale (threshold 8) assumes the reference max is at most 8 above a key");
// Wide-spread items run checked from the start (exp2 units; 0 = never). The unchecked tiles
// overflow fp16 when a later key's score exceeds the first tile's row max by 16; scores whose
// spread is wide (q, k ~ N(0, 1.6^2): a standard deviation near 3.7) reach that late in a few
// rows, and such an item then redoes most of its work. The item's first tile votes: a row is
// wide if each of the four lanes holding its first 32 keys sees a score range above
// FA_PP16_SPREAD (the smallest of the four, so that one dominant key -- an attention sink, an
// outlier -- does not count: the reference max then sits at that key and later keys rarely
// pass it). On q, k ~ N(0, 1) no row of 2^18 reached 7.1; on N(0, 1.6^2) a fifth of the rows
// exceed 9, so every 256-row item is flagged (tests/test_softmax_model.py).
#ifndef FA_PP16_SPREAD
#define FA_PP16_SPREAD 9
#endif
// Per-tile geometry of the 16x16x32 path: D = 128 with 32-key tiles or D = 64 with 64-key
// tiles; either way 32 MFMAs of each kind per wave and tile and 24 fragment reads.
template <class T>
struct M16 {
    static constexpr int D = T::D;
    static constexpr int KB = T::BC / 16;  // 16-key blocks per tile
    static constexpr int QB = 2;           // 16-query blocks per wave
    static constexpr int DC = D / 32;      // 32-deep MFMA steps over D
    static constexpr int DB = D / 16;      // 16-wide feature blocks over D
    static constexpr int KS = T::BC / 32;  // 32-key steps of the P.V product
    static constexpr int ROW = 2 * D;      // bytes per K/V row
    static constexpr int READS = KB * DC + 2 * KS * DB;
    static_assert(KB * QB * DC == 16 && DB * QB * KS == 16, "16 + 16 MFMAs per wave and tile");
};

// Lane-dependent LDS offsets: K fragment (kb, dc) at the 32x32x16 path's fragment address for
// nb = kb / 2, kk = (kb % 2) * DC + dc (the K tile's own layout, fa::geom::m16_kslot_row);
// V^T fragment db: the 4 rows pv16_key(lane, 0, 0..3) (via the tr16 addressing of a 4-row
// block), 16 feature columns from 16db (the second read, keys pv16_key(lane, 0, 4..7), is 8
// rows further; k step t is 32 rows further).
template <class T>
struct Frag16 {
    using G = M16<T>;
    int koff[G::KB][G::DC];
    int voff[G::DB];
    __device__ __forceinline__ explicit Frag16(int lane) {
#pragma unroll
        for (int kb = 0; kb < G::KB; ++kb)
#pragma unroll
            for (int dc = 0; dc < G::DC; ++dc)
                koff[kb][dc] = g::tile_offset(32 * (kb >> 1) + (lane & 31),
                                              2 * ((kb & 1) * G::DC + dc) + (lane >> 5), G::ROW);
#pragma unroll
        for (int db = 0; db < G::DB; ++db) {
            const int row = g::pv16_key(lane, 0, 0) + g::tr16_row(lane);
            const int c = 16 * db + g::tr16_col(lane);  // halves
            voff[db] = g::tile_offset_m16(row, c >> 3, G::D) + 2 * (c & 7);
        }
    }
};

// Q^T operands: qf[qb][dc] holds Q[qw + 16qb + lane%16][8 * m16_kchunk(dc, lane/16) .. +7],
// the feature order of the K operand.
template <class T>
__device__ __forceinline__ void load_q16(const f16* qh, int qw, int n, int lane, int negate_q,
                                         f16x8 (&qf)[M16<T>::QB][M16<T>::DC]) {
    using G = M16<T>;
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb) {
        const int row = min(qw + 16 * qb + (lane & 15), n - 1);
        const f16* src = qh + static_cast<size_t>(row) * G::D;
#pragma unroll
        for (int dc = 0; dc < G::DC; ++dc) {
            qf[qb][dc] =
                *reinterpret_cast<const f16x8*>(src + 8 * g::m16_kchunk(dc, lane >> 4, G::D));
            if (negate_q) qf[qb][dc] = -qf[qb][dc];
        }
    }
}

// K fragments of a tile (KB * DC ds_read_b128) and V^T fragments (2 * KS * DB
// ds_read_b64_tr_b16).
template <class T>
__device__ __forceinline__ void load_k16(const char* kl, const Frag16<T>& fr,
                                         f16x8 (&kf)[M16<T>::KB][M16<T>::DC]) {
    using G = M16<T>;
#pragma unroll
    for (int kb = 0; kb < G::KB; ++kb)
#pragma unroll
        for (int dc = 0; dc < G::DC; ++dc)
            kf[kb][dc] = *reinterpret_cast<const f16x8*>(kl + fr.koff[kb][dc]);
}
template <class T>
__device__ __forceinline__ void load_v16(const char* vl, const Frag16<T>& fr,
                                         f16x8 (&vf)[M16<T>::KS][M16<T>::DB]) {
    using G = M16<T>;
#pragma unroll
    for (int t = 0; t < G::KS; ++t)
#pragma unroll
        for (int db = 0; db < G::DB; ++db) {
            const char* base = vl + fr.voff[db] + 32 * t * G::ROW;
            const f16x4 lo = lds_read_tr16(base);
            const f16x4 up = lds_read_tr16(base + 8 * G::ROW);
            vf[t][db] = f16x8{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
        }
}

// S^T = K Q^T of one tile (the first one, before the steady phases).
template <class T>
__device__ __forceinline__ void qk16(const char* kl, const Frag16<T>& fr,
                                     const f16x8 (&qf)[M16<T>::QB][M16<T>::DC],
                                     f32x4 (&s)[M16<T>::KB][M16<T>::QB]) {
    using G = M16<T>;
    f16x8 kf[G::KB][G::DC];
    load_k16<T>(kl, fr, kf);
#pragma unroll
    for (int kb = 0; kb < G::KB; ++kb)
#pragma unroll
        for (int qb = 0; qb < G::QB; ++qb) {
            s[kb][qb] = f32x4{};
#pragma unroll
            for (int dc = 0; dc < G::DC; ++dc) s[kb][qb] = mfma16(kf[kb][dc], qf[qb][dc], s[kb][qb]);
        }
}

// Keys >= n, and (causal) keys right of the query, get -inf.
template <class T, bool CAUSAL>
__device__ __forceinline__ void mask16(f32x4 (&s)[M16<T>::KB][M16<T>::QB], int kt, int n,
                                       int qw, int lane) {
    using G = M16<T>;
#pragma unroll
    for (int kb = 0; kb < G::KB; ++kb)
#pragma unroll
        for (int qb = 0; qb < G::QB; ++qb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = kt + g::st16_key(lane, kb, r);
                const int query = qw + g::st16_query(lane, qb);
                const bool masked = key >= n || (CAUSAL && key > query);
                s[kb][qb][r] = masked ? -INFINITY : s[kb][qb][r];
            }
}

// P^T operand slot i of k step t of query block qb: score accumulator i % 4 of key block
// 2t + i / 4 (fa::geom::pv16_key).
template <class T>
__device__ __forceinline__ f16x8 pack16(const float (&e)[M16<T>::KB][4], int t) {
    return pack8(e[2 * t][0], e[2 * t][1], e[2 * t][2], e[2 * t][3], e[2 * t + 1][0],
                 e[2 * t + 1][1], e[2 * t + 1][2], e[2 * t + 1][3]);
}

// Unchecked optimistic softmax of a steady tile: p = exp2(s*c - m) against the running max,
// packed to fp16, with neither row sums nor an overflow test here. The matrix phase adds the row
// sums of the packed P (matrix_phase16<T, true>), in the shadow of its MFMAs; an overflowing p
// becomes an infinite fp16 value and so an infinite row sum, which the workgroup tests once per
// item (flash_fwd_pingpong16 then recomputes the item with no unchecked tile: from its true row
// max, non-causal, or with the per-tile checked softmax, causal).
template <class T>
__device__ __forceinline__ void softmax16_unchecked(const f32x4 (&s)[M16<T>::KB][M16<T>::QB],
                                                    float scale_log2,
                                                    const float (&m_run)[M16<T>::QB],
                                                    f16x8 (&p)[M16<T>::QB][M16<T>::KS]) {
    using G = M16<T>;
    float e[G::QB][G::KB][4];
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb)
#pragma unroll
        for (int kb = 0; kb < G::KB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                e[qb][kb][r] = exp2_fast(fmaf(s[kb][qb][r], scale_log2, -m_run[qb]));
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb)
#pragma unroll
        for (int t = 0; t < G::KS; ++t) p[qb][t] = pack16<T>(e[qb], t);
}

// Optimistic softmax against the running max (as softmax_optimistic): P in fp16 and l += row
// sums, unless some p overflowed fp16, in which case `overflow` is set (wave-uniform) and the
// caller redoes the tile exactly. All exponentials are issued first, then the packs and the two
// row sums (interleaved v_dot2 chains): a pack or sum right after the exponentials it reads
// would wait on their latency.
template <class T>
__device__ __forceinline__ void softmax16_optimistic(const f32x4 (&s)[M16<T>::KB][M16<T>::QB],
                                                     float scale_log2,
                                                     const float (&m_run)[M16<T>::QB],
                                                     float (&l_run)[M16<T>::QB], bool& overflow,
                                                     f16x8 (&p)[M16<T>::QB][M16<T>::KS]) {
    using G = M16<T>;
    float e[G::QB][G::KB][4];
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb)
#pragma unroll
        for (int kb = 0; kb < G::KB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                e[qb][kb][r] = exp2_fast(fmaf(s[kb][qb][r], scale_log2, -m_run[qb]));
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb)
#pragma unroll
        for (int t = 0; t < G::KS; ++t) p[qb][t] = pack16<T>(e[qb], t);
    float sum[G::QB] = {0.0F, 0.0F};
    const f16x2 one = {static_cast<f16>(1.0F), static_cast<f16>(1.0F)};
#define FA_SUM2(K)                                                                              \
    for (int qb = 0; qb < G::QB; ++qb)                                                         \
        sum[qb] = __builtin_amdgcn_fdot2(__builtin_shufflevector(p[qb][t], p[qb][t], 2 * (K),  \
                                                                 2 * (K) + 1),                  \
                                         one, sum[qb], false);
#pragma unroll
    for (int t = 0; t < G::KS; ++t) {
        FA_SUM2(0)
        FA_SUM2(1)
        FA_SUM2(2)
        FA_SUM2(3)
    }
#undef FA_SUM2
    overflow = wave_any(!(sum[0] < INFINITY && sum[1] < INFINITY));
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb) l_run[qb] = overflow ? l_run[qb] : l_run[qb] + sum[qb];
}

// The wide-spread vote of an item's first tile (FA_PP16_SPREAD): true, for the whole wave, if
// for some query the smallest of the four lanes' score ranges over the tile's first 32 keys
// (key blocks 0 and 1: lane % 16 + 16 g holds keys m16_key(kb, 4g + 0..3)) exceeds
// FA_PP16_SPREAD exp2 units; 32 keys at either head dim, so one threshold serves both. NaN
// scores are skipped by v_max / v_min.
template <class T>
__device__ __forceinline__ bool softmax16_wide(const f32x4 (&s)[M16<T>::KB][M16<T>::QB],
                                               float scale_log2) {
    using G = M16<T>;
    bool wide = false;
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb) {
        float hi = s[0][qb][0];
        float lo = hi;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                hi = fmaxf(hi, s[kb][qb][r]);
                lo = fminf(lo, s[kb][qb][r]);
            }
        const float range = -max_xor32(max_xor16(-(hi - lo) * scale_log2));  // min over lanes
        wide = wide | (range > static_cast<float>(FA_PP16_SPREAD));
    }
    return wave_any(wide);
}

// Exact online softmax of one tile (as softmax_tile): the tile max of a query spans the four
// lanes lane % 16 + 16*i that hold its keys.
template <class T, bool ADD_SUM = true, int MARGIN = 0>
__device__ __forceinline__ void softmax16_tile(const f32x4 (&s)[M16<T>::KB][M16<T>::QB],
                                               float scale_log2, float (&m_run)[M16<T>::QB],
                                               float (&l_run)[M16<T>::QB],
                                               float (&alpha)[M16<T>::QB], bool& rescale,
                                               f16x8 (&p)[M16<T>::QB][M16<T>::KS]) {
    using G = M16<T>;
    float mx[G::QB];
    bool grow = false;
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb) {
        float x = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < G::KB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) x = fmaxf(x, s[kb][qb][r]);
        mx[qb] = max_xor32(max_xor16(x)) * scale_log2;
        grow = grow || (T::LAZY ? (mx[qb] > m_run[qb] + 8.0F) : (mx[qb] > m_run[qb]));
    }
    rescale = wave_any(grow);
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb) {
        const float m_new = rescale ? fmaxf(m_run[qb], mx[qb] + MARGIN) : m_run[qb];
        const float m_use = (m_new == -INFINITY) ? 0.0F : m_new;
        alpha[qb] = exp2_fast(m_run[qb] - m_use);
        m_run[qb] = m_new;
        float e[G::KB][4];
#pragma unroll
        for (int kb = 0; kb < G::KB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) e[kb][r] = exp2_fast(fmaf(s[kb][qb][r], scale_log2, -m_use));
        float sum = 0.0F;
#pragma unroll
        for (int t = 0; t < G::KS; ++t) {
            p[qb][t] = pack16<T>(e, t);
            if constexpr (ADD_SUM) sum = sum8_f16(p[qb][t], sum);
        }
        // without ADD_SUM the caller adds the row sums of p (matrix_phase16<T, true>)
        l_run[qb] = (rescale ? l_run[qb] * alpha[qb] : l_run[qb]) + sum;
    }
}

template <class T>
__device__ __forceinline__ void rescale16(f32x4 (&oacc)[M16<T>::DB][M16<T>::QB],
                                          const float (&alpha)[M16<T>::QB]) {
#pragma unroll
    for (int db = 0; db < M16<T>::DB; ++db)
#pragma unroll
        for (int qb = 0; qb < M16<T>::QB; ++qb) oacc[db][qb] *= alpha[qb];
}

template <class T>
__device__ __forceinline__ void pv16(const f16x8 (&vf)[M16<T>::KS][M16<T>::DB],
                                     const f16x8 (&p)[M16<T>::QB][M16<T>::KS],
                                     f32x4 (&oacc)[M16<T>::DB][M16<T>::QB]) {
    using G = M16<T>;
#pragma unroll
    for (int t = 0; t < G::KS; ++t)
#pragma unroll
        for (int db = 0; db < G::DB; ++db)
#pragma unroll
            for (int qb = 0; qb < G::QB; ++qb)
                oacc[db][qb] = mfma16(vf[t][db], p[qb][t], oacc[db][qb]);
}

// Matrix phase: S^T_{j+1} (16 MFMAs: KB*QB independent chains of DC, step i on chain i % (KB*QB))
// alternating with O^T += V_j^T P_j^T (16 MFMAs, independent); `mid` (the refill) after pair
// FA_PP16_MID (the second pair: measured best of pairs 0-3 and 7, by about 1 %).
template <class T, bool SUMS, class Mid>
__device__ __forceinline__ void matrix_phase16(const f16x8 (&kf)[M16<T>::KB][M16<T>::DC],
                                               const f16x8 (&qf)[M16<T>::QB][M16<T>::DC],
                                               const f16x8 (&vf)[M16<T>::KS][M16<T>::DB],
                                               const f16x8 (&p)[M16<T>::QB][M16<T>::KS],
                                               f32x4 (&s)[M16<T>::KB][M16<T>::QB],
                                               f32x4 (&oacc)[M16<T>::DB][M16<T>::QB],
                                               float (&l_run)[M16<T>::QB], Mid&& mid) {
    using G = M16<T>;
    constexpr int NCH = G::KB * G::QB;  // QK chains
    static_assert(FA_PP16_SUM_PAIR + 2 * (G::QB * G::KS - 1) < 16, "row sums past the last pair");
#pragma unroll
    for (int kb = 0; kb < G::KB; ++kb)
#pragma unroll
        for (int qb = 0; qb < G::QB; ++qb) s[kb][qb] = f32x4{};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int ch = i % NCH;
        const int kb = ch / G::QB;
        const int qs = ch % G::QB;
        const int dc = i / NCH;
        const int qv = i % G::QB;
        const int db = (i / G::QB) % G::DB;
        const int t = i / (G::QB * G::DB);
        if (FA_PP16_PV_FIRST) {
            oacc[db][qv] = mfma16(vf[t][db], p[qv][t], oacc[db][qv]);
            s[kb][qs] = mfma16(kf[kb][dc], qf[qs][dc], s[kb][qs]);
        } else {
            s[kb][qs] = mfma16(kf[kb][dc], qf[qs][dc], s[kb][qs]);
            oacc[db][qv] = mfma16(vf[t][db], p[qv][t], oacc[db][qv]);
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the alternation
        if (i == FA_PP16_MID) {
            mid();
            __builtin_amdgcn_sched_barrier(0);
        }

        if constexpr (SUMS) {
            // row sum of the packed P of (qb, t), four dependent v_dot2, after pair
            // FA_PP16_SUM_PAIR + 2 (qb KS + t)
#pragma unroll
            for (int qb = 0; qb < G::QB; ++qb)
#pragma unroll
                for (int t = 0; t < G::KS; ++t)
                    if (i == FA_PP16_SUM_PAIR + 2 * (qb * G::KS + t)) {
                        l_run[qb] = sum8_f16(p[qb][t], l_run[qb]);
                        __builtin_amdgcn_sched_barrier(0);
                    }
        }
    }
}

// O = acc / l as fp16 for the lane's two queries (if < n), and the natural-log LSE if lse_h is
// not null. The lane holds features 16db + 4*(lane/16) + 0..3 of each; lanes l and l ^ 16, which
// hold the same query, trade half of them (pair_swap16) so that each lane writes 8 consecutive
// features per 16-byte store: per pair of blocks (2e, 2e + 1) lane group g = lane / 16 stores
// features 32e + 4g + 12 (g % 2) + 0..7, and the four groups cover 64 contiguous bytes.
template <class T>
__device__ __forceinline__ void store16(f16* oh, float* lse_h, int qw, int n, int lane,
                                        const float (&m_run)[M16<T>::QB],
                                        const float (&l_run)[M16<T>::QB],
                                        const f32x4 (&oacc)[M16<T>::DB][M16<T>::QB]) {
    using G = M16<T>;
    float l_tot[G::QB];
    f16x8 out[G::QB][G::DB / 2];
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb) {
        l_tot[qb] = sum_xor32(sum_xor16(l_run[qb]));
        const float inv = (l_tot[qb] > 0.0F) ? (1.0F / l_tot[qb]) : 0.0F;
#pragma unroll
        for (int e = 0; e < G::DB / 2; ++e) {
            const f32x4& a = oacc[2 * e][qb];
            const f32x4& b = oacc[2 * e + 1][qb];
            out[qb][e] = pair_swap16(pack4(a[0] * inv, a[1] * inv, a[2] * inv, a[3] * inv),
                                     pack4(b[0] * inv, b[1] * inv, b[2] * inv, b[3] * inv));
        }
    }
    const int grp = lane >> 4;
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb) {
        const int qrow = qw + g::st16_query(lane, qb);
        if (qrow >= n) continue;
        if (lse_h != nullptr && lane < 16) lse_h[qrow] = row_lse2(m_run[qb], l_tot[qb]) * kLn2;
        f16* dst = oh + static_cast<size_t>(qrow) * G::D + 4 * grp + 12 * (grp & 1);
#pragma unroll
        for (int e = 0; e < G::DB / 2; ++e) *reinterpret_cast<f16x8*>(dst + 32 * e) = out[qb][e];
    }
}

// Split-KV partial of store16: O / l in fp32 and the base-2 LSE (scaled units) of the lane's two
// queries (if < n), at op[qrow][d] and lp[qrow]; a row with no unmasked key in the range gets
// O = 0 and LSE = -inf, which the combine kernel weighs 0. Same layout as the simple kernel's
// store_partial.
template <class T>
__device__ __forceinline__ void store16_partial(float* op, float* lp, int qw, int n, int lane,
                                                const float (&m_run)[M16<T>::QB],
                                                const float (&l_run)[M16<T>::QB],
                                                const f32x4 (&oacc)[M16<T>::DB][M16<T>::QB]) {
    using G = M16<T>;
    float l_tot[G::QB];
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb) l_tot[qb] = sum_xor32(sum_xor16(l_run[qb]));
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb) {
        const int qrow = qw + g::st16_query(lane, qb);
        if (qrow >= n) continue;
        const float inv = (l_tot[qb] > 0.0F) ? (1.0F / l_tot[qb]) : 0.0F;
        if (lane < 16) lp[qrow] = row_lse2(m_run[qb], l_tot[qb]);
        float* dst = op + static_cast<size_t>(qrow) * G::D + 4 * (lane >> 4);
#pragma unroll
        for (int db = 0; db < G::DB; ++db) {
            const f32x4& a = oacc[db][qb];
            *reinterpret_cast<f32x4*>(dst + 16 * db) =
                f32x4{a[0] * inv, a[1] * inv, a[2] * inv, a[3] * inv};
        }
    }
}

// Tiles j .. n_tiles-1 outside the steady phases: one barrier each; K_t
// and V_t in buffer t % 3; refills of K_{j+2} and V_{j+1}.
template <class T, bool CAUSAL>
__device__ __forceinline__ void general_tiles16(
    int j, int n_tiles, int n_act, int n, int qw, int lane, const f16* kh, const f16* vh,
    char* const (&kb)[3], char* const (&vb)[3], const TileDma<T, true>& dma_k,
    const TileDma<T>& dma, const Frag16<T>& fr, const f16x8 (&qf)[M16<T>::QB][M16<T>::DC],
    f32x4 (&s)[M16<T>::KB][M16<T>::QB], f32x4 (&oacc)[M16<T>::DB][M16<T>::QB],
    float scale_log2, float (&m_run)[M16<T>::QB], float (&l_run)[M16<T>::QB]) {
    using G = M16<T>;
    for (; j < n_tiles; ++j) {
        wait_vmem();
        __syncthreads();
        const bool act = j < n_act;
        const bool act_next = j + 1 < n_act;
        f16x8 kf[G::KB][G::DC];
        f16x8 vf[G::KS][G::DB];
        if (act_next) load_k16<T>(kb[(j + 1) % 3], fr, kf);
        if (act) load_v16<T>(vb[j % 3], fr, vf);
        if (j + 2 < n_tiles) load_tile<T>(kh, (j + 2) * T::BC, n, kb[(j + 2) % 3], dma_k);
        if (j + 1 < n_tiles) load_tile<T>(vh, (j + 1) * T::BC, n, vb[(j + 1) % 3], dma);
        if (!act) continue;  // wave-uniform: fully masked for this wave (causal)
        f32x4 s2[G::KB][G::QB];
        if (act_next) {
#pragma unroll
            for (int b = 0; b < G::KB; ++b)
#pragma unroll
                for (int qb = 0; qb < G::QB; ++qb) {
                    s2[b][qb] = f32x4{};
#pragma unroll
                    for (int dc = 0; dc < G::DC; ++dc)
                        s2[b][qb] = mfma16(kf[b][dc], qf[qb][dc], s2[b][qb]);
                }
        }
        const int kt = j * T::BC;
        if (g::tile_needs_mask(n, kt, T::BC, qw, CAUSAL)) mask16<T, CAUSAL>(s, kt, n, qw, lane);
        f16x8 p[G::QB][G::KS];
        float alpha[G::QB];
        bool rescale;
        softmax16_tile<T>(s, scale_log2, m_run, l_run, alpha, rescale, p);
        if (rescale) rescale16<T>(oacc, alpha);
        pv16<T>(vf, p, oacc);
        if (act_next) {
#pragma unroll
            for (int b = 0; b < G::KB; ++b)
#pragma unroll
                for (int qb = 0; qb < G::QB; ++qb) s[b][qb] = s2[b][qb];
        }
    }
}

template <class T, bool CAUSAL, bool SPLIT = false, bool PAIRS = false>
__global__ __launch_bounds__(T::THREADS) void flash_fwd_pingpong16(
    const f16* __restrict__ q, const f16* __restrict__ k, const f16* __restrict__ v,
    f16* __restrict__ o, float* __restrict__ lse, int n, int bh_count, int n_qblocks,
    float scale_log2, int negate_q, int tiles_per_split, float* __restrict__ o_part,
    float* __restrict__ lse_part, unsigned launch_id, int /*group_heads*/) {
    static_assert((T::D == 128 && T::BC == 32) || (T::D == 64 && T::BC == 64),
                  "the 16x16x32 layouts are written for D=128, BC=32 and D=64, BC=64");
    using G = M16<T>;
    static_assert(T::NW == 8, "ping-pong pairs waves w and w+4 on each of the four SIMDs");
    static_assert(T::NBUF == 3, "ping-pong keeps three K and three V tiles in LDS");
    static_assert(T::DMA_ITERS == 1, "one DMA request per tile and wave (vmcnt(2) keeps a pair)");
    constexpr bool PAIRED = CAUSAL && !SPLIT && PAIRS;
    // Items run the unchecked softmax (softmax16_unchecked) on their steady tiles after the
    // first, causal items only up to the diagonal band, whose tiles keep the per-tile checked
    // softmax; an item is recomputed, with every steady tile checked, only if some p overflowed
    // fp16 (then a row sum is infinite). The workgroup sees an overflow in its unchecked run
    // within two to three steps of three tiles and leaves the run early (pp_flags), so that an
    // input on which most items overflow (outlier keys, wide score spreads) costs about one
    // checked pass per item, not two passes.
    constexpr bool UNCHECKED = FA_PP16_UNCHECKED;
    // Overflow flags of the unchecked run (0-1, one per chunk mod 2) and of the item's final
    // test (2), and the first tile's wide-spread vote (3, FA_PP16_SPREAD). Cleared at the start
    // of an item's first pass; read with the lane and wave
    // registers rather than threadIdx or __syncthreads_or, which would keep the work-item ids
    // live across the item loop (past 256 VGPRs, into scratch). Accessed with flag_get and
    // flag_set (LDS instructions).
    __shared__ int pp_flags[4];
    // An item's first pass runs checked from the start (1) after enough overflows in this
    // launch: wave 0 reads pp_overflow_record with the item's prologue loads and writes the
    // decision here before the prologue's barrier, so that every wave takes the same one.
    constexpr bool ADAPT = UNCHECKED && FA_PP16_ADAPT_WGS > 0;
    __shared__ int pp_adapt;
    __shared__ __attribute__((aligned(1024))) char k_lds0[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char k_lds1[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char k_lds2[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char v_lds0[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char v_lds1[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char v_lds2[T::TILE_BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = wave_uniform(threadIdx.x >> 6);
    const int grp = wave >> 2;
    probe_stamp(wave, lane, 0);
    probe_cycles(wave, lane, 11);
    probe_ids(wave, lane);
    int probe_item = 0;  // (FA_PROBE only) items this workgroup has finished
    const int items = bh_count * n_qblocks;
    const int split = SPLIT ? static_cast<int>(blockIdx.x) / items : 0;
    // One (head, query block) item: the whole single-item kernel. With UNCHECKED, a first pass
    // (checked_pass false) runs the unchecked softmax and returns false, having stored nothing,
    // when a row sum came out non-finite; the second pass (checked_pass true) runs the checked
    // softmax in every steady tile, which redoes an overflowing tile with a rescale, and always
    // stores.
    auto run_item = [&](const g::Work w, const bool checked_pass) -> bool {
    probe_stamp(wave, lane, checked_pass ? 12 : 1 + 5 * probe_item);
    constexpr bool FAST = UNCHECKED;
    const size_t head = static_cast<size_t>(w.bh) * n * T::D;
    const int q0 = w.qb * T::BR;
    const int qw = q0 + wave * 32;  // first query of this wave (Q loads, O stores)
    // Split-KV: the workgroup runs its query block's key range `split` (geom::split_range) as
    // if the keys started at key0: K/V pointers, the sequence end nk and the query position qk
    // used by the masks are all taken relative to key0.
    const int n_all = g::num_kv_tiles(n, q0, T::BR, T::BC, CAUSAL);
    const g::KeyRange range = SPLIT ? g::split_range(n_all, tiles_per_split, split)
                                    : g::KeyRange{0, n_all};
    if (SPLIT && range.count == 0) return true;  // workgroup-uniform: no such range
    const int j_begin = range.begin;
    const int key0 = j_begin * T::BC;
    const int nk = n - key0;
    const int qk = qw - key0;
    const f16* kh = k + head + static_cast<size_t>(key0) * T::D;
    const f16* vh = v + head + static_cast<size_t>(key0) * T::D;
    const int n_tiles = range.count;
    // DMA bound: the keys this workgroup visits (its split range, or up to its causal diagonal).
    // The prefetches that run past the last tile still issue, so every wave's vmcnt sequence is
    // unchanged, but they read zeros instead of keys of the next range or right of the diagonal.
    const int nk_load = min(nk, n_tiles * T::BC);
    // (a split can start right of all of this wave's queries: no active tile then)
    const int n_act = (SPLIT && CAUSAL && qk + 31 < 0)
                          ? 0
                          : g::wave_active_tiles(nk, qk, 32, T::BC, n_tiles, CAUSAL);
    // Every tile but the last runs in the steady phases (diagonal and tail tiles masked there).
    // A causal wave computes the first n_busy of them; the non-causal kernel computes all (a
    // wave past the end of the sequence works on masked scores there), which keeps its steady
    // loop free of the idle-tile code.
    const int n_steady = max(0, n_tiles - 1);
    const int n_busy = CAUSAL ? min(n_steady, n_act) : n_steady;

    auto kbuf = [&](auto b) {
        constexpr int B = decltype(b)::value;
        return B == 0 ? k_lds0 : (B == 1 ? k_lds1 : k_lds2);
    };
    auto vbuf = [&](auto b) {
        constexpr int B = decltype(b)::value;
        return B == 0 ? v_lds0 : (B == 1 ? v_lds1 : v_lds2);
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;

    const TileDma<T, true> dma_k(wave, lane);  // K tiles in the layout of Frag16's K reads
    const TileDma<T> dma(wave, lane);          // V tiles, swizzle fa::geom::row_xor_m16
    f16x8 qf[G::QB][G::DC];
    float m_run[G::QB] = {-INFINITY, -INFINITY};
    if constexpr (FAST) {
        // cleared before the prologue's barrier; the previous pass or item read them before
        // its own final barrier
        if (!checked_pass && wave == 0 && lane < 4) flag_set(pp_flags[lane], 0);
    }
    load_tile<T>(kh, 0, nk_load, kbuf(I0{}), dma_k);
    load_tile<T>(vh, 0, nk_load, vbuf(I0{}), dma);
    load_tile<T>(kh, T::BC, nk_load, kbuf(I1{}), dma_k);
    load_tile<T>(kh, 2 * T::BC, nk_load, kbuf(I2{}), dma_k);
    load_tile<T>(vh, T::BC, nk_load, vbuf(I1{}), dma);
    load_q16<T>(q + head, qw, n, lane, negate_q, qf);
    // (after the prologue's loads: its address comes through a scalar load and wait)
    unsigned long long record = 0;
    if constexpr (ADAPT) {
        if (!checked_pass && wave == 0) {
            record = __hip_atomic_load(&pp_overflow_record, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    const Frag16<T> fr(lane);
    probe_stamp(wave, lane, 16 + 5 * probe_item);

    f32x4 oacc[G::DB][G::QB];
#pragma unroll
    for (int db = 0; db < G::DB; ++db)
#pragma unroll
        for (int qb = 0; qb < G::QB; ++qb) oacc[db][qb] = f32x4{};
    float l_run[G::QB] = {0.0F, 0.0F};

    wait_vmem();
    probe_stamp(wave, lane, 17 + 5 * probe_item);
    if constexpr (ADAPT) {
        if (!checked_pass && wave == 0 && lane == 0) {
            pp_adapt = static_cast<unsigned>(record >> 32) == launch_id &&
                               static_cast<unsigned>(record) >= FA_PP16_ADAPT_WGS
                           ? 1
                           : 0;
        }
    }
    __syncthreads();
    probe_stamp(wave, lane, 2 + 5 * probe_item);
    // (workgroup-uniform: one LDS word written before the barrier)
    const bool start_checked =
        ADAPT && !checked_pass && __builtin_amdgcn_readfirstlane(pp_adapt) != 0;
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb)
#pragma unroll
        for (int dc = 0; dc < G::DC; ++dc) asm volatile("" ::"v"(qf[qb][dc]));
    // A wave with no active tile (entirely past the end of the sequence, or left of a split's
    // keys) never computes S, but the non-causal steady loop still runs its softmax on masked
    // scores: start from zeros so that it reads defined values.
    f32x4 s[G::KB][G::QB];
#pragma unroll
    for (int kb = 0; kb < G::KB; ++kb)
#pragma unroll
        for (int qb = 0; qb < G::QB; ++qb) s[kb][qb] = f32x4{};
    if (n_act > 0) qk16<T>(kbuf(I0{}), fr, qf, s);
    probe_stamp(wave, lane, 18 + 5 * probe_item);

    // Returns true when the workgroup left its unchecked run on an overflow (FAST only).
    auto steady = [&](auto group) -> bool {
        constexpr int G = decltype(group)::value;
        bool aborted = false;
        auto refill = [&](int a, auto pa, int b, auto pb) {
            load_tile<T>(kh, a * T::BC, nk_load, kbuf(pa), dma_k);
            load_tile<T>(vh, b * T::BC, nk_load, vbuf(pb), dma);
        };
        end_phase<false>();
        if constexpr (G == 1) {
            refill(3, I0{}, 2, I2{});
            end_phase<false>();
        }
        // kind: 0 the checked optimistic softmax (its own row sums, an overflowing tile redone
        // exactly); with FAST, 1 exact (the item's first tile) and 2 unchecked, both with the row
        // sums added in the matrix phase.
        auto tile = [&](int jj, auto r, auto kind) {
            constexpr int R = decltype(r)::value;
            constexpr bool EXACT = FAST && decltype(kind)::value == 1;
            constexpr bool UNCHECKED_TILE = FAST && decltype(kind)::value == 2;
            using Rj = std::integral_constant<int, R>;
            using Rj1 = std::integral_constant<int, (R + 1) % 3>;
            using Rj2 = std::integral_constant<int, (R + 2) % 3>;
            // softmax phase S_jj. Only causal steady tiles can need a mask: without causality
            // the one tile that can reach past the sequence end is the last, which runs in
            // general_tiles16. (Left to the compiler, the non-causal test is turned into 32
            // unconditional compare/select VALU instructions per tile.) A causal item's
            // unchecked tiles end before the first tile that any of its rows masks.
            if constexpr (CAUSAL && !UNCHECKED_TILE) {
                if (g::tile_needs_mask(nk, jj * T::BC, T::BC, qk, CAUSAL)) {
                    mask16<T, CAUSAL>(s, jj * T::BC, nk, qk, lane);
                }
            }
            f16x8 kf[G::KB][G::DC];
            f16x8 vf[G::KS][G::DB];
            load_k16<T>(kbuf(Rj1{}), fr, kf);
            load_v16<T>(vbuf(Rj{}), fr, vf);
            f16x8 p[G::QB][G::KS];
            bool overflow = false;
            if constexpr (EXACT) {
                float alpha[G::QB];
                bool rescale;
                softmax16_tile<T, false, FA_PP16_UNCHECKED_MARGIN>(s, scale_log2, m_run, l_run,
                                                                   alpha, rescale, p);
                if (rescale) rescale16<T>(oacc, alpha);
                if constexpr (FA_PP16_SPREAD > 0) {
                    // (first pass only; a causal wave votes if all its rows see the whole tile)
                    if (!checked_pass && !start_checked && (!CAUSAL || qk >= T::BC - 1) &&
                        softmax16_wide<T>(s, scale_log2) && lane == 0) {
                        flag_set(pp_flags[3], 1);
                    }
                }
                if constexpr (CAUSAL && SPLIT) {
                    // a split range can start right of some rows' queries: such a row sees no
                    // key in the range, and 0 keeps its later p at exp2(-inf) = 0 (and its
                    // partial LSE at -inf, from l = 0)
#pragma unroll
                    for (int qb = 0; qb < G::QB; ++qb)
                        m_run[qb] = m_run[qb] == -INFINITY ? 0.0F : m_run[qb];
                }
            } else if constexpr (UNCHECKED_TILE) {
                softmax16_unchecked<T>(s, scale_log2, m_run, p);
            } else {
                softmax16_optimistic<T>(s, scale_log2, m_run, l_run, overflow, p);
            }
            using RS = PP16ReadSched<T, CAUSAL, !FAST>;
            static_assert(RS::F <= G::READS && (G::READS - RS::F) % RS::R == 0,
                          "the read groups must cover the 24 fragment reads");
            sched_reads_valu<RS::R, RS::V, (G::READS - RS::F) / RS::R, RS::F>();
            end_phase<G == 1>();
            // matrix phase M_jj
            if (__builtin_expect(overflow, 0)) {
                float alpha[G::QB];
                bool rescale;
                softmax16_tile<T>(s, scale_log2, m_run, l_run, alpha, rescale, p);
                if (rescale) rescale16<T>(oacc, alpha);
            }
            __builtin_amdgcn_s_setprio(FA_PP_PRIO);
            matrix_phase16<T, (EXACT || UNCHECKED_TILE)>(kf, qf, vf, p, s, oacc, l_run, [&] {
                if constexpr (G == 0) {
                    refill(jj + 3, Rj{}, jj + 2, Rj2{});
                } else {
                    refill(jj + 4, Rj1{}, jj + 3, Rj{});
                }
            });
            __builtin_amdgcn_s_setprio(FA_PP_SPRIO);
            end_phase<G == 0>();
        };
        using Checked = std::integral_constant<int, 0>;
        using Exact = std::integral_constant<int, 1>;
        using Unchecked = std::integral_constant<int, 2>;
        int jj = 0;
        if constexpr (FAST) {
            // tile 0 on its own (exact), then tiles 1.. in buffers 1, 2, 0, ...
            auto rest = [&](auto kind, int n_end) {
                for (; jj + 3 <= n_end; jj += 3) {
                    tile(jj, I1{}, kind);
                    tile(jj + 1, I2{}, kind);
                    tile(jj + 2, I0{}, kind);
                }
                if (jj < n_end) tile(jj, I1{}, kind);
                if (jj + 1 < n_end) tile(jj + 1, I2{}, kind);
            };
            if (n_busy > 0) {
                tile(0, I0{}, Exact{});
                jj = 1;
                probe_stamp(wave, lane, 19 + 5 * probe_item);
            }
            // Unchecked tiles in steps of three, in chunks of 1, 2, 4, ... steps, at most
            // FA_PP16_EXIT_STEPS (an overflow tends to come early, as the running max of the
            // keys grows fastest at first). An overflowing p shows as an infinite row sum in the
            // wave's l_run after the matrix phase of its tile. At chunk boundary c (the head of
            // the chunk's first step) every
            // wave first reads flag (c - 1) % 2 and leaves if it is set, then sets flag c % 2 if
            // its own row sums are no longer finite. A flag is read one chunk (at least six
            // barriers) after its writes, each of which has completed by its wave's next barrier
            // (end_phase waits for its LDS writes), and written again one chunk after that read;
            // so all waves read the same value and leave at the same boundary, i.e. after the
            // same number of barriers (tests/test_abort_protocol.py). The workgroup leaves at
            // most two chunks after the first overflow. The read waits at once (an LDS latency
            // per chunk); the inner loop stays the plain three-tile body, whose timing is
            // sensitive to any extra live value.
            // The exit needs every wave in the run. A causal wave that starts past the end of the
            // sequence has no active tile and spends the run in the idle-tile loop below, never
            // reading the flags, so a workgroup with such a wave (only a last query block) keeps
            // to the full pass and its final test: no wave sets a flag there. (Non-causal waves
            // all run every steady tile.)
            const bool exit_ok = !CAUSAL || q0 + T::BR - 32 < n;
            // Unchecked up to n_free, then checked: non-causal, the one to two tiles left over
            // from the steps of three; causal, from the first tile that some row of the workgroup
            // must mask (keys 0..q0 are visible to every row), i.e. the diagonal band. The
            // second pass runs every steady tile checked.
            // A wide-spread vote of the first tile (written in its softmax phase, read here after
            // the barrier that ends both groups' first softmax phases, so every wave sees every
            // vote: tests/test_abort_protocol.py) also runs the item checked.
            const bool wide = FA_PP16_SPREAD > 0 && jj == 1 && !checked_pass && !start_checked &&
                              __builtin_amdgcn_readfirstlane(flag_get(pp_flags[3])) != 0;
            const int n_free =
                (checked_pass || start_checked || wide)
                    ? 0
                    : (CAUSAL ? min(n_busy, max(0, min(q0 - key0 + 1, nk)) / T::BC) : n_busy);
            int slot = 0;
            int chunk = 1;  // steps
            while (jj + 3 <= n_free) {
                // (nothing can be set at the first boundary)
                if (jj > 1 && __builtin_amdgcn_readfirstlane(flag_get(pp_flags[slot ^ 1])) != 0) {
                    aborted = true;
                    break;
                }
                const bool bad = !(l_run[0] < INFINITY && l_run[1] < INFINITY);
                if (exit_ok && wave_any(bad) && lane == 0) flag_set(pp_flags[slot], 1);
                const int chunk_end =
                    FA_PP16_EXIT_STEPS > 0 ? min(n_free, jj + 3 * chunk) : n_free;
                for (; jj + 3 <= chunk_end; jj += 3) {
                    tile(jj, I1{}, Unchecked{});
                    tile(jj + 1, I2{}, Unchecked{});
                    tile(jj + 2, I0{}, Unchecked{});
                }
                slot ^= 1;
                chunk = min(2 * chunk, FA_PP16_EXIT_STEPS);
            }
            rest(Checked{}, aborted ? jj : n_busy);
        } else {
            for (; jj + 3 <= n_busy; jj += 3) {
                tile(jj, I0{}, Checked{});
                tile(jj + 1, I1{}, Checked{});
                tile(jj + 2, I2{}, Checked{});
            }
            if (jj < n_busy) tile(jj, I0{}, Checked{});
            if (jj + 1 < n_busy) tile(jj + 1, I1{}, Checked{});
        }
        // Causal steady tiles whose keys are all masked for this wave (diagonal block, or a wave
        // past the end of the sequence): the wave keeps only its two barriers per tile and its
        // share of the refill DMA, in the order of a busy tile.
        if constexpr (CAUSAL) {
            auto kb_at = [&](int b) { return b == 0 ? k_lds0 : (b == 1 ? k_lds1 : k_lds2); };
            auto vb_at = [&](int b) { return b == 0 ? v_lds0 : (b == 1 ? v_lds1 : v_lds2); };
            // (all waves leave an aborted run after the same tiles, so they skip the rest alike)
            for (int t = aborted ? n_steady : n_busy; t < n_steady; ++t) {
                const int r = t % 3;
                end_phase<G == 1>();
                if constexpr (G == 0) {
                    load_tile<T>(kh, (t + 3) * T::BC, nk_load, kb_at(r), dma_k);
                    load_tile<T>(vh, (t + 2) * T::BC, nk_load, vb_at((r + 2) % 3), dma);
                } else {
                    load_tile<T>(kh, (t + 4) * T::BC, nk_load, kb_at((r + 1) % 3), dma_k);
                    load_tile<T>(vh, (t + 3) * T::BC, nk_load, vb_at(r), dma);
                }
                end_phase<G == 0>();
            }
        }
        if constexpr (G == 0) end_phase<false>();
        return aborted;
    };
    if (n_steady > 0) {
        const bool aborted = grp == 0 ? steady(I0{}) : steady(I1{});
        if (aborted) {
            if constexpr (ADAPT) {
                if (wave == 0 && lane == 0) note_overflow(launch_id);
            }
            // the DMA still in flight lands before the second pass refills the buffers
            wait_vmem();
            __syncthreads();
            return false;
        }
    }
    probe_stamp(wave, lane, 3 + 5 * probe_item);
    char* kb[3];
    char* vb[3];
    kb[0] = k_lds0;
    kb[1] = k_lds1;
    kb[2] = k_lds2;
    vb[0] = v_lds0;
    vb[1] = v_lds1;
    vb[2] = v_lds2;
    {
        // fragment offsets of the last tile's own, which the compiler would otherwise hoist out
        // of the item loop and keep in scratch
        int lane_g = lane;
        asm volatile("" : "+v"(lane_g));
        const Frag16<T> fr_g(lane_g);
        general_tiles16<T, CAUSAL>(n_steady, n_tiles, n_act, nk, qk, lane, kh, vh, kb, vb, dma_k,
                                   dma, fr_g, qf, s, oacc, scale_log2, m_run, l_run);
    }
    probe_stamp(wave, lane, 4 + 5 * probe_item);
    if constexpr (FAST) {
        // an overflowing p makes its row sum infinite (NaN inputs make it NaN): decided for the
        // whole workgroup (flag 2 after a barrier), whose waves then redo the item together.
        // The flag is cleared again only by the next item, after the barrier between a pair's
        // items.
        if (!checked_pass) {
            const bool bad = !(l_run[0] < INFINITY && l_run[1] < INFINITY);
            if (wave_any(bad) && lane == 0) flag_set(pp_flags[2], 1);
            __syncthreads();
            probe_stamp(wave, lane, 20 + 5 * probe_item);
            if (__builtin_amdgcn_readfirstlane(flag_get(pp_flags[2])) != 0) {
                if constexpr (ADAPT) {
                    if (wave == 0 && lane == 0) note_overflow(launch_id);
                }
                return false;
            }
        }
    }
    if constexpr (SPLIT) {
        const size_t part = static_cast<size_t>(split) * bh_count + w.bh;
        // (causal: store offsets of the store's own, as for the last tile above)
        int lane_s = lane;
        int qw_s = qw;
        asm volatile("" : "+v"(lane_s), "+s"(qw_s));
        store16_partial<T>(o_part + part * n * T::D, lse_part + part * n, qw_s, n, lane_s, m_run,
                           l_run, oacc);
    } else {
        store16<T>(o + head, lse ? lse + static_cast<size_t>(w.bh) * n : nullptr, qw, n, lane,
                   m_run, l_run, oacc);
    }
    probe_stamp(wave, lane, 5 + 5 * probe_item);
    ++probe_item;
    return true;
    };
    // With UNCHECKED: a second pass of the same code, every steady tile checked, when some p
    // overflowed fp16 (the final barrier of the failed pass has ended all its LDS reads). One
    // instance of the item code serves both passes.
    auto run = [&](const g::Work w) {
        bool checked_pass = false;
#pragma clang loop unroll(disable)
        while (!run_item(w, checked_pass)) checked_pass = true;
    };
    if constexpr (CAUSAL && !SPLIT) {
        // Causal grids: with PAIRS each workgroup runs the pair of query blocks (long, short) =
        // (n_qblocks - 1 - p, p), so that every workgroup has the same number of tiles
        // (fa::geom::causal_pair); otherwise one query block, longest first (fa::geom::work_of;
        // the launcher picks by fa::geom::causal_pairs_pay).
        g::PairWork pw{};
        if constexpr (PAIRED) {
            pw = g::causal_pair(static_cast<int>(blockIdx.x), bh_count, n_qblocks);
        } else {
            const g::Work w = g::work_of(static_cast<int>(blockIdx.x), bh_count, n_qblocks, true);
            pw = g::PairWork{w.bh, w.qb, -1};
        }
        // One call site of the item code for both items and both passes. The two items of a
        // pair are query blocks of one head, the second seeing a prefix of the first's keys: if
        // the first needed the checked pass, the second runs it at once. (Running the short
        // block first, in every pair or in every other one, measured the same or up to 1.3 %
        // slower.)
        bool second = false;
        bool checked_pass = false;
        bool redone = false;
#pragma clang loop unroll(disable)
        for (;;) {
            if (!run_item(g::Work{pw.bh, second ? pw.qb_short : pw.qb_long}, checked_pass)) {
                checked_pass = true;
                redone = true;
                continue;
            }
            if (second || pw.qb_short < 0) break;
            // the first item's last LDS reads, before the second item's DMA (a barrier that
            // waits for LDS only: __syncthreads would also wait for the first item's O stores)
            end_phase<false>();
            second = true;
            checked_pass = redone;
        }
    } else {
        run(SPLIT ? g::work_of(static_cast<int>(blockIdx.x) - split * items, bh_count,
                               n_qblocks, CAUSAL)
                  : g::work_of_xcd(blockIdx.x, bh_count, n_qblocks, CAUSAL));
    }
    probe_cycles(wave, lane, 13);
}

// ---- kernel, simple schedule on 16x16x32 MFMAs ------------------------------------------------
// S^T = K Q^T of one tile with each K fragment read right before its MFMAs (8 VGPRs of K live at
// a time instead of the 32 that qk16 reads ahead): the simple schedule runs four waves per SIMD
// and so has 128 VGPRs per wave.
template <class T>
__device__ __forceinline__ void qk16_lean(const char* kl, const Frag16<T>& fr,
                                          const f16x8 (&qf)[M16<T>::QB][M16<T>::DC],
                                          f32x4 (&s)[M16<T>::KB][M16<T>::QB]) {
    using G = M16<T>;
#pragma unroll
    for (int kb = 0; kb < G::KB; ++kb) {
        f16x8 kf[G::DC];
#pragma unroll
        for (int dc = 0; dc < G::DC; ++dc)
            kf[dc] = *reinterpret_cast<const f16x8*>(kl + fr.koff[kb][dc]);
#pragma unroll
        for (int qb = 0; qb < G::QB; ++qb) {
            s[kb][qb] = f32x4{};
#pragma unroll
            for (int dc = 0; dc < G::DC; ++dc) s[kb][qb] = mfma16(kf[dc], qf[qb][dc], s[kb][qb]);
        }
    }
}

// O^T += V^T P^T of one tile, V^T fragments of one 32-key step read right before its MFMAs.
template <class T>
__device__ __forceinline__ void pv16_lean(const char* vl, const Frag16<T>& fr,
                                          const f16x8 (&p)[M16<T>::QB][M16<T>::KS],
                                          f32x4 (&oacc)[M16<T>::DB][M16<T>::QB]) {
    using G = M16<T>;
#pragma unroll
    for (int t = 0; t < G::KS; ++t) {
        f16x8 vf[G::DB];
#pragma unroll
        for (int db = 0; db < G::DB; ++db) {
            const char* base = vl + fr.voff[db] + 32 * t * G::ROW;
            const f16x4 lo = lds_read_tr16(base);
            const f16x4 up = lds_read_tr16(base + 8 * G::ROW);
            vf[db] = f16x8{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
        }
#pragma unroll
        for (int db = 0; db < G::DB; ++db)
#pragma unroll
            for (int qb = 0; qb < G::QB; ++qb) oacc[db][qb] = mfma16(vf[db], p[qb][t], oacc[db][qb]);
    }
}

// Optimistic softmax of one tile (as softmax16_optimistic) with each group of 8 exponentials
// (one P^T operand) packed and summed at once: 8 temporaries live instead of 32.
template <class T>
__device__ __forceinline__ void softmax16_optimistic_lean(
    const f32x4 (&s)[M16<T>::KB][M16<T>::QB], float scale_log2, const float (&m_run)[M16<T>::QB],
    float (&l_run)[M16<T>::QB], bool& overflow, f16x8 (&p)[M16<T>::QB][M16<T>::KS]) {
    using G = M16<T>;
    float sum[G::QB] = {0.0F, 0.0F};
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb)
#pragma unroll
        for (int t = 0; t < G::KS; ++t) {
            float e[8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                e[i] = exp2_fast(fmaf(s[2 * t + (i >> 2)][qb][i & 3], scale_log2, -m_run[qb]));
            p[qb][t] = pack8(e[0], e[1], e[2], e[3], e[4], e[5], e[6], e[7]);
            sum[qb] = sum8_f16(p[qb][t], sum[qb]);
        }
    overflow = wave_any(!(sum[0] < INFINITY && sum[1] < INFINITY));
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb) l_run[qb] = overflow ? l_run[qb] : l_run[qb] + sum[qb];
}

// Exact online softmax of one tile (as softmax16_tile with its row sums), each group of 8
// exponentials packed and summed at once.
template <class T>
__device__ __forceinline__ void softmax16_tile_lean(const f32x4 (&s)[M16<T>::KB][M16<T>::QB],
                                                    float scale_log2, float (&m_run)[M16<T>::QB],
                                                    float (&l_run)[M16<T>::QB],
                                                    float (&alpha)[M16<T>::QB], bool& rescale,
                                                    f16x8 (&p)[M16<T>::QB][M16<T>::KS]) {
    using G = M16<T>;
    float mx[G::QB];
    bool grow = false;
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb) {
        float x = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < G::KB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) x = fmaxf(x, s[kb][qb][r]);
        mx[qb] = max_xor32(max_xor16(x)) * scale_log2;
        grow = grow || (T::LAZY ? (mx[qb] > m_run[qb] + 8.0F) : (mx[qb] > m_run[qb]));
    }
    rescale = wave_any(grow);
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb) {
        const float m_new = rescale ? fmaxf(m_run[qb], mx[qb]) : m_run[qb];
        const float m_use = (m_new == -INFINITY) ? 0.0F : m_new;
        alpha[qb] = exp2_fast(m_run[qb] - m_use);
        m_run[qb] = m_new;
        float sum = 0.0F;
#pragma unroll
        for (int t = 0; t < G::KS; ++t) {
            float e[8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                e[i] = exp2_fast(fmaf(s[2 * t + (i >> 2)][qb][i & 3], scale_log2, -m_use));
            p[qb][t] = pack8(e[0], e[1], e[2], e[3], e[4], e[5], e[6], e[7]);
            sum = sum8_f16(p[qb][t], sum);
        }
        l_run[qb] = (rescale ? l_run[qb] * alpha[qb] : l_run[qb]) + sum;
    }
}

// Keys >= n, and (causal) keys right of the query, get -inf (as mask16): one threshold per query
// block and lane (fa::geom::st16_mask_limit), then a compare and a select per score.
template <class T, bool CAUSAL>
__device__ __forceinline__ void mask16_lim(f32x4 (&s)[M16<T>::KB][M16<T>::QB], int kt, int n,
                                           int qw, int lane) {
    using G = M16<T>;
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb) {
        const int lim = g::st16_mask_limit(n, kt, qw, lane, qb, CAUSAL);
#pragma unroll
        for (int kb = 0; kb < G::KB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                s[kb][qb][r] = g::st16_key(0, kb, r) > lim ? -INFINITY : s[kb][qb][r];
    }
}

// Softmax of one tile for flash_fwd_simple16, as softmax_any: optimistic against the running
// max, exact (with the rescale of O) on an overflow; FIRST (the item's first tile, peeled off the
// loop) exact without a rescale.
template <class T, bool FIRST>
__device__ __forceinline__ void softmax16_any(const f32x4 (&s)[M16<T>::KB][M16<T>::QB],
                                              float scale_log2, float (&m_run)[M16<T>::QB],
                                              float (&l_run)[M16<T>::QB],
                                              f32x4 (&oacc)[M16<T>::DB][M16<T>::QB],
                                              f16x8 (&p)[M16<T>::QB][M16<T>::KS]) {
    bool exact = true;
    if constexpr (T::LAZY && FA_OPTIMISTIC && !FIRST) {
        softmax16_optimistic_lean<T>(s, scale_log2, m_run, l_run, exact, p);
    }
    if (exact) {
        float alpha[M16<T>::QB];
        bool rescale;
        softmax16_tile_lean<T>(s, scale_log2, m_run, l_run, alpha, rescale, p);
        if (!FIRST && rescale) rescale16<T>(oacc, alpha);
    }
}

// flash_fwd_kernel's schedule (per tile: barrier, prefetch, then S = QK^T, mask, softmax and
// O += PV in turn; the item's first tile peeled off) on the ping-pong's 16x16x32 MFMAs and
// layouts (K tiles in the Frag16 read layout, V tiles with row_xor_m16, P^T straight from the
// lane's own exponentials). Each wave holds 32 query rows as two 16-row blocks, and each lane
// 4 keys of 2 queries per 16-key block. Same arguments, grid and results as flash_fwd_kernel.
template <class T, bool CAUSAL, bool SPLIT = false>
__global__ __launch_bounds__(T::THREADS) void flash_fwd_simple16(
    const f16* __restrict__ q, const f16* __restrict__ k, const f16* __restrict__ v,
    f16* __restrict__ o, float* __restrict__ lse, int n, int bh_count, int n_qblocks,
    float scale_log2, int negate_q, int tiles_per_split, float* __restrict__ o_part,
    float* __restrict__ lse_part, unsigned /*launch_id*/, int group_heads) {
    static_assert(T::SCHED == SIMPLE16, "16x16x32 simple schedule");
    static_assert((T::D == 128 && T::BC == 32) || (T::D == 64 && T::BC == 64),
                  "the 16x16x32 layouts are written for D=128, BC=32 and D=64, BC=64");
    using G = M16<T>;
    constexpr int NBUF = T::NBUF;
    __shared__ __attribute__((aligned(1024))) char k_lds0[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char k_lds1[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char k_lds2[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char v_lds0[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char v_lds1[T::TILE_BYTES];
    __shared__ __attribute__((aligned(1024))) char v_lds2[T::TILE_BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = wave_uniform(threadIdx.x >> 6);
    const int items = bh_count * n_qblocks;
    const int split = SPLIT ? static_cast<int>(blockIdx.x) / items : 0;
    auto run_item = [&](const g::Work w) {
    const size_t head = static_cast<size_t>(w.bh) * n * T::D;
    const f16* kh = k + head;
    const f16* vh = v + head;
    const int q0 = w.qb * T::BR;
    const int qw = q0 + wave * 32;  // first query of this wave
    const int n_all = g::num_kv_tiles(n, q0, T::BR, T::BC, CAUSAL);
    const g::KeyRange range = SPLIT ? g::split_range(n_all, tiles_per_split, split)
                                    : g::KeyRange{0, n_all};
    const int j_begin = range.begin;
    const int n_tiles = range.begin + range.count;  // absolute: tiles [j_begin, n_tiles)
    if (SPLIT && range.count == 0) return;           // workgroup-uniform

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    auto kbuf = [&](auto b) {
        constexpr int B = decltype(b)::value;
        return B == 0 ? k_lds0 : (B == 1 ? k_lds1 : k_lds2);
    };
    auto vbuf = [&](auto b) {
        constexpr int B = decltype(b)::value;
        return B == 0 ? v_lds0 : (B == 1 ? v_lds1 : v_lds2);
    };

    constexpr int PRIO = T::D == 128 ? FA_SIMPLE_PRIO_D128 : FA_SIMPLE_PRIO_D64;
    const TileDma<T, true> dma_k(wave, lane);  // K tiles in the layout of Frag16's K reads
    const TileDma<T> dma(wave, lane);          // V tiles, swizzle fa::geom::row_xor_m16
    load_tile<T>(kh, j_begin * T::BC, n, kbuf(I0{}), dma_k);
    load_tile<T>(vh, j_begin * T::BC, n, vbuf(I0{}), dma);
    if constexpr (NBUF == 3) {
        if (j_begin + 1 < n_tiles) {
            load_tile<T>(kh, (j_begin + 1) * T::BC, n, kbuf(I1{}), dma_k);
            load_tile<T>(vh, (j_begin + 1) * T::BC, n, vbuf(I1{}), dma);
        }
    }
    f16x8 qf[G::QB][G::DC];
    // (a negative scale negates Q by one sign XOR per register: load_q16's conditional negation
    // is turned into selects here, with a wait for the Q loads early in the prologue)
    load_q16<T>(q + head, qw, n, lane, 0, qf);
    const unsigned qsign = negate_q != 0 ? 0x80008000U : 0U;
#pragma unroll
    for (int qb = 0; qb < G::QB; ++qb)
#pragma unroll
        for (int dc = 0; dc < G::DC; ++dc) qf[qb][dc] = xor_sign8(qf[qb][dc], qsign);
    const Frag16<T> fr(lane);

    f32x4 oacc[G::DB][G::QB];
#pragma unroll
    for (int db = 0; db < G::DB; ++db)
#pragma unroll
        for (int qb = 0; qb < G::QB; ++qb) oacc[db][qb] = f32x4{};
    float m_run[G::QB] = {-INFINITY, -INFINITY};  // running maxima, log2 domain (scaled)
    float l_run[G::QB] = {0.0F, 0.0F};            // the lane's partial row sums (its keys)

    // Tile j in buffer B, as in flash_fwd_kernel.
    auto tile = [&](int j, auto b, auto first) {
        constexpr int B = decltype(b)::value;
        using Refill = std::integral_constant<int, (B + NBUF - 1) % NBUF>;
        if (NBUF == 3 && j > j_begin && j + 1 < n_tiles) {
            // vmcnt(2 * DMA_ITERS) lgkmcnt(0): only the next tile's requests stay in flight
            __builtin_amdgcn_s_waitcnt(static_cast<short>(0x0070 | (2 * T::DMA_ITERS)));
        } else {
            wait_vmem();
        }
        __syncthreads();  // tile j is in LDS for every wave; tile j-1's buffers are free
        if (j + NBUF - 1 < n_tiles) {
            load_tile<T>(kh, (j + NBUF - 1) * T::BC, n, kbuf(Refill{}), dma_k);
            load_tile<T>(vh, (j + NBUF - 1) * T::BC, n, vbuf(Refill{}), dma);
        }
        const int kt = j * T::BC;
        if (qw >= n || g::tile_fully_masked(kt, qw, 32, CAUSAL)) return;  // wave-uniform
        f32x4 s[G::KB][G::QB];
        if constexpr (PRIO & 1) __builtin_amdgcn_s_setprio(1);
        qk16_lean<T>(kbuf(b), fr, qf, s);
        if constexpr (PRIO & 1) __builtin_amdgcn_s_setprio(0);
        if (g::tile_needs_mask(n, kt, T::BC, qw, CAUSAL)) mask16_lim<T, CAUSAL>(s, kt, n, qw, lane);
        f16x8 p[G::QB][G::KS];
        softmax16_any<T, decltype(first)::value>(s, scale_log2, m_run, l_run, oacc, p);
        if constexpr (PRIO & 2) __builtin_amdgcn_s_setprio(1);
        pv16_lean<T>(vbuf(b), fr, p, oacc);
        if constexpr (PRIO & 2) __builtin_amdgcn_s_setprio(0);
    };
    using Later = std::false_type;
    tile(j_begin, I0{}, std::true_type{});
    int j = j_begin + 1;
    if constexpr (NBUF == 3) {
        for (; j + 3 <= n_tiles; j += 3) {
            tile(j, I1{}, Later{});
            tile(j + 1, I2{}, Later{});
            tile(j + 2, I0{}, Later{});
        }
        if (j < n_tiles) tile(j, I1{}, Later{});
        if (j + 1 < n_tiles) tile(j + 1, I2{}, Later{});
    } else {
        // (the odd last tile inside the loop: a second instance of the tile code after it would
        // keep its own copies of the fragment offsets live across the loop)
        for (; j < n_tiles; j += 2) {
            tile(j, I1{}, Later{});
            if (j + 1 < n_tiles) tile(j + 1, I0{}, Later{});
        }
    }
    if constexpr (SPLIT) {
        const size_t part = static_cast<size_t>(split) * bh_count + w.bh;
        store16_partial<T>(o_part + part * n * T::D, lse_part + part * n, qw, n, lane, m_run,
                           l_run, oacc);
    } else {
        store16<T>(o + head, lse ? lse + static_cast<size_t>(w.bh) * n : nullptr, qw, n, lane,
                   m_run, l_run, oacc);
    }
    };
    run_item(SPLIT ? g::work_of(static_cast<int>(blockIdx.x) - split * items, bh_count,
                                n_qblocks, CAUSAL)
                   : g::work_of_xcd(blockIdx.x, bh_count, n_qblocks, CAUSAL, group_heads));
}

// ---- tile table -------------------------------------------------------------------------------
// Counterpart of the reference's per-(variant, d, causal) `using` lines
// (csrc/kernels/flash_fwd.cu:597-612). On MI355X the best tile also depends on the sequence
// length and the grid size, so the "opt" / "fp16acc" rows are split by N at thresholds found by
// the tile sweep (FA2-paper shapes, B*N = 16k tokens, and interleaved A/B of the candidates):
//   * d = 64: the 8-wave simple schedule (256-row workgroups, 64-key tiles, two workgroups per
//     CU) on 16x16x32 MFMAs (SIMPLE16); causal up to 2048 keys on 32x32x16 MFMAs (SIMPLE).
//     SIMPLE16 against SIMPLE: non-causal +1.2 / +3.9 / +4.8 / +3.8 % at 512 / 1024 / 2048 /
//     4096 keys, causal +1.8 / +2.0 / +3.4 % at 3072 / 4096 (two grids); against the d = 64
//     ping-pong that the table ran on long sequences: non-causal +2.9 / +2.4 / +0.5 / +1.7 %
//     (4x16x4096, 2x32x8192, 1x16x16384, 1x32x16384), causal +1.6 / +6.1 / +4.0 / -0.7 %
//     (2x16x8192, 2x32x8192, 1x32x16384, 1x16x16384). Causal at 1024 and 2048 keys it measured
//     -1.3 to +0.8 % (and -0.8 to -2.5 % on the many-heads shape with outlier keys);
//   * d = 128: the 16x16x32 ping-pong for long sequences; up to 1536 keys (causal 3072) the
//     4-wave simple tile, which has no pipeline prologue and epilogue per workgroup (and, when
//     causal, fewer diagonal tiles): on 16x16x32 MFMAs above 256 keys (causal 512; +3.3 / +5.2 %
//     at 512 / 768, causal +1.0 / +2.7 / +3.8 % at 1024 / 1536 / 2048 against 32x32x16), else
//     on 32x32x16 (-1.8 % at 256, causal -1.2 % at 512 on 16x16x32). Against the ping-pong the
//     4-wave tile on 16x16x32 MFMAs measured +9.2 / +1.5 / -1.2 / -3.9 % at 1024 / 1536 / 2048 /
//     4096 keys, causal +6.0 / +0.3 / -3.6 % at 3072 / 4096 / 8192;
//   * small grids (fewer 8-wave workgroups than the 256 CUs, e.g. B*H = 16 at N = 1000): the
//     key-split schedule with 64-row workgroups (two waves per 32 query rows, each on half the
//     key tiles), so the same grid keeps twice the SIMDs busy.
// Each entry is "BC, NW, LAZY, SCHED" and can be overridden at build time with
// -DFA_<NAME>="..." (the counterpart of bench/tune.sh, which rewrites the `using` lines with
// sed); so can each threshold (a row applies while N <= its FA_*_MAX_N).
#ifndef FA_BASE_D64
#define FA_BASE_D64 64, 4, false, SIMPLE
#endif
#ifndef FA_BASE_D128
#define FA_BASE_D128 64, 4, false, SIMPLE
#endif
#ifndef FA_OPT_D64_SMALL
#define FA_OPT_D64_SMALL 64, 2, true, KSPLIT
#endif
#ifndef FA_OPT_D128_SMALL
#define FA_OPT_D128_SMALL 32, 2, true, KSPLIT
#endif
// Grids of at most FA_TINY_GRID_WGS 64-row query blocks (one round of one workgroup per CU)
// whose key loop has at least FA_TINY_MIN_TILES tiles: four waves per 32 query rows, each on
// every fourth key tile (128 KiB of LDS, eight waves). Against the two-way split, interleaved on
// one box: 1x8x2048 d=64 causal +12.7 %, 2x4x1500 d=128 causal +11.8 %, 2x8x1000 d=128 causal
// +4.5 %, 1x16x1024 d=128 +1.7 %, 2x8x1000 d=64 causal (16 tiles) +1.9 %; with 8 tiles
// (4x8x500 d=64) -7.7 %, with 4 (1x4x256 d=64) -13.8 %.
#ifndef FA_OPT_D64_TINY
#define FA_OPT_D64_TINY 64, 2, true, KSPLIT4
#endif
#ifndef FA_OPT_D128_TINY
#define FA_OPT_D128_TINY 32, 2, true, KSPLIT4
#endif
#ifndef FA_TINY_GRID_WGS
#define FA_TINY_GRID_WGS 256
#endif
#ifndef FA_TINY_MIN_TILES
#define FA_TINY_MIN_TILES 16
#endif
#ifndef FA_OPT_D64
#define FA_OPT_D64 64, 8, true, SIMPLE16
#endif
// Non-causal d = 64 grids of exactly one round of one workgroup per CU (B*H*ceil(N/256) = 256
// items, which is also how the head split runs its first heads when they fill one round): the
// simple schedule would hold one of its two workgroups per CU there, and the ping-pong, built for
// one, is faster (1x8x8192 +9.9 %, 1x16x4096 +7.8 %, 1x4x16384 +12.9 %, 2x8x4096 +8.6 %).
#ifndef FA_OPT_D64_ONE_ROUND
#define FA_OPT_D64_ONE_ROUND 64, 8, true, PINGPONG16
#endif
#ifndef FA_D64_ONE_ROUND_MIN_N
#define FA_D64_ONE_ROUND_MIN_N 4096
#endif
#ifndef FA_OPT_D64_CAUSAL_SHORT
#define FA_OPT_D64_CAUSAL_SHORT 64, 8, true, SIMPLE
#endif
#ifndef FA_OPT_D64_CAUSAL
#define FA_OPT_D64_CAUSAL 64, 8, true, SIMPLE16
#endif
#ifndef FA_D64_CAUSAL_SHORT_MAX_N
#define FA_D64_CAUSAL_SHORT_MAX_N 2048
#endif
// Causal d = 64 grids of at most FA_D64_CAUSAL_ROUND_MAX_WGS items (B*H*ceil(N/256); one round
// of the 64-key tiles' two workgroups per CU) at N >= FA_D64_CAUSAL_ROUND_MIN_N: such a grid
// lasts as long as its longest items, and 128-key tiles halve their tile steps (1x16x4096 +21 %,
// 1x8x8192 +23 %, 2x16x4096 +12 %, 4x16x1536 +13 %, 4x16x2048 +5 %), although their 167 VGPRs
// leave one workgroup per CU. On larger grids the longer tile's diagonal waste and the lost
// second workgroup cost more than the steps save (5x16x2048 -6 %, 3x16x4096 -4 %), and at
// N = 1024 it gains or loses with the grid's fill (+10 % to -2 %).
#ifndef FA_OPT_D64_CAUSAL_ROUND
#define FA_OPT_D64_CAUSAL_ROUND 128, 8, true, SIMPLE
#endif
#ifndef FA_D64_CAUSAL_ROUND_MIN_N
#define FA_D64_CAUSAL_ROUND_MIN_N 1536
#endif
#ifndef FA_D64_CAUSAL_ROUND_MAX_WGS
#define FA_D64_CAUSAL_ROUND_MAX_WGS 512
#endif
#ifndef FA_OPT_D128_VSHORT
#define FA_OPT_D128_VSHORT 32, 4, true, SIMPLE
#endif
#ifndef FA_OPT_D128_SHORT
#define FA_OPT_D128_SHORT 32, 4, true, SIMPLE16
#endif
#ifndef FA_OPT_D128
#define FA_OPT_D128 32, 8, true, PINGPONG16
#endif
#ifndef FA_OPT_D128_CAUSAL_VSHORT
#define FA_OPT_D128_CAUSAL_VSHORT 32, 4, true, SIMPLE
#endif
#ifndef FA_OPT_D128_CAUSAL_SHORT
#define FA_OPT_D128_CAUSAL_SHORT 32, 4, true, SIMPLE16
#endif
#ifndef FA_OPT_D128_CAUSAL
#define FA_OPT_D128_CAUSAL 32, 8, true, PINGPONG16
#endif
#ifndef FA_D128_VSHORT_MAX_N
#define FA_D128_VSHORT_MAX_N 256
#endif
#ifndef FA_D128_SHORT_MAX_N
#define FA_D128_SHORT_MAX_N 1536
#endif
#ifndef FA_D128_CAUSAL_VSHORT_MAX_N
#define FA_D128_CAUSAL_VSHORT_MAX_N 512
#endif
#ifndef FA_D128_CAUSAL_SHORT_MAX_N
#define FA_D128_CAUSAL_SHORT_MAX_N 3072
#endif
// ... and up to this N where the grid runs in head groups (fa::geom::causal_group_heads: 256
// heads or more), which make the 16x16x32 simple tile faster than the ping-pong there:
// 16x16x3500 +5.5 %, 16x16x4096 +3.8 %, 8x32x4096 +3.5 % in interleaved A/B; even at 5000 and
// 6144 (-0.6 to +0.1 %).
#ifndef FA_D128_CAUSAL_GROUPED_MAX_N
#define FA_D128_CAUSAL_GROUPED_MAX_N 4096
#endif
#ifndef FA_SMALL_GRID_WGS
#define FA_SMALL_GRID_WGS 256
#endif

// One kernel instance per row: the tile and whether it is the causal build.
template <class T_, bool CAUSAL_>
struct Entry {
    using T = T_;
    static constexpr bool CAUSAL = CAUSAL_;
};
enum TileId : int {
    BASE_D64, BASE_D64_C, BASE_D128, BASE_D128_C,
    OPT_D64_SMALL, OPT_D64_C_SMALL, OPT_D128_SMALL, OPT_D128_C_SMALL,
    OPT_D64_TINY, OPT_D64_C_TINY, OPT_D128_TINY, OPT_D128_C_TINY,
    OPT_D64, OPT_D64_ONE_ROUND, OPT_D64_C_SHORT, OPT_D64_C, OPT_D64_C_ROUND, OPT_D128_VSHORT,
    OPT_D128_SHORT, OPT_D128,
    OPT_D128_C_VSHORT, OPT_D128_C_SHORT, OPT_D128_C,
};
template <int ID> struct Row;
template <> struct Row<BASE_D64> : Entry<Tile<64, FA_BASE_D64>, false> {};
template <> struct Row<BASE_D64_C> : Entry<Tile<64, FA_BASE_D64>, true> {};
template <> struct Row<BASE_D128> : Entry<Tile<128, FA_BASE_D128>, false> {};
template <> struct Row<BASE_D128_C> : Entry<Tile<128, FA_BASE_D128>, true> {};
template <> struct Row<OPT_D64_SMALL> : Entry<Tile<64, FA_OPT_D64_SMALL>, false> {};
template <> struct Row<OPT_D64_C_SMALL> : Entry<Tile<64, FA_OPT_D64_SMALL>, true> {};
template <> struct Row<OPT_D128_SMALL> : Entry<Tile<128, FA_OPT_D128_SMALL>, false> {};
template <> struct Row<OPT_D128_C_SMALL> : Entry<Tile<128, FA_OPT_D128_SMALL>, true> {};
template <> struct Row<OPT_D64_TINY> : Entry<Tile<64, FA_OPT_D64_TINY>, false> {};
template <> struct Row<OPT_D64_C_TINY> : Entry<Tile<64, FA_OPT_D64_TINY>, true> {};
template <> struct Row<OPT_D128_TINY> : Entry<Tile<128, FA_OPT_D128_TINY>, false> {};
template <> struct Row<OPT_D128_C_TINY> : Entry<Tile<128, FA_OPT_D128_TINY>, true> {};
template <> struct Row<OPT_D64> : Entry<Tile<64, FA_OPT_D64>, false> {};
template <> struct Row<OPT_D64_ONE_ROUND> : Entry<Tile<64, FA_OPT_D64_ONE_ROUND>, false> {};
template <> struct Row<OPT_D64_C_SHORT> : Entry<Tile<64, FA_OPT_D64_CAUSAL_SHORT>, true> {};
template <> struct Row<OPT_D64_C> : Entry<Tile<64, FA_OPT_D64_CAUSAL>, true> {};
template <> struct Row<OPT_D64_C_ROUND> : Entry<Tile<64, FA_OPT_D64_CAUSAL_ROUND>, true> {};
template <> struct Row<OPT_D128_VSHORT> : Entry<Tile<128, FA_OPT_D128_VSHORT>, false> {};
template <> struct Row<OPT_D128_SHORT> : Entry<Tile<128, FA_OPT_D128_SHORT>, false> {};
template <> struct Row<OPT_D128> : Entry<Tile<128, FA_OPT_D128>, false> {};
template <> struct Row<OPT_D128_C_VSHORT> : Entry<Tile<128, FA_OPT_D128_CAUSAL_VSHORT>, true> {};
template <> struct Row<OPT_D128_C_SHORT> : Entry<Tile<128, FA_OPT_D128_CAUSAL_SHORT>, true> {};
template <> struct Row<OPT_D128_C> : Entry<Tile<128, FA_OPT_D128_CAUSAL>, true> {};

// The row for (head_dim in {64, 128}, causal, variant, seqlen >= 1, batch * heads >= 1).
TileId tile_id(int head_dim, bool causal, int variant, int n, int64_t bh) {
    if (variant == FA_VARIANT_BASELINE) {
        if (head_dim == 64) return causal ? BASE_D64_C : BASE_D64;
        return causal ? BASE_D128_C : BASE_D128;
    }
    if (bh * ((static_cast<int64_t>(n) + 255) / 256) < FA_SMALL_GRID_WGS) {
        const int bc =
            head_dim == 64 ? Tile<64, FA_OPT_D64_TINY>::BC : Tile<128, FA_OPT_D128_TINY>::BC;
        if (bh * ((static_cast<int64_t>(n) + 63) / 64) <= FA_TINY_GRID_WGS &&
            (n + bc - 1) / bc >= FA_TINY_MIN_TILES) {
            if (head_dim == 64) return causal ? OPT_D64_C_TINY : OPT_D64_TINY;
            return causal ? OPT_D128_C_TINY : OPT_D128_TINY;
        }
        if (head_dim == 64) return causal ? OPT_D64_C_SMALL : OPT_D64_SMALL;
        return causal ? OPT_D128_C_SMALL : OPT_D128_SMALL;
    }
    if (head_dim == 64) {
        if (!causal) {
            const int64_t items = bh * ((static_cast<int64_t>(n) + 255) / 256);
            return n >= FA_D64_ONE_ROUND_MIN_N && items <= g::kCus ? OPT_D64_ONE_ROUND : OPT_D64;
        }
        if (n >= FA_D64_CAUSAL_ROUND_MIN_N &&
            bh * ((static_cast<int64_t>(n) + 255) / 256) <= FA_D64_CAUSAL_ROUND_MAX_WGS)
            return OPT_D64_C_ROUND;
        return n <= FA_D64_CAUSAL_SHORT_MAX_N ? OPT_D64_C_SHORT : OPT_D64_C;
    }
    if (!causal) {
        if (n <= FA_D128_VSHORT_MAX_N) return OPT_D128_VSHORT;
        return n <= FA_D128_SHORT_MAX_N ? OPT_D128_SHORT : OPT_D128;
    }
    if (n <= FA_D128_CAUSAL_VSHORT_MAX_N) return OPT_D128_C_VSHORT;
    if (n <= FA_D128_CAUSAL_SHORT_MAX_N) return OPT_D128_C_SHORT;
    return n <= FA_D128_CAUSAL_GROUPED_MAX_N && g::causal_group_heads(128, bh) > 0
               ? OPT_D128_C_SHORT
               : OPT_D128_C;
}

// Calls f(Row<id>{}) with the row as a compile-time type.
template <class F>
decltype(auto) with_row(TileId id, F&& f) {
    switch (id) {
        case BASE_D64: return f(Row<BASE_D64>{});
        case BASE_D64_C: return f(Row<BASE_D64_C>{});
        case BASE_D128: return f(Row<BASE_D128>{});
        case BASE_D128_C: return f(Row<BASE_D128_C>{});
        case OPT_D64_SMALL: return f(Row<OPT_D64_SMALL>{});
        case OPT_D64_C_SMALL: return f(Row<OPT_D64_C_SMALL>{});
        case OPT_D128_SMALL: return f(Row<OPT_D128_SMALL>{});
        case OPT_D128_C_SMALL: return f(Row<OPT_D128_C_SMALL>{});
        case OPT_D64_TINY: return f(Row<OPT_D64_TINY>{});
        case OPT_D64_C_TINY: return f(Row<OPT_D64_C_TINY>{});
        case OPT_D128_TINY: return f(Row<OPT_D128_TINY>{});
        case OPT_D128_C_TINY: return f(Row<OPT_D128_C_TINY>{});
        case OPT_D64: return f(Row<OPT_D64>{});
        case OPT_D64_ONE_ROUND: return f(Row<OPT_D64_ONE_ROUND>{});
        case OPT_D64_C_SHORT: return f(Row<OPT_D64_C_SHORT>{});
        case OPT_D64_C: return f(Row<OPT_D64_C>{});
        case OPT_D64_C_ROUND: return f(Row<OPT_D64_C_ROUND>{});
        case OPT_D128_VSHORT: return f(Row<OPT_D128_VSHORT>{});
        case OPT_D128_SHORT: return f(Row<OPT_D128_SHORT>{});
        case OPT_D128: return f(Row<OPT_D128>{});
        case OPT_D128_C_VSHORT: return f(Row<OPT_D128_C_VSHORT>{});
        case OPT_D128_C_SHORT: return f(Row<OPT_D128_C_SHORT>{});
        default: return f(Row<OPT_D128_C>{});
    }
}

template <class T>
constexpr fa_tile_info info_of() {
    return fa_tile_info{T::BR, T::BC, T::NW * T::KS, T::LDS_BYTES, T::SCHED};
}

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

// Scale handling shared by every entry point. scale * log2(e) is folded into one FMA per score.
// A negative scale is applied by negating Q (exact in fp16) so the kernel's row max can use
// scale > 0; a zero scale becomes the smallest normal float, which leaves every exp2 argument at
// exactly 0 after rounding but keeps masked scores at -inf (0 * -inf would be NaN).
struct Scale {
    float log2e_scaled;
    int negate_q;
};
Scale scale_of(float softmax_scale) {
    Scale r{softmax_scale, 0};
    if (softmax_scale < 0.0F) {
        r.log2e_scaled = -softmax_scale;
        r.negate_q = 1;
    }
    r.log2e_scaled *= 1.44269504088896340736F;
    if (r.log2e_scaled < 1.17549435e-38F) r.log2e_scaled = 1.17549435e-38F;
    return r;
}

// Id of a kernel launch, for pp_overflow_record: process-wide, never 0. (A launch captured in a
// HIP graph keeps its id in every replay, so replays after one whose items overflowed may start
// their items checked: the same results, at the checked softmax's speed.)
unsigned next_launch_id() {
    static std::atomic<unsigned> seq{0};
    unsigned id = seq.fetch_add(1, std::memory_order_relaxed) + 1;
    if (id == 0) id = seq.fetch_add(1, std::memory_order_relaxed) + 1;
    return id;
}

// One launch of kernel T (SPLIT: the split-KV partial pass over n_splits * items workgroups).
template <class T, bool CAUSAL, bool SPLIT = false>
int launch(const fa_params& p, float* lse, hipStream_t stream, Scale sc, int n_splits = 1,
           int tiles_per_split = 0, float* o_part = nullptr, float* lse_part = nullptr) {
    const int n_qblocks = g::ceil_div(p.seqlen, T::BR);
    int n = p.seqlen;
    int bh = p.batch * p.heads;
    const auto* qp = static_cast<const f16*>(p.q);
    const auto* kp = static_cast<const f16*>(p.k);
    const auto* vp = static_cast<const f16*>(p.v);
    auto* op = static_cast<f16*>(p.o);
    int nqb = n_qblocks;
    float scale_log2 = sc.log2e_scaled;
    int negate_q = sc.negate_q;
    unsigned launch_id = next_launch_id();
    // head groups of a causal simple-schedule grid (the ping-pong's causal grids run pairs or
    // single blocks of their own order, the key split is for small grids; the baseline variant
    // keeps the first kernel's global order, as the yardstick the other variants are measured by)
    int group_heads = CAUSAL && !SPLIT && (T::SCHED == SIMPLE || T::SCHED == SIMPLE16) &&
                              p.variant != FA_VARIANT_BASELINE
                          ? g::causal_group_heads(T::D, bh)
                          : 0;
    void* args[] = {&qp, &kp, &vp, &op, &lse, &n, &bh, &nqb, &scale_log2, &negate_q,
                    &tiles_per_split, &o_part, &lse_part, &launch_id, &group_heads};
    dim3 grid(static_cast<unsigned>(n_qblocks) * static_cast<unsigned>(bh) *
              static_cast<unsigned>(n_splits));
    const void* fn;
    if constexpr (SPLIT) {
        static_assert(T::SCHED == SIMPLE || T::SCHED == SIMPLE16 || T::SCHED == PINGPONG16,
                      "split-KV runs a simple or the 16x16x32 ping-pong schedule");
        if constexpr (T::SCHED == PINGPONG16) {
            fn = reinterpret_cast<const void*>(&flash_fwd_pingpong16<T, CAUSAL, true>);
        } else if constexpr (T::SCHED == SIMPLE16) {
            fn = reinterpret_cast<const void*>(&flash_fwd_simple16<T, CAUSAL, true>);
        } else {
            fn = reinterpret_cast<const void*>(&flash_fwd_kernel<T, CAUSAL, true>);
        }
    } else if constexpr (T::SCHED == PINGPONG16) {
        fn = reinterpret_cast<const void*>(&flash_fwd_pingpong16<T, CAUSAL>);
        if constexpr (CAUSAL && FA_CAUSAL_PAIRS) {
            if (g::causal_pairs_pay(bh, n_qblocks, g::kCus)) {
                grid = dim3(static_cast<unsigned>(bh) * static_cast<unsigned>((n_qblocks + 1) / 2));
                fn = reinterpret_cast<const void*>(&flash_fwd_pingpong16<T, CAUSAL, false, true>);
            }
        }
    } else if constexpr (T::SCHED == KSPLIT || T::SCHED == KSPLIT4) {
        fn = reinterpret_cast<const void*>(&flash_fwd_ksplit<T, CAUSAL>);
    } else if constexpr (T::SCHED == SIMPLE16) {
        fn = reinterpret_cast<const void*>(&flash_fwd_simple16<T, CAUSAL>);
    } else {
        fn = reinterpret_cast<const void*>(&flash_fwd_kernel<T, CAUSAL>);
    }
    const hipError_t err = hipLaunchKernel(fn, grid, dim3(T::THREADS), args, 0, stream);
    if (err != hipSuccess) {
        return fail(FA_EHIP, std::string("flash_fwd: HIP launch failed: ") + hipGetErrorString(err));
    }
    return FA_OK;
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15U) == 0; }

// ---- split-KV ---------------------------------------------------------------------------------
// Rows of the split-KV partial pass, by (d, causal): the tile, and the automatic plan's target
// number of workgroups with work and minimum keys per range. The 16x16x32 ping-pong runs the
// long rows' tile over each key range; it wants about one workgroup per CU when not causal.
// Causal d=64 keeps the 4-wave simple tile, whose smaller workgroups balance the ragged causal
// ranges better (measured on few-head long shapes against the other candidates of this table).
#ifndef FA_SPLIT_D64
#define FA_SPLIT_D64 64, 8, true, PINGPONG16
#endif
#ifndef FA_SPLIT_D64_CAUSAL
#define FA_SPLIT_D64_CAUSAL 64, 4, true, SIMPLE
#endif
#ifndef FA_SPLIT_D128
#define FA_SPLIT_D128 32, 8, true, PINGPONG16
#endif
#ifndef FA_SPLIT_D128_CAUSAL
#define FA_SPLIT_D128_CAUSAL 32, 8, true, PINGPONG16
#endif
#ifndef FA_SPLIT_PLAN
#define FA_SPLIT_PLAN 256, 512  // non-causal: target workgroups, minimum keys per range
#endif
#ifndef FA_SPLIT_PLAN_D64_CAUSAL
#define FA_SPLIT_PLAN_D64_CAUSAL 1024, 256
#endif
#ifndef FA_SPLIT_PLAN_D128_CAUSAL
#define FA_SPLIT_PLAN_D128_CAUSAL 512, 1024
#endif
template <class T_, bool CAUSAL_, int TARGET_WGS_, int MIN_KEYS_>
struct SplitRow {
    using T = T_;
    static constexpr bool CAUSAL = CAUSAL_;
    static constexpr int TARGET_WGS = TARGET_WGS_;
    static constexpr int MIN_KEYS = MIN_KEYS_;
};
using SplitD64 = SplitRow<Tile<64, FA_SPLIT_D64>, false, FA_SPLIT_PLAN>;
using SplitD64C = SplitRow<Tile<64, FA_SPLIT_D64_CAUSAL>, true, FA_SPLIT_PLAN_D64_CAUSAL>;
using SplitD128 = SplitRow<Tile<128, FA_SPLIT_D128>, false, FA_SPLIT_PLAN>;
using SplitD128C = SplitRow<Tile<128, FA_SPLIT_D128_CAUSAL>, true, FA_SPLIT_PLAN_D128_CAUSAL>;
// Causal d = 128 on grids of fewer 256-row query blocks than CUs (the shapes fa.forward routes
// to split-KV): the 4-wave simple tile, two or more workgroups per CU hiding each other's
// prologue and epilogue, beats the ping-pong there (1x1x16384 +9.0 %, 1x4x8192 +11.1 %,
// 1x2x16384 +2.1 %) and loses on larger grids (1x2x32768 -6.4 %); on 16x16x32 MFMAs it gains
// another 1.4-2.9 % (1x2x16384, 1x4x8192, 1x1x16384). (The other split rows keep their tiles:
// the simple schedule on 16x16x32 MFMAs measured -4.6 to -7.4 % on the non-causal d = 64 split
// pass, one workgroup per CU, and -7.4 to +1.7 % on the causal one.)
#ifndef FA_SPLIT_D128_CAUSAL_SMALL
#define FA_SPLIT_D128_CAUSAL_SMALL 32, 4, true, SIMPLE16
#endif
#ifndef FA_SPLIT_PLAN_D128_CAUSAL_SMALL
#define FA_SPLIT_PLAN_D128_CAUSAL_SMALL 1024, 512
#endif
using SplitD128CSmall =
    SplitRow<Tile<128, FA_SPLIT_D128_CAUSAL_SMALL>, true, FA_SPLIT_PLAN_D128_CAUSAL_SMALL>;

template <class F>
auto with_split_row(const fa_params& p, F&& f) {
    if (p.head_dim == 64) return p.causal ? f(SplitD64C{}) : f(SplitD64{});
    if (!p.causal) return f(SplitD128{});
    const int64_t blocks = static_cast<int64_t>(p.batch) * p.heads * ((p.seqlen + 255) / 256);
    return blocks < FA_SMALL_GRID_WGS ? f(SplitD128CSmall{}) : f(SplitD128C{});
}

struct SplitPlan {
    int n_splits;
    int tiles_per_split;
    int block_q;
    int block_k;
    uint64_t workspace_bytes;
};

// Splits the key tiles of every query block into ranges of tiles_per_split tiles. With
// requested == 0 the range length is the total number of (query block, key tile) pairs over
// the row's TARGET_WGS (at least MIN_KEYS keys), so that about that many workgroups have work;
// otherwise the longest query block's tiles are cut into `requested` ranges. Workspace: fp32 O
// and LSE per split and row.
bool causal_round_split(const fa_params& p);

SplitPlan split_plan(const fa_params& p, int requested) {
    struct Consts {
        int br, bc, target_wgs, min_keys;
    };
    const Consts rc = with_split_row(p, [](auto row) {
        using R = decltype(row);
        return Consts{R::T::BR, R::T::BC, R::TARGET_WGS, R::MIN_KEYS};
    });
    const int br = rc.br;
    const int bc = rc.bc;
    const int64_t bh = static_cast<int64_t>(p.batch) * p.heads;
    const int nqb = g::ceil_div(p.seqlen, br);
    const int max_tiles = g::ceil_div(p.seqlen, bc);
    int tps;
    if (requested > 0) {
        tps = g::ceil_div(max_tiles, min(requested, max_tiles));
    } else if (p.head_dim == 128 && causal_round_split(p)) {
        tps = g::ceil_div(max_tiles, 2);  // one-round causal grids: two ranges
    } else {
        int64_t pairs = 0;
        for (int qb = 0; qb < nqb; ++qb) {
            pairs += g::num_kv_tiles(p.seqlen, qb * br, br, bc, p.causal != 0);
        }
        pairs *= bh;
        const int64_t want = (pairs + rc.target_wgs - 1) / rc.target_wgs;
        const int64_t min_tiles = g::ceil_div(rc.min_keys, bc);
        tps = static_cast<int>(std::min<int64_t>(std::max<int64_t>(min_tiles, want),
                                                 max_tiles));
    }
    SplitPlan sp{};
    sp.tiles_per_split = tps;
    sp.n_splits = g::ceil_div(max_tiles, tps);
    sp.block_q = br;
    sp.block_k = bc;
    sp.workspace_bytes = static_cast<uint64_t>(sp.n_splits) * bh * p.seqlen * (p.head_dim + 1) * 4;
    return sp;
}

// Whether fa_flash_fwd leaves most of the GPU idle on these params and the automatic split-KV
// plan is expected to be faster (measured on MI355X over few-head shapes at d = 64 and 128:
// the split path wins from N = 4096 on grids of fewer 8-wave workgroups than CUs; causal
// d = 64, whose partial pass keeps the 4-wave simple tile, only from N = 16384: 1x1x16384
// +48 %, 1x2x16384 +9 %, but 1x4x8192 -4 % and 1x8x4096 -20 %).
#ifndef FA_SPLITKV_MIN_N
#define FA_SPLITKV_MIN_N 4096
#endif
#ifndef FA_SPLITKV_MIN_N_D64_CAUSAL
#define FA_SPLITKV_MIN_N_D64_CAUSAL 16384
#endif
// Causal grids of about one round of 256-row query blocks (FA_SMALL_GRID_WGS to
// FA_SPLITKV_ROUND_MAX_WGS blocks) from FA_SPLITKV_ROUND_MIN_N keys: a single launch lasts as
// long as its longest query block, which holds every key tile, while most CUs finish early.
// Split-KV halves that block. Measured on MI355X with dev/fa_dev, single launch against the
// split pair (interleaved, 3 rounds), d = 128 with two ranges: 1x8x8192 +11.4 to +12.6 %,
// 1x4x16384 +22.1 %, 2x2x16384 +27.5 %, 1x2x32768 +31.8 %, 1x1x65536 +36.3 %, 1x6x12288 (288
// blocks) +12.7 %, 1x9x8192 (288) +5.1 %; the automatic plan's 3-4 ranges gained less. d = 64
// with the automatic plan: 1x8x8192 +12.5 %, 1x4x16384 +24.0 %, 1x2x32768 +29.9 %, 1x9x8192
// +7.2 %. Past the bounds: 1x16x4096 -1.5 % (d = 128) and -1.3 % (d = 64); 320 blocks
// (1x10x8192, 1x5x16384) +1.6 and +5.2 %; 512 blocks (1x16x8192 d = 128, 2x4x16384 d = 64)
// -12 % and -15 %.
#ifndef FA_SPLITKV_ROUND_MIN_N
#define FA_SPLITKV_ROUND_MIN_N 8192
#endif
#ifndef FA_SPLITKV_ROUND_MAX_WGS
#define FA_SPLITKV_ROUND_MAX_WGS 288
#endif
bool causal_round_split(const fa_params& p) {
    if (p.variant == FA_VARIANT_BASELINE || !p.causal || p.seqlen < FA_SPLITKV_ROUND_MIN_N)
        return false;
    const int64_t blocks =
        static_cast<int64_t>(p.batch) * p.heads * ((static_cast<int64_t>(p.seqlen) + 255) / 256);
    return blocks >= FA_SMALL_GRID_WGS && blocks <= FA_SPLITKV_ROUND_MAX_WGS;
}

bool splitkv_preferred(const fa_params& p) {
    if (p.variant == FA_VARIANT_BASELINE || p.seqlen < FA_SPLITKV_MIN_N) return false;
    if (causal_round_split(p)) return true;
    if (p.head_dim == 64 && p.causal && p.seqlen < FA_SPLITKV_MIN_N_D64_CAUSAL) return false;
    const int64_t bh = static_cast<int64_t>(p.batch) * p.heads;
    if (bh * ((static_cast<int64_t>(p.seqlen) + 255) / 256) >= FA_SMALL_GRID_WGS) return false;
    return split_plan(p, 0).n_splits >= 2;
}

// Non-causal head split for grids whose last round of ping-pong workgroups (one per CU) is
// mostly empty: the first `heads` (b, h) heads run as one launch whose items fill whole rounds,
// the rest through the split-KV pair, whose key ranges fill the CUs. Returns that head count, or
// 0 to keep the single launch (causal grids choose pairs or single blocks instead). Measured on
// MI355X, d = 128, through the binding against the single launch (one process, alternating):
// 1x9x8192 (288 items: 1.1 rounds) +37.5 %, 1x17x4096 +34.9 %, 1x17x8192 (2.1 rounds) +21.9 %,
// 1x36x4096 +14.7 %, 1x20x10000 +11.5 %, 1x40x5000 +9.6 %.
int64_t tail_heads(const fa_params& p) {
    if (p.variant == FA_VARIANT_BASELINE || p.causal || p.seqlen < FA_SPLITKV_MIN_N) return 0;
    const int64_t bh = static_cast<int64_t>(p.batch) * p.heads;
    const TileId id = tile_id(p.head_dim, false, p.variant, p.seqlen, bh);
    // the one-workgroup-per-CU rows, and the d = 64 row of long sequences (measured with the
    // d = 64 ping-pong on the first heads: d=64 1x9x8192 +36 %, 1x17x8192 +24 %, 1x20x10000
    // +12 %, 1x36x4096 +10 %, 1x40x5000 +6 % against its single launch)
    const bool d64_long = id == OPT_D64 && p.seqlen >= FA_SPLITKV_MIN_N;
    if (id != OPT_D128 && !d64_long) return 0;
    if (splitkv_preferred(p)) return 0;
    const int64_t nqb = (static_cast<int64_t>(p.seqlen) + 255) / 256;
    const int64_t items = bh * nqb;
    const int64_t full = items / g::kCus;  // whole rounds
    const int64_t last = items - full * g::kCus;
    // a last round at most a third full (the split pass and its merge run the rest at a lower
    // rate than the single launch: with the last round 3/8 full the split gained 2 %, with it
    // half full it lost 4 %)
    if (full < 1 || last == 0 || 3 * last > g::kCus) return 0;
    const int64_t heads = full * g::kCus / nqb;
    // the first heads must still fill the CUs (and keep this row of the tile table)
    if (heads * nqb < FA_SMALL_GRID_WGS || heads >= bh) return 0;
    return heads;
}

template <int D>
int combine(const fa_params& p, const SplitPlan& sp, const float* o_part, const float* lse_part,
            float* lse, hipStream_t stream) {
    const int64_t rows = static_cast<int64_t>(p.batch) * p.heads * p.seqlen;
    constexpr int ROWS_PER_BLOCK = CombineGeom<D>::ROWS;
    const auto blocks = static_cast<unsigned>((rows + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK);
    auto* op = static_cast<f16*>(p.o);
    int n = p.seqlen, bh = p.batch * p.heads, ns = sp.n_splits, tps = sp.tiles_per_split;
    int causal = p.causal, bq = sp.block_q, bk = sp.block_k;
    void* args[] = {&o_part, &lse_part, &op, &lse, &n, &bh, &ns, &tps, &causal, &bq, &bk};
    const hipError_t err = hipLaunchKernel(reinterpret_cast<const void*>(&flash_fwd_combine<D>),
                                           dim3(blocks), dim3(256), args, 0, stream);
    if (err != hipSuccess) {
        return fail(FA_EHIP, std::string("flash_fwd_splitkv: HIP launch failed: ") +
                                 hipGetErrorString(err));
    }
    return FA_OK;
}

template <class R>
int splitkv(const fa_params& p, float* lse, const SplitPlan& sp, void* workspace, Scale sc,
            hipStream_t stream) {
    using T = typename R::T;
    auto* o_part = static_cast<float*>(workspace);
    float* lse_part = o_part + static_cast<size_t>(sp.n_splits) * p.batch * p.heads * p.seqlen *
                                   T::D;
    const int rc = launch<T, R::CAUSAL, true>(p, nullptr, stream, sc, sp.n_splits,
                                              sp.tiles_per_split, o_part, lse_part);
    if (rc != FA_OK) return rc;
    return combine<T::D>(p, sp, o_part, lse_part, lse, stream);
}

// ---- static scratch of the allocation-free split-KV entry point -------------------------------
// fa_flash_fwd_splitkv_static takes its partial-O / LSE workspace from `scratch`, a file-scope
// device array that every GPU the library runs on holds until the process ends. In host code
// the array's name only stands for the symbol; its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and kept in g_scratch_ptr. The partial pass
// writes every (range, row) entry the combine kernel reads, so nothing needs clearing between
// calls; calls that overlap on one GPU share the array and race.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int static_scratch(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        return fail(FA_EHIP, std::string("flash_fwd_splitkv_static: hipGetDevice failed: ") +
                                 hipGetErrorString(e));
    }
    if (dev < 0 || dev >= kMaxDevices) {
        return fail(FA_EHIP, "flash_fwd_splitkv_static: device index " + std::to_string(dev) +
                                 " beyond the " + std::to_string(kMaxDevices) + " supported");
    }
    const std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            return fail(FA_EHIP, std::string("flash_fwd_splitkv_static: hipGetSymbolAddress of "
                                             "the scratch array failed: ") +
                                     hipGetErrorString(e));
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return FA_OK;
}

bool tile_of(int head_dim, bool causal, int variant, int seqlen, int64_t bh, fa_tile_info* out) {
    if (head_dim != 64 && head_dim != 128) return false;
    *out = with_row(tile_id(head_dim, causal, variant, seqlen, bh),
                    [](auto row) { return info_of<typename decltype(row)::T>(); });
    return true;
}

}  // namespace
}  // namespace fa

extern "C" {

const char* fa_last_error(void) { return fa::g_last_error.c_str(); }

#define FA_STR_(x) #x
#define FA_STR(x) FA_STR_(x)
// The softmax build options follow the version, so that a caller (and the CPU tests' model of
// the ping-pong arithmetic) can read how this library was compiled.
const char* fa_version(void) {
    return "fa_hip 0.2.0 gfx950 pp16_unchecked=" FA_STR(FA_PP16_UNCHECKED) " pp16_margin=" FA_STR(
        FA_PP16_UNCHECKED_MARGIN) " pp16_spread=" FA_STR(FA_PP16_SPREAD);
}

int fa_tile_config(const fa_params* params, fa_tile_info* out) {
    fa::g_last_error.clear();
    if (params == nullptr || out == nullptr) {
        return fa::fail(FA_EINVAL, "fa_tile_config: params and out must not be NULL");
    }
    const fa_params& p = *params;
    if (p.variant > FA_VARIANT_FP16ACC) return fa::fail(FA_EINVAL, "fa_tile_config: unknown variant");
    if (p.batch <= 0 || p.heads <= 0 || p.seqlen <= 0) {
        return fa::fail(FA_EINVAL, "fa_tile_config: batch, heads and seqlen must be positive");
    }
    const int64_t bh = static_cast<int64_t>(p.batch) * p.heads;
    if (!fa::tile_of(p.head_dim, p.causal != 0, p.variant, p.seqlen, bh, out)) {
        return fa::fail(FA_EINVAL, "fa_tile_config: head_dim must be 64 or 128, got " +
                                       std::to_string(p.head_dim));
    }
    return FA_OK;
}

// Argument checks follow csrc/kernels/flash_fwd.cu:626-651 (same conditions and message
// keywords), extended with the checks a C caller needs (NULL pointers, reserved bytes,
// non-finite scale, 32-bit index limits of this kernel).
static int validate(const fa_params* params, const char* who) {
    using fa::fail;
    const std::string w = std::string(who) + ": ";
    if (params == nullptr) return fail(FA_EINVAL, w + "params must not be NULL");
    const fa_params& p = *params;
    if (p.batch <= 0 || p.heads <= 0 || p.seqlen <= 0) {
        return fail(FA_EINVAL, w + "batch, heads and seqlen must be positive");
    }
    if (p.head_dim != 64 && p.head_dim != 128) {
        return fail(FA_EINVAL, w + "head_dim must be 64 or 128, got " + std::to_string(p.head_dim));
    }
    if (p.variant > FA_VARIANT_FP16ACC) return fail(FA_EINVAL, w + "unknown variant");
    if (p.causal > 1 || p.reserved[0] != 0 || p.reserved[1] != 0) {
        return fail(FA_EINVAL, w + "causal must be 0 or 1 and reserved bytes zero");
    }
    if (p.q == nullptr || p.k == nullptr || p.v == nullptr || p.o == nullptr) {
        return fail(FA_EINVAL, w + "q, k, v and o must be non-null");
    }
    if (!fa::aligned16(p.q) || !fa::aligned16(p.k) || !fa::aligned16(p.v) ||
        !fa::aligned16(p.o)) {
        return fail(FA_EINVAL, w + "tensors must be 16-byte aligned (16-byte loads)");
    }
    if (!std::isfinite(p.softmax_scale)) return fail(FA_EINVAL, w + "softmax_scale must be finite");
    // Offsets inside one head are 32-bit; the grid is one-dimensional.
    if (static_cast<int64_t>(p.seqlen) * p.head_dim > INT32_MAX) {
        return fail(FA_EINVAL, w + "seqlen * head_dim must be below 2^31");
    }
    // The smallest workgroup has 64 query rows: this bounds the grid of every tile.
    const int64_t blocks = static_cast<int64_t>(p.batch) * p.heads *
                           ((static_cast<int64_t>(p.seqlen) + 63) / 64);
    if (blocks > INT32_MAX) {
        return fail(FA_EINVAL, w + "batch * heads * query blocks exceeds the grid limit");
    }
    return FA_OK;
}

static int run(const fa_params& p, float* lse, void* stream) {
    const fa::Scale sc = fa::scale_of(p.softmax_scale);
    auto s = static_cast<hipStream_t>(stream);
    const int64_t bh = static_cast<int64_t>(p.batch) * p.heads;
    return fa::with_row(fa::tile_id(p.head_dim, p.causal != 0, p.variant, p.seqlen, bh),
                        [&](auto row) {
        using R = decltype(row);
        return fa::launch<typename R::T, R::CAUSAL>(p, lse, s, sc);
    });
}

int fa_flash_fwd(const fa_params* params, void* stream) {
    fa::g_last_error.clear();
    const int rc = validate(params, "flash_fwd");
    return rc != FA_OK ? rc : run(*params, nullptr, stream);
}

int fa_flash_fwd_lse(const fa_params* params, float* lse, void* stream) {
    fa::g_last_error.clear();
    const int rc = validate(params, "flash_fwd_lse");
    if (rc != FA_OK) return rc;
    if (lse == nullptr || (reinterpret_cast<uintptr_t>(lse) & 3U) != 0) {
        return fa::fail(FA_EINVAL, "flash_fwd_lse: lse must be a non-null, 4-byte aligned float*");
    }
    return run(*params, lse, stream);
}

int fa_tail_plan(const fa_params* params, int64_t* single_heads) {
    fa::g_last_error.clear();
    if (single_heads == nullptr) {
        return fa::fail(FA_EINVAL, "fa_tail_plan: single_heads must not be NULL");
    }
    *single_heads = 0;
    if (params == nullptr) return fa::fail(FA_EINVAL, "fa_tail_plan: params must not be NULL");
    const fa_params& p = *params;
    if (p.batch <= 0 || p.heads <= 0 || p.seqlen <= 0) {
        return fa::fail(FA_EINVAL, "fa_tail_plan: batch, heads and seqlen must be positive");
    }
    if (p.head_dim != 64 && p.head_dim != 128) {
        return fa::fail(FA_EINVAL, "fa_tail_plan: head_dim must be 64 or 128, got " +
                                       std::to_string(p.head_dim));
    }
    if (static_cast<int64_t>(p.seqlen) * p.head_dim > INT32_MAX) {
        return fa::fail(FA_EINVAL, "fa_tail_plan: seqlen * head_dim must be below 2^31");
    }
    if (p.variant > FA_VARIANT_FP16ACC) {
        return fa::fail(FA_EINVAL, "fa_tail_plan: unknown variant " + std::to_string(p.variant));
    }
    *single_heads = fa::tail_heads(p);
    return FA_OK;
}

int fa_splitkv_plan(const fa_params* params, int32_t num_splits, fa_splitkv_info* out) {
    fa::g_last_error.clear();
    if (out == nullptr) return fa::fail(FA_EINVAL, "fa_splitkv_plan: out must not be NULL");
    if (params == nullptr) return fa::fail(FA_EINVAL, "fa_splitkv_plan: params must not be NULL");
    const fa_params& p = *params;
    if (p.batch <= 0 || p.heads <= 0 || p.seqlen <= 0) {
        return fa::fail(FA_EINVAL, "fa_splitkv_plan: batch, heads and seqlen must be positive");
    }
    if (p.head_dim != 64 && p.head_dim != 128) {
        return fa::fail(FA_EINVAL, "fa_splitkv_plan: head_dim must be 64 or 128, got " +
                                       std::to_string(p.head_dim));
    }
    if (static_cast<int64_t>(p.seqlen) * p.head_dim > INT32_MAX) {
        return fa::fail(FA_EINVAL, "fa_splitkv_plan: seqlen * head_dim must be below 2^31");
    }
    if (num_splits < 0) return fa::fail(FA_EINVAL, "fa_splitkv_plan: num_splits must be >= 0");
    const fa::SplitPlan sp = fa::split_plan(p, num_splits);
    *out = fa_splitkv_info{sp.n_splits, sp.tiles_per_split, sp.block_q, sp.block_k,
                           sp.workspace_bytes, fa::splitkv_preferred(p) ? 1 : 0, 0};
    return FA_OK;
}

// Checks shared by the two split-KV entry points (before any HIP call); the plan on success.
static int splitkv_checks(const fa_params* params, float* lse, int32_t num_splits, const char* who,
                          fa::SplitPlan* plan) {
    const std::string w = std::string(who) + ": ";
    const int rc = validate(params, who);
    if (rc != FA_OK) return rc;
    const fa_params& p = *params;
    if (num_splits < 0) return fa::fail(FA_EINVAL, w + "num_splits must be >= 0");
    if (lse != nullptr && (reinterpret_cast<uintptr_t>(lse) & 3U) != 0) {
        return fa::fail(FA_EINVAL, w + "lse must be 4-byte aligned");
    }
    *plan = fa::split_plan(p, num_splits);
    if (static_cast<int64_t>(p.batch) * p.heads * fa::g::ceil_div(p.seqlen, plan->block_q) *
            plan->n_splits > INT32_MAX) {
        return fa::fail(FA_EINVAL, w + "splits * query blocks exceed the grid limit");
    }
    return FA_OK;
}

static int splitkv_run(const fa_params& p, float* lse, const fa::SplitPlan& sp, void* workspace,
                       void* stream) {
    const fa::Scale sc = fa::scale_of(p.softmax_scale);
    auto s = static_cast<hipStream_t>(stream);
    return fa::with_split_row(p, [&](auto row) {
        return fa::splitkv<decltype(row)>(p, lse, sp, workspace, sc, s);
    });
}

int fa_flash_fwd_splitkv(const fa_params* params, float* lse, int32_t num_splits,
                         void* workspace, uint64_t workspace_bytes, void* stream) {
    fa::g_last_error.clear();
    fa::SplitPlan sp{};
    const int rc = splitkv_checks(params, lse, num_splits, "flash_fwd_splitkv", &sp);
    if (rc != FA_OK) return rc;
    if (workspace == nullptr || !fa::aligned16(workspace)) {
        return fa::fail(FA_EINVAL, "flash_fwd_splitkv: workspace must be non-null and 16-byte aligned");
    }
    if (workspace_bytes < sp.workspace_bytes) {
        return fa::fail(FA_EINVAL, "flash_fwd_splitkv: workspace too small: need " +
                                       std::to_string(sp.workspace_bytes) + " bytes");
    }
    return splitkv_run(*params, lse, sp, workspace, stream);
}

int fa_flash_fwd_splitkv_static(const fa_params* params, float* lse, int32_t num_splits,
                                void* stream) {
    fa::g_last_error.clear();
    fa::SplitPlan sp{};
    const int rc = splitkv_checks(params, lse, num_splits, "flash_fwd_splitkv_static", &sp);
    if (rc != FA_OK) return rc;
    if (sp.workspace_bytes > FA_STATIC_SCRATCH_BYTES) {
        return fa::fail(FA_EINVAL, "flash_fwd_splitkv_static: the plan needs " +
                                       std::to_string(sp.workspace_bytes) +
                                       " bytes of workspace, more than the static scratch of " +
                                       std::to_string(FA_STATIC_SCRATCH_BYTES) +
                                       " bytes; pass a smaller num_splits or call "
                                       "fa_flash_fwd_splitkv with a workspace");
    }
    void* ws = nullptr;
    const int src = fa::static_scratch(&ws);
    if (src != FA_OK) return src;
    return splitkv_run(*params, lse, sp, ws, stream);
}

}  // extern "C"

#if FA_PROBE
// Development build only (FA_PROBE 1): the ping-pong's timeline stamps of the current device.
extern "C" __attribute__((visibility("default"))) int fa_probe_clear(void) {
    static unsigned long long zeros[kProbeWorkgroups * kProbeSlots];
    return hipMemcpyToSymbol(HIP_SYMBOL(probe_stamps), zeros, sizeof(zeros), 0,
                             hipMemcpyHostToDevice) == hipSuccess ? 0 : 1;
}
extern "C" __attribute__((visibility("default"))) int fa_probe_read(void* dst, uint64_t bytes) {
    const uint64_t size = sizeof(unsigned long long) * kProbeWorkgroups * kProbeSlots;
    return hipMemcpyFromSymbol(dst, HIP_SYMBOL(probe_stamps), bytes < size ? bytes : size, 0,
                               hipMemcpyDeviceToHost) == hipSuccess ? 0 : 1;
}
#endif
