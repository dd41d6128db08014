// FlashAttention-2 forward for AMD MI355X (gfx950, CDNA4), written for the hardware:
//
//   O = softmax(Q K^T * scale) V        Q, K, V, O: [B, H, N, D] fp16, fp32 accumulation
//
// Work decomposition
//   * A workgroup of NW wave64s owns BR = 32*NW consecutive query rows of one (batch, head);
//     each wave owns 32 of them for the whole kernel, so a row's softmax statistics never leave
//     the wave (the FA2 split-Q scheme of csrc/kernels/flash_fwd.cu:7-12).
//   * The workgroup streams over keys in tiles of BC rows, double-buffered in LDS and filled by
//     global_load_lds_dwordx4 (direct HBM/L2 -> LDS, no VGPR staging): tile j+1 is in flight
//     while tile j is computed, with one workgroup barrier per tile.
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
//   * Causal: tiles right of the diagonal are never loaded; masking runs only on diagonal and
//     tail tiles; longest query blocks launch first.
//   * Ragged N: K/V/Q row indices are clamped to N-1 (always in bounds); clamped keys are
//     masked to -inf and so contribute exactly 0, clamped query rows are never stored.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>

#include "fa_device.h"
#include "fa_geometry.h"
#include "fa_hip.h"

namespace fa {
namespace {

using namespace fa::dev;
namespace g = fa::geom;

// Compile-time tile shape and options. Counterpart of the reference's Config/Opt pair
// (csrc/kernels/flash_fwd.cu:70-100), re-derived for 64-wide waves and 32x32 MFMA blocks.
template <int D_, int BC_, int NW_, bool LAZY_>
struct Tile {
    static constexpr int D = D_;            // head dim (64 or 128)
    static constexpr int BC = BC_;          // keys per K/V tile
    static constexpr int NW = NW_;          // wave64s per workgroup
    static constexpr bool LAZY = LAZY_;     // rescale O only when a row max grows by > 2^8
    static constexpr int BR = 32 * NW;      // query rows per workgroup
    static constexpr int THREADS = 64 * NW;
    static constexpr int ROW_BYTES = 2 * D;
    static constexpr int CPR = D / 8;                  // 16-byte chunks per row
    static constexpr int TILE_BYTES = BC * ROW_BYTES;  // one K or V tile
    static constexpr int LDS_BYTES = 4 * TILE_BYTES;   // {K, V} x 2 buffers
    static constexpr int NB = BC / 32;                 // 32-key MFMA blocks per tile
    static constexpr int KK = D / 16;                  // 16-deep MFMA steps over D
    static constexpr int DB = D / 32;                  // 32-wide output blocks over D
    static constexpr int DMA_ITERS = (BC * CPR) / (64 * NW);
    static_assert(D == 64 || D == 128, "head dim must be 64 or 128");
    static_assert(BC % 32 == 0, "BC must be a multiple of the 32-key MFMA block");
    static_assert((BC * CPR) % (64 * NW) == 0, "tile must split evenly over the waves");
    static_assert(LDS_BYTES <= 64 * 1024, "static LDS budget");
};

// Copies K or V rows [kt, kt + BC) of one head into a swizzled LDS tile. Each wave issues
// DMA_ITERS 16-byte-per-lane direct loads covering 64 consecutive physical chunk slots; the
// lane picks the global chunk whose swizzled home is its slot. Rows >= n re-read row n-1
// (masked later), so no load is ever out of bounds.
template <class T>
__device__ __forceinline__ void load_tile(const f16* __restrict__ src, int kt, int n, char* lds,
                                          int wave, int lane) {
#pragma unroll
    for (int it = 0; it < T::DMA_ITERS; ++it) {
        const int slot0 = (it * T::NW + wave) * 64;  // wave-uniform
        const int slot = slot0 + lane;
        const int row = slot / T::CPR;
        const int chunk = g::swizzle_chunk(row, slot % T::CPR);
        const int grow = min(kt + row, n - 1);
        lds_dma16(src + static_cast<size_t>(grow) * T::D + chunk * 8, lds + slot0 * 16);
    }
}

template <class T, bool CAUSAL>
__global__ __launch_bounds__(T::THREADS) void flash_fwd_kernel(
    const f16* __restrict__ q, const f16* __restrict__ k, const f16* __restrict__ v,
    f16* __restrict__ o, int n, int bh_count, int n_qblocks, float scale_log2, int negate_q) {
    __shared__ __attribute__((aligned(1024))) char smem[T::LDS_BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = wave_uniform(threadIdx.x >> 6);
    const int col = lane & 31;  // this lane's query within the wave's 32
    const int hi = lane >> 5;   // which half of the wave

    const g::Work w = g::work_of(blockIdx.x, bh_count, n_qblocks, CAUSAL);
    const size_t head = static_cast<size_t>(w.bh) * n * T::D;
    const f16* qh = q + head;
    const f16* kh = k + head;
    const f16* vh = v + head;
    f16* oh = o + head;

    const int q0 = w.qb * T::BR;
    const int qw = q0 + wave * 32;  // first query of this wave
    const int qrow = qw + col;      // this lane's query
    const int n_tiles = g::num_kv_tiles(n, q0, T::BR, T::BC, CAUSAL);

    // LDS: [K0 | K1 | V0 | V1]; buffer b of K at b*TILE_BYTES, of V at (2+b)*TILE_BYTES.
    auto kbuf = [&](int b) { return smem + b * T::TILE_BYTES; };
    auto vbuf = [&](int b) { return smem + (2 + b) * T::TILE_BYTES; };

    // Prefetch tile 0 while Q is fetched into registers.
    load_tile<T>(kh, 0, n, kbuf(0), wave, lane);
    load_tile<T>(vh, 0, n, vbuf(0), wave, lane);

    // Q^T operand: lane holds Q[qrow][16*kk + 8*hi .. +7] for every kk (32 VGPRs at D=128).
    f16x8 qf[T::KK];
    {
        const f16* src = qh + static_cast<size_t>(min(qrow, n - 1)) * T::D + 8 * hi;
#pragma unroll
        for (int kk = 0; kk < T::KK; ++kk) {
            qf[kk] = *reinterpret_cast<const f16x8*>(src + 16 * kk);
            if (negate_q) qf[kk] = -qf[kk];
        }
    }

    // Per-lane LDS byte offsets. K fragment (nb, kk): row 32*nb + col, logical chunk 2*kk + hi.
    // Only the low 3 chunk bits are swizzled, so chunk 2*kk+hi splits into an immediate part
    // 8*(kk/4) and a lane part ((2*(kk%4)+hi) ^ row_xor(col)).
    int koff[4];
#pragma unroll
    for (int kq = 0; kq < 4; ++kq)
        koff[kq] = col * T::ROW_BYTES + 16 * ((2 * kq + hi) ^ g::row_xor(col));
    // V^T fragment (nb, h, db, half-read e): rows 32*nb + 16*h + 8*e + 4*hi + tr16_row(lane),
    // columns 32*db + 16*((lane>>4)&1) + tr16_col(lane). row & 7 = 4*hi + tr16_row(lane).
    const int vrow = 4 * hi + g::tr16_row(lane);
    int voff[2];
#pragma unroll
    for (int dpar = 0; dpar < 2; ++dpar) {
        const int c = 32 * dpar + 16 * ((lane >> 4) & 1) + g::tr16_col(lane);  // column in halves
        voff[dpar] = vrow * T::ROW_BYTES + 16 * ((c >> 3) ^ g::row_xor(vrow)) + 2 * (c & 7);
    }

    f32x16 oacc[T::DB];
#pragma unroll
    for (int db = 0; db < T::DB; ++db) oacc[db] = f32x16{};
    float m_run = -INFINITY;  // running max of this lane's query, log2 domain (scaled)
    float l_run = 0.0F;       // this lane's partial row sum (its 16 keys of each 32-key block)

    for (int j = 0; j < n_tiles; ++j) {
        wait_vmem();
        __syncthreads();  // tile j is in LDS for every wave; tile j-1's buffers are free
        if (j + 1 < n_tiles) {
            load_tile<T>(kh, (j + 1) * T::BC, n, kbuf((j + 1) & 1), wave, lane);
            load_tile<T>(vh, (j + 1) * T::BC, n, vbuf((j + 1) & 1), wave, lane);
        }
        const int kt = j * T::BC;
        if (qw >= n || g::tile_fully_masked(kt, qw, 32, CAUSAL)) continue;  // wave-uniform
        const char* kl = kbuf(j & 1);
        const char* vl = vbuf(j & 1);

        // ---- S^T = K Q^T ------------------------------------------------------------------
        f32x16 s[T::NB];
#pragma unroll
        for (int nb = 0; nb < T::NB; ++nb) {
            s[nb] = f32x16{};
#pragma unroll
            for (int kk = 0; kk < T::KK; ++kk) {
                const f16x8 a = *reinterpret_cast<const f16x8*>(
                    kl + koff[kk & 3] + nb * 32 * T::ROW_BYTES + 128 * (kk >> 2));
                s[nb] = mfma32(a, qf[kk], s[nb]);
            }
        }

        // ---- mask (tail tile, causal diagonal) ---------------------------------------------
        if (g::tile_needs_mask(n, kt, T::BC, qw, CAUSAL)) {
#pragma unroll
            for (int nb = 0; nb < T::NB; ++nb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kt + g::st_key(lane, nb, r);
                    const bool masked = key >= n || (CAUSAL && key > qrow);
                    s[nb][r] = masked ? -INFINITY : s[nb][r];
                }
        }

        // ---- online softmax (base 2) -------------------------------------------------------
        float mx = -INFINITY;
#pragma unroll
        for (int nb = 0; nb < T::NB; ++nb)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[nb][r]);
        mx = max_xor32(mx) * scale_log2;  // both halves now agree on the query's tile max

        const bool grow = T::LAZY ? (mx > m_run + 8.0F) : (mx > m_run);
        if (wave_any(grow)) {
            const float m_new = fmaxf(m_run, mx);
            // m_new is -inf only for a row that has seen nothing but masked keys; use 0 there so
            // that -inf - -inf never forms a NaN (its p values are exp2(-inf) = 0).
            const float alpha = exp2_fast(m_run - (m_new == -INFINITY ? 0.0F : m_new));
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < T::DB; ++db) oacc[db] *= alpha;
        }
        const float m_use = (m_run == -INFINITY) ? 0.0F : m_run;

        f16x8 p[T::NB][2];
#pragma unroll
        for (int nb = 0; nb < T::NB; ++nb) {
            float e[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                e[r] = exp2_fast(fmaf(s[nb][r], scale_log2, -m_use));
                l_run += e[r];
            }
            p[nb][0] = pack8(e[0], e[1], e[2], e[3], e[4], e[5], e[6], e[7]);
            p[nb][1] = pack8(e[8], e[9], e[10], e[11], e[12], e[13], e[14], e[15]);
        }

        // ---- O^T += V^T P^T ----------------------------------------------------------------
#pragma unroll
        for (int nb = 0; nb < T::NB; ++nb)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int db = 0; db < T::DB; ++db) {
                    const char* base =
                        vl + voff[db & 1] + (32 * nb + 16 * h) * T::ROW_BYTES + 128 * (db >> 1);
                    const f16x4 lo = lds_read_tr16(base);
                    const f16x4 up = lds_read_tr16(base + 8 * T::ROW_BYTES);
                    const f16x8 a = {lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
                    oacc[db] = mfma32(a, p[nb][h], oacc[db]);
                }
    }

    // ---- epilogue: O = acc / l, fp16 (RNE), rows < n ----------------------------------------
    const float l_tot = sum_xor32(l_run);
    const float inv = (l_tot > 0.0F) ? (1.0F / l_tot) : 0.0F;
    if (qrow < n) {
        f16* dst = oh + static_cast<size_t>(qrow) * T::D + 4 * hi;
#pragma unroll
        for (int db = 0; db < T::DB; ++db)
#pragma unroll
            for (int rq = 0; rq < 4; ++rq) {
                const f32x16& a = oacc[db];
                *reinterpret_cast<f16x4*>(dst + 32 * db + 8 * rq) =
                    pack4(a[4 * rq] * inv, a[4 * rq + 1] * inv, a[4 * rq + 2] * inv,
                          a[4 * rq + 3] * inv);
            }
    }
}

// ---- tile table -------------------------------------------------------------------------------
// Counterpart of the reference's per-(variant, d, causal) `using` lines
// (csrc/kernels/flash_fwd.cu:597-612), chosen for MI355X.
using BaseD64 = Tile<64, 64, 4, false>;
using BaseD128 = Tile<128, 64, 4, false>;
using OptD64 = Tile<64, 64, 4, true>;
using OptD128 = Tile<128, 64, 4, true>;

template <class T>
constexpr fa_tile_info info_of() {
    return fa_tile_info{T::BR, T::BC, T::NW, T::LDS_BYTES};
}

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

template <class T, bool CAUSAL>
int launch(const fa_params& p, hipStream_t stream, float scale_log2, int negate_q) {
    const int n_qblocks = g::ceil_div(p.seqlen, T::BR);
    int n = p.seqlen;
    int bh = p.batch * p.heads;
    const auto* qp = static_cast<const f16*>(p.q);
    const auto* kp = static_cast<const f16*>(p.k);
    const auto* vp = static_cast<const f16*>(p.v);
    auto* op = static_cast<f16*>(p.o);
    int nqb = n_qblocks;
    void* args[] = {&qp, &kp, &vp, &op, &n, &bh, &nqb, &scale_log2, &negate_q};
    const dim3 grid(static_cast<unsigned>(n_qblocks) * static_cast<unsigned>(bh));
    const hipError_t err =
        hipLaunchKernel(reinterpret_cast<const void*>(&flash_fwd_kernel<T, CAUSAL>), grid,
                        dim3(T::THREADS), args, 0, stream);
    if (err != hipSuccess) {
        return fail(FA_EHIP, std::string("flash_fwd: HIP launch failed: ") + hipGetErrorString(err));
    }
    return FA_OK;
}

template <class T64, class T128>
int dispatch(const fa_params& p, hipStream_t s, float scale_log2, int negate_q) {
    if (p.head_dim == 64) {
        return p.causal ? launch<T64, true>(p, s, scale_log2, negate_q)
                        : launch<T64, false>(p, s, scale_log2, negate_q);
    }
    return p.causal ? launch<T128, true>(p, s, scale_log2, negate_q)
                    : launch<T128, false>(p, s, scale_log2, negate_q);
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15U) == 0; }

bool tile_of(int head_dim, int variant, fa_tile_info* out) {
    if (head_dim != 64 && head_dim != 128) return false;
    if (variant == FA_VARIANT_BASELINE) {
        *out = head_dim == 64 ? info_of<BaseD64>() : info_of<BaseD128>();
    } else {
        *out = head_dim == 64 ? info_of<OptD64>() : info_of<OptD128>();
    }
    return true;
}

}  // namespace
}  // namespace fa

extern "C" {

const char* fa_last_error(void) { return fa::g_last_error.c_str(); }

const char* fa_version(void) { return "fa_hip 0.1.0 gfx950"; }

int fa_tile_config(int32_t head_dim, int32_t causal, int32_t variant, fa_tile_info* out) {
    fa::g_last_error.clear();
    (void)causal;
    if (out == nullptr) return fa::fail(FA_EINVAL, "fa_tile_config: out must not be NULL");
    if (variant < FA_VARIANT_BASELINE || variant > FA_VARIANT_FP16ACC) {
        return fa::fail(FA_EINVAL, "fa_tile_config: unknown variant");
    }
    if (!fa::tile_of(head_dim, variant, out)) {
        return fa::fail(FA_EINVAL, "fa_tile_config: head_dim must be 64 or 128, got " +
                                       std::to_string(head_dim));
    }
    return FA_OK;
}

// Argument checks follow csrc/kernels/flash_fwd.cu:626-651 (same conditions and message
// keywords), extended with the checks a C caller needs (NULL pointers, reserved bytes,
// non-finite scale, 32-bit index limits of this kernel).
int fa_flash_fwd(const fa_params* params, void* stream) {
    using fa::fail;
    fa::g_last_error.clear();
    if (params == nullptr) return fail(FA_EINVAL, "flash_fwd: params must not be NULL");
    const fa_params& p = *params;
    if (p.batch <= 0 || p.heads <= 0 || p.seqlen <= 0) {
        return fail(FA_EINVAL, "flash_fwd: batch, heads and seqlen must be positive");
    }
    if (p.head_dim != 64 && p.head_dim != 128) {
        return fail(FA_EINVAL,
                    "flash_fwd: head_dim must be 64 or 128, got " + std::to_string(p.head_dim));
    }
    if (p.variant > FA_VARIANT_FP16ACC) return fail(FA_EINVAL, "flash_fwd: unknown variant");
    if (p.causal > 1 || p.reserved[0] != 0 || p.reserved[1] != 0) {
        return fail(FA_EINVAL, "flash_fwd: causal must be 0 or 1 and reserved bytes zero");
    }
    if (p.q == nullptr || p.k == nullptr || p.v == nullptr || p.o == nullptr) {
        return fail(FA_EINVAL, "flash_fwd: q, k, v and o must be non-null");
    }
    if (!fa::aligned16(p.q) || !fa::aligned16(p.k) || !fa::aligned16(p.v) ||
        !fa::aligned16(p.o)) {
        return fail(FA_EINVAL, "flash_fwd: tensors must be 16-byte aligned (16-byte loads)");
    }
    if (!std::isfinite(p.softmax_scale)) {
        return fail(FA_EINVAL, "flash_fwd: softmax_scale must be finite");
    }
    // Offsets inside one head are 32-bit; the grid is one-dimensional.
    if (static_cast<int64_t>(p.seqlen) * p.head_dim > INT32_MAX) {
        return fail(FA_EINVAL, "flash_fwd: seqlen * head_dim must be below 2^31");
    }
    fa_tile_info t{};
    fa::tile_of(p.head_dim, p.variant, &t);
    const int64_t blocks = static_cast<int64_t>(p.batch) * p.heads *
                           ((static_cast<int64_t>(p.seqlen) + t.block_q - 1) / t.block_q);
    if (blocks > INT32_MAX) {
        return fail(FA_EINVAL, "flash_fwd: batch * heads * query blocks exceeds the grid limit");
    }

    // scale * log2(e), folded into one FMA per score. A negative scale is applied by negating Q
    // (exact in fp16) so the kernel's row max can use scale > 0; a zero scale becomes the
    // smallest normal float, which leaves every exp2 argument at exactly 0 after rounding but
    // keeps masked scores at -inf (0 * -inf would be NaN).
    float scale = p.softmax_scale;
    int negate_q = 0;
    if (scale < 0.0F) {
        scale = -scale;
        negate_q = 1;
    }
    float scale_log2 = scale * 1.44269504088896340736F;
    if (scale_log2 < 1.17549435e-38F) scale_log2 = 1.17549435e-38F;

    auto s = static_cast<hipStream_t>(stream);
    if (p.variant == FA_VARIANT_BASELINE) {
        return fa::dispatch<fa::BaseD64, fa::BaseD128>(p, s, scale_log2, negate_q);
    }
    return fa::dispatch<fa::OptD64, fa::OptD128>(p, s, scale_log2, negate_q);
}

}  // extern "C"
