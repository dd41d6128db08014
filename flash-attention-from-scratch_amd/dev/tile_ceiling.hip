// Synthetic ceiling of the d = 64 simple tile on MI355X: the per-tile work of flash_fwd_kernel
// (32x32x16 MFMAs) and flash_fwd_simple16 (16x16x32 MFMAs) with nothing else around it.
//
//     dev/tile_ceiling [iters]          (built by fa_build.py --only dev)
//
// One "tile" per loop iteration and wave, as in the kernels at d = 64 with 64-key tiles and 32
// query rows per wave: a barrier; S = K Q^T (K fragments read from LDS, Q in registers); the
// optimistic softmax (p = exp2(s * c - m), packed to fp16, row sums by v_dot2); O += V^T P^T.
// Variants add the transposed V fragment reads from LDS (+V) and the overflow vote with its
// exact branch (+check, never taken here), and take away the softmax (MFMA only: p = fp16(s)) or
// the MFMAs (VALU only: s from the K fragments). Two more rows start the QK^T MFMAs from a block
// of -m (their C operand) so that the exponential needs no FMA in front of it (FULL_CMAX), with
// and without the V reads and the vote. The grid is 512 workgroups of 8 waves, two per
// CU and four waves per SIMD, as the d = 64 simple tile runs. Operands are pseudo-random fp16
// values in [-2, 2]: the chip runs at its power limit and the clock depends on the switching
// activity of the data (structured small values run faster). Not included: the K/V DMA refills,
// the per-item prologue and O stores, causal masks. Prints TFLOPS by the 4 B H N^2 d count of the
// tile's two products (16 32x32x16 MFMA equivalents per wave and tile).
// Every LDS access stays inside the two 16 KiB arrays; the only global access is one store per
// thread into `out`.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __fp16 h4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
#define TC_LDS __attribute__((address_space(3)))

// FULL_CMAX: as FULL, but the QK^T MFMAs start from a register block that holds -m in every
// element (C operand) instead of zero, so that they return s * c - m directly (Q taken as already
// scaled by c) and the exponential needs no FMA in front of it.
enum Mode { FULL = 0, MFMA_ONLY = 1, VALU_ONLY = 2, FULL_CMAX = 3 };

__device__ __forceinline__ f16x8 pack8(const float* e) {
    f16x8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = static_cast<_Float16>(e[i]);
    return r;
}

__device__ __forceinline__ float sum8(f16x8 p, float s) {
    const f16x2 one = {static_cast<_Float16>(1.0F), static_cast<_Float16>(1.0F)};
    s = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 0, 1), one, s, false);
    s = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 2, 3), one, s, false);
    s = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 4, 5), one, s, false);
    s = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 6, 7), one, s, false);
    return s;
}

// Two transposed 4x16 reads 1024 halves apart, as a V^T operand.
__device__ __forceinline__ f16x8 vread(const _Float16* base) {
    const h4 TC_LDS* p0 = (const h4 TC_LDS*)(base);
    const h4 TC_LDS* p1 = (const h4 TC_LDS*)(base + 1024);
    const f16x4 lo = __builtin_bit_cast(
        f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(const_cast<h4 TC_LDS*>(p0)));
    const f16x4 up = __builtin_bit_cast(
        f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(const_cast<h4 TC_LDS*>(p1)));
    return f16x8{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
}

// Pseudo-random value in [-2, 2) with a full fp16 mantissa (an integer hash of x).
__device__ __forceinline__ float prand(unsigned x) {
    x ^= x >> 16;
    x *= 0x7feb352dU;
    x ^= x >> 15;
    x *= 0x846ca68bU;
    x ^= x >> 16;
    return (static_cast<float>(x & 0xFFFFFFU) / 16777216.0F - 0.5F) * 4.0F;
}

__device__ __forceinline__ f32x16 m32(f16x8 a, f16x8 b, f32x16 c, int mode) {
    return mode == VALU_ONLY ? c : __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 m16(f16x8 a, f16x8 b, f32x4 c, int mode) {
    return mode == VALU_ONLY ? c : __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float expo(float s, float c, float m, int mode) {
    return mode == MFMA_ONLY   ? s
           : mode == FULL_CMAX ? __builtin_amdgcn_exp2f(s)
                               : __builtin_amdgcn_exp2f(__builtin_fmaf(s, c, -m));
}

template <int SHAPE, bool V, bool CHK, int MODE>
__global__ __launch_bounds__(512) void tile_loop(float* out, int iters, float c) {
    const int lane = threadIdx.x & 63;
    __shared__ __attribute__((aligned(16))) _Float16 kl[8192];
    __shared__ __attribute__((aligned(16))) _Float16 vl[8192];
    for (int i = threadIdx.x; i < 8192; i += blockDim.x) {
        kl[i] = static_cast<_Float16>(prand(2 * i + 1));
        vl[i] = static_cast<_Float16>(prand(2 * i + 2));
    }
    __syncthreads();
    f16x8 a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            a[i][j] = static_cast<_Float16>(prand(100000 + threadIdx.x * 64 + i * 8 + j));
            b[i][j] = static_cast<_Float16>(prand(900000 + threadIdx.x * 64 + i * 8 + j));
        }
    float m = 0.0F, l = 0.0F;
    // K offsets: (it & 1) * 4096 + lane * 8 + 7 * 512 + 7 < 8192; V offsets (tile half, lane
    // part < 256, block part < 800, second read + 1024, 4 halves) < 8192.
    const int voff = (lane & 15) * 4 + (lane >> 4) * 64;
    float t = 0.0F;
    if constexpr (SHAPE == 32) {
        f32x16 o[2] = {};
        f32x16 mblk;
#pragma unroll
        for (int r = 0; r < 16; ++r) mblk[r] = -m;
        for (int it = 0; it < iters; ++it) {
            __syncthreads();
            const _Float16* kb0 = kl + (it & 1) * 4096 + lane * 8;
            f32x16 s[2];
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                s[nb] = MODE == FULL_CMAX ? mblk : f32x16{};
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    const f16x8 kf = *reinterpret_cast<const f16x8*>(kb0 + (nb * 4 + kk) * 512);
                    s[nb] = m32(kf, b[kk], s[nb], MODE);
                    if (MODE == VALU_ONLY) s[nb][kk] += static_cast<float>(kf[kk]);
                }
            }
            f16x8 p[2][2];
            float sum0 = 0.0F, sum1 = 0.0F;
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    float e[8];
#pragma unroll
                    for (int r = 0; r < 8; ++r) e[r] = expo(s[nb][8 * h + r], c, m, MODE);
                    p[nb][h] = pack8(e);
                    if (MODE != MFMA_ONLY) {
                        if (h == 0) sum0 = sum8(p[nb][h], sum0);
                        else sum1 = sum8(p[nb][h], sum1);
                    }
                }
            if constexpr (CHK) {
                if (__builtin_amdgcn_ballot_w64(!(sum0 + sum1 < INFINITY)) != 0) {
                    float mx = -INFINITY;
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[nb][r]);
                    m = mx * c;
#pragma unroll
                    for (int r = 0; r < 16; ++r) mblk[r] = -m;
#pragma unroll
                    for (int db = 0; db < 2; ++db) o[db] *= 0.5F;
                }
            }
            l += sum0 + sum1;
            const _Float16* vb0 = vl + (it & 1) * 4096 + voff;
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int db = 0; db < 2; ++db) {
                        const f16x8 vf = V ? vread(vb0 + (nb * 2 + h) * 256 + db * 16)
                                           : a[(nb + h + db) & 3];
                        o[db] = m32(vf, p[nb][h], o[db], MODE);
                        if (MODE == VALU_ONLY) o[db][h] += static_cast<float>(p[nb][h][db]);
                    }
            if (MODE != FULL_CMAX) m = m + 1e-7F;
        }
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) t += o[db][r];
    } else {
        f32x4 o[4][2] = {};
        f32x4 mblk = {-m, -m, -m, -m};
        for (int it = 0; it < iters; ++it) {
            __syncthreads();
            const _Float16* kb0 = kl + (it & 1) * 4096 + lane * 8;
            f32x4 s[4][2];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                f16x8 kf[2];
#pragma unroll
                for (int dc = 0; dc < 2; ++dc)
                    kf[dc] = *reinterpret_cast<const f16x8*>(kb0 + (kb * 2 + dc) * 512);
#pragma unroll
                for (int qb = 0; qb < 2; ++qb) {
                    s[kb][qb] = MODE == FULL_CMAX ? mblk : f32x4{};
#pragma unroll
                    for (int dc = 0; dc < 2; ++dc) {
                        s[kb][qb] = m16(kf[dc], b[(qb * 2 + dc) & 3], s[kb][qb], MODE);
                        if (MODE == VALU_ONLY) s[kb][qb][dc] += static_cast<float>(kf[dc][qb]);
                    }
                }
            }
            f16x8 p[2][2];
            float sum[2] = {0.0F, 0.0F};
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    float e[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        e[i] = expo(s[2 * tt + (i >> 2)][qb][i & 3], c, m, MODE);
                    p[qb][tt] = pack8(e);
                    if (MODE != MFMA_ONLY) sum[qb] = sum8(p[qb][tt], sum[qb]);
                }
            if constexpr (CHK) {
                if (__builtin_amdgcn_ballot_w64(!(sum[0] < INFINITY && sum[1] < INFINITY)) != 0) {
                    float mx = -INFINITY;
#pragma unroll
                    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
                            for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[kb][qb][r]);
                    m = mx * c;
                    mblk = f32x4{-m, -m, -m, -m};
#pragma unroll
                    for (int db = 0; db < 4; ++db)
#pragma unroll
                        for (int qb = 0; qb < 2; ++qb) o[db][qb] *= 0.5F;
                }
            }
            l += sum[0] + sum[1];
            const _Float16* vb0 = vl + (it & 1) * 4096 + voff;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                f16x8 vf[4];
#pragma unroll
                for (int db = 0; db < 4; ++db)
                    vf[db] = V ? vread(vb0 + tt * 512 + db * 16) : a[(tt + db) & 3];
#pragma unroll
                for (int db = 0; db < 4; ++db)
#pragma unroll
                    for (int qb = 0; qb < 2; ++qb) {
                        o[db][qb] = m16(vf[db], p[qb][tt], o[db][qb], MODE);
                        if (MODE == VALU_ONLY) o[db][qb][tt] += static_cast<float>(p[qb][tt][db]);
                    }
            }
            if (MODE != FULL_CMAX) m = m + 1e-7F;
        }
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
#pragma unroll
                for (int r = 0; r < 4; ++r) t += o[db][qb][r];
    }
    out[blockIdx.x * blockDim.x + threadIdx.x] = t + l;
}

constexpr int kWgs = 512;      // two 8-wave workgroups per CU on 256 CUs
constexpr int kThreads = 512;

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
        std::exit(2);
    }
}

template <int SHAPE, bool V, bool CHK, int MODE>
float time_ms(float* out, int iters) {
    hipEvent_t e0, e1;
    check(hipEventCreate(&e0), "hipEventCreate");
    check(hipEventCreate(&e1), "hipEventCreate");
    for (int w = 0; w < 3; ++w) tile_loop<SHAPE, V, CHK, MODE><<<kWgs, kThreads>>>(out, iters, 0.125F);
    check(hipEventRecord(e0), "hipEventRecord");
    constexpr int reps = 5;
    for (int r = 0; r < reps; ++r) tile_loop<SHAPE, V, CHK, MODE><<<kWgs, kThreads>>>(out, iters, 0.125F);
    check(hipEventRecord(e1), "hipEventRecord");
    check(hipEventSynchronize(e1), "hipEventSynchronize");
    float ms = 0.0F;
    check(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
    check(hipEventDestroy(e0), "hipEventDestroy");
    check(hipEventDestroy(e1), "hipEventDestroy");
    return ms / reps;
}

}  // namespace

int main(int argc, char** argv) {
    const int iters = argc > 1 ? std::atoi(argv[1]) : 4000;
    if (iters <= 0 || iters > 1000000) {
        std::fprintf(stderr, "usage: tile_ceiling [iters in 1..1000000]\n");
        return 1;
    }
    float* out = nullptr;
    check(hipMalloc(&out, sizeof(float) * kWgs * kThreads), "hipMalloc");
    const double flops = 2.0 * 16 * 32 * 32 * 16 * static_cast<double>(iters) * kWgs * (kThreads / 64);
    auto row = [&](const char* name, float t32, float t16) {
        std::printf("%-26s 32x32x16 %7.3f ms %6.0f TFLOPS   16x16x32 %7.3f ms %6.0f TFLOPS\n", name,
                    t32, flops / t32 / 1e9, t16, flops / t16 / 1e9);
    };
    std::printf("d=64 tile, 512 workgroups x 8 waves, %d tiles per wave\n", iters);
    row("MFMA only", time_ms<32, false, false, MFMA_ONLY>(out, iters),
        time_ms<16, false, false, MFMA_ONLY>(out, iters));
    row("VALU only", time_ms<32, false, false, VALU_ONLY>(out, iters),
        time_ms<16, false, false, VALU_ONLY>(out, iters));
    row("MFMA + softmax", time_ms<32, false, false, FULL>(out, iters),
        time_ms<16, false, false, FULL>(out, iters));
    row("+ V^T reads", time_ms<32, true, false, FULL>(out, iters),
        time_ms<16, true, false, FULL>(out, iters));
    row("+ overflow vote", time_ms<32, false, true, FULL>(out, iters),
        time_ms<16, false, true, FULL>(out, iters));
    row("+ V^T reads + vote", time_ms<32, true, true, FULL>(out, iters),
        time_ms<16, true, true, FULL>(out, iters));
    row("  same, -m in the C operand", time_ms<32, true, true, FULL_CMAX>(out, iters),
        time_ms<16, true, true, FULL_CMAX>(out, iters));
    row("MFMA + softmax, -m in C", time_ms<32, false, false, FULL_CMAX>(out, iters),
        time_ms<16, false, false, FULL_CMAX>(out, iters));
    check(hipFree(out), "hipFree");
    return 0;
}
