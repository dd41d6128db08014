// Measurement probes for MI355X (gfx950): how fast can a CU stream fp16 MFMAs when the power
// limit, not the schedule, sets the clock? Not part of the attention library; built into
// fa/libfa_probe.so by fa_build.py (target "probe") and run by `python -m fa.probe`.
//
// probe_kernel<VALU, LDS>: 8 waves per workgroup (two per SIMD), one workgroup per CU slot,
// each wave streaming v_mfma_f32_32x32x16_f16 (SHAPE 0) or v_mfma_f32_16x16x32_f16 (SHAPE 1,
// twice as many of half the FLOPs) on operands drawn from random fp16 data (the data activity
// of attention, which sets the power draw). Per 16 MFMAs a wave optionally adds
//   VALU: the VALU work of one softmax tile (16 v_exp_f32, 16 fma, adds), and
//   LDS:  the fragment reads of one K/V tile (8 ds_read_b128 + 16 ds_read_b64_tr_b16, with the
//         conflict-free access pattern of the attention kernel) feeding the MFMA operands.
// Each workgroup records shader cycles (s_memtime) and 100 MHz real time (s_memrealtime), so
// the effective clock is measured, not assumed.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "fa_device.h"
#include "fa_geometry.h"

namespace {

using namespace fa::dev;
typedef unsigned uint4_t __attribute__((ext_vector_type(4)));
typedef unsigned uint2_t __attribute__((ext_vector_type(2)));

template <int VALU, int LDS, int SHAPE = 0>
__global__ __launch_bounds__(512) void probe_kernel(const f16x8* __restrict__ src, float* out,
                                                    unsigned long long* clk, int iters) {
    __shared__ __attribute__((aligned(1024))) char lds[32768];
    const int t = threadIdx.x;
    for (int i = t; i < 32768 / 16; i += 512) reinterpret_cast<f16x8*>(lds)[i] = src[i & 4095];
    __syncthreads();
    f16x8 a[8], b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = src[(t * 16 + i) & 4095];
        b[i] = src[(t * 16 + 8 + i) & 4095];
    }
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    f32x4 h[8] = {};  // SHAPE 1: eight 16x16 accumulators
    float e[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) e[i] = (t & 63) * 1e-3F - i * 0.1F;
    const int lane = t & 63;
    // K-fragment and V^T-fragment offsets with the 64-bank swizzle of the attention kernel;
    // every address stays inside the 32 KiB array.
    const unsigned kbase = (lane & 31) * 256 + 16 * ((lane >> 5) ^ ((lane & 31) & 15));
    const unsigned vbase = 16384 + ((lane & 15) >> 2) * 256 + 8 * (lane & 3) + 64 * (lane >> 4);
    const unsigned long long s0 = __builtin_amdgcn_s_memtime();
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    float acc = 0.0F;
    for (int it = 0; it < iters; ++it) {
        if (LDS) {
            f32x4 r[8];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                r[k] = *reinterpret_cast<const f32x4*>(lds + ((kbase + k * 32 + (it & 1) * 8192) & 16383));
            f16x4 w[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) w[k] = lds_read_tr16(lds + ((vbase + k * 1024) & 32767));
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                a[k] = __builtin_bit_cast(f16x8, r[k]);
                b[k] = f16x8{w[2 * k][0], w[2 * k][1], w[2 * k][2], w[2 * k][3],
                             w[2 * k + 1][0], w[2 * k + 1][1], w[2 * k + 1][2], w[2 * k + 1][3]};
            }
        }
        if (SHAPE == 0) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                c0 = mfma32(a[m], b[m], c0);
                c1 = mfma32(a[m + 4], b[m + 1], c1);
                c2 = mfma32(a[(m + 2) & 7], b[m + 2], c2);
                c3 = mfma32(a[(m + 5) & 7], b[m + 3], c3);
            }
        } else {
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int j = 0; j < 8; ++j) h[j] = mfma16(a[(m + j) & 7], b[(m * 3 + j) & 7], h[j]);
        }
        if (VALU) {
            float sum = 0.0F;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float ci = SHAPE == 0 ? c0[i] : h[i >> 2][i & 3];
                const float x = exp2_fast(fmaf(ci, 0.125F, -e[i]));
                e[i] = x * 0.5F;
                sum += x;
            }
            acc += sum;
        }
        if (!LDS) asm volatile("" : "+v"(a[0]), "+v"(b[0]), "+v"(a[1]), "+v"(b[1]));
    }
    const unsigned long long s1 = __builtin_amdgcn_s_memtime();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    float hs = 0.0F;
#pragma unroll
    for (int j = 0; j < 8; ++j) hs += h[j][j & 3];
    out[blockIdx.x * 512 + t] = c0[0] + c1[1] + c2[2] + c3[3] + hs + acc;
    if (t == 0) {
        clk[blockIdx.x * 2] = s1 - s0;
        clk[blockIdx.x * 2 + 1] = r1 - r0;
    }
}

// LDS read throughput alone: every wave of a 512-thread workgroup issues `iters` rounds of
// 8 independent reads at distinct addresses (the 16x16x32 patterns vary by an XOR of whole
// 16-byte chunks, which keeps each lane in its row and the pattern's bank structure)
// (MODE 0: ds_read_b128 with the K-fragment pattern, MODE 1:
// ds_read_b64_tr_b16 with the V^T pattern; MODE 2 / 3: the same for the 16x16x32 layout;
// MODE 4: its V^T rows without the swizzle), folding the results with one xor per read so
// that nothing waits on a read before the next one issues. The addresses move every round
// (the LDS contents never change, so repeated addresses would let the compiler fold reads).
template <int MODE>
__global__ __launch_bounds__(512) void probe_lds_kernel(float* out, unsigned long long* clk,
                                                        int iters) {
    __shared__ __attribute__((aligned(1024))) char lds[32768];
    const int t = threadIdx.x;
    for (int i = t; i < 32768 / 4; i += 512) reinterpret_cast<unsigned*>(lds)[i] = i * 2654435761U;
    __syncthreads();
    const int lane = t & 63;
    const unsigned kbase = (lane & 31) * 256 + 16 * ((lane >> 5) ^ ((lane & 31) & 15));
    const unsigned vbase = ((lane & 15) >> 2) * 256 + 8 * (lane & 3) + 64 * (lane >> 4);
    // 16x16x32 patterns with contiguous 16-row key blocks and row xor 2*(row%8) + (row/8)%2:
    // MODE 2 K (16 rows x one chunk per 16 lanes), MODE 3 V^T (rows 4*(lane/16) + 0..3, 32 bytes
    // per row), MODE 4 the same V^T rows unswizzled.
    auto xa = [](int row) { return ((row & 7) << 1) | ((row >> 3) & 1); };
    const unsigned k16base = (lane & 15) * 256 + 16 * ((lane >> 4) ^ xa(lane & 15));
    const int v16row = 4 * (lane >> 4) + ((lane & 15) >> 2);
    const unsigned v16base = v16row * 256 + 16 * (((lane & 3) >> 1) ^ xa(v16row)) + 8 * (lane & 1);
    const unsigned v16plain = v16row * 256 + 8 * (lane & 3);
    // MODE 5 / 6: the layout the 16x16x32 kernel uses (fa::geom::m16_key / tile_offset_m16:
    // key blocks split over both 4 KiB halves of the tile).
    const unsigned k5base =
        fa::geom::tile_offset_m16(fa::geom::m16_key(0, lane & 15), lane >> 4, 128);
    const int v6row = fa::geom::pv16_key(lane, 0, 0) + fa::geom::tr16_row(lane);
    const unsigned v6base = fa::geom::tile_offset_m16(v6row, fa::geom::tr16_col(lane) >> 3, 128) +
                            2 * (fa::geom::tr16_col(lane) & 7);
    unsigned acc = 0;
    const unsigned long long s0 = __builtin_amdgcn_s_memtime();
    const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
        // New addresses every round (repeated ones would let the compiler fold reads): whole
        // 8 KiB steps, which keep every pattern's alignment to 32 rows, made opaque to the
        // compiler so that it cannot see they repeat every four rounds.
        unsigned shift = (static_cast<unsigned>(it) * 8192U) & 32767U;
        asm volatile("" : "+v"(shift));
        if (MODE == 0 || MODE == 2 || MODE == 5) {
            f32x4 r[8];
#pragma unroll
            for (int k = 0; k < 8; ++k)
                r[k] = *reinterpret_cast<const f32x4*>(
                    lds + ((MODE == 0 ? kbase + k * 32
                                      : ((MODE == 2 ? k16base : k5base) ^ (16U * k)) +
                                            8192U * (k & 3)) +
                               shift &
                           32752));
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const auto u = __builtin_bit_cast(uint4_t, r[k]);
                acc ^= u[0] ^ u[1] ^ u[2] ^ u[3];
            }
        } else {
            f16x4 w[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const unsigned a =
                    MODE == 1 ? vbase + k * 1024
                              : ((MODE == 6 ? v6base : (MODE == 3 ? v16base : v16plain)) ^
                                 (16U * k)) + 8192U * (k & 3);
                w[k] = lds_read_tr16(lds + ((a + shift) & 32760));
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const auto u = __builtin_bit_cast(uint2_t, w[k]);
                acc ^= u[0] ^ u[1];
            }
        }
    }
    const unsigned long long s1 = __builtin_amdgcn_s_memtime();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    out[blockIdx.x * 512 + t] = static_cast<float>(acc);
    if (t == 0) {
        clk[blockIdx.x * 2] = s1 - s0;
        clk[blockIdx.x * 2 + 1] = r1 - r0;
    }
}

}  // namespace

extern "C" {

// LDS read probe: mode 0 = ds_read_b128, 1 = ds_read_b64_tr_b16 (the 32x32x16 layout's K and
// V^T patterns), 2 / 3 = the same for the 16x16x32 layout, 4 = its V^T rows unswizzled; `blocks` workgroups of 8
// waves, `iters` rounds of 8 reads per wave. *cycles: mean shader cycles per workgroup.
int fa_probe_lds(int mode, int blocks, int iters, float* ms, double* ghz, double* cycles) {
    if (blocks <= 0 || blocks > 65536 || iters <= 0 || mode < 0 || mode > 6) {
        return static_cast<int>(hipErrorInvalidValue);
    }
    float* d = nullptr;
    unsigned long long* c = nullptr;
    hipError_t err = hipMalloc(&d, static_cast<size_t>(blocks) * 512 * sizeof(float));
    if (err == hipSuccess) err = hipMalloc(&c, static_cast<size_t>(blocks) * 2 * sizeof(unsigned long long));
    if (err != hipSuccess) return static_cast<int>(err);
    auto launch = [&](int it) {
        switch (mode) {
            case 0: hipLaunchKernelGGL((probe_lds_kernel<0>), dim3(blocks), dim3(512), 0, 0, d, c, it); break;
            case 1: hipLaunchKernelGGL((probe_lds_kernel<1>), dim3(blocks), dim3(512), 0, 0, d, c, it); break;
            case 2: hipLaunchKernelGGL((probe_lds_kernel<2>), dim3(blocks), dim3(512), 0, 0, d, c, it); break;
            case 3: hipLaunchKernelGGL((probe_lds_kernel<3>), dim3(blocks), dim3(512), 0, 0, d, c, it); break;
            case 4: hipLaunchKernelGGL((probe_lds_kernel<4>), dim3(blocks), dim3(512), 0, 0, d, c, it); break;
            case 5: hipLaunchKernelGGL((probe_lds_kernel<5>), dim3(blocks), dim3(512), 0, 0, d, c, it); break;
            default: hipLaunchKernelGGL((probe_lds_kernel<6>), dim3(blocks), dim3(512), 0, 0, d, c, it); break;
        }
    };
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    launch(iters);
    (void)hipEventRecord(e0, nullptr);
    launch(iters);
    (void)hipEventRecord(e1, nullptr);
    err = hipEventSynchronize(e1);
    (void)hipEventElapsedTime(ms, e0, e1);
    unsigned long long* hc = new unsigned long long[2 * static_cast<size_t>(blocks)];
    (void)hipMemcpy(hc, c, static_cast<size_t>(blocks) * 2 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
    double sg = 0.0;
    double sc = 0.0;
    for (int i = 0; i < blocks; ++i) {
        sg += static_cast<double>(hc[2 * i]) / (static_cast<double>(hc[2 * i + 1]) * 10.0);
        sc += static_cast<double>(hc[2 * i]);
    }
    *ghz = sg / blocks;
    *cycles = sc / blocks;
    delete[] hc;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    (void)hipFree(d);
    (void)hipFree(c);
    return err == hipSuccess ? static_cast<int>(hipGetLastError()) : static_cast<int>(err);
}


// Runs the probe: `blocks` workgroups of 8 waves, `iters` iterations of 16 MFMAs per wave
// (shape 0: v_mfma_f32_32x32x16_f16) or of 32 MFMAs of half the FLOPs (shape 1:
// v_mfma_f32_16x16x32_f16, eight independent chains), the same FLOPs per iteration.
// Returns the HIP status; *ms is the kernel time, *ghz the mean measured clock, *cycles the mean
// shader cycles per workgroup.
int fa_probe_ceiling(int valu, int lds, int shape, int blocks, int iters, float* ms, double* ghz,
                     double* cycles) {
    if (blocks <= 0 || blocks > 65536 || iters <= 0 || shape < 0 || shape > 1) {
        return static_cast<int>(hipErrorInvalidValue);
    }
    f16x8* src = nullptr;
    float* d = nullptr;
    unsigned long long* c = nullptr;
    hipError_t err = hipMalloc(&src, 4096 * sizeof(f16x8));
    if (err == hipSuccess) err = hipMalloc(&d, static_cast<size_t>(blocks) * 512 * sizeof(float));
    if (err == hipSuccess) err = hipMalloc(&c, static_cast<size_t>(blocks) * 2 * sizeof(unsigned long long));
    if (err != hipSuccess) return static_cast<int>(err);
    // Random fp16 in [-2, 2) from a 32-bit LCG.
    static f16x8 host[4096];
    uint32_t x = 12345U;
    for (auto& h : host)
        for (int j = 0; j < 8; ++j) {
            x = x * 1103515245U + 12345U;
            h[j] = static_cast<f16>(static_cast<float>((x >> 8) & 0xffffU) / 16384.0F - 2.0F);
        }
    (void)hipMemcpy(src, host, sizeof(host), hipMemcpyHostToDevice);
    auto launch = [&](int it) {
        if (shape == 1) {
            if (valu && lds) hipLaunchKernelGGL((probe_kernel<1, 1, 1>), dim3(blocks), dim3(512), 0, 0, src, d, c, it);
            else if (valu) hipLaunchKernelGGL((probe_kernel<1, 0, 1>), dim3(blocks), dim3(512), 0, 0, src, d, c, it);
            else if (lds) hipLaunchKernelGGL((probe_kernel<0, 1, 1>), dim3(blocks), dim3(512), 0, 0, src, d, c, it);
            else hipLaunchKernelGGL((probe_kernel<0, 0, 1>), dim3(blocks), dim3(512), 0, 0, src, d, c, it);
        } else {
            if (valu && lds) hipLaunchKernelGGL((probe_kernel<1, 1>), dim3(blocks), dim3(512), 0, 0, src, d, c, it);
            else if (valu) hipLaunchKernelGGL((probe_kernel<1, 0>), dim3(blocks), dim3(512), 0, 0, src, d, c, it);
            else if (lds) hipLaunchKernelGGL((probe_kernel<0, 1>), dim3(blocks), dim3(512), 0, 0, src, d, c, it);
            else hipLaunchKernelGGL((probe_kernel<0, 0>), dim3(blocks), dim3(512), 0, 0, src, d, c, it);
        }
    };
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    launch(200);
    launch(iters);  // ramp the clock before the timed launch
    (void)hipEventRecord(e0, nullptr);
    launch(iters);
    (void)hipEventRecord(e1, nullptr);
    err = hipEventSynchronize(e1);
    (void)hipEventElapsedTime(ms, e0, e1);
    unsigned long long* hc = new unsigned long long[2 * static_cast<size_t>(blocks)];
    (void)hipMemcpy(hc, c, static_cast<size_t>(blocks) * 2 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
    double sg = 0.0;
    double sc = 0.0;
    for (int i = 0; i < blocks; ++i) {
        sg += static_cast<double>(hc[2 * i]) / (static_cast<double>(hc[2 * i + 1]) * 10.0);
        sc += static_cast<double>(hc[2 * i]);
    }
    *ghz = sg / blocks;
    *cycles = sc / blocks;
    delete[] hc;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    (void)hipFree(src);
    (void)hipFree(d);
    (void)hipFree(c);
    return err == hipSuccess ? static_cast<int>(hipGetLastError()) : static_cast<int>(err);
}

}  // extern "C"
