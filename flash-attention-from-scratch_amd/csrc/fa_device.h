// gfx950 (CDNA4) device primitives of the FlashAttention-2 forward. Each wraps one
// instruction the kernel is built from; tests/blocks/fa_blocks.hip pins their lane layouts and
// numerics on the GPU.
//
// Counterparts of the reference's Ampere primitives (csrc/common.cuh), not translations:
//   cp.async 16 B (common.cuh:57-68)        -> lds_dma16: global_load_lds_dwordx4
//   ldmatrix_x4 (common.cuh:73-79)          -> plain ds_read_b128 of a swizzled row chunk
//   ldmatrix_x4_trans (common.cuh:80-84)    -> lds_read_tr16: ds_read_b64_tr_b16
//   mma_16816 f32 acc (common.cuh:91-98)    -> mfma32: v_mfma_f32_32x32x16_f16
//   __shfl_xor row reductions (flash_fwd.cu:359-363, 535-537)
//                                           -> max_xor32 / sum_xor32: v_permlane32_swap,
//                                              max_xor16 / sum_xor16: v_permlane16_swap
//   exp2f / ex2.approx (common.cuh:124-128) -> exp2_fast: v_exp_f32
//   pack_half2 RN (common.cuh:113-117)      -> pack8: v_cvt_pk_f16_f32 (round to nearest even)
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace fa::dev {

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __fp16 fp16x4_t __attribute__((__vector_size__(4 * sizeof(__fp16))));

#define FA_LDS __attribute__((address_space(3)))

// D(32x32, fp32) += A(32x16, fp16) * B(16x32, fp16); 32 cycles per wave on one SIMD.
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// D(16x16, fp32) += A(16x32, fp16) * B(32x16, fp16).
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Transposing LDS read: see fa::geom::tr16_row / tr16_col for the addressing.
__device__ __forceinline__ f16x4 lds_read_tr16(const char* lds_generic) {
    const fp16x4_t FA_LDS* p = (const fp16x4_t FA_LDS*)(lds_generic);
    return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                                         const_cast<fp16x4_t FA_LDS*>(p)));
}

// 16-byte global -> LDS copy that bypasses VGPRs. Lane i of the wave writes its 16 bytes to
// lds_wave_base + 16*i; lds_wave_base must be wave-uniform. Completion is tracked by vmcnt.
__device__ __forceinline__ void lds_dma16(const void* global_src, char* lds_wave_base) {
    __builtin_amdgcn_global_load_lds(global_src, (void FA_LDS*)(lds_wave_base), 16, 0, 0);
}

// Buffer resource for raw (stride 0) buffer loads of `bytes` bytes from `base`; the hardware
// range check returns zeros for any access at or past `bytes` (4th descriptor dword of gfx9
// parts: 0x00020000, 32-bit data format).
// `bytes` is the 32-bit num_records field, unsigned: a range of up to 2^32 - 1 bytes.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, unsigned bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0,
                                             __builtin_bit_cast(int, bytes), 0x00020000);
}

// 16-byte buffer -> LDS copy (buffer_load_dwordx4 ... lds): lane i reads rsrc + voffset and
// writes lds_wave_base + 16*i (lds_wave_base wave-uniform). Out-of-range lanes write zeros.
__device__ __forceinline__ void lds_dma16_buf(__amdgpu_buffer_rsrc_t rsrc, int voffset,
                                              char* lds_wave_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (void FA_LDS*)(lds_wave_base), 16, voffset, 0,
                                             0, 0);
}

// Wait until every global load of this wave (including LDS DMA) has landed.
__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Combine a per-lane value with the one held by lane ^ 32 (the other half of the wave). The
// swap yields the pair {x[l], x[l^32]} in every lane, so max and sum need no lane select.
__device__ __forceinline__ float max_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The same with lane ^ 16 (v_permlane16_swap: the neighbouring 16-lane row).
__device__ __forceinline__ float max_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Eight fp32 values -> eight fp16 (RNE), as one MFMA operand.
__device__ __forceinline__ f16x8 pack8(float a0, float a1, float a2, float a3, float a4,
                                       float a5, float a6, float a7) {
    const f16x2 p0 = __builtin_convertvector(f32x2{a0, a1}, f16x2);
    const f16x2 p1 = __builtin_convertvector(f32x2{a2, a3}, f16x2);
    const f16x2 p2 = __builtin_convertvector(f32x2{a4, a5}, f16x2);
    const f16x2 p3 = __builtin_convertvector(f32x2{a6, a7}, f16x2);
    return f16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// 16-byte output stores from two lanes that hold halves of the same row. v_permlane16_swap
// swaps the odd 16-lane rows of its first operand with the even rows of its second (lanes l and
// l ^ 16); v_permlane32_swap swaps lanes 32..63 of the first operand with lanes 0..31 of the
// second (l and l ^ 32). Lane l of the lower row of a pair thus receives {a[l], a[partner]} and
// lane l of the upper row {b[partner], b[l]}: if the lower lane holds 4 consecutive values a
// and the partner the 4 that follow them, and likewise for b one block further, each lane ends
// with 8 consecutive values of one block (a for the lower lane, b for the upper one).
__device__ __forceinline__ f16x8 pair_swap16(f16x4 a, f16x4 b) {
    const auto ua = __builtin_bit_cast(uint2, a);
    const auto ub = __builtin_bit_cast(uint2, b);
    const auto r0 = __builtin_amdgcn_permlane16_swap(ua.x, ub.x, false, false);
    const auto r1 = __builtin_amdgcn_permlane16_swap(ua.y, ub.y, false, false);
    return __builtin_bit_cast(f16x8, uint4{r0[0], r1[0], r0[1], r1[1]});
}
__device__ __forceinline__ f16x8 pair_swap32(f16x4 a, f16x4 b) {
    const auto ua = __builtin_bit_cast(uint2, a);
    const auto ub = __builtin_bit_cast(uint2, b);
    const auto r0 = __builtin_amdgcn_permlane32_swap(ua.x, ub.x, false, false);
    const auto r1 = __builtin_amdgcn_permlane32_swap(ua.y, ub.y, false, false);
    return __builtin_bit_cast(f16x8, uint4{r0[0], r1[0], r0[1], r1[1]});
}

__device__ __forceinline__ f16x4 pack4(float a0, float a1, float a2, float a3) {
    const f16x2 p0 = __builtin_convertvector(f32x2{a0, a1}, f16x2);
    const f16x2 p1 = __builtin_convertvector(f32x2{a2, a3}, f16x2);
    return f16x4{p0[0], p0[1], p1[0], p1[1]};
}

// Sum of the eight fp16 values of a packed MFMA operand, accumulated in fp32 onto acc
// (four v_dot2_f32_f16 against (1, 1)).
__device__ __forceinline__ float sum8_f16(f16x8 p, float acc) {
    const f16x2 one = {static_cast<f16>(1.0F), static_cast<f16>(1.0F)};
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 0, 1), one, acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 2, 3), one, acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 4, 5), one, acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(p, p, 6, 7), one, acc, false);
    return acc;
}

__device__ __forceinline__ bool wave_any(bool pred) {
    return __builtin_amdgcn_ballot_w64(pred) != 0;
}

__device__ __forceinline__ int wave_uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// x with the sign bits of its eight halves XORed with `sign` (0x80008000 negates every half,
// exactly; 0 leaves x as it is): one v_xor per register, without a branch.
__device__ __forceinline__ f16x8 xor_sign8(f16x8 x, unsigned sign) {
    uint4 u = __builtin_bit_cast(uint4, x);
    u.x ^= sign;
    u.y ^= sign;
    u.z ^= sign;
    u.w ^= sign;
    return __builtin_bit_cast(f16x8, u);
}

}  // namespace fa::dev
