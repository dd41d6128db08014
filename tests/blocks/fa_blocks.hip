// Building-block kernels for the GPU unit tests (tests/test_blocks.py): each runs one wave64
// over one instruction the FlashAttention kernel relies on, so a wrong lane layout shows up as
// a small, exact failure instead of a wrong attention output. Counterpart of the reference's
// tests/cpp/test_ptx.cu (mma fragment layout :93-167, ldmatrix :173-250, cp.async zero-fill
// :318-352, exp2 accuracy :357-424), re-targeted to the gfx950 instructions.
//
// Every entry point allocates its own device buffers, copies the host inputs in, runs one
// 64-thread workgroup, copies the result out and returns a hipError_t value (0 = success).
// All indices stay inside the buffers sized here.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>

#include "fa_device.h"
#include "fa_geometry.h"

using namespace fa::dev;

namespace {

typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

// Whole-vector bit casts only: a bit cast of a single vector element (an lvalue) miscompiles
// with this clang (it reads element 0), so results are reinterpreted as a vector first.
__device__ inline u16x4 bits4(f16x4 v) { return __builtin_bit_cast(u16x4, v); }
__device__ inline u16x8 bits8(f16x8 v) { return __builtin_bit_cast(u16x8, v); }

// ds_read_b64_tr_b16: LDS holds 256 halves with value i at index i; lane l reads the 8 bytes
// at half index 4*l. out[4*l + e] = element e returned to lane l.
__global__ void k_tr16_probe(uint16_t* out) {
    __shared__ __attribute__((aligned(16))) f16 lds[256];
    const int l = threadIdx.x;
    for (int i = l; i < 256; i += 64) lds[i] = static_cast<f16>(i);
    __syncthreads();
    const u16x4 r = bits4(lds_read_tr16(reinterpret_cast<const char*>(lds + 4 * l)));
    for (int e = 0; e < 4; ++e) out[4 * l + e] = r[e];
}

// Transposed read as the kernel uses it: a [16 rows][64 cols] fp16 tile (row-major, no
// swizzle). Each 16-lane group j4 = lane/16 reads the 4-row block starting at row 4*j4 and
// columns [16*j4, 16*j4 + 16), addressed through fa::geom::tr16_row / tr16_col, so lane l
// should receive tile[4*j4 + e][16*j4 + l%16], e = 0..3. out[4*l + e].
__global__ void k_tr16_block(const uint16_t* tile, uint16_t* out) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[16 * 64];
    const int l = threadIdx.x;
    for (int i = l; i < 16 * 64; i += 64) lds[i] = tile[i];
    __syncthreads();
    const int grp = l >> 4;
    const int row = 4 * grp + fa::geom::tr16_row(l);
    const int colh = 16 * grp + fa::geom::tr16_col(l);
    const u16x4 r = bits4(lds_read_tr16(reinterpret_cast<const char*>(lds + row * 64 + colh)));
    for (int e = 0; e < 4; ++e) out[4 * l + e] = r[e];
}

// C(32x32) = A(32x16) B(16x32), fragments loaded in the layout of fa::geom (A, B row-major).
__global__ void k_mfma32(const uint16_t* a, const uint16_t* b, float* c) {
    const int l = threadIdx.x;
    f16x8 fa_, fb;
    for (int i = 0; i < 8; ++i) {
        fa_[i] = __builtin_bit_cast(f16, a[(l % 32) * 16 + 8 * (l / 32) + i]);
        fb[i] = __builtin_bit_cast(f16, b[(8 * (l / 32) + i) * 32 + (l % 32)]);
    }
    const f32x16 acc = mfma32(fa_, fb, f32x16{});
    for (int r = 0; r < 16; ++r) c[fa::geom::mfma32_c_row(l, r) * 32 + fa::geom::mfma32_c_col(l)] = acc[r];
}

// C(16x16) = A(16x32) B(32x16).
__global__ void k_mfma16(const uint16_t* a, const uint16_t* b, float* c) {
    const int l = threadIdx.x;
    f16x8 fa_, fb;
    for (int i = 0; i < 8; ++i) {
        fa_[i] = __builtin_bit_cast(f16, a[(l % 16) * 32 + 8 * (l / 16) + i]);
        fb[i] = __builtin_bit_cast(f16, b[(8 * (l / 16) + i) * 16 + (l % 16)]);
    }
    const f32x4 acc = mfma16(fa_, fb, f32x4{});
    for (int r = 0; r < 4; ++r) c[fa::geom::mfma16_c_row(l, r) * 16 + fa::geom::mfma16_c_col(l)] = acc[r];
}

__global__ void k_xor32(const float* in, float* out_max, float* out_sum) {
    const int l = threadIdx.x;
    out_max[l] = max_xor32(in[l]);
    out_sum[l] = sum_xor32(in[l]);
}

__global__ void k_xor16(const float* in, float* out_max, float* out_sum) {
    const int l = threadIdx.x;
    out_max[l] = max_xor16(in[l]);
    out_sum[l] = sum_xor16(in[l]);
}

// pair_swap16 / pair_swap32 (the 16-byte output stores): lane l passes a = in[8l .. 8l+3] and
// b = in[8l+4 .. 8l+7] (as fp16) and writes the 8 halves it gets back to out[8l .. 8l+7].
__global__ void k_pair_swap(const uint16_t* in, uint16_t* out, int dist) {
    const int l = threadIdx.x;
    const u16x8 x = *reinterpret_cast<const u16x8*>(in + 8 * l);
    const f16x4 a = __builtin_bit_cast(f16x4, u16x4{x[0], x[1], x[2], x[3]});
    const f16x4 b = __builtin_bit_cast(f16x4, u16x4{x[4], x[5], x[6], x[7]});
    const u16x8 r = bits8(dist == 16 ? pair_swap16(a, b) : pair_swap32(a, b));
    *reinterpret_cast<u16x8*>(out + 8 * l) = r;
}

__global__ void k_exp2(const float* x, float* y, int n) {
    for (int i = threadIdx.x; i < n; i += 64) y[i] = exp2_fast(x[i]);
}

// pack8 (v_cvt_pk_f16_f32): n must be a multiple of 8.
__global__ void k_pack8(const float* x, uint16_t* y, int n) {
    for (int i = 8 * threadIdx.x; i < n; i += 8 * 64) {
        const u16x8 p = bits8(pack8(x[i], x[i + 1], x[i + 2], x[i + 3], x[i + 4], x[i + 5],
                                    x[i + 6], x[i + 7]));
        for (int e = 0; e < 8; ++e) y[i + e] = p[e];
    }
}

// lds_dma16: lane l copies 16-byte chunk src_chunk[l] of a 64-chunk source to LDS slot l;
// out = the 1 KiB LDS image.
__global__ void k_lds_dma(const uint16_t* src, const int* src_chunk, uint16_t* out) {
    __shared__ __attribute__((aligned(1024))) char lds[1024];
    const int l = threadIdx.x;
    lds_dma16(src + 8 * src_chunk[l], lds);
    wait_vmem();
    __syncthreads();
    const uint16_t* lh = reinterpret_cast<const uint16_t*>(lds);
    for (int i = l; i < 512; i += 64) out[i] = lh[i];
}

// lds_dma16_buf: as k_lds_dma through a buffer resource covering the first `bytes` bytes of
// src; lanes whose chunk starts at or past `bytes` must write zeros. The LDS image is first
// filled with 0xFFFF (NaN) so that a skipped write would show.
__global__ void k_lds_dma_buf(const uint16_t* src, const int* src_chunk, int bytes,
                              uint16_t* out) {
    __shared__ __attribute__((aligned(1024))) uint16_t lds[512];
    const int l = threadIdx.x;
    for (int i = l; i < 512; i += 64) lds[i] = 0xFFFF;
    __syncthreads();
    const auto rsrc = make_rsrc(src, bytes);
    lds_dma16_buf(rsrc, 16 * src_chunk[l], reinterpret_cast<char*>(lds));
    wait_vmem();
    __syncthreads();
    for (int i = l; i < 512; i += 64) out[i] = lds[i];
}

// sum8_f16: fp32 sum of the eight fp16 values of each 8-element group of x.
__global__ void k_sum8(const uint16_t* x, float* y, int groups) {
    for (int gi = threadIdx.x; gi < groups; gi += 64) {
        f16x8 v;
        for (int e = 0; e < 8; ++e) v[e] = __builtin_bit_cast(f16, x[8 * gi + e]);
        y[gi] = sum8_f16(v, 0.0F);
    }
}

template <class T>
struct DevBuf {
    T* p = nullptr;
    hipError_t err = hipSuccess;
    explicit DevBuf(size_t count) { err = hipMalloc(&p, count * sizeof(T)); }
    ~DevBuf() {
        if (p != nullptr) (void)hipFree(p);
    }
};

#define FAB_TRY(expr)                       \
    do {                                    \
        const hipError_t e_ = (expr);       \
        if (e_ != hipSuccess) return e_;    \
    } while (0)

template <class T>
hipError_t to_dev(DevBuf<T>& d, const T* h, size_t count) {
    FAB_TRY(d.err);
    return hipMemcpy(d.p, h, count * sizeof(T), hipMemcpyHostToDevice);
}
template <class T>
hipError_t to_host(T* h, const DevBuf<T>& d, size_t count) {
    return hipMemcpy(h, d.p, count * sizeof(T), hipMemcpyDeviceToHost);
}

}  // namespace

extern "C" {

int fab_tr16_probe(uint16_t* out) {
    DevBuf<uint16_t> d(256);
    FAB_TRY(d.err);
    hipLaunchKernelGGL(k_tr16_probe, dim3(1), dim3(64), 0, 0, d.p);
    FAB_TRY(hipGetLastError());
    FAB_TRY(hipDeviceSynchronize());
    return to_host(out, d, 256);
}

int fab_tr16_block(const uint16_t* tile, uint16_t* out) {
    DevBuf<uint16_t> t(16 * 64), d(256);
    FAB_TRY(to_dev(t, tile, 16 * 64));
    FAB_TRY(d.err);
    hipLaunchKernelGGL(k_tr16_block, dim3(1), dim3(64), 0, 0, t.p, d.p);
    FAB_TRY(hipGetLastError());
    FAB_TRY(hipDeviceSynchronize());
    return to_host(out, d, 256);
}

int fab_mfma32(const uint16_t* a, const uint16_t* b, float* c) {
    DevBuf<uint16_t> da(32 * 16), db(16 * 32);
    DevBuf<float> dc(32 * 32);
    FAB_TRY(to_dev(da, a, 32 * 16));
    FAB_TRY(to_dev(db, b, 16 * 32));
    FAB_TRY(dc.err);
    hipLaunchKernelGGL(k_mfma32, dim3(1), dim3(64), 0, 0, da.p, db.p, dc.p);
    FAB_TRY(hipGetLastError());
    FAB_TRY(hipDeviceSynchronize());
    return to_host(c, dc, 32 * 32);
}

int fab_mfma16(const uint16_t* a, const uint16_t* b, float* c) {
    DevBuf<uint16_t> da(16 * 32), db(32 * 16);
    DevBuf<float> dc(16 * 16);
    FAB_TRY(to_dev(da, a, 16 * 32));
    FAB_TRY(to_dev(db, b, 32 * 16));
    FAB_TRY(dc.err);
    hipLaunchKernelGGL(k_mfma16, dim3(1), dim3(64), 0, 0, da.p, db.p, dc.p);
    FAB_TRY(hipGetLastError());
    FAB_TRY(hipDeviceSynchronize());
    return to_host(c, dc, 16 * 16);
}

int fab_xor32(const float* in, float* out_max, float* out_sum) {
    DevBuf<float> di(64), dm(64), ds(64);
    FAB_TRY(to_dev(di, in, 64));
    FAB_TRY(dm.err);
    FAB_TRY(ds.err);
    hipLaunchKernelGGL(k_xor32, dim3(1), dim3(64), 0, 0, di.p, dm.p, ds.p);
    FAB_TRY(hipGetLastError());
    FAB_TRY(hipDeviceSynchronize());
    FAB_TRY(to_host(out_max, dm, 64));
    return to_host(out_sum, ds, 64);
}

int fab_xor16(const float* in, float* out_max, float* out_sum) {
    DevBuf<float> di(64), dm(64), ds(64);
    FAB_TRY(to_dev(di, in, 64));
    FAB_TRY(dm.err);
    FAB_TRY(ds.err);
    hipLaunchKernelGGL(k_xor16, dim3(1), dim3(64), 0, 0, di.p, dm.p, ds.p);
    FAB_TRY(hipGetLastError());
    FAB_TRY(hipDeviceSynchronize());
    FAB_TRY(to_host(out_max, dm, 64));
    return to_host(out_sum, ds, 64);
}

int fab_pair_swap(const uint16_t* in, uint16_t* out, int dist) {
    DevBuf<uint16_t> di(512), dout(512);
    FAB_TRY(to_dev(di, in, 512));
    FAB_TRY(dout.err);
    hipLaunchKernelGGL(k_pair_swap, dim3(1), dim3(64), 0, 0, di.p, dout.p, dist);
    FAB_TRY(hipGetLastError());
    FAB_TRY(hipDeviceSynchronize());
    return to_host(out, dout, 512);
}

int fab_exp2(const float* x, float* y, int n) {
    if (n <= 0) return 0;
    DevBuf<float> dx(n), dy(n);
    FAB_TRY(to_dev(dx, x, n));
    FAB_TRY(dy.err);
    hipLaunchKernelGGL(k_exp2, dim3(1), dim3(64), 0, 0, dx.p, dy.p, n);
    FAB_TRY(hipGetLastError());
    FAB_TRY(hipDeviceSynchronize());
    return to_host(y, dy, n);
}

int fab_pack8(const float* x, uint16_t* y, int n) {
    if (n <= 0 || n % 8 != 0) return static_cast<int>(hipErrorInvalidValue);
    DevBuf<float> dx(n);
    DevBuf<uint16_t> dy(n);
    FAB_TRY(to_dev(dx, x, n));
    FAB_TRY(dy.err);
    hipLaunchKernelGGL(k_pack8, dim3(1), dim3(64), 0, 0, dx.p, dy.p, n);
    FAB_TRY(hipGetLastError());
    FAB_TRY(hipDeviceSynchronize());
    return to_host(y, dy, n);
}

int fab_lds_dma(const uint16_t* src, const int* src_chunk, uint16_t* out) {
    for (int i = 0; i < 64; ++i)
        if (src_chunk[i] < 0 || src_chunk[i] >= 64) return static_cast<int>(hipErrorInvalidValue);
    DevBuf<uint16_t> ds(512), dout(512);
    DevBuf<int> dc(64);
    FAB_TRY(to_dev(ds, src, 512));
    FAB_TRY(to_dev(dc, src_chunk, 64));
    FAB_TRY(dout.err);
    hipLaunchKernelGGL(k_lds_dma, dim3(1), dim3(64), 0, 0, ds.p, dc.p, dout.p);
    FAB_TRY(hipGetLastError());
    FAB_TRY(hipDeviceSynchronize());
    return to_host(out, dout, 512);
}

int fab_lds_dma_buf(const uint16_t* src, const int* src_chunk, int bytes, uint16_t* out) {
    for (int i = 0; i < 64; ++i)
        if (src_chunk[i] < 0 || src_chunk[i] >= 128) return static_cast<int>(hipErrorInvalidValue);
    if (bytes < 0 || bytes > 1024) return static_cast<int>(hipErrorInvalidValue);
    // 4 KiB allocation: even a lane the range check failed to stop would stay inside it.
    DevBuf<uint16_t> ds(2048), dout(512);
    DevBuf<int> dc(64);
    FAB_TRY(ds.err);
    FAB_TRY(hipMemset(ds.p, 0x7F, 2048 * sizeof(uint16_t)));
    FAB_TRY(to_dev(ds, src, 512));
    FAB_TRY(to_dev(dc, src_chunk, 64));
    FAB_TRY(dout.err);
    hipLaunchKernelGGL(k_lds_dma_buf, dim3(1), dim3(64), 0, 0, ds.p, dc.p, bytes, dout.p);
    FAB_TRY(hipGetLastError());
    FAB_TRY(hipDeviceSynchronize());
    return to_host(out, dout, 512);
}

int fab_sum8(const uint16_t* x, float* y, int groups) {
    if (groups <= 0) return static_cast<int>(hipErrorInvalidValue);
    DevBuf<uint16_t> dx(8 * groups);
    DevBuf<float> dy(groups);
    FAB_TRY(to_dev(dx, x, 8 * static_cast<size_t>(groups)));
    FAB_TRY(dy.err);
    hipLaunchKernelGGL(k_sum8, dim3(1), dim3(64), 0, 0, dx.p, dy.p, groups);
    FAB_TRY(hipGetLastError());
    FAB_TRY(hipDeviceSynchronize());
    return to_host(y, dy, groups);
}

}  // extern "C"
