// Machine calibration for bench.py (not part of the op library): the bf16 MFMA rate and the
// HBM streaming rate this GPU reaches, measured with the same clock settling as the kernels,
// to read the rooflines' published peaks against.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Four independent 32x32x16 bf16 accumulation chains per wave, iters rounds each; one block of
// four waves per SIMD quad. The sum keeps the chains live.
__global__ void __launch_bounds__(256) mfma_rate_kernel(float* __restrict__ out, int iters) {
    bf16x8 a, b;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        a[i] = (__bf16)(threadIdx.x * 0.001f + i);
        b[i] = (__bf16)(i * 0.5f);
    }
    f32x16 c[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < 16; i++) c[j][i] = 0.f;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int j = 0; j < 4; j++) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c[j], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int i = 0; i < 16; i++) s += c[j][i];
    out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// 16-byte copy, four transfers per thread with all loads ahead of the stores; one pass over
// the buffer (bytes a multiple of 16 KiB per 256-thread block).
__global__ void __launch_bounds__(256) copy_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n16) {
    const size_t base = (size_t)blockIdx.x * 1024 + threadIdx.x;
    uint4 r[4];
#pragma unroll
    for (int j = 0; j < 4; j++) r[j] = base + 256 * j < n16 ? src[base + 256 * j] : uint4{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 4; j++)
        if (base + 256 * j < n16) dst[base + 256 * j] = r[j];
}

}  // namespace

// out: blocks * 256 floats. Each block performs 4 * 4 waves * 4 chains * iters MFMAs of
// 2 * 32 * 32 * 16 flop.
extern "C" int q35cal_mfma(float* out, int blocks, int iters, void* stream) {
    if (!out || blocks <= 0 || iters <= 0) return hipErrorInvalidValue;
    mfma_rate_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(out, iters);
    return hipGetLastError();
}

// Copies bytes (a multiple of 16, 16-byte aligned buffers) from src to dst.
extern "C" int q35cal_copy(const void* src, void* dst, size_t bytes, void* stream) {
    if (!src || !dst || bytes % 16 || (reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16)
        return hipErrorInvalidValue;
    const size_t n16 = bytes / 16;
    copy_kernel<<<(unsigned)((n16 + 1023) / 1024), 256, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint4*>(src), static_cast<uint4*>(dst), n16);
    return hipGetLastError();
}
