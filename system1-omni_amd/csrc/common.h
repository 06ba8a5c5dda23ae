// Device helpers shared by the gfx950 kernels: bfloat16 storage and rounding, wave64
// reductions, MFMA operand types, and the PyTorch-compatible activations.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <initializer_list>

#include "qwen3_5_ops.h"

namespace q35 {

// Operand pointers of a call that launches work: each must be set (a null operand is an
// argument error, not a GPU fault).
inline bool all_set(std::initializer_list<const void*> ps) {
    for (const void* p : ps)
        if (p == nullptr) return false;
    return true;
}

// bfloat16 values are carried as raw 16-bit patterns in memory.
using bf16 = uint16_t;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float f32(bf16 x) { return __uint_as_float((uint32_t)x << 16); }

// Round to nearest even through the hardware conversion (v_cvt_pk_bf16_f32).
__device__ __forceinline__ bf16 to_bf16(float x) {
    __bf16 b = (__bf16)x;
    return __builtin_bit_cast(uint16_t, b);
}
__device__ __forceinline__ float round_bf16(float x) { return f32(to_bf16(x)); }
// Two floats to a packed bf16 pair (round to nearest even), one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), bf16x2));
}
__device__ __forceinline__ float lo_f32(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float hi_f32(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }

// PyTorch's float32 SiLU and sigmoid: x / (1 + e^-x) and 1 / (1 + e^-x) with expf.
__device__ __forceinline__ float silu(float x) { return x / (1.f + expf(-x)); }
__device__ __forceinline__ float sigmoid(float x) { return 1.f / (1.f + expf(-x)); }
// The attention output gate's sigmoid, 1 / (1 + 2^(-x log2 e)), on the hardware exp2 and
// reciprocal (each within 1 ulp): a few float32 ulps from the expf form, which can move the
// gate factor by one bf16 step near a rounding boundary. Every gate path (the fused attention
// epilogues and cs1_sigmoid_gate) uses it, so fused and separate gating agree bit for bit.
__device__ __forceinline__ float gate_sigmoid(float x) {
    return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}
// The GDN conv's SiLU in the same form, x / (1 + 2^(-x log2 e)) with the hardware exp2 and
// reciprocal; its output is rounded to bf16, so it differs from the expf form by at most one
// bf16 step, next to a rounding boundary (for x above -87; further down both are -0 or a
// denormal). It halves the conv's arithmetic, which otherwise bounds that kernel.
__device__ __forceinline__ float conv_silu(float x) {
    return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// GDN gates: beta = bf16(sigmoid(b)); g = -exp(A_log) * softplus(a + dt_bias), softplus(x) = x
// above 20 (reference elementwise.cu:50-54; float32, expf/log1pf as PyTorch evaluates them).
// Shared by cs1_gdn_gates and the gated GDN prefill, so the two give the same bits.
__device__ __forceinline__ void gate_values(float b, float a, float neg_a_exp, float dt, bf16& beta, float& g) {
    beta = to_bf16(sigmoid(b));
    const float x = a + dt;
    g = neg_a_exp * (x > 20.f ? x : log1pf(expf(x)));
}

// Butterfly sum over `width` consecutive lanes of a wave64 (width a power of two <= 64).
template <int width>
__device__ __forceinline__ float lane_sum(float x) {
#pragma unroll
    for (int o = width / 2; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

template <int width>
__device__ __forceinline__ float lane_max(float x) {
#pragma unroll
    for (int o = width / 2; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
    return x;
}

// 8 bf16 as one 16-byte access.
struct alignas(16) Pack8 {
    uint32_t w[4];
};

__device__ __forceinline__ void unpack8(const Pack8& p, float out[8]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        out[2 * i] = lo_f32(p.w[i]);
        out[2 * i + 1] = hi_f32(p.w[i]);
    }
}

__device__ __forceinline__ Pack8 pack8(const float in[8]) {
    Pack8 p;
#pragma unroll
    for (int i = 0; i < 4; i++) p.w[i] = pack2(in[2 * i], in[2 * i + 1]);
    return p;
}

// MFMA 16x16x32 bf16 -> f32 (gfx950). Operand layout for a wave:
//   A (16 x 32): lane l holds row l % 16, k = 8 * (l / 16) + 0..7
//   B (32 x 16): lane l holds col l % 16, k = 8 * (l / 16) + 0..7
//   D (16 x 16): lane l holds col l % 16, rows 4 * (l / 16) + 0..3
__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

// Wait until every outstanding vector memory load of this wave has completed (vmcnt(0),
// lgkm/exp counters untouched). Placed before a loop so the compiler's wait analysis knows
// one-time loads issued before it are done and does not re-wait on them every iteration.
__device__ __forceinline__ void wait_vm_all() { __builtin_amdgcn_s_waitcnt(0x0f70); }

inline unsigned cdiv(size_t n, unsigned d) { return (unsigned)((n + d - 1) / d); }

// CU count of the current device (looked up once per device; 0 if it cannot be read).
inline int device_cus() {
    constexpr int MAX_DEV = 64;
    static std::atomic<int> cus_of[MAX_DEV];  // 0: not looked up yet
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) return 0;
    int n = cus_of[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
        cus_of[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

}  // namespace q35
