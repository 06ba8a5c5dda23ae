// RMSNorm variants of the Qwen3.5 prefill (norm.cu:11-99 semantics):
//   cs1_rms_norm / cs1_add_rms_norm: zero-centred x * rsqrt(mean x^2 + eps) * (1 + w),
//     float32 math, one bf16 rounding (the residual add rounds first);
//   cs1_gated_rms_norm: the GDN output norm, D = 128, round(x * inv), round(w * .),
//     times silu(z), rounded.
// MI355X layout: rows of the residual stream go one block of 256 lanes per row with
// 16-byte accesses; the gated norm packs four 128-wide rows into one wave64 (16 lanes x
// 8 values per row) so a wave moves 1 KiB per instruction.
#include "common.h"

namespace q35 {
namespace {

constexpr int NORM_THREADS = 256;

__device__ __forceinline__ float block_sum256(float x, float* red) {
    x = lane_sum<64>(x);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = x;
    __syncthreads();
    const float total = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return total;
}

// Vector path: D % 8 == 0 and 16-byte aligned rows; each lane keeps its packs in
// registers (up to MAXP packs per lane, i.e. D <= 256 * 8 * MAXP).
template <int MAXP, bool ADD>
__global__ void __launch_bounds__(NORM_THREADS)
    rms_norm_vec_kernel(Pack8* __restrict__ residual, const Pack8* __restrict__ delta, const Pack8* __restrict__ x,
                        const Pack8* __restrict__ w, Pack8* __restrict__ out, int packs, float inv_d, float eps) {
    __shared__ float red[4];
    const size_t row = (size_t)blockIdx.x * packs;
    float v[MAXP][8];
    float ss = 0.f;
#pragma unroll
    for (int m = 0; m < MAXP; m++) {
        const int p = threadIdx.x + m * NORM_THREADS;
        if (p < packs) {
            if (ADD) {
                float a[8], b[8];
                unpack8(residual[row + p], a);
                unpack8(delta[row + p], b);
#pragma unroll
                for (int e = 0; e < 8; e++) v[m][e] = round_bf16(a[e] + b[e]);
                residual[row + p] = pack8(v[m]);
            } else {
                unpack8(x[row + p], v[m]);
            }
#pragma unroll
            for (int e = 0; e < 8; e++) ss += v[m][e] * v[m][e];
        }
    }
    const float inv = rsqrtf(block_sum256(ss, red) * inv_d + eps);
#pragma unroll
    for (int m = 0; m < MAXP; m++) {
        const int p = threadIdx.x + m * NORM_THREADS;
        if (p < packs) {
            float wv[8];
            unpack8(w[p], wv);
#pragma unroll
            for (int e = 0; e < 8; e++) v[m][e] = v[m][e] * inv * (1.f + wv[e]);
            out[row + p] = pack8(v[m]);
        }
    }
}

// Scalar path for any D (re-reads the row).
template <bool ADD>
__global__ void __launch_bounds__(NORM_THREADS)
    rms_norm_scalar_kernel(bf16* __restrict__ residual, const bf16* __restrict__ delta, const bf16* __restrict__ x,
                           const bf16* __restrict__ w, bf16* __restrict__ out, int D, float eps) {
    __shared__ float red[4];
    const size_t row = (size_t)blockIdx.x * D;
    const bf16* src = ADD ? residual : x;
    float ss = 0.f;
    for (int i = threadIdx.x; i < D; i += NORM_THREADS) {
        float val;
        if (ADD) {
            const bf16 r = to_bf16(f32(residual[row + i]) + f32(delta[row + i]));
            residual[row + i] = r;
            val = f32(r);
        } else {
            val = f32(src[row + i]);
        }
        ss += val * val;
    }
    const float inv = rsqrtf(block_sum256(ss, red) / D + eps);
    for (int i = threadIdx.x; i < D; i += NORM_THREADS)
        out[row + i] = to_bf16(f32(src[row + i]) * inv * (1.f + f32(w[i])));
}

// Gated RMSNorm, D = 128: 16 lanes per row, 4 rows per wave, 16 rows per block.
__global__ void __launch_bounds__(NORM_THREADS)
    gated_rms_norm_kernel(const bf16* __restrict__ x, const bf16* __restrict__ z, int ldz, const bf16* __restrict__ w,
                          bf16* __restrict__ out, int rows, int H, float eps) {
    const int row = blockIdx.x * (NORM_THREADS / 16) + threadIdx.x / 16, sub = threadIdx.x & 15;
    const bool valid = row < rows;
    const int r = valid ? row : rows - 1;
    const size_t base = (size_t)r * 128 + sub * 8;
    const size_t zbase = (size_t)(r / H) * ldz + (size_t)(r % H) * 128 + sub * 8;
    float v[8], zv[8], wv[8];
    unpack8(*reinterpret_cast<const Pack8*>(x + base), v);
    unpack8(*reinterpret_cast<const Pack8*>(z + zbase), zv);
    unpack8(*reinterpret_cast<const Pack8*>(w + sub * 8), wv);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) ss += v[i] * v[i];
    const float inv = rsqrtf(lane_sum<16>(ss) * (1.f / 128.f) + eps);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float normed = round_bf16(v[i] * inv);
        const float scaled = round_bf16(wv[i] * normed);
        v[i] = scaled * silu(zv[i]);
    }
    if (valid) *reinterpret_cast<Pack8*>(out + base) = pack8(v);
}

__global__ void __launch_bounds__(NORM_THREADS)
    gated_rms_norm_scalar_kernel(const bf16* __restrict__ x, const bf16* __restrict__ z, int ldz,
                                 const bf16* __restrict__ w, bf16* __restrict__ out, int rows, int H, float eps) {
    const int row = blockIdx.x * (NORM_THREADS / 16) + threadIdx.x / 16, sub = threadIdx.x & 15;
    const bool valid = row < rows;
    const int r = valid ? row : rows - 1;
    const size_t base = (size_t)r * 128 + sub * 8;
    const size_t zbase = (size_t)(r / H) * ldz + (size_t)(r % H) * 128 + sub * 8;
    float v[8];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        v[i] = f32(x[base + i]);
        ss += v[i] * v[i];
    }
    const float inv = rsqrtf(lane_sum<16>(ss) * (1.f / 128.f) + eps);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float normed = round_bf16(v[i] * inv);
        const float scaled = round_bf16(f32(w[sub * 8 + i]) * normed);
        if (valid) out[base + i] = to_bf16(scaled * silu(f32(z[zbase + i])));
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <bool ADD>
int launch_rms(void* residual, const void* delta, const void* x, const void* w, void* out, int rows, int D, float eps,
               hipStream_t st) {
    const bool vec = D % 8 == 0 && D <= 256 * 8 * 4 && aligned16(residual) && aligned16(delta) && aligned16(x) &&
                     aligned16(w) && aligned16(out);
    if (vec) {
        const int packs = D / 8;
        auto* r = static_cast<Pack8*>(residual);
        auto* d = static_cast<const Pack8*>(delta);
        auto* xx = static_cast<const Pack8*>(x);
        auto* ww = static_cast<const Pack8*>(w);
        auto* o = static_cast<Pack8*>(out);
        if (packs <= 256)
            rms_norm_vec_kernel<1, ADD><<<rows, NORM_THREADS, 0, st>>>(r, d, xx, ww, o, packs, 1.f / D, eps);
        else if (packs <= 512)
            rms_norm_vec_kernel<2, ADD><<<rows, NORM_THREADS, 0, st>>>(r, d, xx, ww, o, packs, 1.f / D, eps);
        else
            rms_norm_vec_kernel<4, ADD><<<rows, NORM_THREADS, 0, st>>>(r, d, xx, ww, o, packs, 1.f / D, eps);
    } else {
        rms_norm_scalar_kernel<ADD><<<rows, NORM_THREADS, 0, st>>>(
            static_cast<bf16*>(residual), static_cast<const bf16*>(delta), static_cast<const bf16*>(x),
            static_cast<const bf16*>(w), static_cast<bf16*>(out), D, eps);
    }
    return hipGetLastError();
}

}  // namespace
}  // namespace q35

using namespace q35;

extern "C" int cs1_rms_norm(const void* x, const void* w, void* out, int rows, int D, float eps, void* stream) {
    if (rows <= 0 || D <= 0) return hipSuccess;
    if (!all_set({x, w, out})) return hipErrorInvalidValue;
    return launch_rms<false>(nullptr, nullptr, x, w, out, rows, D, eps, static_cast<hipStream_t>(stream));
}

extern "C" int cs1_add_rms_norm(void* residual, const void* delta, const void* w, void* out, int rows, int D,
                                float eps, void* stream) {
    if (rows <= 0 || D <= 0) return hipSuccess;
    if (!all_set({residual, delta, w, out})) return hipErrorInvalidValue;
    return launch_rms<true>(residual, delta, nullptr, w, out, rows, D, eps, static_cast<hipStream_t>(stream));
}

extern "C" int cs1_gated_rms_norm(const void* x, const void* z, int ldz, const void* w, void* out, int T, int H,
                                  int D, float eps, void* stream) {
    if (D != 128 || ldz < H * D) return hipErrorInvalidValue;
    const int rows = T * H;
    if (rows <= 0) return hipSuccess;
    if (!all_set({x, z, w, out})) return hipErrorInvalidValue;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const unsigned blocks = cdiv((size_t)rows, NORM_THREADS / 16);
    if (ldz % 8 == 0 && aligned16(x) && aligned16(z) && aligned16(w) && aligned16(out))
        gated_rms_norm_kernel<<<blocks, NORM_THREADS, 0, st>>>(static_cast<const bf16*>(x), static_cast<const bf16*>(z),
                                                               ldz, static_cast<const bf16*>(w), static_cast<bf16*>(out),
                                                               rows, H, eps);
    else
        gated_rms_norm_scalar_kernel<<<blocks, NORM_THREADS, 0, st>>>(
            static_cast<const bf16*>(x), static_cast<const bf16*>(z), ldz, static_cast<const bf16*>(w),
            static_cast<bf16*>(out), rows, H, eps);
    return hipGetLastError();
}
