// Full-attention layers of the Qwen3.5 hybrid prefill on gfx950.
//
// attn_prep: per-(token, head) zero-centred RMSNorm x (1 + w) and rotate_half RoPE on
// the first 2*half dims, rounding where the reference does (attention.cu:21-71).  A row of
// Dh values is spread over Dh/8 lanes of a wave64 (8 values per lane, 16-byte accesses);
// the RoPE partner value comes from lane +- half/8 by a cross-lane read.
//
// flash_kernel: causal GQA attention, FlashAttention-2 structure, designed around the
// wave64 MFMA v_mfma_f32_16x16x32_bf16:
//   * a workgroup owns 64 queries of one head (four waves of 16 queries) and walks the
//     keys up to its last query in tiles of 64, K row-major and V transposed in LDS;
//   * each wave computes S^T = K Q^T (keys on the MFMA M side, its 16 queries on N) so the
//     accumulator layout (lane = query column, 4 consecutive keys per lane) is already the
//     B-operand layout of O^T = V^T P^T: the probabilities never leave registers and every
//     softmax statistic of a query lives in the 4 lanes {q, q+16, q+32, q+48};
//   * online softmax in base 2 with float32 running max/sum, P rounded to bf16 for the
//     MFMA and the running sum kept in float32 (the reference's rounding points,
//     attention.cu:146-205), epilogue out = bf16(o / l) or
//     bf16(round(o / l) * round(sigmoid(gate))) (attention.cu:221-231), optional float32
//     log-sum-exp [Hq, T];
//   * blocks are issued longest-first (the diagonal blocks of the causal triangle last).
#include "common.h"

namespace q35 {
namespace {

// ---------------------------------------------------------------- attn_prep

template <int DH>
__global__ void __launch_bounds__(256)
    attn_prep_kernel(const bf16* __restrict__ qg, const bf16* __restrict__ kr, int ld, const bf16* __restrict__ qw,
                     const bf16* __restrict__ kw, const bf16* __restrict__ cs, const bf16* __restrict__ sn,
                     bf16* __restrict__ q, bf16* __restrict__ gate, bf16* __restrict__ k, int T, int Hq, int Hk,
                     int half, float eps) {
    constexpr int LPR = DH / 8;  // lanes per row
    constexpr int RPB = 256 / LPR;
    const int heads = Hq + Hk;
    const int item = blockIdx.x * RPB + threadIdx.x / LPR, sub = threadIdx.x % LPR;
    const bool valid = item < T * heads;
    const int it = valid ? item : T * heads - 1;
    const int t = it / heads, hh = it % heads;
    const bool is_q = hh < Hq;
    const int h = is_q ? hh : hh - Hq;
    const bf16* src = is_q ? qg + (size_t)t * ld + (size_t)h * 2 * DH : kr + (size_t)t * ld + (size_t)h * DH;
    const bf16* w = is_q ? qw : kw;
    const int d0 = sub * 8;
    float x[8], wv[8];
    unpack8(*reinterpret_cast<const Pack8*>(src + d0), x);
    unpack8(*reinterpret_cast<const Pack8*>(w + d0), wv);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) ss += x[i] * x[i];
    const float inv = rsqrtf(lane_sum<LPR>(ss) / DH + eps);
#pragma unroll
    for (int i = 0; i < 8; i++) x[i] = round_bf16(x[i] * inv * (1.f + wv[i]));
    // partner lane: dims d < half pair with d + half, dims in [half, 2 half) with d - half
    const int lane = threadIdx.x & 63;
    const int hl = half / 8;
    const bool lower = d0 < half;
    const int src_lane = lower ? lane + hl : lane - hl;
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float partner = __shfl(x[i], (src_lane & 63), 64);
        y[i] = x[i];
        if (d0 < 2 * half) {
            const int fi = (d0 + i) % half;
            const float c = f32(cs[(size_t)t * half + fi]), s = f32(sn[(size_t)t * half + fi]);
            const float r = lower ? -partner : partner;
            y[i] = round_bf16(round_bf16(x[i] * c) + round_bf16(r * s));
        }
    }
    if (!valid) return;
    if (is_q) {
        *reinterpret_cast<Pack8*>(q + ((size_t)t * Hq + h) * DH + d0) = pack8(y);
        *reinterpret_cast<Pack8*>(gate + ((size_t)t * Hq + h) * DH + d0) =
            *reinterpret_cast<const Pack8*>(src + DH + d0);
    } else {
        *reinterpret_cast<Pack8*>(k + ((size_t)t * Hk + h) * DH + d0) = pack8(y);
    }
}

// ---------------------------------------------------------------- flash attention

constexpr int BM = 64, BN = 64, FA_THREADS = 256;

template <int D>
struct FaSmem {
    static constexpr int KLD = D + 8;   // bf16 row stride of K [BN][D]
    static constexpr int VLD = BN + 8;  // bf16 row stride of V^T [D][BN]
    static constexpr int BYTES = (BN * KLD + D * VLD) * 2;
};

template <int D>
struct TileRegs {
    // this thread's share of one K tile and one V tile (16-byte packs)
    static constexpr int KP = BN * D / 8 / FA_THREADS;        // K packs per thread
    static constexpr int VP = BN / 2 * D / 8 / FA_THREADS;    // V key-pairs x 8 dims per thread
    Pack8 k[KP];
    Pack8 v[VP][2];
};

template <int D>
__device__ __forceinline__ void load_tile(TileRegs<D>& r, const bf16* __restrict__ k, const bf16* __restrict__ v,
                                          int ldk, int ldv, int k0, int T) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < TileRegs<D>::KP; i++) {
        const int x = tid + i * FA_THREADS;
        const int row = x / (D / 8), col = (x % (D / 8)) * 8, s = k0 + row;
        if (s < T)
            r.k[i] = *reinterpret_cast<const Pack8*>(k + (size_t)s * ldk + col);
        else
            r.k[i] = Pack8{{0u, 0u, 0u, 0u}};
    }
#pragma unroll
    for (int i = 0; i < TileRegs<D>::VP; i++) {
        const int x = tid + i * FA_THREADS;
        const int pair = x / (D / 8), col = (x % (D / 8)) * 8, s = k0 + 2 * pair;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            if (s + j < T)
                r.v[i][j] = *reinterpret_cast<const Pack8*>(v + (size_t)(s + j) * ldv + col);
            else
                r.v[i][j] = Pack8{{0u, 0u, 0u, 0u}};
        }
    }
}

template <int D>
__device__ __forceinline__ void store_tile(const TileRegs<D>& r, bf16* ks, bf16* vt) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < TileRegs<D>::KP; i++) {
        const int x = tid + i * FA_THREADS;
        const int row = x / (D / 8), col = (x % (D / 8)) * 8;
        *reinterpret_cast<Pack8*>(ks + row * FaSmem<D>::KLD + col) = r.k[i];
    }
#pragma unroll
    for (int i = 0; i < TileRegs<D>::VP; i++) {
        const int x = tid + i * FA_THREADS;
        const int pair = x / (D / 8), col = (x % (D / 8)) * 8;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            // dims col + 2e and col + 2e + 1 of keys 2 pair, 2 pair + 1
            const uint32_t a = r.v[i][0].w[e], b = r.v[i][1].w[e];
            const uint32_t lo = (a & 0xffffu) | (b << 16);
            const uint32_t hi = (a >> 16) | (b & 0xffff0000u);
            *reinterpret_cast<uint32_t*>(vt + (col + 2 * e) * FaSmem<D>::VLD + 2 * pair) = lo;
            *reinterpret_cast<uint32_t*>(vt + (col + 2 * e + 1) * FaSmem<D>::VLD + 2 * pair) = hi;
        }
    }
}

template <int D, bool GATED>
__global__ void __launch_bounds__(FA_THREADS)
    flash_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v, int ldv,
                 const bf16* __restrict__ gate, bf16* __restrict__ out, float* __restrict__ lse, int T, int Hq, int Hk,
                 float scale_log2, int q_base) {
    extern __shared__ __align__(16) unsigned char smem[];
    bf16* ks = reinterpret_cast<bf16*>(smem);
    bf16* vt = ks + BN * FaSmem<D>::KLD;
    const int h = blockIdx.y, hk = h / (Hq / Hk);
    const int q0 = q_base + (gridDim.x - 1 - blockIdx.x) * BM;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int col = lane & 15, grp = lane >> 4;
    const int qrow = q0 + wave * 16 + col;  // this lane's query
    const bf16* kh = k + (size_t)hk * D;
    const bf16* vh = v + (size_t)hk * D;
    const int ldk = Hk * D;

    // Q^T fragments (B operand): query qrow, dims 32 s + 8 grp .. + 7
    constexpr int KS = D / 32;
    u32x4 qf[KS];
    {
        const bf16* qr = q + ((size_t)min(qrow, T - 1) * Hq + h) * D + 8 * grp;
#pragma unroll
        for (int s = 0; s < KS; s++) {
            const Pack8 p = *reinterpret_cast<const Pack8*>(qr + 32 * s);
            qf[s] = u32x4{p.w[0], p.w[1], p.w[2], p.w[3]};
        }
    }

    constexpr int DT = D / 16;
    f32x4 o[DT];
#pragma unroll
    for (int i = 0; i < DT; i++) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;

    const int kv_end = min(T, q0 + BM);
    const int ntiles = (kv_end + BN - 1) / BN;
    TileRegs<D> regs;
    load_tile<D>(regs, kh, vh, ldk, ldv, 0, T);
    for (int tile = 0; tile < ntiles; tile++) {
        const int k0 = tile * BN;
        __syncthreads();  // the previous tile is consumed
        store_tile<D>(regs, ks, vt);
        __syncthreads();
        if (tile + 1 < ntiles) load_tile<D>(regs, kh, vh, ldk, ldv, k0 + BN, T);

        // S^T = K Q^T: 4 sub-tiles of 16 keys
        f32x4 st[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            st[t] = f32x4{0.f, 0.f, 0.f, 0.f};
            const bf16* kr = ks + (16 * t + col) * FaSmem<D>::KLD + 8 * grp;
#pragma unroll
            for (int s = 0; s < KS; s++) {
                const Pack8 p = *reinterpret_cast<const Pack8*>(kr + 32 * s);
                st[t] = mfma16(u32x4{p.w[0], p.w[1], p.w[2], p.w[3]}, qf[s], st[t]);
            }
        }
        // mask, scale, running max
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int key = k0 + 16 * t + 4 * grp + r;
                const float sv = (key <= qrow && key < T) ? st[t][r] * scale_log2 : -INFINITY;
                st[t][r] = sv;
                mx = fmaxf(mx, sv);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mn = fmaxf(m, mx);
        const float base = mn == -INFINITY ? 0.f : mn;
        const float alpha = exp2f(m - base);
        m = mn;
        l *= alpha;
#pragma unroll
        for (int i = 0; i < DT; i++) o[i] *= alpha;
        u32x4 pf[2];
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = exp2f(st[t][r] - base);
                st[t][r] = p;
                l += p;
            }
#pragma unroll
        for (int s2 = 0; s2 < 2; s2++)
            pf[s2] = u32x4{pack2(st[2 * s2][0], st[2 * s2][1]), pack2(st[2 * s2][2], st[2 * s2][3]),
                           pack2(st[2 * s2 + 1][0], st[2 * s2 + 1][1]), pack2(st[2 * s2 + 1][2], st[2 * s2 + 1][3])};
        // O^T += V^T P^T; the k index 8 grp + e maps to key 32 s2 + 4 grp + e (e < 4) or
        // 32 s2 + 16 + 4 grp + e - 4 (e >= 4), the same mapping on both operands
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            const bf16* vr = vt + (16 * dt + col) * FaSmem<D>::VLD + 4 * grp;
#pragma unroll
            for (int s2 = 0; s2 < 2; s2++) {
                const u32x2 a0 = *reinterpret_cast<const u32x2*>(vr + 32 * s2);
                const u32x2 a1 = *reinterpret_cast<const u32x2*>(vr + 32 * s2 + 16);
                o[dt] = mfma16(u32x4{a0[0], a0[1], a1[0], a1[1]}, pf[s2], o[dt]);
            }
        }
    }

    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (qrow >= T) return;
    const float inv = 1.f / l;
    bf16* dst = out + ((size_t)qrow * Hq + h) * D + 4 * grp;
#pragma unroll
    for (int dt = 0; dt < DT; dt++) {
        float a[4];
#pragma unroll
        for (int r = 0; r < 4; r++) a[r] = o[dt][r] * inv;
        if (GATED) {
            const u32x2 gp = *reinterpret_cast<const u32x2*>(gate + ((size_t)qrow * Hq + h) * D + 16 * dt + 4 * grp);
            a[0] = round_bf16(a[0]) * round_bf16(sigmoid(lo_f32(gp[0])));
            a[1] = round_bf16(a[1]) * round_bf16(sigmoid(hi_f32(gp[0])));
            a[2] = round_bf16(a[2]) * round_bf16(sigmoid(lo_f32(gp[1])));
            a[3] = round_bf16(a[3]) * round_bf16(sigmoid(hi_f32(gp[1])));
        }
        *reinterpret_cast<u32x2*>(dst + 16 * dt) = u32x2{pack2(a[0], a[1]), pack2(a[2], a[3])};
    }
    if (lse != nullptr && grp == 0) lse[(size_t)h * T + qrow] = (m + log2f(l)) * 0.69314718055994531f;
}

template <int D, bool GATED>
int launch_flash(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out, float* lse, int T,
                 int Hq, int Hk, float scale, int q_base, hipStream_t st) {
    static const hipError_t configured = hipFuncSetAttribute(
        reinterpret_cast<const void*>(flash_kernel<D, GATED>), hipFuncAttributeMaxDynamicSharedMemorySize,
        FaSmem<D>::BYTES);
    if (configured != hipSuccess) return configured;
    constexpr float LOG2E = 1.4426950408889634f;
    flash_kernel<D, GATED><<<dim3((T - q_base + BM - 1) / BM, Hq), FA_THREADS, FaSmem<D>::BYTES, st>>>(
        static_cast<const bf16*>(q), static_cast<const bf16*>(k), static_cast<const bf16*>(v), ldv,
        static_cast<const bf16*>(gate), static_cast<bf16*>(out), lse, T, Hq, Hk, scale * LOG2E, q_base);
    return hipGetLastError();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int attention_run(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out, float* lse,
                  int T, int Hq, int Hk, int Dh, float scale, int q_base, void* stream) {
    if ((Dh != 128 && Dh != 256) || Hk <= 0 || Hq <= 0 || Hq % Hk != 0 || ldv % 8 != 0 || ldv < Hk * Dh || T < 0)
        return hipErrorInvalidValue;
    if (q_base < 0 || q_base % BM || q_base > T) return hipErrorInvalidValue;
    if (T == q_base) return hipSuccess;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || (gate && !aligned16(gate)))
        return hipErrorInvalidValue;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (Dh == 128)
        return gate ? launch_flash<128, true>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, st)
                    : launch_flash<128, false>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, st);
    return gate ? launch_flash<256, true>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, st)
                : launch_flash<256, false>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, st);
}

}  // namespace
}  // namespace q35

using namespace q35;

extern "C" int cs1_attn_prep(const void* qg, const void* kr, int ld, const void* qw, const void* kw, const void* cos,
                             const void* sin, void* q, void* gate, void* k, int T, int Hq, int Hk, int Dh, int half,
                             float eps, void* stream) {
    if (ld % 8 != 0 || T < 0 || Hq < 0 || Hk < 0) return hipErrorInvalidValue;
    if ((Dh != 128 && Dh != 256) || half < 0 || half % 8 != 0 || 2 * half > Dh) return hipErrorInvalidValue;
    const int rows = T * (Hq + Hk);
    if (rows == 0) return hipSuccess;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    auto args = [&](auto kernel, int rpb) {
        kernel<<<cdiv((size_t)rows, rpb), 256, 0, st>>>(
            static_cast<const bf16*>(qg), static_cast<const bf16*>(kr), ld, static_cast<const bf16*>(qw),
            static_cast<const bf16*>(kw), static_cast<const bf16*>(cos), static_cast<const bf16*>(sin),
            static_cast<bf16*>(q), static_cast<bf16*>(gate), static_cast<bf16*>(k), T, Hq, Hk, half, eps);
    };
    if (Dh == 256)
        args(attn_prep_kernel<256>, 256 / 32);
    else
        args(attn_prep_kernel<128>, 256 / 16);
    return hipGetLastError();
}

extern "C" int cs1_attention(const void* q, const void* k, const void* v, int ldv, void* out, int T, int Hq, int Hk,
                             int Dh, float scale, void* stream) {
    if (Dh != 256) return hipErrorInvalidValue;
    return attention_run(q, k, v, ldv, nullptr, out, nullptr, T, Hq, Hk, Dh, scale, 0, stream);
}

extern "C" int cs1_attention_gated(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out,
                                   int T, int Hq, int Hk, int Dh, float scale, void* stream) {
    if (Dh != 256) return hipErrorInvalidValue;
    if (T > 0 && gate == nullptr) return hipErrorInvalidValue;
    return attention_run(q, k, v, ldv, gate, out, nullptr, T, Hq, Hk, Dh, scale, 0, stream);
}

extern "C" int cs1_attention_gated_prefix(const void* q, const void* k, const void* v, int ldv, const void* gate,
                                          void* out, int T, int Hq, int Hk, int Dh, float scale, int q_base,
                                          void* stream) {
    if (Dh != 256) return hipErrorInvalidValue;
    if (T > q_base && gate == nullptr) return hipErrorInvalidValue;
    return attention_run(q, k, v, ldv, gate, out, nullptr, T, Hq, Hk, Dh, scale, q_base, stream);
}

extern "C" int cs1_attention_ex(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out,
                                float* lse, int T, int Hq, int Hk, int Dh, float scale, int q_base, void* stream) {
    return attention_run(q, k, v, ldv, gate, out, lse, T, Hq, Hk, Dh, scale, q_base, stream);
}
