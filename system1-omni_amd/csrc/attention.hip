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

constexpr int BN = 64;          // keys per tile
constexpr int QW = 32;          // queries per wave (two 16-query MFMA column tiles)
constexpr int FA_THREADS = 256; // four waves

template <int D>
struct FaSmem {
    static constexpr int KLD = D + 8;   // bf16 row stride of K [BN][D]
    static constexpr int VLD = BN + 8;  // bf16 row stride of V^T [D][BN]
    static constexpr int STAGE = BN * KLD + D * VLD;  // bf16 elements per stage
    static constexpr int BYTES = 2 * STAGE * 2;        // two stages
};

template <int D>
struct TileRegs {
    // this thread's share of one K tile and one V tile (16-byte packs)
    static constexpr int KP = BN * D / 8 / FA_THREADS;        // K packs per thread
    static constexpr int VP = BN / 2 * D / 8 / FA_THREADS;    // V key-pairs x 8 dims per thread
    u32x4 k[KP];
    u32x4 v[VP][2];
};

__device__ __forceinline__ u32x4 ldg16(const bf16* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

// V^T column swizzle: key pair p of row d is stored at pair p ^ 2 ((d / 8) % 16). Groups of
// four keys stay contiguous (fragment reads are unchanged in shape) while the transposing
// stores of one wave, which cover rows 8c + 2e for c = 0..15, spread over all 64 banks.
__device__ __forceinline__ int vt_pair(int d, int pair) { return pair ^ (((d >> 3) & 15) << 1); }

template <int D>
__device__ __forceinline__ void load_tile(TileRegs<D>& r, const bf16* __restrict__ k, const bf16* __restrict__ v,
                                          int ldk, int ldv, int k0, int T) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < TileRegs<D>::KP; i++) {
        const int x = tid + i * FA_THREADS;
        const int row = x / (D / 8), col = (x % (D / 8)) * 8, s = min(k0 + row, T - 1);
        r.k[i] = ldg16(k + (size_t)s * ldk + col);
    }
#pragma unroll
    for (int i = 0; i < TileRegs<D>::VP; i++) {
        const int x = tid + i * FA_THREADS;
        const int pair = x / (D / 8), col = (x % (D / 8)) * 8;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int s = min(k0 + 2 * pair + j, T - 1);  // rows past T are masked out
            r.v[i][j] = ldg16(v + (size_t)s * ldv + col);
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
        *reinterpret_cast<u32x4*>(ks + row * FaSmem<D>::KLD + col) = r.k[i];
    }
#pragma unroll
    for (int i = 0; i < TileRegs<D>::VP; i++) {
        const int x = tid + i * FA_THREADS;
        const int pair = x / (D / 8), col = (x % (D / 8)) * 8;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            // dims col + 2e and col + 2e + 1 of keys 2 pair, 2 pair + 1
            const uint32_t a = r.v[i][0][e], b = r.v[i][1][e];
            const uint32_t lo = (a & 0xffffu) | (b << 16);
            const uint32_t hi = (a >> 16) | (b & 0xffff0000u);
            const int d0 = col + 2 * e, d1 = d0 + 1;
            *reinterpret_cast<uint32_t*>(vt + d0 * FaSmem<D>::VLD + 2 * vt_pair(d0, pair)) = lo;
            *reinterpret_cast<uint32_t*>(vt + d1 * FaSmem<D>::VLD + 2 * vt_pair(d1, pair)) = hi;
        }
    }
}

#ifdef Q35_PHASE_TIMING
// Development aid: per-phase shader-clock ticks of the tile loop, summed over blocks.
__device__ unsigned long long q35_fa_ticks[8];
#define FA_T0() uint64_t fa_t0 = __builtin_amdgcn_s_memtime(), fa_acc[4] = {0, 0, 0, 0}
#define FA_T(i)                                                 \
    do {                                                        \
        const uint64_t fa_t1 = __builtin_amdgcn_s_memtime();    \
        fa_acc[i] += fa_t1 - fa_t0;                             \
        fa_t0 = fa_t1;                                          \
    } while (0)
#define FA_FLUSH()                                                                                   \
    do {                                                                                             \
        if (threadIdx.x == 0) {                                                                      \
            for (int fa_i = 0; fa_i < 4; fa_i++) atomicAdd(&q35_fa_ticks[fa_i], fa_acc[fa_i]);       \
            atomicAdd(&q35_fa_ticks[4], (unsigned long long)ntiles);                                 \
        }                                                                                            \
    } while (0)
#else
#define FA_T0() (void)0
#define FA_T(i) (void)0
#define FA_FLUSH() (void)0
#endif

// Work split. GQA4 (Hq / Hk a multiple of 4): the four waves are four q-heads of one GQA
// group on the same 32 query rows, so every K/V tile in LDS serves four heads. Otherwise
// the four waves are four consecutive 32-row blocks of one head.
template <int D, bool GATED, bool GQA4, int QT>
__global__ void __launch_bounds__(FA_THREADS, D == 128 ? 2 : 1)
    flash_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v, int ldv,
                 const bf16* __restrict__ gate, bf16* __restrict__ out, float* __restrict__ lse, int T, int Hq, int Hk,
                 float scale_log2, int q_base) {
    extern __shared__ __align__(16) unsigned char smem[];
    bf16* stage0 = reinterpret_cast<bf16*>(smem);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int col = lane & 15, grp = lane >> 4;
    constexpr int QWW = 16 * QT;             // query rows per wave
    const int nrows = GQA4 ? QWW : 4 * QWW;  // query rows per block
    const int nblk = (T - q_base + nrows - 1) / nrows;
    const int units = GQA4 ? Hq / 4 : Hq;  // head units per row block
    const int b = blockIdx.x;
    const int rblk = nblk - 1 - b / units;  // longest blocks first
    const int unit = b % units;
    const int h = GQA4 ? unit * 4 + wave : unit;
    const int hk = (GQA4 ? unit * 4 : unit) / (Hq / Hk);
    const int blk_q0 = q_base + rblk * nrows;
    const int q0 = blk_q0 + (GQA4 ? 0 : wave * QWW);  // this wave's first query
    const bf16* kh = k + (size_t)hk * D;
    const bf16* vh = v + (size_t)hk * D;
    const int ldk = Hk * D;

    // Q^T fragments (B operand): query q0 + 16 qt + col, dims 32 s + 8 grp .. + 7
    constexpr int KS = D / 32;
    u32x4 qf[QT][KS];
#pragma unroll
    for (int qt = 0; qt < QT; qt++) {
        const bf16* qr = q + ((size_t)min(q0 + 16 * qt + col, T - 1) * Hq + h) * D + 8 * grp;
#pragma unroll
        for (int s = 0; s < KS; s++) {
            const Pack8 p = *reinterpret_cast<const Pack8*>(qr + 32 * s);
            qf[qt][s] = u32x4{p.w[0], p.w[1], p.w[2], p.w[3]};
        }
    }

    constexpr int DT = D / 16;
    f32x4 o[QT][DT];
#pragma unroll
    for (int qt = 0; qt < QT; qt++)
#pragma unroll
        for (int i = 0; i < DT; i++) o[qt][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m[QT], l[QT];
#pragma unroll
    for (int qt = 0; qt < QT; qt++) m[qt] = -INFINITY, l[qt] = 0.f;

    const int kv_end = min(T, blk_q0 + nrows);
    const int ntiles = (kv_end + BN - 1) / BN;
    TileRegs<D> regs;
    load_tile<D>(regs, kh, vh, ldk, ldv, 0, T);
    wait_vm_all();  // Q fragments and tile 0 are in registers
    store_tile<D>(regs, stage0, stage0 + BN * FaSmem<D>::KLD);
    if (ntiles > 1) load_tile<D>(regs, kh, vh, ldk, ldv, BN, T);
    __syncthreads();
    FA_T0();
    for (int tile = 0; tile < ntiles; tile++) {
        const int k0 = tile * BN;
        const bf16* ks = stage0 + (tile & 1) * FaSmem<D>::STAGE;
        const bf16* vt = ks + BN * FaSmem<D>::KLD;
        // S^T = K Q^T: 4 sub-tiles of 16 keys x 2 query tiles; each K fragment feeds both
        f32x4 st[4][QT];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            #pragma unroll
            for (int qt = 0; qt < QT; qt++) st[t][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
            const bf16* kr = ks + (16 * t + col) * FaSmem<D>::KLD + 8 * grp;
#pragma unroll
            for (int s = 0; s < KS; s++) {
                const Pack8 p = *reinterpret_cast<const Pack8*>(kr + 32 * s);
                const u32x4 a = u32x4{p.w[0], p.w[1], p.w[2], p.w[3]};
                #pragma unroll
                for (int qt = 0; qt < QT; qt++) st[t][qt] = mfma16(a, qf[qt][s], st[t][qt]);
            }
        }
        FA_T(0);
        u32x4 pf[QT][2];
        // Only the tiles that reach the diagonal of this wave's rows or past T need the mask
        // (wave-uniform test); elsewhere every key is visible to every row.
        const bool masked = k0 + BN - 1 > q0 || k0 + BN > T;
#pragma unroll
        for (int qt = 0; qt < QT; qt++) {
            const int qrow = q0 + 16 * qt + col;
            // running max of the raw scores (scale > 0), over the 4 lanes {q, q+16, q+32, q+48}
            float mx = -INFINITY;
            if (masked) {
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int key = k0 + 16 * t + 4 * grp + r;
                        if (key > qrow || key >= T) st[t][qt][r] = -INFINITY;
                    }
            }
#pragma unroll
            for (int t = 0; t < 4; t++)
                mx = fmaxf(mx, fmaxf(fmaxf(st[t][qt][0], st[t][qt][1]), fmaxf(st[t][qt][2], st[t][qt][3])));
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mn = fmaxf(m[qt], mx * scale_log2);
            const float base = mn == -INFINITY ? 0.f : mn;
            const float alpha = __builtin_amdgcn_exp2f(m[qt] - base);
            m[qt] = mn;
            l[qt] *= alpha;
            // rescale only when some row's maximum moved (alpha == 1 is exact otherwise)
            if (!__all(alpha == 1.f)) {
#pragma unroll
                for (int i = 0; i < DT; i++) o[qt][i] *= alpha;
            }
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float p = __builtin_amdgcn_exp2f(fmaf(st[t][qt][r], scale_log2, -base));
                    st[t][qt][r] = p;
                    l[qt] += p;
                }
            // P^T as the B operand of V^T P^T: key k index 8 grp + e is key 32 s2 + 4 grp + e
            // (e < 4) or 32 s2 + 16 + 4 grp + e - 4 (e >= 4), the same order V^T is read in
#pragma unroll
            for (int s2 = 0; s2 < 2; s2++)
                pf[qt][s2] = u32x4{pack2(st[2 * s2][qt][0], st[2 * s2][qt][1]), pack2(st[2 * s2][qt][2], st[2 * s2][qt][3]),
                                   pack2(st[2 * s2 + 1][qt][0], st[2 * s2 + 1][qt][1]),
                                   pack2(st[2 * s2 + 1][qt][2], st[2 * s2 + 1][qt][3])};
        }
        FA_T(1);
        // O^T += V^T P^T; each V^T fragment feeds both query tiles
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            const int d = 16 * dt + col;
            const bf16* vr = vt + d * FaSmem<D>::VLD;
#pragma unroll
            for (int s2 = 0; s2 < 2; s2++) {
                // keys 32 s2 + 4 grp .. + 3 and 32 s2 + 16 + 4 grp .. + 3 (pairs 16 s2 + 2 grp, + 8)
                const u32x2 a0 = *reinterpret_cast<const u32x2*>(vr + 2 * vt_pair(d, 16 * s2 + 2 * grp));
                const u32x2 a1 = *reinterpret_cast<const u32x2*>(vr + 2 * vt_pair(d, 16 * s2 + 8 + 2 * grp));
                const u32x4 a = u32x4{a0[0], a0[1], a1[0], a1[1]};
                #pragma unroll
                for (int qt = 0; qt < QT; qt++) o[qt][dt] = mfma16(a, pf[qt][s2], o[qt][dt]);
            }
        }
        FA_T(2);
        // next stage: tile + 1 from registers to LDS, then fetch tile + 2
        if (tile + 1 < ntiles) {
            bf16* nk = stage0 + ((tile + 1) & 1) * FaSmem<D>::STAGE;
            store_tile<D>(regs, nk, nk + BN * FaSmem<D>::KLD);
            if (tile + 2 < ntiles) load_tile<D>(regs, kh, vh, ldk, ldv, k0 + 2 * BN, T);
        }
        __syncthreads();
        FA_T(3);
    }
    FA_FLUSH();

#pragma unroll
    for (int qt = 0; qt < QT; qt++) {
        float lt = l[qt];
        lt += __shfl_xor(lt, 16, 64);
        lt += __shfl_xor(lt, 32, 64);
        const int qrow = q0 + 16 * qt + col;
        if (qrow >= T) continue;
        const float inv = 1.f / lt;
        bf16* dst = out + ((size_t)qrow * Hq + h) * D + 4 * grp;
#pragma unroll
        for (int dt = 0; dt < DT; dt++) {
            float a[4];
#pragma unroll
            for (int r = 0; r < 4; r++) a[r] = o[qt][dt][r] * inv;
            if (GATED) {
                const u32x2 gp =
                    *reinterpret_cast<const u32x2*>(gate + ((size_t)qrow * Hq + h) * D + 16 * dt + 4 * grp);
                a[0] = round_bf16(a[0]) * round_bf16(sigmoid(lo_f32(gp[0])));
                a[1] = round_bf16(a[1]) * round_bf16(sigmoid(hi_f32(gp[0])));
                a[2] = round_bf16(a[2]) * round_bf16(sigmoid(lo_f32(gp[1])));
                a[3] = round_bf16(a[3]) * round_bf16(sigmoid(hi_f32(gp[1])));
            }
            *reinterpret_cast<u32x2*>(dst + 16 * dt) = u32x2{pack2(a[0], a[1]), pack2(a[2], a[3])};
        }
        if (lse != nullptr && grp == 0) lse[(size_t)h * T + qrow] = (m[qt] + log2f(lt)) * 0.69314718055994531f;
    }
}

template <int D, bool GATED, bool GQA4, int QT>
int launch_flash(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out, float* lse, int T,
                 int Hq, int Hk, float scale, int q_base, hipStream_t st) {
    static const hipError_t configured = hipFuncSetAttribute(
        reinterpret_cast<const void*>(flash_kernel<D, GATED, GQA4, QT>), hipFuncAttributeMaxDynamicSharedMemorySize,
        FaSmem<D>::BYTES);
    if (configured != hipSuccess) return configured;
    constexpr float LOG2E = 1.4426950408889634f;
    const int nrows = (GQA4 ? 1 : 4) * 16 * QT;
    const int blocks = (T - q_base + nrows - 1) / nrows * (GQA4 ? Hq / 4 : Hq);
    flash_kernel<D, GATED, GQA4, QT><<<blocks, FA_THREADS, FaSmem<D>::BYTES, st>>>(
        static_cast<const bf16*>(q), static_cast<const bf16*>(k), static_cast<const bf16*>(v), ldv,
        static_cast<const bf16*>(gate), static_cast<bf16*>(out), lse, T, Hq, Hk, scale * LOG2E, q_base);
    return hipGetLastError();
}

template <int D, bool GATED>
int launch_flash_any(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out, float* lse,
                     int T, int Hq, int Hk, float scale, int q_base, hipStream_t st) {
    if ((Hq / Hk) % 4 == 0)
        return launch_flash<D, GATED, true, 1>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, st);
    return launch_flash<D, GATED, false, 2>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, st);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int attention_run(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out, float* lse,
                  int T, int Hq, int Hk, int Dh, float scale, int q_base, void* stream) {
    if ((Dh != 128 && Dh != 256) || Hk <= 0 || Hq <= 0 || Hq % Hk != 0 || ldv % 8 != 0 || ldv < Hk * Dh || T < 0)
        return hipErrorInvalidValue;
    if (q_base < 0 || q_base % 64 || q_base > T) return hipErrorInvalidValue;
    if (T == q_base) return hipSuccess;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || (gate && !aligned16(gate)))
        return hipErrorInvalidValue;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (Dh == 128)
        return gate ? launch_flash_any<128, true>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, st)
                    : launch_flash_any<128, false>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, st);
    return gate ? launch_flash_any<256, true>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, st)
                : launch_flash_any<256, false>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, st);
}

}  // namespace
}  // namespace q35

using namespace q35;

#ifdef Q35_PHASE_TIMING
extern "C" int q35_debug_fa_ticks(unsigned long long* out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(q35_fa_ticks), sizeof(q35_fa_ticks));
}
#endif

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
