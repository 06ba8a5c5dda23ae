// Full-attention layers of the Qwen3.5 hybrid prefill on gfx950.
//
// attn_prep: per-(token, head) zero-centred RMSNorm x (1 + w) and rotate_half RoPE on
// the first 2*half dims, rounding where the reference does (attention.cu:21-71).  A row of
// Dh values is spread over Dh/8 lanes of a wave64 (8 values per lane, 16-byte accesses);
// the RoPE partner value comes from lane +- half/8 by a cross-lane read.
//
// flash_kernel: causal GQA attention, FlashAttention-2 structure, designed around the
// wave64 MFMA v_mfma_f32_16x16x32_bf16:
//   * a workgroup of eight waves owns 16 query rows of the four q-heads of a GQA group (or
//     128 rows of one head); its key range is split by tile parity between two groups of
//     four waves, halving the serial chain, and the partial softmax states are merged at
//     the end; K row-major and V transposed (bank-swizzled) are double-buffered in LDS;
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
#include <type_traits>

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

constexpr int FA_WAVES = 8;                  // two groups of four waves
constexpr int FA_THREADS = 64 * FA_WAVES;
constexpr int GROUP_THREADS = 256;

template <int D>
struct FaCfg {
    static constexpr int BN = D == 128 ? 64 : 32;  // keys per tile
    static constexpr int NSUB = BN / 16;           // 16-key score sub-tiles
    static constexpr int KS2 = BN / 32;            // 32-key steps of P V
    static constexpr int KLD = D + 8;              // bf16 row stride of K [BN][D]
    static constexpr int VLD = BN + 8;             // bf16 row stride of V^T [D][BN]
    static constexpr int NCH = BN / 8;             // 16-byte key chunks per V^T row
    // V^T layout: 16-byte key chunks in MFMA k order (64-key tiles), or key pairs with a
    // pair swizzle (32-key tiles, where four chunks per row cannot spread the stores)
    static constexpr bool CHUNKED = BN == 64;
    static constexpr int STAGE = BN * KLD + D * VLD;           // bf16 elements per stage
    static constexpr int BYTES = 4 * STAGE * 2;                // 2 groups x 2 stages
    static constexpr int KP = BN * D / 8 / GROUP_THREADS;      // K packs per thread
    static constexpr int VP = BN / 2 * D / 8 / GROUP_THREADS;  // V key pairs x 8 dims per thread
};

template <int D>
struct TileRegs {
    u32x4 k[FaCfg<D>::KP];
    u32x4 v[FaCfg<D>::VP][2];
};

__device__ __forceinline__ u32x4 ldg16(const bf16* p) { return *reinterpret_cast<const u32x4*>(p); }

// Chunked V^T layout (64-key tiles). Row d holds the tile's keys in the MFMA's k order:
// within each 32-key step s2,
// lane group g's eight keys {4g .. 4g+3, 16+4g .. 16+4g+3} form one 16-byte chunk
// c = 4 s2 + g, so a lane's A operand of V^T P^T is a single 16-byte read. Chunk c of row d
// sits at slot c ^ ((d / 8) mod NCH): the transposing stores of one wave (rows 8c + 2e)
// spread over the banks, and since the XOR only mixes d / 8 into the chunk bits, a reader's
// address is one of two per-lane bases (by the parity of its 16-row block) plus a constant.
template <int D>
__device__ __forceinline__ int vt_slot(int d, int chunk) {
    return chunk ^ ((d >> 3) & (FaCfg<D>::NCH - 1));
}

// Pair layout (32-key tiles): key pair p of row d is stored at pair p ^ 2 ((d / 8) % 8):
// groups of four keys stay contiguous, and the transposing stores of one wave
// (rows 8c + 2e) spread over the banks.
template <int D>
__device__ __forceinline__ int vt_pair(int d, int pair) {
    return pair ^ ((((d >> 3) & 15) << 1) & (FaCfg<D>::BN / 2 - 1));
}

// element offset, within row d, of key j of the tile (j even: the pair j, j + 1 is one word)
template <int D>
__device__ __forceinline__ int vt_pos(int d, int j) {
    if (FaCfg<D>::CHUNKED) {
        const int jj = j & 31, chunk = 4 * (j >> 5) + ((jj & 15) >> 2), e = (jj & 3) + (jj & 16 ? 4 : 0);
        return 8 * vt_slot<D>(d, chunk) + e;
    }
    return 2 * vt_pair<D>(d, j >> 1);
}

// Buffer descriptor over rows [k0, T) of a row-major bf16 tensor with row stride ld and
// rows of D elements: rows at or past T fall outside the descriptor and read as zero (those
// keys are masked, and their probabilities are exactly zero). Based at row k0, so every
// offset stays small whatever T is.
template <int D>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const bf16* base, int ld, int k0, int T) {
    const uint64_t a = (uint64_t)(base + (size_t)k0 * ld);
    const uint64_t ua = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a) |
                        ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)) << 32);
    const int rows = min(T - k0, FaCfg<D>::BN);
    const int bytes = rows > 0 ? ((rows - 1) * ld + D) * 2 : 0;
    return __builtin_amdgcn_make_buffer_rsrc((void*)ua, (short)0, __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

__device__ __forceinline__ u32x4 bload16(__amdgpu_buffer_rsrc_t r, int voff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0));
}

template <int D>
__device__ __forceinline__ void load_tile(TileRegs<D>& r, const bf16* __restrict__ k, const bf16* __restrict__ v,
                                          int ldk, int ldv, int k0, int T, int tg) {
    const __amdgpu_buffer_rsrc_t kr = tile_rsrc<D>(k, ldk, k0, T), vr = tile_rsrc<D>(v, ldv, k0, T);
#pragma unroll
    for (int i = 0; i < FaCfg<D>::KP; i++) {
        const int x = tg + i * GROUP_THREADS;
        const int row = x / (D / 8), col = (x % (D / 8)) * 8;
        r.k[i] = bload16(kr, (row * ldk + col) * 2);
    }
#pragma unroll
    for (int i = 0; i < FaCfg<D>::VP; i++) {
        const int x = tg + i * GROUP_THREADS;
        const int pair = x / (D / 8), col = (x % (D / 8)) * 8;
#pragma unroll
        for (int j = 0; j < 2; j++) r.v[i][j] = bload16(vr, ((2 * pair + j) * ldv + col) * 2);
    }
}

template <int D>
__device__ __forceinline__ void store_tile(const TileRegs<D>& r, bf16* ks, int tg) {
    bf16* vt = ks + FaCfg<D>::BN * FaCfg<D>::KLD;
#pragma unroll
    for (int i = 0; i < FaCfg<D>::KP; i++) {
        const int x = tg + i * GROUP_THREADS;
        const int row = x / (D / 8), col = (x % (D / 8)) * 8;
        *reinterpret_cast<u32x4*>(ks + row * FaCfg<D>::KLD + col) = r.k[i];
    }
#pragma unroll
    for (int i = 0; i < FaCfg<D>::VP; i++) {
        const int x = tg + i * GROUP_THREADS;
        const int pair = x / (D / 8), col = (x % (D / 8)) * 8;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            // dims col + 2e and col + 2e + 1 of keys 2 pair, 2 pair + 1
            const uint32_t a = r.v[i][0][e], b = r.v[i][1][e];
            const uint32_t lo = __builtin_amdgcn_perm(b, a, 0x05040100u);
            const uint32_t hi = __builtin_amdgcn_perm(b, a, 0x07060302u);
            const int d0 = col + 2 * e, d1 = d0 + 1;
            *reinterpret_cast<uint32_t*>(vt + d0 * FaCfg<D>::VLD + vt_pos<D>(d0, 2 * pair)) = lo;
            *reinterpret_cast<uint32_t*>(vt + d1 * FaCfg<D>::VLD + vt_pos<D>(d1, 2 * pair)) = hi;
        }
    }
}

#ifdef Q35_PHASE_TIMING
__device__ unsigned long long q35_fa_ticks[8];
#endif

// Work split of a block (eight waves): wave = 4 g + w. Group g processes the key tiles
// t = g, g + 2, ... of the block's key range, so the block's serial chain is half its
// length and the two groups interleave on every SIMD; their partial softmax states are
// merged at the end. GQA4 (Hq / Hk a multiple of 4): w indexes four q-heads of one GQA group
// on the same 16 query rows (every K/V tile in LDS serves four heads); otherwise w indexes
// four consecutive 32-row (16 for Dh = 256) blocks of one head. Tile boundaries are fixed multiples of BN from
// key 0 and the split is by tile parity, so a query row's arithmetic does not depend on how
// rows are grouped into blocks (the windowed pass repeats the full pass bit for bit).
// Packed sequences of a varlen launch (up to SEQS_MAX per launch, passed by value): sequence
// s is rows cu[s] .. cu[s + 1] - 1 of q, k, v, gate and out, causal within itself; its
// blocks are blockIdx.x in [blk[s], blk[s + 1]). n == 0: one sequence of T rows.
constexpr int SEQS_MAX = 64;
// With a shared prefix (pre > 0, a multiple of 64): sequence s continues pre prefix rows
// whose post-prep K and V are kp (rows of Hk * D) and vp (rows of ldvp): its queries are its
// own rows at positions pre .. pre + len - 1, its keys positions 0 .. pre - 1 from the prefix
// and pre .. from its own rows.
struct Seqs {
    int n, lse_ld;
    int cu[SEQS_MAX + 1], blk[SEQS_MAX + 1];
    int pre, ldvp;
    const bf16* kp;
    const bf16* vp;
};

template <int D, bool GATED, bool GQA4>
__global__ void __launch_bounds__(FA_THREADS, 1)
    flash_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v, int ldv,
                 const bf16* __restrict__ gate, bf16* __restrict__ out, float* __restrict__ lse, int T, int Hq, int Hk,
                 float scale_log2, int q_base, const Seqs seqs) {
    using Cfg = FaCfg<D>;
    int b = blockIdx.x, lse_ld = T;
    if (seqs.n > 0) {
        // varlen: find this block's sequence (a scalar scan) and address it as a whole call
        int sq = 0;
        while (sq + 1 < seqs.n && b >= seqs.blk[sq + 1]) sq++;
        b -= seqs.blk[sq];
        // rows are addressed by position: position P + i is the sequence's row i
        const int r0 = seqs.cu[sq], P = seqs.pre;
        T = seqs.cu[sq + 1] - r0 + P;
        q_base = P;
        lse_ld = seqs.lse_ld;
        const ptrdiff_t sh = (ptrdiff_t)r0 - P;
        q += sh * Hq * D;
        k += sh * Hk * D;
        v += sh * ldv;
        if (GATED) gate += sh * Hq * D;
        out += sh * Hq * D;
        if (lse != nullptr) lse += sh;
    }
    constexpr int BN = Cfg::BN, QT = (GQA4 || D == 256) ? 1 : 2;
    extern __shared__ __align__(16) unsigned char smem[];
    bf16* lds = reinterpret_cast<bf16*>(smem);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int grp_id = __builtin_amdgcn_readfirstlane(wave >> 2), w = wave & 3, tg = tid & (GROUP_THREADS - 1);
    const int col = lane & 15, grp = lane >> 4;
    constexpr int QWW = 16 * QT;                   // query rows per wave
    constexpr int NROWS = GQA4 ? QWW : 4 * QWW;    // query rows per block
    const int nblk = (T - q_base + NROWS - 1) / NROWS;
    const int units = GQA4 ? Hq / 4 : Hq;
    const int rblk = nblk - 1 - b / units;  // longest blocks first
    const int unit = b % units;
    const int h = GQA4 ? unit * 4 + w : unit;
    const int hk = (GQA4 ? unit * 4 : unit) / (Hq / Hk);
    const int blk_q0 = q_base + rblk * NROWS;
    const int q0 = blk_q0 + (GQA4 ? 0 : w * QWW);  // this wave's first query
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
        for (int s = 0; s < KS; s++) qf[qt][s] = ldg16(qr + 32 * s);
    }

    constexpr int DT = D / 16;
    f32x4 o[QT][DT];
    float m[QT], l[QT];
#pragma unroll
    for (int qt = 0; qt < QT; qt++) {
        m[qt] = -INFINITY;
        l[qt] = 0.f;
#pragma unroll
        for (int i = 0; i < DT; i++) o[qt][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    const int kv_end = min(T, blk_q0 + NROWS);
    const int ntiles = (kv_end + BN - 1) / BN;
    const int nt0 = (ntiles + 1) / 2;                // group 0's tiles (>= group 1's)
    const int ntg = grp_id == 0 ? nt0 : ntiles / 2;  // this group's tiles
    bf16* gstage = lds + grp_id * 2 * Cfg::STAGE;

    // Pipeline, one barrier per step: at step it a group first stores its tile it + 1 (in
    // registers since the previous step) to its other stage and issues the loads of tile
    // it + 2, then computes tile it. The barrier closing step it - 1 guarantees nobody still
    // reads that other stage, and the one closing step it publishes tile it + 1.
    TileRegs<D> regs;
    // keys below the shared prefix length come from the prefix buffers
    const bf16* kph = seqs.kp + (size_t)hk * D;
    const bf16* vph = seqs.vp + (size_t)hk * D;
    auto load = [&](int k0) {
        if (k0 < seqs.pre) load_tile<D>(regs, kph, vph, ldk, seqs.ldvp, k0, seqs.pre, tg);
        else load_tile<D>(regs, kh, vh, ldk, ldv, k0, T, tg);
    };
    if (ntg > 0) load(grp_id * BN);
    // Unconditional: the compiler's wait analysis must see the Q fragments complete on every
    // path into the loop, or it waits on the in-loop prefetches before each QK^T MFMA.
    wait_vm_all();
    if (ntg > 0) {
        store_tile<D>(regs, gstage, tg);
        if (ntg > 1) load((2 + grp_id) * BN);
    }
    __syncthreads();
    for (int it = 0; it < nt0; it++) {
        if (it + 1 < ntg) {
            store_tile<D>(regs, gstage + ((it + 1) & 1) * Cfg::STAGE, tg);
            if (it + 2 < ntg) load((2 * (it + 2) + grp_id) * BN);
        }
        const int tile = 2 * it + grp_id;
        const bool live = it < ntg;  // wave-uniform
        const bf16* ks = gstage + (it & 1) * Cfg::STAGE;
        const bf16* vt = ks + BN * Cfg::KLD;
        if (live) {
            const int k0 = tile * BN;
            // V^T fragment (dt, s2) of this lane: row d = 16 dt + col; chunked layout: chunk
            // 4 s2 + grp at slot (4 s2 + grp) ^ ((2 dt + col / 8) mod NCH), i.e. a per-lane base for
            // each parity of dt plus a constant.
            auto read_v = [&](int dt, int s2) {
                if (Cfg::CHUNKED) {
                    const bf16* vr =
                        vt + (16 * dt + col) * Cfg::VLD + 8 * (grp ^ (((col >> 3) | ((dt & 1) << 1)) & 3));
                    return *reinterpret_cast<const u32x4*>(vr + 32 * (s2 ^ ((dt >> 1) & 1)));
                }
                // keys 32 s2 + 4 grp .. + 3 and 32 s2 + 16 + 4 grp .. + 3
                const int d = 16 * dt + col;
                const bf16* vr = vt + d * Cfg::VLD;
                const u32x2 a0 = *reinterpret_cast<const u32x2*>(vr + 2 * vt_pair<D>(d, 16 * s2 + 2 * grp));
                const u32x2 a1 = *reinterpret_cast<const u32x2*>(vr + 2 * vt_pair<D>(d, 16 * s2 + 8 + 2 * grp));
                return u32x4{a0[0], a0[1], a1[0], a1[1]};
            };
            // S^T = K Q^T: NSUB sub-tiles of 16 keys x QT query tiles
            f32x4 st[Cfg::NSUB][QT];
#pragma unroll
            for (int t = 0; t < Cfg::NSUB; t++) {
#pragma unroll
                for (int qt = 0; qt < QT; qt++) st[t][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
                const bf16* kr = ks + (16 * t + col) * Cfg::KLD + 8 * grp;
#pragma unroll
                for (int s = 0; s < KS; s++) {
                    const u32x4 a = *reinterpret_cast<const u32x4*>(kr + 32 * s);
#pragma unroll
                    for (int qt = 0; qt < QT; qt++) st[t][qt] = mfma16(a, qf[qt][s], st[t][qt]);
                }
            }
            u32x4 pf[QT][Cfg::KS2];
            // only tiles reaching the diagonal of this wave's rows or past T need the mask
            const bool masked = k0 + BN - 1 > q0 || k0 + BN > T;
#pragma unroll
            for (int qt = 0; qt < QT; qt++) {
                const int qrow = q0 + 16 * qt + col;
                if (masked) {
#pragma unroll
                    for (int t = 0; t < Cfg::NSUB; t++)
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const int key = k0 + 16 * t + 4 * grp + r;
                            if (key > qrow || key >= T) st[t][qt][r] = -INFINITY;
                        }
                }
                // running max of the raw scores (scale > 0) over the lanes {q, q+16, q+32, q+48}
                float mx = -INFINITY;
#pragma unroll
                for (int t = 0; t < Cfg::NSUB; t++)
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
                for (int t = 0; t < Cfg::NSUB; t++)
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const float p = __builtin_amdgcn_exp2f(fmaf(st[t][qt][r], scale_log2, -base));
                        st[t][qt][r] = p;
                        l[qt] += p;
                    }
                // P^T as the B operand of V^T P^T: k index 8 grp + e is key 32 s2 + 4 grp + e
                // (e < 4) or 32 s2 + 16 + 4 grp + e - 4 (e >= 4), the order V^T is read in
#pragma unroll
                for (int s2 = 0; s2 < Cfg::KS2; s2++)
                    pf[qt][s2] = u32x4{pack2(st[2 * s2][qt][0], st[2 * s2][qt][1]), pack2(st[2 * s2][qt][2], st[2 * s2][qt][3]),
                                       pack2(st[2 * s2 + 1][qt][0], st[2 * s2 + 1][qt][1]),
                                       pack2(st[2 * s2 + 1][qt][2], st[2 * s2 + 1][qt][3])};
            }
            // O^T += V^T P^T; each V^T fragment feeds every query tile
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int s2 = 0; s2 < Cfg::KS2; s2++) {
                    const u32x4 a = read_v(dt, s2);
#pragma unroll
                    for (int qt = 0; qt < QT; qt++) o[qt][dt] = mfma16(a, pf[qt][s2], o[qt][dt]);
                }
        }
        __syncthreads();
    }

    // merge the two groups' partial states through LDS: group 1 publishes, group 0 finishes
    __syncthreads();
    float* part = reinterpret_cast<float*>(smem) + (size_t)w * 64 * (QT * (DT * 4 + 2));
    if (grp_id == 1) {
#pragma unroll
        for (int qt = 0; qt < QT; qt++) {
            float* pp = part + qt * (DT * 4 + 2) * 64;
#pragma unroll
            for (int i = 0; i < DT; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) pp[(i * 4 + r) * 64 + lane] = o[qt][i][r];
            pp[(DT * 4) * 64 + lane] = m[qt];
            pp[(DT * 4 + 1) * 64 + lane] = l[qt];
        }
    }
    __syncthreads();
    if (grp_id == 1) return;
#pragma unroll
    for (int qt = 0; qt < QT; qt++) {
        const float* pp = part + qt * (DT * 4 + 2) * 64;
        const float m1 = pp[(DT * 4) * 64 + lane], l1 = pp[(DT * 4 + 1) * 64 + lane];
        const float mm = fmaxf(m[qt], m1);
        const float base = mm == -INFINITY ? 0.f : mm;
        const float a0 = __builtin_amdgcn_exp2f(m[qt] - base), a1 = __builtin_amdgcn_exp2f(m1 - base);
        float lt = l[qt] * a0 + l1 * a1;
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
            for (int r = 0; r < 4; r++) a[r] = (o[qt][dt][r] * a0 + pp[(dt * 4 + r) * 64 + lane] * a1) * inv;
            if (GATED) {
                const u32x2 gp =
                    *reinterpret_cast<const u32x2*>(gate + ((size_t)qrow * Hq + h) * D + 16 * dt + 4 * grp);
                a[0] = round_bf16(a[0]) * round_bf16(gate_sigmoid(lo_f32(gp[0])));
                a[1] = round_bf16(a[1]) * round_bf16(gate_sigmoid(hi_f32(gp[0])));
                a[2] = round_bf16(a[2]) * round_bf16(gate_sigmoid(lo_f32(gp[1])));
                a[3] = round_bf16(a[3]) * round_bf16(gate_sigmoid(hi_f32(gp[1])));
            }
            *reinterpret_cast<u32x2*>(dst + 16 * dt) = u32x2{pack2(a[0], a[1]), pack2(a[2], a[3])};
        }
        if (lse != nullptr && grp == 0) lse[(size_t)h * lse_ld + qrow] = (mm + log2f(lt)) * 0.69314718055994531f;
    }
}

// ---------------------------------------------------------------- flash attention, Dh 128, GQA4
//
// flash32_kernel: the Dh = 128 GQA path (q heads per kv head a multiple of 4) on the
// 32x32x16 MFMA (v_mfma_f32_32x32x16_bf16). A wave owns 16 query rows of two q heads (32
// query columns), so one K or V fragment read from LDS feeds a 32x32 output tile. A block
// owns 32 rows of the four q heads of one GQA group; its eight waves are 2 key groups x 2 row
// halves x 2 head pairs, group g taking the 32-key tiles g, g + 2, ... of the block's key
// range through its own four LDS stages. Tiles move
// from global memory straight into LDS (buffer_load_dwordx4 ... lds, no registers, no LDS
// stores): K and V keep their row-major layout, 16-byte chunks permuted within each row so
// fragment reads spread over the banks, and V^T fragments come out of ds_read_b64_tr_b16.
// The two key groups' partial softmax states are merged through LDS: a wave publishes the
// half of its output the other group finishes and merges its own half from registers, each
// group finishing 64 dims. Tile boundaries are fixed multiples of 32 from key 0 and the
// merge order is fixed, so a row's arithmetic does not depend on its block (windowed and
// packed launches repeat the full pass bit for bit).
namespace fa32 {
constexpr int BN = 32;                     // keys per tile
constexpr int ROWS = 32;                   // query rows per block
constexpr int KG = 2;                      // key groups per block
constexpr int NSTAGE = 4;                  // LDS stages per key group
constexpr int ROW = 256;                   // bytes per K or V row (128 bf16)
constexpr int K_BYTES = BN * ROW;          // 8192
constexpr int STAGE = 2 * K_BYTES;         // one K tile and one V tile
constexpr int XS = 36;                     // floats per lane of a published half state: o (32), m, l, pad
constexpr int BYTES = KG * NSTAGE * STAGE;  // the stages (131072); the exchange reuses them
static_assert(8 * 64 * XS * 4 <= BYTES, "the exchange fits in the stages");
// s_waitcnt with at most 8 vector memory operations outstanding (a wave issues four
// transfers per step): vmcnt 8 (bits 3:0 = 8, bits 15:14 = 0), lgkmcnt and expcnt untouched
constexpr int VMCNT_TWO_STEPS = 0x0f78;
// how far (log2 units) a row's maximum may exceed the exponent base before the base moves
constexpr float RESCALE_SLACK = 8.f;

// Chunk placement, conflict-free whether the LDS serves 128 or 256 bytes per cycle: 16-byte
// chunk c of K row r sits at slot c ^ (r & 15) (8 or 16 consecutive rows read at one chunk hit
// distinct slots); of V row r at slot c ^ f(r & 3), f = {0, 6, 12, 10}, which separates the
// four rows of a transposing read both within 8 slots (two adjacent chunks per row, one lane
// group) and within 16 (four chunks per row, two lane groups).
__device__ __forceinline__ int k_slot(int r, int c) { return c ^ (r & 15); }
__device__ __forceinline__ int v_slot(int r, int c) { return c ^ ((0xAC60 >> (4 * (r & 3))) & 15); }

__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
}

// Buffer descriptor over rows [k0, min(T, k0 + BN)) of a row-major bf16 tensor (row stride
// ld, rows of 128 elements); rows past T, and every row when !valid, read as zero.
__device__ __forceinline__ u32x4 rsrc(const bf16* base, int ld, int k0, int T, bool valid) {
    const uint64_t a = (uint64_t)(base + (size_t)k0 * ld);
    const int rows = valid ? min(T - k0, BN) : 0;
    const int bytes = rows > 0 ? ((rows - 1) * ld + 128) * 2 : 0;
    // word 1: base bits 32..47, stride 0; word 3: the raw-buffer format word
    return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                 (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)) & 0xffffu,
                 (uint32_t)__builtin_amdgcn_readfirstlane(bytes), 0x00020000u};
}

// One 16-byte-per-lane LDS DMA (buffer_load_dwordx4 ... lds): lane l's chunk lands at LDS
// byte lds + 16 l. Issued as inline asm so the compiler does not treat the in-flight LDS write
// as aliasing this step's fragment reads (it would wait for the transfer before them); the
// kernel orders it explicitly, waiting for all transfers before the barrier that publishes
// them. The asm is the only user of M0 in the kernel.
__device__ __forceinline__ void dma16(const u32x4& rsrc, uint32_t lds, int voff, int soff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds), "v"(voff), "s"(rsrc),
                 "s"(soff)
                 : "memory");
}

// One of a key group's four waves moves its quarter of a tile: rows 8 p .. 8 p + 7, two 1 KB
// instructions of four rows each; lane l fills slot l % 16 of row 4 n + l / 16 with the chunk
// that belongs there. voff[j]: per-lane byte offset within a four-row instruction (j = n for
// K, whose permutation depends on r & 15; V's depends only on r & 3).
__device__ __forceinline__ void dma(const u32x4& r, uint32_t dst, int ld, int p, const int* voff, bool is_k) {
#pragma unroll
    for (int n = 0; n < 2; n++) {
        const int row0 = 8 * p + 4 * n;
        dma16(r, dst + row0 * ROW, voff[is_k ? n : 0], row0 * ld * 2);
    }
}

// Maximum over the two lane halves (lanes l and l ^ 32): one v_permlane32_swap, no LDS trip.
__device__ __forceinline__ float max_halves(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 read_tr(const unsigned char* p) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                         (__attribute__((address_space(3))) s16x4*)(p)));
}
}  // namespace fa32

// PREFIX: the launch has a shared prefix (a compile-time flag, so launches without one carry
// no per-tile selection)
template <bool GATED, bool PREFIX>
__global__ void __launch_bounds__(512, 1)
    flash32_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v, int ldv,
                   const bf16* __restrict__ gate, bf16* __restrict__ out, float* __restrict__ lse, int T, int Hq,
                   int Hk, float scale_log2, int q_base, const Seqs seqs) {
    using namespace fa32;
    constexpr int D = 128;
    int b = blockIdx.x, lse_ld = T;
    if (seqs.n > 0) {
        int sq = 0;
        while (sq + 1 < seqs.n && b >= seqs.blk[sq + 1]) sq++;
        b -= seqs.blk[sq];
        // rows are addressed by position: position P + i is the sequence's row i
        const int r0 = seqs.cu[sq], P = seqs.pre;
        T = seqs.cu[sq + 1] - r0 + P;
        q_base = P;
        lse_ld = seqs.lse_ld;
        const ptrdiff_t sh = (ptrdiff_t)r0 - P;
        q += sh * Hq * D;
        k += sh * Hk * D;
        v += sh * ldv;
        if (GATED) gate += sh * Hq * D;
        out += sh * Hq * D;
        if (lse != nullptr) lse += sh;
    }
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // wave = 4 kg + 2 rh + pair: key group kg, row half rh, head pair
    const int kg = __builtin_amdgcn_readfirstlane(wave >> 2), gw = __builtin_amdgcn_readfirstlane(wave & 3);
    const int rh = gw >> 1, pair = gw & 1;
    // key group 0's waves lead on the SIMD they share with key group 1's
    if (kg == 0) __builtin_amdgcn_s_setprio(1);
    const int c32 = lane & 31, hh = lane >> 5;  // query column, lane half
    const int units = Hq / 4;
    const int nblk = (T - q_base + ROWS - 1) / ROWS;
    const int unit = b % units;
    const int q0 = q_base + (nblk - 1 - b / units) * ROWS;  // longest blocks first
    const int hk = unit * 4 / (Hq / Hk);
    const int h = unit * 4 + 2 * pair + (c32 >> 4);  // this lane's q head
    const int qrow = q0 + 16 * rh + (c32 & 15);      // this lane's query row
    const int wq0 = q0 + 16 * rh;                     // this wave's first query row
    const bf16* kh = k + (size_t)hk * D;
    const bf16* vh = v + (size_t)hk * D;
    const int ldk = Hk * D;

    const int kv_end = min(T, q0 + ROWS);
    const int ntiles = (kv_end + BN - 1) / BN;
    const int nit = (ntiles + KG - 1) / KG;                        // group 0's tiles (the most)
    const int ntg = ntiles > kg ? (ntiles - kg + KG - 1) / KG : 0;  // this group's tiles
    unsigned char* const gstage = smem + kg * NSTAGE * STAGE;
    // LDS byte address of a stage (the DMA destination, a wave-uniform M0 value)
    auto lds_addr = [&](const unsigned char* p) {
        return (uint32_t)__builtin_amdgcn_readfirstlane(
            (int)(uint32_t)(uintptr_t)(__attribute__((address_space(3))) const unsigned char*)p);
    };

    // DMA lane offsets within a four-row instruction: row l / 16, slot l % 16
    const int drow = lane >> 4, dslot = lane & 15;
    int kvoff[2], vvoff[1];
#pragma unroll
    for (int j = 0; j < 2; j++) kvoff[j] = drow * ldk * 2 + (k_slot(8 * gw + 4 * j + drow, dslot) << 4);
    vvoff[0] = drow * ldv * 2 + (v_slot(drow, dslot) << 4);
    int vvoff_p[1] = {drow * seqs.ldvp * 2 + (v_slot(drow, dslot) << 4)};
    // the group's four waves move one tile each of K and V as eight four-row instructions
    // tile j of the group goes to stage sidx = j % 4 (passed separately: a constant in the
    // unrolled main loop)
    const uint32_t gbase = lds_addr(gstage);
    // keys below the shared prefix length come from the prefix buffers (a tile never
    // straddles it: the prefix length is a multiple of the tile)
    const bf16* kph = seqs.kp + (size_t)hk * D;
    const bf16* vph = seqs.vp + (size_t)hk * D;
    auto dma_k = [&](int j, int sidx, bool valid) {
        const int k0 = (kg + KG * j) * BN;
        if (PREFIX && k0 < seqs.pre)
            dma(rsrc(kph, ldk, k0, seqs.pre, valid), gbase + sidx * STAGE, ldk, gw, kvoff, true);
        else
            dma(rsrc(kh, ldk, k0, T, valid), gbase + sidx * STAGE, ldk, gw, kvoff, true);
    };
    auto dma_v = [&](int j, int sidx, bool valid) {
        const int k0 = (kg + KG * j) * BN;
        if (PREFIX && k0 < seqs.pre)
            dma(rsrc(vph, seqs.ldvp, k0, seqs.pre, valid), gbase + sidx * STAGE + K_BYTES, seqs.ldvp, gw, vvoff_p, false);
        else
            dma(rsrc(vh, ldv, k0, T, valid), gbase + sidx * STAGE + K_BYTES, ldv, gw, vvoff, false);
    };

    // Pipeline prologue: K(0) and V(-1) (zeros: step 0's P V runs on an empty tile) first, the
    // Q fragments beside them, then K(1), K(2), V(0), V(1).
    dma_k(0, 0, ntg > 0);
    dma_v(-1, 3, false);
    // Q^T (B operand): column c32, dims 16 s + 8 hh .. + 7. The wave's 32 (row, head) rows
    // move to LDS as whole lines (two heads of a row are 512 contiguous bytes; read directly,
    // a fragment takes 32 bytes of 32 rows) into the four 2 KB pieces that the wave itself
    // fills with K(1), V(1), K(2) and V(2) once the fragments are in registers. Row-head
    // i = 2 r + hb (row wq0 + r, head 2 pair + hb of the unit) sits at piece i / 8, row i % 8,
    // its 16-byte chunk c at slot c ^ r.
    u32x4 qf[8];
    {
        const int rb = min(wq0, T - 1);
        const uint64_t a = (uint64_t)(q + ((size_t)rb * Hq + unit * 4 + 2 * pair) * D);
        const u32x4 qd = {(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                          (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)) & 0xffffu, 0x7fffffffu,
                          0x00020000u};
#pragma unroll
        for (int n = 0; n < 8; n++) {
            const int i = 4 * n + (lane >> 4), r = i >> 1, hb = i & 1;
            const int voff = ((min(wq0 + r, T - 1) - rb) * Hq + hb) * D * 2 + (((lane & 15) ^ r) << 4);
            const int p = n >> 1;
            dma16(qd, gbase + (1 + (p >> 1)) * STAGE + (p & 1) * K_BYTES + gw * 2048 + (n & 1) * 1024, voff, 0);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const int r = c32 & 15, i = 2 * r + (c32 >> 4), p = i >> 3;
        const unsigned char* qs = gstage + (1 + (p >> 1)) * STAGE + (p & 1) * K_BYTES + gw * 2048 + (i & 7) * ROW;
#pragma unroll
        for (int s = 0; s < 8; s++) qf[s] = *reinterpret_cast<const u32x4*>(qs + (((2 * s + hh) ^ r) << 4));
    }
    // The Q fragments must be complete before the loop, and read before this wave's transfers
    // into their pieces: an empty asm that uses them pins the reads (and the wait for them)
    // here, so the compiler neither sinks them into the loop nor waits on counts there.
#pragma unroll
    for (int i = 0; i < 8; i++) asm volatile("" ::"v"(qf[i]));
    wait_vm_all();
    dma_k(1, 1, ntg > 1);
    dma_v(0, 0, ntg > 0);
    dma_k(2, 2, ntg > 2);
    dma_v(1, 1, ntg > 1);
    __syncthreads();

    f32x16 o[4];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) o[t][i] = 0.f;
    float m = -INFINITY, l = 0.f;

    // fragment read offsets. K (A operand of S^T = K Q^T): row c32, chunk 2 ks + hh.
    // V^T (A operand of O^T += V^T P^T) for dim tile t and k step s: lane i of lane group
    // g = lane / 16 reads 8 bytes of row 16 s + 8 e + 4 (g / 2) + (i / 4) at dims
    // 32 t + 16 (g % 2) + 4 (i % 4); the transposing read hands lane i the four keys of its dim.
    const int kf = c32 * ROW;
    const int gi = lane & 15, gg = lane >> 4;
    const int vrow = 4 * (gg >> 1) + (gi >> 2);     // + 16 s + 8 e
    const int vdim = 16 * (gg & 1) + 4 * (gi & 3);  // + 32 t
    auto vt = [&](int t, int s, int e) {
        const int r = 16 * s + 8 * e + vrow, dim = 32 * t + vdim;
        return r * ROW + (v_slot(r, dim >> 3) << 4) + 2 * (dim & 7);
    };

    // Software pipeline, one barrier per step. Step it computes S = K Q^T of tile it on the
    // MFMA while the VALU finishes the softmax of tile it - 1 and then issues its P V, so a
    // wave always has independent MFMA work in flight. Stage j % 4 holds K(j) and V(j); step it
    // issues K(it + 3) and V(it + 2) into the stage whose K (it - 1) and V (it - 2) the barrier
    // closing step it - 1 released, and before its own barrier waits for the transfers of step
    // it - 2 (K(it + 1), V(it)), which step it + 1 reads: two steps of transfers stay in flight.
    // Transfers are unconditional: tiles past the group's range read as zero and land in slots
    // nobody reads. Every step runs the same code: a tile past the group's range (or the
    // "previous tile" of step 0, whose scores start at -inf) lies beyond every query row of the
    // wave, so the causal mask sends all its scores to -inf and it adds exact zeros.
    //
    // The exponent base m moves lazily: only when some row's maximum exceeds it by more than
    // RESCALE_SLACK (log2 units), so a probability is at most 2^RESCALE_SLACK and O and l are
    // rescaled a few times per row instead of at nearly every step.
    f32x16 s;  // scores of the tile whose softmax is pending
#pragma unroll
    for (int i = 0; i < 16; i++) s[i] = -INFINITY;
    // sc = it % 4; may_mask: tile it - 1 can reach the diagonal or T (the general loop)
    auto step = [&](int it, int sc, bool may_mask) {
        // Issue order within a step (all eight waves start it together after the barrier):
        // the K fragment reads, the K(it + 3) transfer, the softmax statistics of tile it - 1
        // while those reads are in flight, the V fragment reads, QK^T of tile it beside the
        // exponentials, the V(it + 2) transfer, then P V. Spreading the two transfers through
        // the step keeps a wave from stalling on a full memory queue when every wave issues at
        // once.
        const unsigned char* kb = gstage + sc * STAGE;
        const unsigned char* vb = gstage + ((sc + 3) & 3) * STAGE + K_BYTES;
        u32x4 kfr[8], vfr[4][2];
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
            kfr[ks] = *reinterpret_cast<const u32x4*>(kb + kf + (k_slot(c32, 2 * ks + hh) << 4));
        __builtin_amdgcn_sched_barrier(0);
        dma_k(it + 3, (sc + 3) & 3, it + 3 < ntg);
        __builtin_amdgcn_sched_barrier(0);
        // softmax statistics of tile it - 1: s[i] is key k0 + 8 (i / 4) + 4 hh + i % 4
        const int k0 = (kg + KG * (it - 1)) * BN;
        if (may_mask && (k0 + BN - 1 > wq0 || k0 + BN > T)) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int key = k0 + 8 * (i >> 2) + 4 * hh + (i & 3);
                if (key > qrow || key >= T) s[i] = -INFINITY;
            }
        }
        float mx = s[0];
#pragma unroll
        for (int i = 1; i < 16; i++) mx = fmaxf(mx, s[i]);
        mx = max_halves(mx) * scale_log2;
        if (!__all(mx <= m + RESCALE_SLACK)) {
            const float mn = fmaxf(m, mx);
            const float alpha = __builtin_amdgcn_exp2f(m - (mn == -INFINITY ? 0.f : mn));
            m = mn;
            l *= alpha;
#pragma unroll
            for (int t = 0; t < 4; t++) o[t] *= alpha;
        }
        const float base = m == -INFINITY ? 0.f : m;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const u32x2 lo = read_tr(vb + vt(t, j, 0)), hi = read_tr(vb + vt(t, j, 1));
                vfr[t][j] = u32x4{lo[0], lo[1], hi[0], hi[1]};
            }
        __builtin_amdgcn_sched_barrier(0);
        // QK^T of tile it on the MFMA beside the exponentials of tile it - 1
        f32x16 sn;
#pragma unroll
        for (int i = 0; i < 16; i++) sn[i] = 0.f;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) sn = mfma32(kfr[ks], qf[ks], sn);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            s[i] = __builtin_amdgcn_exp2f(fmaf(s[i], scale_log2, -base));
            l += s[i];
        }
        // P^T (B operand) of k step j: k index 8 hh + e is key 16 j + 4 hh + e (e < 4) or
        // 16 j + 8 + 4 hh + e - 4, i.e. s[8 j + e]
        u32x4 pf[2];
#pragma unroll
        for (int j = 0; j < 2; j++)
            pf[j] = u32x4{pack2(s[8 * j], s[8 * j + 1]), pack2(s[8 * j + 2], s[8 * j + 3]),
                          pack2(s[8 * j + 4], s[8 * j + 5]), pack2(s[8 * j + 6], s[8 * j + 7])};
        __builtin_amdgcn_sched_barrier(0);
        dma_v(it + 2, (sc + 2) & 3, it + 2 < ntg);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int j = 0; j < 2; j++) o[t] = mfma32(vfr[t][j], pf[j], o[t]);
        s = sn;
        // the transfers of step it - 2 (issued before this step's four) have landed
        __builtin_amdgcn_s_waitcnt(VMCNT_TWO_STEPS);
        __syncthreads();
    };
    // Steps 0 .. n_main - 1 see no masked tile: step 0's previous tile is the empty one, and
    // the group's tiles kg + 2 m with 32 (kg + 2 m) <= lim lie wholly below this wave's first
    // row and below T; the remaining steps (diagonal, tail, past the range) run the general
    // loop with the mask.
    const int lim = min(wq0 + 1, T) - BN;
    const int ulast = lim >= 0 ? lim / BN : -1;  // last unmasked tile index
    const int n_main = ulast >= kg ? (ulast - kg) / KG + 2 : 1;
    int it = 0;
    for (; it < n_main; it++) step(it, it & 3, false);
    for (; it <= nit; it++) step(it, it & 3, true);
    wait_vm_all();  // trailing transfers (all zero-length) land before the stages are reused
    __syncthreads();

    // o[t][i]: dim 32 t + 8 (i / 4) + 4 hh + i % 4 of query column c32. Key group kg finishes
    // dims [64 kg, 64 kg + 64) of its rows and head pair from the two groups' partial states.
    u32x2 gp[8];
    const size_t orow = ((size_t)min(qrow, T - 1) * Hq + h) * D + 64 * kg + 4 * hh;
    if (GATED) {
#pragma unroll
        for (int j = 0; j < 8; j++) gp[j] = *reinterpret_cast<const u32x2*>(gate + orow + 8 * j);
    }
    // Exchange: each wave publishes the half of its partial output the other key group
    // finishes (o[2 (1 - kg)], o[2 (1 - kg) + 1]) and its m and l, lane-contiguous (XS floats
    // per lane: 16-byte accesses, conflict-free), and merges its own half from registers.
    float* xch = reinterpret_cast<float*>(smem);
    auto finish = [&](auto kgc) {
        constexpr int K = decltype(kgc)::value;  // this wave's key group
        {
            f32x4* px = reinterpret_cast<f32x4*>(xch + (wave * 64 + lane) * XS);
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++)
                    px[4 * t + q4] = f32x4{o[2 * (1 - K) + t][4 * q4], o[2 * (1 - K) + t][4 * q4 + 1],
                                          o[2 * (1 - K) + t][4 * q4 + 2], o[2 * (1 - K) + t][4 * q4 + 3]};
            px[8] = f32x4{m, l, 0.f, 0.f};
        }
        __syncthreads();
        const f32x4* qx = reinterpret_cast<const f32x4*>(xch + ((4 * (1 - K) + gw) * 64 + lane) * XS);
        const f32x4 pml = qx[8];
        const float mk[KG] = {K == 0 ? m : pml[0], K == 0 ? pml[0] : m};
        const float lk[KG] = {K == 0 ? l : pml[1], K == 0 ? pml[1] : l};
        float ak[KG];
        float mm = -INFINITY;
#pragma unroll
        for (int g = 0; g < KG; g++) mm = fmaxf(mm, mk[g]);
        const float base = mm == -INFINITY ? 0.f : mm;
        float lt = 0.f;
#pragma unroll
        for (int g = 0; g < KG; g++) {
            ak[g] = __builtin_amdgcn_exp2f(mk[g] - base);
            lt += lk[g] * ak[g];
        }
        lt += __shfl_xor(lt, 32, 64);
        if (qrow >= T) return;
        const float inv = 1.f / lt;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const f32x4 pv = qx[j];  // the other group's values of dims 64 K + 8 j + 4 hh + r
            float a[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float mine = o[2 * K + j / 4][4 * (j % 4) + r];
                const float p0 = K == 0 ? mine : pv[r], p1 = K == 0 ? pv[r] : mine;
                float acc = 0.f;
                acc += p0 * ak[0];
                acc += p1 * ak[1];
                a[r] = acc * inv;
            }
            if (GATED) {
                a[0] = round_bf16(a[0]) * round_bf16(gate_sigmoid(lo_f32(gp[j][0])));
                a[1] = round_bf16(a[1]) * round_bf16(gate_sigmoid(hi_f32(gp[j][0])));
                a[2] = round_bf16(a[2]) * round_bf16(gate_sigmoid(lo_f32(gp[j][1])));
                a[3] = round_bf16(a[3]) * round_bf16(gate_sigmoid(hi_f32(gp[j][1])));
            }
            *reinterpret_cast<u32x2*>(out + orow + 8 * j) = u32x2{pack2(a[0], a[1]), pack2(a[2], a[3])};
        }
        if (lse != nullptr && K == 0 && hh == 0) lse[(size_t)h * lse_ld + qrow] = (mm + log2f(lt)) * 0.69314718055994531f;
    };
    if (kg == 0)
        finish(std::integral_constant<int, 0>{});
    else
        finish(std::integral_constant<int, 1>{});
}

template <bool GATED, bool PREFIX>
int launch_flash32_as(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out, float* lse,
                      int T, int Hq, int Hk, float scale, int q_base, int blocks, const Seqs& sq, hipStream_t st) {
    static const hipError_t configured =
        hipFuncSetAttribute(reinterpret_cast<const void*>(flash32_kernel<GATED, PREFIX>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, fa32::BYTES);
    if (configured != hipSuccess) return configured;
    flash32_kernel<GATED, PREFIX><<<blocks, 512, fa32::BYTES, st>>>(
        static_cast<const bf16*>(q), static_cast<const bf16*>(k), static_cast<const bf16*>(v), ldv,
        static_cast<const bf16*>(gate), static_cast<bf16*>(out), lse, T, Hq, Hk, scale * 1.4426950408889634f, q_base,
        sq);
    return hipGetLastError();
}

template <bool GATED>
int launch_flash32(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out, float* lse, int T,
                   int Hq, int Hk, float scale, int q_base, int blocks, const Seqs& sq, hipStream_t st) {
    return sq.pre > 0 ? launch_flash32_as<GATED, true>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, blocks, sq, st)
                      : launch_flash32_as<GATED, false>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, blocks, sq,
                                                        st);
}

// flash256_kernel: the Dh = 256 path (q heads per kv head even) on the 32x32x16 MFMA, built
// like flash32_kernel. A block owns 64 rows of one q-head pair; its eight waves are 4 row
// quarters x 2 dim halves, and a wave owns 16 query rows of the pair (32 query columns) and
// one half of the 256 dims. Per 32-key tile a wave computes its half of S^T = K Q^T (8 MFMAs
// over its 128 dims), the two waves of a dim pair exchange those partial scores through LDS
// and both add them in the same order (dims 0-127 first), so they hold identical scores,
// softmax statistics and P; each then accumulates O^T += V^T P^T for its own 128 dims. Every
// K/V tile in LDS serves 128 query columns. Tiles move global -> LDS by buffer_load ... lds
// with flash32's chunk permutations (K: c ^ (r & 15), V: c ^ f(r & 3)) through three stages
// (K two steps ahead, V one), and the partial scores alternate between two exchange buffers,
// so a step needs one barrier. Tile boundaries are fixed multiples of 32 from key 0, so a row's
// arithmetic does not depend on its block (windowed and packed launches repeat the full pass
// bit for bit).
namespace fa256 {
constexpr int BN = 32;                     // keys per tile
constexpr int ROWS = 64;                   // query rows per block
constexpr int NSTAGE = 3;                  // K two steps ahead, V one
constexpr int ROW = 512;                   // bytes per K or V row (256 bf16)
constexpr int K_BYTES = BN * ROW;          // 16384
constexpr int STAGE = 2 * K_BYTES;
constexpr int XCH = 8 * 4096;              // one partial-score tile per wave
constexpr int BYTES = NSTAGE * STAGE + 2 * XCH;  // the stages and two exchange buffers (160 KB)
// at most one step of transfers (four per wave) outstanding before a step's barrier
constexpr int VMCNT_ONE_STEP = 0x0f74;
}  // namespace fa256

template <bool GATED, bool PREFIX>
__global__ void __launch_bounds__(512, 1)
    flash256_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v, int ldv,
                    const bf16* __restrict__ gate, bf16* __restrict__ out, float* __restrict__ lse, int T, int Hq,
                    int Hk, float scale_log2, int q_base, const Seqs seqs) {
    using namespace fa256;
    using fa32::k_slot;
    using fa32::v_slot;
    using fa32::mfma32;
    using fa32::max_halves;
    using fa32::read_tr;
    using fa32::dma16;
    constexpr int D = 256;
    int b = blockIdx.x, lse_ld = T;
    if (seqs.n > 0) {
        int sq = 0;
        while (sq + 1 < seqs.n && b >= seqs.blk[sq + 1]) sq++;
        b -= seqs.blk[sq];
        // rows are addressed by position: position P + i is the sequence's row i
        const int r0 = seqs.cu[sq], P = seqs.pre;
        T = seqs.cu[sq + 1] - r0 + P;
        q_base = P;
        lse_ld = seqs.lse_ld;
        const ptrdiff_t sh = (ptrdiff_t)r0 - P;
        q += sh * Hq * D;
        k += sh * Hk * D;
        v += sh * ldv;
        if (GATED) gate += sh * Hq * D;
        out += sh * Hq * D;
        if (lse != nullptr) lse += sh;
    }
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // wave = 2 rq + dh: row quarter rq, dim half dh
    const int rq = __builtin_amdgcn_readfirstlane(wave >> 1), dh = __builtin_amdgcn_readfirstlane(wave & 1);
    const int c32 = lane & 31, hh = lane >> 5;  // query column, lane half
    const int units = Hq / 2;
    const int nblk = (T - q_base + ROWS - 1) / ROWS;
    const int unit = b % units;
    const int q0 = q_base + (nblk - 1 - b / units) * ROWS;  // longest blocks first
    const int hk = unit * 2 / (Hq / Hk);
    const int h = unit * 2 + (c32 >> 4);           // this lane's q head
    const int qrow = q0 + 16 * rq + (c32 & 15);    // this lane's query row
    const int wq0 = q0 + 16 * rq;                   // this wave's first query row
    const bf16* kh = k + (size_t)hk * D;
    const bf16* vh = v + (size_t)hk * D;
    const int ldk = Hk * D;

    const int kv_end = min(T, q0 + ROWS);
    const int ntiles = (kv_end + BN - 1) / BN;
    auto lds_addr = [&](const unsigned char* p) {
        return (uint32_t)__builtin_amdgcn_readfirstlane(
            (int)(uint32_t)(uintptr_t)(__attribute__((address_space(3))) const unsigned char*)p);
    };
    // DMA: wave w moves rows 4 w .. 4 w + 3 of a K or V tile as two 1 KB instructions of two
    // rows each; lane l fills slot l % 32 of row l / 32 with the chunk that belongs there
    const int drow = lane >> 5, dslot = lane & 31;
    int kvoff[2], vvoff[2], vvoff_p[2];
#pragma unroll
    for (int n = 0; n < 2; n++) {
        const int r = 4 * wave + 2 * n + drow;
        kvoff[n] = drow * ldk * 2 + (k_slot(r, dslot) << 4);
        vvoff[n] = drow * ldv * 2 + (v_slot(r, dslot) << 4);
        vvoff_p[n] = drow * seqs.ldvp * 2 + (v_slot(r, dslot) << 4);
    }
    const uint32_t gbase = lds_addr(smem);
    const bf16* kph = seqs.kp + (size_t)hk * D;
    const bf16* vph = seqs.vp + (size_t)hk * D;
    auto rsrc = [&](const bf16* base, int ld, int k0, int lim, bool valid) {
        const uint64_t a = (uint64_t)(base + (size_t)k0 * ld);
        const int rows = valid ? min(lim - k0, BN) : 0;
        const int bytes = rows > 0 ? ((rows - 1) * ld + D) * 2 : 0;
        return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                     (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)) & 0xffffu,
                     (uint32_t)__builtin_amdgcn_readfirstlane(bytes), 0x00020000u};
    };
    const int uwave = __builtin_amdgcn_readfirstlane(wave);
    auto dma_tile = [&](const u32x4& r, uint32_t dst, int ld, const int* voff) {
#pragma unroll
        for (int n = 0; n < 2; n++) {
            const int row0 = 4 * uwave + 2 * n;
            dma16(r, dst + row0 * ROW, voff[n], row0 * ld * 2);
        }
    };
    auto dma_k = [&](int j, int sidx, bool valid) {
        const int k0 = j * BN;
        if (PREFIX && k0 < seqs.pre)
            dma_tile(rsrc(kph, ldk, k0, seqs.pre, valid), gbase + sidx * STAGE, ldk, kvoff);
        else
            dma_tile(rsrc(kh, ldk, k0, T, valid), gbase + sidx * STAGE, ldk, kvoff);
    };
    auto dma_v = [&](int j, int sidx, bool valid) {
        const int k0 = j * BN;
        if (PREFIX && k0 < seqs.pre)
            dma_tile(rsrc(vph, seqs.ldvp, k0, seqs.pre, valid), gbase + sidx * STAGE + K_BYTES, seqs.ldvp, vvoff_p);
        else
            dma_tile(rsrc(vh, ldv, k0, T, valid), gbase + sidx * STAGE + K_BYTES, ldv, vvoff);
    };

    // Pipeline prologue: K(0) and an empty V(-1), the Q fragments, then K(1) and V(0).
    dma_k(0, 0, ntiles > 0);
    dma_v(-1, 2, false);
    // Q^T (B operand): column c32, dims 128 dh + 16 s + 8 hh .. + 7 (this wave's half)
    u32x4 qf[8];
    {
        const bf16* qr = q + ((size_t)min(qrow, T - 1) * Hq + h) * D + 128 * dh + 8 * hh;
#pragma unroll
        for (int s = 0; s < 8; s++) qf[s] = ldg16(qr + 16 * s);
    }
#pragma unroll
    for (int i = 0; i < 8; i++) asm volatile("" ::"v"(qf[i]));
    wait_vm_all();
    dma_k(1, 1, ntiles > 1);
    dma_v(0, 0, ntiles > 0);
    __syncthreads();

    f32x16 o[4];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) o[t][i] = 0.f;
    float m = -INFINITY, l = 0.f;

    const int kf = c32 * ROW;
    const int gi = lane & 15, gg = lane >> 4;
    const int vrow = 4 * (gg >> 1) + (gi >> 2);                 // + 16 s + 8 e
    const int vdim = 128 * dh + 16 * (gg & 1) + 4 * (gi & 3);   // + 32 t
    auto vt = [&](int t, int s, int e) {
        const int r = 16 * s + 8 * e + vrow, dim = 32 * t + vdim;
        return r * ROW + (v_slot(r, dim >> 3) << 4) + 2 * (dim & 7);
    };

    // Partial scores are exchanged through LDS: buffer it % 2, 4 KB per wave, holds a wave's
    // partial S of tile it as [4][64 lanes] x 16 bytes. A partner reads tile it's partial in
    // step it + 1, and the buffer is rewritten in step it + 2, after that step's barrier.
    unsigned char* const xch = smem + NSTAGE * STAGE;
    unsigned char* const xown = xch + wave * 4096 + lane * 16;
    const unsigned char* const xpart = xch + (wave ^ 1) * 4096 + lane * 16;
    f32x16 sp;  // this wave's partial scores of the tile whose softmax is pending
#pragma unroll
    for (int i = 0; i < 16; i++) sp[i] = 0.f;
    // sc = it % 3
    auto step = [&](int it, int sc, bool may_mask) {
        const unsigned char* kb = smem + sc * STAGE;
        const unsigned char* vb = smem + (sc == 0 ? 2 : sc - 1) * STAGE + K_BYTES;
        const int xr = ((it + 1) & 1) * XCH, xw = (it & 1) * XCH;
        u32x4 kfr[8], vfr[4][2];
        // the partner's partial scores of tile it - 1 (step 0: of the empty tile, whose scores
        // are masked below), read ahead of the K fragments so the softmax does not wait for them
        f32x16 s;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const f32x4 x = *reinterpret_cast<const f32x4*>(xpart + xr + j * 1024);
#pragma unroll
            for (int e = 0; e < 4; e++) s[4 * j + e] = x[e];
        }
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
            kfr[ks] = *reinterpret_cast<const u32x4*>(kb + kf + (k_slot(c32, 16 * dh + 2 * ks + hh) << 4));
        __builtin_amdgcn_sched_barrier(0);
        dma_k(it + 2, sc == 0 ? 2 : sc - 1, it + 2 < ntiles);
        __builtin_amdgcn_sched_barrier(0);
        // QK^T of tile it over this wave's dims
        f32x16 sn;
#pragma unroll
        for (int i = 0; i < 16; i++) sn[i] = 0.f;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) sn = mfma32(kfr[ks], qf[ks], sn);
        // full scores of tile it - 1 (the same order in both waves of the pair: dims 0-127
        // first), then the softmax statistics: s[i] is key k0 + 8 (i / 4) + 4 hh + i % 4
        s = dh == 0 ? sp + s : s + sp;
        const int k0 = (it - 1) * BN;
        if (it == 0 || (may_mask && (k0 + BN - 1 > wq0 || k0 + BN > T))) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int key = k0 + 8 * (i >> 2) + 4 * hh + (i & 3);
                if (it == 0 || key > qrow || key >= T) s[i] = -INFINITY;
            }
        }
        float mx = s[0];
#pragma unroll
        for (int i = 1; i < 16; i++) mx = fmaxf(mx, s[i]);
        mx = max_halves(mx) * scale_log2;
        if (!__all(mx <= m + fa32::RESCALE_SLACK)) {
            const float mn = fmaxf(m, mx);
            const float alpha = __builtin_amdgcn_exp2f(m - (mn == -INFINITY ? 0.f : mn));
            m = mn;
            l *= alpha;
#pragma unroll
            for (int t = 0; t < 4; t++) o[t] *= alpha;
        }
        const float base = m == -INFINITY ? 0.f : m;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            s[i] = __builtin_amdgcn_exp2f(fmaf(s[i], scale_log2, -base));
            l += s[i];
        }
        u32x4 pf[2];
#pragma unroll
        for (int j = 0; j < 2; j++)
            pf[j] = u32x4{pack2(s[8 * j], s[8 * j + 1]), pack2(s[8 * j + 2], s[8 * j + 3]),
                          pack2(s[8 * j + 4], s[8 * j + 5]), pack2(s[8 * j + 6], s[8 * j + 7])};
        // publish this wave's partial of tile it
#pragma unroll
        for (int j = 0; j < 4; j++)
            *reinterpret_cast<f32x4*>(xown + xw + j * 1024) =
                f32x4{sn[4 * j], sn[4 * j + 1], sn[4 * j + 2], sn[4 * j + 3]};
        sp = sn;
        __builtin_amdgcn_sched_barrier(0);
        dma_v(it + 1, sc == 2 ? 0 : sc + 1, it + 1 < ntiles);
        __builtin_amdgcn_sched_barrier(0);
        // P V for this wave's 128 dims: every V^T fragment is read before the first MFMA, so
        // the reads of later dim tiles overlap the MFMAs of earlier ones
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const u32x2 lo = read_tr(vb + vt(t, j, 0)), hi = read_tr(vb + vt(t, j, 1));
                vfr[t][j] = u32x4{lo[0], lo[1], hi[0], hi[1]};
            }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int j = 0; j < 2; j++) o[t] = mfma32(vfr[t][j], pf[j], o[t]);
        __builtin_amdgcn_s_waitcnt(VMCNT_ONE_STEP);
        __syncthreads();
    };
    // Steps 0 .. n_main - 1 see no masked tile (tiles 0 .. ulast lie wholly below this wave's
    // first row and below T); every wave runs ntiles + 1 steps in all.
    const int lim = min(wq0 + 1, T) - BN;
    const int ulast = lim >= 0 ? lim / BN : -1;  // last unmasked tile index
    const int n_main = ulast >= 0 ? ulast + 2 : 1;
    int it = 0, sc = 0;
    for (; it < n_main; it++, sc = sc == 2 ? 0 : sc + 1) step(it, sc, false);
    for (; it <= ntiles; it++, sc = sc == 2 ? 0 : sc + 1) step(it, sc, true);
    wait_vm_all();

    // o[t][i]: dim 128 dh + 32 t + 8 (i / 4) + 4 hh + i % 4 of query column c32
    if (qrow >= T) return;
    const float lt = l + __shfl_xor(l, 32, 64);
    const float inv = 1.f / lt;
    const size_t orow = ((size_t)qrow * Hq + h) * D + 128 * dh + 4 * hh;
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int off = 32 * t + 8 * j;
            float a[4];
#pragma unroll
            for (int r = 0; r < 4; r++) a[r] = o[t][4 * j + r] * inv;
            if (GATED) {
                const u32x2 gp = *reinterpret_cast<const u32x2*>(gate + orow + off);
                a[0] = round_bf16(a[0]) * round_bf16(gate_sigmoid(lo_f32(gp[0])));
                a[1] = round_bf16(a[1]) * round_bf16(gate_sigmoid(hi_f32(gp[0])));
                a[2] = round_bf16(a[2]) * round_bf16(gate_sigmoid(lo_f32(gp[1])));
                a[3] = round_bf16(a[3]) * round_bf16(gate_sigmoid(hi_f32(gp[1])));
            }
            *reinterpret_cast<u32x2*>(out + orow + off) = u32x2{pack2(a[0], a[1]), pack2(a[2], a[3])};
        }
    if (lse != nullptr && dh == 0 && hh == 0) lse[(size_t)h * lse_ld + qrow] = (m + log2f(lt)) * 0.69314718055994531f;
}

template <bool GATED, bool PREFIX>
int launch_flash256_as(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out, float* lse,
                       int T, int Hq, int Hk, float scale, int q_base, int blocks, const Seqs& sq, hipStream_t st) {
    static const hipError_t configured =
        hipFuncSetAttribute(reinterpret_cast<const void*>(flash256_kernel<GATED, PREFIX>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, fa256::BYTES);
    if (configured != hipSuccess) return configured;
    flash256_kernel<GATED, PREFIX><<<blocks, 512, fa256::BYTES, st>>>(
        static_cast<const bf16*>(q), static_cast<const bf16*>(k), static_cast<const bf16*>(v), ldv,
        static_cast<const bf16*>(gate), static_cast<bf16*>(out), lse, T, Hq, Hk, scale * 1.4426950408889634f, q_base,
        sq);
    return hipGetLastError();
}

template <bool GATED>
int launch_flash256(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out, float* lse,
                    int T, int Hq, int Hk, float scale, int q_base, int blocks, const Seqs& sq, hipStream_t st) {
    return sq.pre > 0
               ? launch_flash256_as<GATED, true>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, blocks, sq, st)
               : launch_flash256_as<GATED, false>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, blocks, sq,
                                                  st);
}

template <int D, bool GATED, bool GQA4>
int launch_flash(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out, float* lse, int T,
                 int Hq, int Hk, float scale, int q_base, hipStream_t st) {
    static const hipError_t configured = hipFuncSetAttribute(
        reinterpret_cast<const void*>(flash_kernel<D, GATED, GQA4>), hipFuncAttributeMaxDynamicSharedMemorySize,
        FaCfg<D>::BYTES);
    if (configured != hipSuccess) return configured;
    constexpr float LOG2E = 1.4426950408889634f;
    const int nrows = GQA4 ? 16 : (D == 256 ? 64 : 128);
    const int blocks = (T - q_base + nrows - 1) / nrows * (GQA4 ? Hq / 4 : Hq);
    Seqs one;
    one.n = 0;
    one.pre = 0;
    one.ldvp = 0;
    one.kp = one.vp = nullptr;
    if (D == 128 && GQA4)
        return launch_flash32<GATED>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base,
                                     (T - q_base + fa32::ROWS - 1) / fa32::ROWS * (Hq / 4), one, st);
    if (D == 256 && (Hq / Hk) % 2 == 0)
        return launch_flash256<GATED>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base,
                                      (T - q_base + fa256::ROWS - 1) / fa256::ROWS * (Hq / 2), one, st);
    flash_kernel<D, GATED, GQA4><<<blocks, FA_THREADS, FaCfg<D>::BYTES, st>>>(
        static_cast<const bf16*>(q), static_cast<const bf16*>(k), static_cast<const bf16*>(v), ldv,
        static_cast<const bf16*>(gate), static_cast<bf16*>(out), lse, T, Hq, Hk, scale * LOG2E, q_base, one);
    return hipGetLastError();
}

// Packed sequences: groups of up to SEQS_MAX sequences per launch.
template <int D, bool GATED, bool GQA4>
int launch_flash_varlen(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out, float* lse,
                        const int32_t* cu, int nseq, int Hq, int Hk, float scale, int pre, const void* kp,
                        const void* vp, int ldvp, hipStream_t st) {
    static const hipError_t configured = hipFuncSetAttribute(
        reinterpret_cast<const void*>(flash_kernel<D, GATED, GQA4>), hipFuncAttributeMaxDynamicSharedMemorySize,
        FaCfg<D>::BYTES);
    if (configured != hipSuccess) return configured;
    constexpr float LOG2E = 1.4426950408889634f;
    const bool pairs256 = D == 256 && (Hq / Hk) % 2 == 0;
    const int nrows = (D == 128 && GQA4) ? fa32::ROWS : pairs256 ? fa256::ROWS : GQA4 ? 16 : (D == 256 ? 64 : 128);
    const int units = pairs256 ? Hq / 2 : GQA4 ? Hq / 4 : Hq;
    for (int s0 = 0; s0 < nseq; s0 += SEQS_MAX) {
        Seqs sq;
        sq.n = min(SEQS_MAX, nseq - s0);
        sq.lse_ld = cu[nseq];
        sq.pre = pre;
        sq.ldvp = ldvp;
        sq.kp = static_cast<const bf16*>(kp);
        sq.vp = static_cast<const bf16*>(vp);
        int blocks = 0;
        for (int i = 0; i < sq.n; i++) {
            sq.cu[i] = cu[s0 + i];
            sq.blk[i] = blocks;
            blocks += (cu[s0 + i + 1] - cu[s0 + i] + nrows - 1) / nrows * units;
        }
        sq.cu[sq.n] = cu[s0 + sq.n];
        sq.blk[sq.n] = blocks;
        if (blocks == 0) continue;
        if (D == 128 && GQA4) {
            const int e = launch_flash32<GATED>(q, k, v, ldv, gate, out, lse, 0, Hq, Hk, scale, 0, blocks, sq, st);
            if (e != hipSuccess) return e;
            continue;
        }
        if (pairs256) {
            const int e = launch_flash256<GATED>(q, k, v, ldv, gate, out, lse, 0, Hq, Hk, scale, 0, blocks, sq, st);
            if (e != hipSuccess) return e;
            continue;
        }
        flash_kernel<D, GATED, GQA4><<<blocks, FA_THREADS, FaCfg<D>::BYTES, st>>>(
            static_cast<const bf16*>(q), static_cast<const bf16*>(k), static_cast<const bf16*>(v), ldv,
            static_cast<const bf16*>(gate), static_cast<bf16*>(out), lse, 0, Hq, Hk, scale * LOG2E, 0, sq);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

template <int D, bool GATED>
int launch_flash_any(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out, float* lse,
                     int T, int Hq, int Hk, float scale, int q_base, hipStream_t st) {
    if ((Hq / Hk) % 4 == 0)
        return launch_flash<D, GATED, true>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, st);
    return launch_flash<D, GATED, false>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, st);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int attention_run(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out, float* lse,
                  int T, int Hq, int Hk, int Dh, float scale, int q_base, void* stream) {
    if ((Dh != 128 && Dh != 256) || Hk <= 0 || Hq <= 0 || Hq % Hk != 0 || ldv % 8 != 0 || ldv < Hk * Dh || T < 0)
        return hipErrorInvalidValue;
    if (q_base < 0 || q_base % 64 || q_base > T) return hipErrorInvalidValue;
    if (T == q_base) return hipSuccess;
    if (!all_set({q, k, v, out})) return hipErrorInvalidValue;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || (gate && !aligned16(gate)))
        return hipErrorInvalidValue;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (Dh == 128)
        return gate ? launch_flash_any<128, true>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, st)
                    : launch_flash_any<128, false>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, st);
    return gate ? launch_flash_any<256, true>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, st)
                : launch_flash_any<256, false>(q, k, v, ldv, gate, out, lse, T, Hq, Hk, scale, q_base, st);
}

// Packed sequences, optionally continuing a shared prefix (pre rows of kp / vp).
int attention_varlen_run(const void* q, const void* k, const void* v, int ldv, const void* kp, const void* vp,
                         int ldvp, int pre, const void* gate, void* out, float* lse, const int32_t* cu_seqlens,
                         int nseq, int Hq, int Hk, int Dh, float scale, void* stream) {
    if ((Dh != 128 && Dh != 256) || Hk <= 0 || Hq <= 0 || Hq % Hk != 0 || ldv % 8 != 0 || ldv < Hk * Dh || nseq < 0)
        return hipErrorInvalidValue;
    if (pre < 0 || pre % 64 != 0) return hipErrorInvalidValue;
    if (pre > 0 && (!kp || !vp || !aligned16(kp) || !aligned16(vp) || ldvp % 8 != 0 || ldvp < Hk * Dh))
        return hipErrorInvalidValue;
    if (nseq == 0) return hipSuccess;
    if (!cu_seqlens || cu_seqlens[0] != 0) return hipErrorInvalidValue;
    for (int i = 0; i < nseq; i++)
        if (cu_seqlens[i + 1] < cu_seqlens[i]) return hipErrorInvalidValue;
    if (cu_seqlens[nseq] > 0 && !all_set({q, k, v, out})) return hipErrorInvalidValue;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || (gate && !aligned16(gate)))
        return hipErrorInvalidValue;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const bool g4 = (Hq / Hk) % 4 == 0;
    auto run = [&](auto d, auto gated) {
        constexpr int DD = decltype(d)::value;
        constexpr bool GG = decltype(gated)::value;
        return g4 ? launch_flash_varlen<DD, GG, true>(q, k, v, ldv, gate, out, lse, cu_seqlens, nseq, Hq, Hk, scale,
                                                      pre, kp, vp, ldvp, st)
                  : launch_flash_varlen<DD, GG, false>(q, k, v, ldv, gate, out, lse, cu_seqlens, nseq, Hq, Hk, scale,
                                                       pre, kp, vp, ldvp, st);
    };
    using T128 = std::integral_constant<int, 128>;
    using T256 = std::integral_constant<int, 256>;
    using Yes = std::true_type;
    using No = std::false_type;
    if (Dh == 128) return gate ? run(T128{}, Yes{}) : run(T128{}, No{});
    return gate ? run(T256{}, Yes{}) : run(T256{}, No{});
}

}  // namespace
}  // namespace q35

using namespace q35;

#ifdef Q35_PHASE_TIMING
extern "C" int q35_debug_fa_ticks(unsigned long long* out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(q35_fa_ticks), sizeof(q35_fa_ticks));
}
#endif

extern "C" int cs1_attention_varlen(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out,
                                    float* lse, const int32_t* cu_seqlens, int nseq, int Hq, int Hk, int Dh, float scale,
                                    void* stream) {
    return attention_varlen_run(q, k, v, ldv, nullptr, nullptr, 0, 0, gate, out, lse, cu_seqlens, nseq, Hq, Hk, Dh,
                                scale, stream);
}

extern "C" int cs1_attention_prefix_varlen(const void* q, const void* k, const void* v, int ldv, const void* kp,
                                           const void* vp, int ldvp, int pre, const void* gate, void* out, float* lse,
                                           const int32_t* cu_seqlens, int nseq, int Hq, int Hk, int Dh, float scale,
                                           void* stream) {
    return attention_varlen_run(q, k, v, ldv, kp, vp, ldvp, pre, gate, out, lse, cu_seqlens, nseq, Hq, Hk, Dh, scale,
                                stream);
}

extern "C" int cs1_attn_prep(const void* qg, const void* kr, int ld, const void* qw, const void* kw, const void* cos,
                             const void* sin, void* q, void* gate, void* k, int T, int Hq, int Hk, int Dh, int half,
                             float eps, void* stream) {
    if (ld % 8 != 0 || T < 0 || Hq < 0 || Hk < 0) return hipErrorInvalidValue;
    if ((Dh != 128 && Dh != 256) || half < 0 || half % 8 != 0 || 2 * half > Dh) return hipErrorInvalidValue;
    const int rows = T * (Hq + Hk);
    if (rows == 0) return hipSuccess;
    if (!all_set({qg, kr, qw, kw, cos, sin, q, gate, k})) return hipErrorInvalidValue;
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
