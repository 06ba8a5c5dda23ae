// Chunked Gated DeltaNet prefill (chunk 64, dk = dv = 128, batch 1) on gfx950.
//
// Arithmetic of record: transformers' torch_chunk_gated_delta_rule (modeling_qwen3_5.py
// 249-328) with the rounding points of the reference CUDA kernel (gdn_prefill.cu):
//   per chunk and head:  cum = sequential float32 cumsum of g, decay = e^cum_last;
//     q^ = q rsqrt(|q|^2 + 1e-6) scale, k^ = k rsqrt(|k|^2 + 1e-6)  (float32);
//     A_ij = (beta_i (k^_i . k^_j)) e^(cum_i - cum_j) for j < i, P_ij = (q^_i . k^_j) e^(...)
//       for j <= i, the pair products on TF32-rounded operands with float32 sums;
//     T = (I + A)^-1 by the blocked float32 substitution of gdn_prefill.cu:250-287;
//     u = bf16(bf16(T beta) v), w = bf16(bf16(T beta) bf16(k^ e^cum)),
//     qd = bf16(q^ e^cum), kd = bf16(k^ e^(cum_last - cum)), pb = bf16(P);
//   scan over chunks:  Sb = bf16(S); v_new = bf16(u - w Sb); o = bf16(qd Sb + pb v_new);
//     S = S decay + kd^T v_new (float32).
//
// MI355X design (not the reference's three-kernel split):
//   gdn_prep  grid (chunk, head), 8 waves.  TF32 operands are split exactly into two
//     bf16 planes (hi = rne(x), lo = x - hi, exact since TF32 has 11 significant bits) so
//     the TF32 pair products run on the bf16 MFMA (four products per term reproduce the
//     TF32 product exactly); u and w are MFMA products of the triangular T with V and
//     k e^cum staged transposed in LDS.
//   gdn_scan  grid (head x 8 value slices of 16 columns), 4 waves.  The float32 state
//     slice 128 x 16 lives in MFMA accumulators; each chunk reads w, qd, pb, kd^T rows
//     straight from HBM/L2 into MFMA operand registers (prefetched one chunk ahead) and
//     exchanges only bf16(S) and v_new through LDS.  The output o = qd Sb + pb v_new is
//     produced in the same pass, so the per-chunk state copies and v_new never go to
//     memory.  Slices of one head are issued to the same XCD (block = slice * H + head).
#include "common.h"

namespace q35 {
namespace {

constexpr int C = 64;    // chunk length
constexpr int DK = 128;  // key / value head dim

// ------------------------------------------------------------ workspace layout

// Per (head, chunk) records, 256-byte aligned parts:
//   w, u, qd  [64][128] bf16 row-major;  kdT [128][64] bf16 (kd transposed);
//   pb [64][64] bf16 (zero above the diagonal);  decay float.
struct Work {
    bf16* w;
    bf16* u;
    bf16* qd;
    bf16* kdt;
    bf16* pb;
    float* decay;
};

struct Layout {
    size_t w, u, qd, kdt, pb, decay, total;
    Layout(int T, int H) {
        const size_t NC = (size_t)((T + C - 1) / C), n = (size_t)H * NC;
        size_t at = 0;
        auto take = [&](size_t bytes) {
            const size_t off = at;
            at = (at + bytes + 255) / 256 * 256;
            return off;
        };
        w = take(n * C * DK * 2);
        u = take(n * C * DK * 2);
        qd = take(n * C * DK * 2);
        kdt = take(n * C * DK * 2);
        pb = take(n * C * C * 2);
        decay = take(n * 4);
        total = at;
    }
};

Work split(float* workspace, int T, int H) {
    const Layout l(T, H);
    unsigned char* b = reinterpret_cast<unsigned char*>(workspace);
    return Work{reinterpret_cast<bf16*>(b + l.w),   reinterpret_cast<bf16*>(b + l.u),
                reinterpret_cast<bf16*>(b + l.qd),  reinterpret_cast<bf16*>(b + l.kdt),
                reinterpret_cast<bf16*>(b + l.pb),  reinterpret_cast<float*>(b + l.decay)};
}

// cvt.rna.tf32.f32: 10 explicit mantissa bits, round half away from zero.
__device__ __forceinline__ float tf32_rna(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7f800000u) != 0x7f800000u) u = (u + 0x1000u) & 0xffffe000u;
    return __uint_as_float(u);
}

__device__ __forceinline__ u32x4 ld16(const bf16* p) {
    const Pack8 v = *reinterpret_cast<const Pack8*>(p);
    return u32x4{v.w[0], v.w[1], v.w[2], v.w[3]};
}

// ------------------------------------------------------------------ gdn_prep

constexpr int PT = 512;          // threads
constexpr int PW = PT / 64;      // waves
constexpr int PLD = DK + 8;      // bf16 stride of the split planes [64][128]
constexpr int TLD = C + 8;       // bf16 stride of [128][64] transposes and of Tb [64][64]
constexpr int FLD = C + 1;       // float stride of A and T [64][64]

// LDS map (bytes). Region 0 holds the four split planes during the pair products, then
// T (float), the level scratch, Tb (bf16) and v^T (bf16).
constexpr int PLANE = C * PLD * 2;                 // 17408
constexpr int R0 = 0;                              // 4 planes: k hi, k lo, q hi, q lo
constexpr int R0_TM = 0;                           // T float [64][65]
constexpr int R0_SC = R0_TM + C * FLD * 4;         // level scratch float [3][256]
constexpr int R0_TB = R0_SC + 3 * 256 * 4;         // Tb bf16 [64][72]
constexpr int R0_VT = R0_TB + C * TLD * 2;         // v^T bf16 [128][72]
constexpr int R1 = R0 + 4 * PLANE;                 // kw^T bf16 [128][72]
constexpr int R2 = R1 + DK * TLD * 2;              // kd^T bf16 [128][72]
constexpr int R3 = R2 + DK * TLD * 2;              // A float [64][65]
constexpr int R4 = R3 + C * FLD * 4;               // cum, beta, e^cum, e^(last-cum)
constexpr int PREP_SMEM = R4 + 4 * C * 4;
static_assert(R0_VT + DK * TLD * 2 <= R1, "region 0 overlay fits");

__global__ void __launch_bounds__(PT)
    gdn_prep(const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
             const float* __restrict__ g, const bf16* __restrict__ beta, Work ws, int T, int H, int HK, float scale) {
    extern __shared__ __align__(16) unsigned char sm[];
    bf16* khi = reinterpret_cast<bf16*>(sm + R0);
    bf16* klo = khi + C * PLD;
    bf16* qhi = klo + C * PLD;
    bf16* qlo = qhi + C * PLD;
    float* tm = reinterpret_cast<float*>(sm + R0_TM);
    float* sc = reinterpret_cast<float*>(sm + R0_SC);
    bf16* tb = reinterpret_cast<bf16*>(sm + R0_TB);
    bf16* vt = reinterpret_cast<bf16*>(sm + R0_VT);
    bf16* kwt = reinterpret_cast<bf16*>(sm + R1);
    bf16* kdt = reinterpret_cast<bf16*>(sm + R2);
    float* am = reinterpret_cast<float*>(sm + R3);
    float* cum = reinterpret_cast<float*>(sm + R4);
    float* bet = cum + C;
    float* ecum = bet + C;
    float* erem = ecum + C;

    const int c = blockIdx.x, h = blockIdx.y, NC = gridDim.x;
    const int hk = h / (H / HK);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 15, grp = lane >> 4;
    const size_t rec = (size_t)h * NC + c;

    // 1. cumulative log-decay: lane i of wave 0 sums g_0 .. g_i in index order
    if (wave == 0) {
        const int t = c * C + lane;
        const float gv = t < T ? g[(size_t)t * H + h] : 0.f;
        bet[lane] = t < T ? f32(beta[(size_t)t * H + h]) : 0.f;
        float s = 0.f;
        for (int j = 0; j < C; j++) {
            const float gj = __shfl(gv, j, 64);
            if (j <= lane) s = s + gj;
        }
        cum[lane] = s;
        const float last = __shfl(s, C - 1, 64);
        ecum[lane] = expf(s);
        erem[lane] = expf(last - s);
        if (lane == C - 1) ws.decay[rec] = expf(s);
    }
    __syncthreads();

    // 2. L2 norms (16 lanes x 8 dims per row), TF32 split planes, qd, kw^T, kd^T
    for (int r0 = 0; r0 < C; r0 += PT / 16) {
        const int r = r0 + tid / 16, sub = tid & 15, d0 = sub * 8;
        const int t = c * C + r;
        float kv[8], qv[8];
        if (t < T) {
            unpack8(*reinterpret_cast<const Pack8*>(k + ((size_t)t * HK + hk) * DK + d0), kv);
            unpack8(*reinterpret_cast<const Pack8*>(q + ((size_t)t * HK + hk) * DK + d0), qv);
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) kv[e] = qv[e] = 0.f;
        }
        float ks = 0.f, qs = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            ks += kv[e] * kv[e];
            qs += qv[e] * qv[e];
        }
        ks = lane_sum<16>(ks);
        qs = lane_sum<16>(qs);
        const float kinv = rsqrtf(ks + 1e-6f), qinv = rsqrtf(qs + 1e-6f) * scale;
        float khv[8], klv[8], qhv[8], qlv[8], qdv[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float kx = kv[e] * kinv, qx = qv[e] * qinv;
            const float kt = tf32_rna(kx), qt = tf32_rna(qx);
            khv[e] = round_bf16(kt);
            klv[e] = kt - khv[e];
            qhv[e] = round_bf16(qt);
            qlv[e] = qt - qhv[e];
            qdv[e] = qx * ecum[r];
            kwt[(d0 + e) * TLD + r] = to_bf16(kx * ecum[r]);
            kdt[(d0 + e) * TLD + r] = to_bf16(kx * erem[r]);
        }
        *reinterpret_cast<Pack8*>(khi + r * PLD + d0) = pack8(khv);
        *reinterpret_cast<Pack8*>(klo + r * PLD + d0) = pack8(klv);
        *reinterpret_cast<Pack8*>(qhi + r * PLD + d0) = pack8(qhv);
        *reinterpret_cast<Pack8*>(qlo + r * PLD + d0) = pack8(qlv);
        *reinterpret_cast<Pack8*>(ws.qd + (rec * C + r) * DK + d0) = pack8(qdv);
    }
    __syncthreads();

    // kd^T to the workspace, 16-byte stores
    for (int x = tid; x < DK * C / 8; x += PT) {
        const int d = x / (C / 8), j0 = (x % (C / 8)) * 8;
        *reinterpret_cast<Pack8*>(ws.kdt + (rec * DK + d) * C + j0) = *reinterpret_cast<const Pack8*>(kdt + d * TLD + j0);
    }

    // 3. pair products on the lower 16x16 tiles: e < 10 -> k.k (A), else q.k (P)
    bf16* pbg = ws.pb + rec * C * C;
    for (int e = wave; e < 20; e += PW) {
        const int tile = e % 10;
        const int it = tile < 1 ? 0 : tile < 3 ? 1 : tile < 6 ? 2 : 3;
        const int jt = tile - it * (it + 1) / 2;
        const bf16* ah = e < 10 ? khi : qhi;
        const bf16* al = e < 10 ? klo : qlo;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < DK / 32; s++) {
            const int ao = (16 * it + col) * PLD + 32 * s + 8 * grp;
            const int bo = (16 * jt + col) * PLD + 32 * s + 8 * grp;
            const u32x4 a_h = ld16(ah + ao), a_l = ld16(al + ao);
            const u32x4 b_h = ld16(khi + bo), b_l = ld16(klo + bo);
            acc = mfma16(a_l, b_l, acc);
            acc = mfma16(a_l, b_h, acc);
            acc = mfma16(a_h, b_l, acc);
            acc = mfma16(a_h, b_h, acc);
        }
        const int j = 16 * jt + col;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int i = 16 * it + 4 * grp + r;
            const float dec = j <= i ? expf(cum[i] - cum[j]) : 0.f;
            if (e < 10)
                am[i * FLD + j] = j < i ? bet[i] * acc[r] * dec : 0.f;
            else
                pbg[i * C + j] = j <= i ? to_bf16(acc[r] * dec) : (bf16)0;
        }
    }
    // the six tiles above the diagonal of pb are zero
    for (int x = tid; x < 6 * 256; x += PT) {
        const int tile = x / 256, r = (x % 256) / 16, cc = x % 16;
        const int it = tile < 3 ? 0 : tile < 5 ? 1 : 2;
        const int jt = tile < 3 ? tile + 1 : tile < 5 ? tile - 1 : 3;
        pbg[(16 * it + r) * C + 16 * jt + cc] = 0;
    }
    __syncthreads();

    // 4. T = (I + A)^-1: 16x16 diagonal blocks by forward substitution, then three levels
    for (int x = tid; x < C * FLD; x += PT) tm[x] = 0.f;
    __syncthreads();
    if (tid < C) {
        const int base = 16 * (tid / 16), cc = tid % 16;
        float xs[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            float acc = r == cc ? 1.f : 0.f;
#pragma unroll
            for (int j = 0; j < r; j++) acc = fmaf(-am[(base + r) * FLD + base + j], xs[j], acc);
            xs[r] = acc;
        }
#pragma unroll
        for (int r = 0; r < 16; r++) tm[(base + r) * FLD + base + cc] = xs[r];
    }
    __syncthreads();
    for (int lv = 1; lv < 4; lv++) {
        const int nb = 4 - lv;
        for (int x = tid; x < nb * 256; x += PT) {
            const int bi = lv + x / 256, bj = bi - lv, r = (x % 256) / 16, cc = x % 16;
            float acc = 0.f;
            for (int kb = bj; kb < bi; kb++)
#pragma unroll
                for (int m = 0; m < 16; m++)
                    acc = fmaf(am[(16 * bi + r) * FLD + 16 * kb + m], tm[(16 * kb + m) * FLD + 16 * bj + cc], acc);
            sc[x] = acc;
        }
        __syncthreads();
        for (int x = tid; x < nb * 256; x += PT) {
            const int bi = lv + x / 256, bj = bi - lv, r = (x % 256) / 16, cc = x % 16;
            const float* s0 = sc + (x / 256) * 256 + cc;
            float acc = 0.f;
            for (int m = 0; m <= r; m++) acc = fmaf(tm[(16 * bi + r) * FLD + 16 * bi + m], s0[m * 16], acc);
            tm[(16 * bi + r) * FLD + 16 * bj + cc] = -acc;
        }
        __syncthreads();
    }

    // 5. Tb = bf16(T beta_j); v^T; then u = Tb v and w = Tb kw on the MFMA
    for (int x = tid; x < C * C; x += PT) {
        const int i = x / C, j = x % C;
        tb[i * TLD + j] = to_bf16(tm[i * FLD + j] * bet[j]);
    }
    for (int x = tid; x < C * DK / 8; x += PT) {
        const int j = x / (DK / 8), d0 = (x % (DK / 8)) * 8;
        const int t = c * C + j;
        Pack8 p = Pack8{{0u, 0u, 0u, 0u}};
        if (t < T) p = *reinterpret_cast<const Pack8*>(v + ((size_t)t * H + h) * DK + d0);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            vt[(d0 + 2 * e) * TLD + j] = (bf16)(p.w[e] & 0xffffu);
            vt[(d0 + 2 * e + 1) * TLD + j] = (bf16)(p.w[e] >> 16);
        }
    }
    __syncthreads();
    for (int e = wave; e < 64; e += PW) {
        const bool is_u = e < 32;
        const int it = (e % 32) / 8, dt = e % 8;
        const bf16* bsrc = is_u ? vt : kwt;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s <= it / 2; s++) {  // T is lower triangular
            const u32x4 a = ld16(tb + (16 * it + col) * TLD + 32 * s + 8 * grp);
            const u32x4 b = ld16(bsrc + (16 * dt + col) * TLD + 32 * s + 8 * grp);
            acc = mfma16(a, b, acc);
        }
        bf16* dst = (is_u ? ws.u : ws.w) + rec * C * DK + 16 * dt + col;
#pragma unroll
        for (int r = 0; r < 4; r++) dst[(16 * it + 4 * grp + r) * DK] = to_bf16(acc[r]);
    }
}

// ------------------------------------------------------------------ gdn_scan

constexpr int ST = 256;   // threads, 4 waves
constexpr int BV = 16;    // value columns per block
constexpr int NS = DK / BV;
constexpr int SLD = DK + 8;  // bf16 stride of Sb^T [16][128]
constexpr int VLD = C + 8;   // bf16 stride of v_new^T [16][64]

struct ChunkOps {
    u32x4 w[4];    // w rows 16 wave + col, dims 32 s + 8 grp
    u32x4 qd[4];   // qd rows, same layout
    u32x4 pb[2];   // pb rows, tokens 32 s + 8 grp
    u32x4 kd[2][2];// kd^T rows 32 wave + 16 i + col, tokens 32 s + 8 grp
    bf16 u[4];     // u rows 16 wave + 4 grp + r, column v0 + col
    float decay;
};

__device__ __forceinline__ void load_chunk(ChunkOps& op, const Work& ws, size_t rec, int wave, int col, int grp,
                                           int v0) {
    const bf16* wr = ws.w + (rec * C + 16 * wave + col) * DK + 8 * grp;
    const bf16* qr = ws.qd + (rec * C + 16 * wave + col) * DK + 8 * grp;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        op.w[s] = ld16(wr + 32 * s);
        op.qd[s] = ld16(qr + 32 * s);
    }
    const bf16* pr = ws.pb + (rec * C + 16 * wave + col) * C + 8 * grp;
    op.pb[0] = ld16(pr);
    op.pb[1] = ld16(pr + 32);
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const bf16* kr = ws.kdt + (rec * DK + 32 * wave + 16 * i + col) * C + 8 * grp;
        op.kd[i][0] = ld16(kr);
        op.kd[i][1] = ld16(kr + 32);
    }
    const bf16* ur = ws.u + (rec * C + 16 * wave + 4 * grp) * DK + v0 + col;
#pragma unroll
    for (int r = 0; r < 4; r++) op.u[r] = ur[r * DK];
    op.decay = ws.decay[rec];
}

__global__ void __launch_bounds__(ST)
    gdn_scan(Work ws, bf16* __restrict__ o, int T, int H, int NC, const float* __restrict__ s_in,
             float* __restrict__ s_out) {
    __shared__ __align__(16) bf16 sbt[BV * SLD];
    __shared__ __align__(16) bf16 vnt[BV * VLD];
    const int h = blockIdx.x % H, slice = blockIdx.x / H, v0 = slice * BV;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 15, grp = lane >> 4;

    // state rows 32 wave + 16 i + 4 grp + r, column v0 + col
    f32x4 st[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
#pragma unroll
        for (int r = 0; r < 4; r++)
            st[i][r] = s_in ? s_in[((size_t)h * DK + 32 * wave + 16 * i + 4 * grp + r) * DK + v0 + col] : 0.f;
    }

    ChunkOps cur, nxt;
    load_chunk(cur, ws, (size_t)h * NC, wave, col, grp, v0);
    for (int c = 0; c < NC; c++) {
        if (c + 1 < NC) load_chunk(nxt, ws, (size_t)h * NC + c + 1, wave, col, grp, v0);
        // 1. bf16(S)^T to LDS
#pragma unroll
        for (int i = 0; i < 2; i++)
            *reinterpret_cast<u32x2*>(sbt + col * SLD + 32 * wave + 16 * i + 4 * grp) =
                u32x2{pack2(st[i][0], st[i][1]), pack2(st[i][2], st[i][3])};
        __syncthreads();
        // 2. v_new = bf16(u - w Sb) and qd Sb for rows 16 wave ..
        f32x4 ws_acc = {0.f, 0.f, 0.f, 0.f}, oacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const u32x4 b = ld16(sbt + col * SLD + 32 * s + 8 * grp);
            ws_acc = mfma16(cur.w[s], b, ws_acc);
            oacc = mfma16(cur.qd[s], b, oacc);
        }
        float vn[4];
#pragma unroll
        for (int r = 0; r < 4; r++) vn[r] = f32(cur.u[r]) - ws_acc[r];
        *reinterpret_cast<u32x2*>(vnt + col * VLD + 16 * wave + 4 * grp) = u32x2{pack2(vn[0], vn[1]), pack2(vn[2], vn[3])};
        __syncthreads();
        // 3. o = qd Sb + pb v_new
#pragma unroll
        for (int s = 0; s < 2; s++) oacc = mfma16(cur.pb[s], ld16(vnt + col * VLD + 32 * s + 8 * grp), oacc);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int t = c * C + 16 * wave + 4 * grp + r;
            if (t < T) o[((size_t)t * H + h) * DK + v0 + col] = to_bf16(oacc[r]);
        }
        // 4. S = S decay + kd^T v_new
#pragma unroll
        for (int i = 0; i < 2; i++) {
            st[i] *= cur.decay;
#pragma unroll
            for (int s = 0; s < 2; s++) st[i] = mfma16(cur.kd[i][s], ld16(vnt + col * VLD + 32 * s + 8 * grp), st[i]);
        }
        cur = nxt;
    }
    if (s_out) {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int r = 0; r < 4; r++)
                s_out[((size_t)h * DK + 32 * wave + 16 * i + 4 * grp + r) * DK + v0 + col] = st[i][r];
    }
}

// T == 0: s_out = s_in, or zero (a kernel rather than a memset/memcpy node, so that a
// captured graph re-executes it).
__global__ void __launch_bounds__(256) state_pass(const float4* __restrict__ s_in, float4* __restrict__ s_out, size_t n4) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n4) s_out[i] = s_in ? s_in[i] : float4{0.f, 0.f, 0.f, 0.f};
}

int gdn_run(const void* q, const void* k, const void* v, const float* g, const void* beta, void* o, float* workspace,
            int T, int H, int HK, float scale, const void* s_in, void* s_out, void* stream) {
    if (T < 0 || H <= 0 || HK <= 0 || H % HK != 0) return hipErrorInvalidValue;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const float* si = static_cast<const float*>(s_in);
    float* so = static_cast<float*>(s_out);
    if (T == 0) {
        if (so == nullptr) return hipSuccess;
        const size_t n4 = (size_t)H * DK * DK / 4;
        state_pass<<<cdiv(n4, 256), 256, 0, st>>>(reinterpret_cast<const float4*>(si), reinterpret_cast<float4*>(so),
                                                  n4);
        return hipGetLastError();
    }
    if (((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
          reinterpret_cast<uintptr_t>(workspace)) & 15) != 0)
        return hipErrorInvalidValue;
    static const hipError_t configured = hipFuncSetAttribute(reinterpret_cast<const void*>(gdn_prep),
                                                             hipFuncAttributeMaxDynamicSharedMemorySize, PREP_SMEM);
    if (configured != hipSuccess) return configured;
    const int NC = (T + C - 1) / C;
    const Work ws = split(workspace, T, H);
    gdn_prep<<<dim3(NC, H), PT, PREP_SMEM, st>>>(static_cast<const bf16*>(q), static_cast<const bf16*>(k),
                                                 static_cast<const bf16*>(v), g, static_cast<const bf16*>(beta), ws, T,
                                                 H, HK, scale);
    gdn_scan<<<H * NS, ST, 0, st>>>(ws, static_cast<bf16*>(o), T, H, NC, si, so);
    return hipGetLastError();
}

}  // namespace
}  // namespace q35

using namespace q35;

extern "C" size_t cs1_gdn_workspace_floats(int T, int H) {
    if (T < 0 || H < 0) return 0;
    return (Layout(T, H).total + 3) / 4;
}

extern "C" int cs1_gdn_prefill(const void* q, const void* k, const void* v, const float* g, const void* beta, void* o,
                               float* workspace, int T, int H, int HK, float scale, void* stream) {
    return gdn_run(q, k, v, g, beta, o, workspace, T, H, HK, scale, nullptr, nullptr, stream);
}

extern "C" int cs1_gdn_prefill_x(const void* q, const void* k, const void* v, const float* g, const void* beta,
                                 void* o, float* workspace, int T, int H, int HK, float scale, const void* s_in,
                                 void* s_out, void* stream) {
    return gdn_run(q, k, v, g, beta, o, workspace, T, H, HK, scale, s_in, s_out, stream);
}
