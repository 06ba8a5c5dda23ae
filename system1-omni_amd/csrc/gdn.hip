// Chunked Gated DeltaNet prefill (chunk 64, dk = dv = 128, batch 1) on gfx950.
//
// Arithmetic of record: transformers' torch_chunk_gated_delta_rule (modeling_qwen3_5.py
// 249-328) with the rounding points of the reference CUDA kernel (gdn_prefill.cu):
//   per chunk and head:  cum = sequential float32 cumsum of g, decay = e^cum_last;
//     q^ = q rsqrt(|q|^2 + 1e-6) scale, k^ = k rsqrt(|k|^2 + 1e-6)  (float32);
//     A_ij = (beta_i (k^_i . k^_j)) e^(cum_i - cum_j) for j < i, P_ij = (q^_i . k^_j) e^(...)
//       for j <= i, the pair products on TF32-rounded operands with float32 sums;
//     T = (I + A)^-1 (float32, 16x16 blocks); tb = bf16(T_ij beta_j);
//     u = bf16(tb v), w = bf16(tb bf16(k^ e^cum)), qd = bf16(q^ e^cum),
//     kd = bf16(k^ e^(cum_last - cum)), pb = bf16(P);
//   scan over chunks:  Sb = bf16(S); v_new = bf16(u - w Sb); o = bf16(qd Sb + pb v_new);
//     S = S decay + kd^T v_new (float32).
//
// MI355X design.  Everything is organised around the operand layouts of the wave64 MFMA
// v_mfma_f32_16x16x32_bf16 (lane l: A row / B column l % 16, k = 8 (l / 16) + e):
//
//   * One k ordering everywhere: within each 32-wide k step, lane group g holds
//     k = {4g .. 4g+3, 16+4g .. 16+4g+3}.  With that ordering the accumulators of two
//     16-row tiles (rows 4g + r of each) are, lane for lane, the B (or A) operand of the
//     next MFMA, so products chain without moving data between lanes.
//   * gdn_prep, grid (chunk, head), 4 waves, ~50 KB LDS (three blocks per CU); gdn_prep8, the
//     same arithmetic on 8 waves, when every item of the launch has a CU of its own:
//       - TF32 pair products on the bf16 MFMA: each TF32 operand is split exactly into
//         hi = rne_bf16(x) and lo = x - hi (TF32 has 11 significant bits), and the four
//         products hi.hi + hi.lo + lo.hi + lo.lo reproduce the TF32 product exactly;
//       - token-major inputs are transposed on the MFMA (a product with a 0/1 selection
//         matrix, exact in bf16), not through LDS;
//       - the triangular inverse: diagonal 16x16 blocks by forward substitution (the
//         reference order), off-diagonal levels T_ij = -T_ii sum_k A_ik T_kj on the
//         float32 MFMA v_mfma_f32_16x16x4_f32;
//       - every scan operand is written to the workspace in the exact per-lane order the
//         scan's MFMA consumes it (1 KB per wave per store, fully coalesced).
//   * gdn_scan, grid (head x 8 slices of 16 value columns, or x 4 slices of 32 when that
//     needs fewer rounds of blocks), 4 chain waves + 4 output waves (16-column slices: two
//     sets of 4 output waves taking alternate chunks).  The float32 state
//     slice 128 x 16 (per half) lives in MFMA accumulators; each chunk streams its operand
//     fragments from HBM/L2 straight into registers (three chunks ahead) and exchanges only
//     bf16(S) and v_new through LDS.  The output o = qd Sb + pb v_new is produced in the
//     same pass, so per-chunk states and v_new never go to memory.  The slices of one head
//     run on the same XCD (block = slice * H + head) and share its L2.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <mutex>

#include "common.h"

namespace q35 {
namespace {

constexpr int C = 64;    // chunk length
constexpr int DK = 128;  // key / value head dim
constexpr uint32_t BF16_ONE = 0x3f80u;

// ------------------------------------------------------------ workspace layout

// Per (head, chunk) record rec = head * NC + chunk; a "fragment" is 64 lanes x 8 bf16.
//   w   [4 row blocks][4 dim steps]   fragments: lane = (row 16 it + l%16, dims 32 s + perm)
//   qd  [4][4]                        same layout
//   kd  [8 dim blocks][2 token steps] fragments: lane = (dim 16 b + l%16, tokens 32 s + perm)
//   pb  [4 row blocks][2 token steps] fragments: lane = (row, tokens 32 s + perm), zero above
//   u   [4 row blocks][8 dim blocks]  accumulator tiles: lane = (dim 16 dt + l%16,
//                                     rows 16 it + 4 (l/16) + r), 4 bf16 per lane
//   decay float
struct Work {
    u32x4* w;
    u32x4* qd;
    u32x4* kd;
    u32x4* pb;
    u32x2* u;
    float* decay;
};

constexpr size_t FRAG = 64;  // lanes per fragment (u32x4 or u32x2 each)

struct Layout {
    size_t w, qd, kd, pb, u, decay, total;
    // NC chunks (records per head)
    Layout(size_t NC, int H) {
        const size_t n = (size_t)H * NC;
        size_t at = 0;
        auto take = [&](size_t bytes) {
            const size_t off = at;
            at = (at + bytes + 255) / 256 * 256;
            return off;
        };
        w = take(n * 16 * 1024);
        qd = take(n * 16 * 1024);
        kd = take(n * 16 * 1024);
        pb = take(n * 8 * 1024);
        u = take(n * 32 * 512);
        decay = take(n * 4);
        total = at;
    }
};

// packed sequences of one launch (up to GSEQS_MAX): sequence s is token rows tok[s] ..
// tok[s + 1] - 1 and workspace chunks chk[s] .. chk[s + 1] - 1; n == 0: one sequence
constexpr int GSEQS_MAX = 64;
struct GSeqs {
    int n;
    int tok[GSEQS_MAX + 1], chk[GSEQS_MAX + 1];
};

// The per-token gates of a launch: either precomputed (g float32, beta bf16, [T, H]) or, for
// the gated entry points, the raw projections b and a (bf16 rows of stride ld, head h at
// column h) with the per-head A_log and dt_bias, from which the prep computes beta and g with
// the arithmetic of cs1_gdn_gates (gate_values), so both routes give the same bits.
struct Gates {
    const float* g;
    const bf16* beta;
    const bf16* b;
    const bf16* a;
    int ld;
    const bf16* A_log;
    const bf16* dt_bias;
    // the gates of token rows from r0 on
    __host__ __device__ Gates from_row(size_t r0, int H) const {
        Gates x = *this;
        if (b) {
            x.b += r0 * ld;
            x.a += r0 * ld;
        } else {
            x.g += r0 * H;
            x.beta += r0 * H;
        }
        return x;
    }
};

Work split(float* workspace, size_t NC, int H) {
    const Layout l(NC, H);
    unsigned char* b = reinterpret_cast<unsigned char*>(workspace);
    return Work{reinterpret_cast<u32x4*>(b + l.w),  reinterpret_cast<u32x4*>(b + l.qd),
                reinterpret_cast<u32x4*>(b + l.kd), reinterpret_cast<u32x4*>(b + l.pb),
                reinterpret_cast<u32x2*>(b + l.u),  reinterpret_cast<float*>(b + l.decay)};
}

// cvt.rna.tf32.f32 for finite x: 10 explicit mantissa bits, round half away from zero (the
// operands here are L2-normalised rows, always finite).
__device__ __forceinline__ float tf32_rna(float x) {
    return __uint_as_float((__float_as_uint(x) + 0x1000u) & 0xffffe000u);
}

// The exact two-term bf16 split of eight TF32-rounded values: hi = rne_bf16(t) (a TF32 value
// has 11 significant bits, so lo = t - hi is exact in bf16), both packed in operand order. The
// packed hi comes straight from the pairwise conversion and is unpacked once for the
// subtraction.
__device__ __forceinline__ void split_tf32(const float t[8], u32x4& hi, u32x4& lo) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t h = pack2(t[2 * i], t[2 * i + 1]);
        hi[i] = h;
        lo[i] = pack2(t[2 * i] - lo_f32(h), t[2 * i + 1] - hi_f32(h));
    }
}

// 8 bf16 of a row in the permuted k order of lane group g: k = 32 s + {4g..4g+3, 16+4g..}
__device__ __forceinline__ u32x4 load_perm(const bf16* row, int s, int g) {
    const u32x2 a = *reinterpret_cast<const u32x2*>(row + 32 * s + 4 * g);
    const u32x2 b = *reinterpret_cast<const u32x2*>(row + 32 * s + 16 + 4 * g);
    return u32x4{a[0], a[1], b[0], b[1]};
}

__device__ __forceinline__ void unpack8v(const u32x4& p, float out[8]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        out[2 * i] = lo_f32(p[i]);
        out[2 * i + 1] = hi_f32(p[i]);
    }
}

__device__ __forceinline__ u32x4 pack8v(const float x[8]) {
    return u32x4{pack2(x[0], x[1]), pack2(x[2], x[3]), pack2(x[4], x[5]), pack2(x[6], x[7])};
}

// two accumulator tiles (rows 4g + r of tile 0 and of tile 1) as one operand in perm order
__device__ __forceinline__ u32x4 pack_pair(const f32x4& t0, const f32x4& t1) {
    return u32x4{pack2(t0[0], t0[1]), pack2(t0[2], t0[3]), pack2(t1[0], t1[1]), pack2(t1[2], t1[3])};
}

// B operand selecting k = 16 half + (l % 16) in perm order: D = A B copies 16 columns of A.
__device__ __forceinline__ u32x4 select_op(int half, int col, int grp) {
    uint32_t v[4] = {0u, 0u, 0u, 0u};
    const int d = col - 4 * grp;  // position within the lane group's run of four
    if (d >= 0 && d < 4) {
        const int e = d + 4 * half;
        v[e >> 1] = BF16_ONE << (16 * (e & 1));
    }
    return u32x4{v[0], v[1], v[2], v[3]};
}

__device__ __forceinline__ int tid_of_block() { return threadIdx.x; }

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------ gdn_prep

constexpr int PT = 256;          // threads, 4 waves
constexpr int FLD = C + 1;       // float stride of A and T [64][65]
constexpr int TLD = C + 8;       // bf16 stride of Tb [64][72]

// LDS map (bytes). Region 0: split planes of k^ in fragment order during the pair
// products; afterwards T (float), Tb (bf16) and a per-wave 16x16 float scratch.
constexpr int R0 = 0;
constexpr int PLANE = 4 * 4 * 1024;                // [4 blocks][4 steps] fragments
constexpr int R0_TM = 0;
constexpr int R0_TB = R0_TM + C * FLD * 4;         // 16640
constexpr int R0_SC = R0_TB + C * TLD * 2;         // 25856
constexpr int R1 = R0 + 2 * PLANE;                 // A float [64][65]; then raw k fragments
static_assert(C * FLD * 4 >= 16 * (int)FRAG * 16, "region 1 holds the 16 raw k fragments");
static_assert(C * FLD * 4 >= C * DK * 2, "region 1 holds the staged v rows of gdn_prep");
constexpr int R2 = R1 + C * FLD * 4;               // cum, beta, e^cum, e^(last-cum), k inverse norm
constexpr int PREP_SMEM = R2 + 5 * C * 4;
static_assert(R0_SC + 4 * 256 * 4 <= R1, "region 0 overlay fits");

#ifdef Q35_PHASE_TIMING
// Development aid: per-phase shader-clock ticks summed over all blocks.
__device__ unsigned long long q35_phase_ticks[16];
#define Q35_PHASE_START() uint64_t q35_t0 = __builtin_amdgcn_s_memtime()
#define Q35_PHASE(i)                                                             \
    do {                                                                         \
        const uint64_t q35_t1 = __builtin_amdgcn_s_memtime();                    \
        if (threadIdx.x == 0) atomicAdd(&q35_phase_ticks[i], q35_t1 - q35_t0);   \
        q35_t0 = q35_t1;                                                         \
    } while (0)
// per wave of gdn_prep8: clocks from the block's start to point i, summed over blocks
__device__ unsigned long long q35_wave_ticks[64];
#define Q35_WSTART() uint64_t q35_w0 = __builtin_amdgcn_s_memtime(), q35_ws[8] = {0, 0, 0, 0, 0, 0, 0, 0}
#define Q35_WSTAMP(i) q35_ws[i] = __builtin_amdgcn_s_memtime() - q35_w0
#define Q35_WFLUSH()                                                                             \
    do {                                                                                         \
        if ((threadIdx.x & 63) == 0)                                                             \
            for (int q35_i = 0; q35_i < 8; q35_i++) atomicAdd(&q35_wave_ticks[(threadIdx.x >> 6) * 8 + q35_i], q35_ws[q35_i]); \
    } while (0)
#define Q35_LPHASE_START() uint64_t q35_t0 = __builtin_amdgcn_s_memtime(), q35_acc[5] = {0, 0, 0, 0, 0}
#define Q35_LPHASE(i)                                          \
    do {                                                       \
        const uint64_t q35_t1 = __builtin_amdgcn_s_memtime();  \
        q35_acc[(i) - 8] += q35_t1 - q35_t0;                   \
        q35_t0 = q35_t1;                                       \
    } while (0)
#define Q35_LPHASE_FLUSH()                                                                             \
    do {                                                                                               \
        if (threadIdx.x == 0)                                                                          \
            for (int q35_i = 0; q35_i < 5; q35_i++) atomicAdd(&q35_phase_ticks[8 + q35_i], q35_acc[q35_i]); \
    } while (0)
#else
#define Q35_PHASE_START() (void)0
#define Q35_WSTART() (void)0
#define Q35_WSTAMP(i) (void)0
#define Q35_WFLUSH() (void)0
#define Q35_PHASE(i) (void)0
#define Q35_LPHASE_START() (void)0
#define Q35_LPHASE(i) (void)0
#define Q35_LPHASE_FLUSH() (void)0
#endif

// Off-diagonal level LV of the blocked inverse for the wave owning row block bi >= LV:
// T_{bi, bi - LV} = -T_ii (sum_k A_ik T_kj), k over the LV blocks bi - LV .. bi - 1, on the f32
// MFMA (A operand: lane = row l%16, k = l/16; B operand: lane = column l%16, k = l/16). The
// level's trip counts are constants, so every operand is read from LDS ahead of the MFMA chain
// (the products and their order are those of a loop over the blocks). The partial product
// passes through the wave's own scratch, whose writes precede its reads in the wave's LDS order.
// The block goes to T (float) and to Tb = bf16(T_ij beta_j), the scan operand's factor.
template <int LV>
__device__ __forceinline__ void inverse_level(int bi, const float* am, float* tm, bf16* tb, const float* bet,
                                              float* scr, int col, int grp) {
    const int bj = bi - LV;
    float a[4 * LV], t[4 * LV], tii[4];
#pragma unroll
    for (int m = 0; m < LV; m++)
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            const int kb = bj + m;
            a[4 * m + kk] = am[(16 * bi + col) * FLD + 16 * kb + 4 * kk + grp];
            t[4 * m + kk] = tm[(16 * kb + 4 * kk + grp) * FLD + 16 * bj + col];
        }
#pragma unroll
    for (int kk = 0; kk < 4; kk++) tii[kk] = tm[(16 * bi + col) * FLD + 16 * bi + 4 * kk + grp];
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int x = 0; x < 4 * LV; x++) acc = mfma_f32(a[x], t[x], acc);
#pragma unroll
    for (int r = 0; r < 4; r++) scr[(4 * grp + r) * 16 + col] = acc[r];
    acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; kk++) acc = mfma_f32(tii[kk], scr[(4 * kk + grp) * 16 + col], acc);
    const float bj_beta = bet[16 * bj + col];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        tm[(16 * bi + 4 * grp + r) * FLD + 16 * bj + col] = -acc[r];
        tb[(16 * bi + 4 * grp + r) * TLD + 16 * bj + col] = to_bf16(-acc[r] * bj_beta);
    }
}

constexpr int STG_ROW = DK * 2;  // bytes of a staged input row

// A buffer load of 16 bytes per lane straight into LDS: lane l's chunk lands at lds + 16 l.
// (A __device__ function: the builtin used inside a kernel's lambda kept the host pass from
// emitting the kernel's launch stub.)
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, unsigned char* lds, int voff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

// Rows rl0 .. rl0 + 15 of a chunk (token t0 + rl at base + t ld, 256 bytes; rows past T read
// row T - 1) into the staging area stg as whole cache lines: 16-byte chunk c of row rl sits at
// chunk position c ^ (rl % 16), so the permuted reads of staged_perm hit distinct banks.
__device__ __forceinline__ void stage_rows(const bf16* base, int ld, int t0, int rl0, int T, unsigned char* stg,
                                           int lane) {
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(base), (short)0, 0x7fffffff, 0x00020000);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int rl = rl0 + 4 * i + (lane >> 4);
        const int c = (lane & 15) ^ (rl & 15);
        const int t = min(t0 + rl, T - 1);
        lds_load16(rs, stg + (rl0 + 4 * i) * STG_ROW, t * ld * 2 + 16 * c);
    }
}

// load_perm's 8 values of staged row rl: dims 32 s + 4 g .. + 3 and 32 s + 16 + 4 g .. + 3
__device__ __forceinline__ u32x4 staged_perm(const unsigned char* stg, int rl, int s, int g) {
    const unsigned char* rp = stg + rl * STG_ROW + 8 * (g & 1);
    const u32x2 a = *reinterpret_cast<const u32x2*>(rp + (((4 * s + (g >> 1)) ^ (rl & 15)) << 4));
    const u32x2 b = *reinterpret_cast<const u32x2*>(rp + (((4 * s + 2 + (g >> 1)) ^ (rl & 15)) << 4));
    return u32x4{a[0], a[1], b[0], b[1]};
}

template <bool GATED>
__global__ void __launch_bounds__(PT)
    gdn_prep(const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v, Gates gt, Work ws,
             int T, int H, int HK, float scale, const GSeqs gs) {
    extern __shared__ __align__(16) unsigned char sm[];
    u32x4* khi_pl = reinterpret_cast<u32x4*>(sm + R0);
    u32x4* klo_pl = reinterpret_cast<u32x4*>(sm + R0 + PLANE);
    float* tm = reinterpret_cast<float*>(sm + R0_TM);
    bf16* tb = reinterpret_cast<bf16*>(sm + R0_TB);
    float* am = reinterpret_cast<float*>(sm + R1);
    float* cum = reinterpret_cast<float*>(sm + R2);
    float* bet = cum + C;
    float* ecum = bet + C;
    float* erem = ecum + C;
    float* kinv_s = erem + C;

    const int c = blockIdx.x, h = blockIdx.y, NC = gridDim.x;
    int cl = c;  // chunk within its sequence
    if (gs.n > 0) {
        // packed sequences: find this chunk's sequence (a scalar scan) and address it alone
        int sq = 0;
        while (sq + 1 < gs.n && c >= gs.chk[sq + 1]) sq++;
        cl = c - gs.chk[sq];
        const int r0 = gs.tok[sq];
        T = gs.tok[sq + 1] - r0;
        q += (size_t)r0 * HK * DK;
        k += (size_t)r0 * HK * DK;
        v += (size_t)r0 * H * DK;
        gt = gt.from_row(r0, H);
    }
    const int hk = h / (H / HK);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 15, grp = lane >> 4;
    float* scr = reinterpret_cast<float*>(sm + R0_SC) + wave * 256;
    const size_t rec = (size_t)h * NC + c;
    const int t0 = cl * C;
    Q35_PHASE_START();

    // 0. loads: own k rows (block `wave`), q rows (block 3 - wave), and the v columns of dim
    //    step `wave` for all 64 tokens; gates for all tokens (lane = token). The k columns
    //    step 6 needs are the other waves' raw k rows, passed through LDS there rather than
    //    loaded a second time.
    //    Every load is unconditional (rows past T read row T - 1) and the rows past T are zeroed
    //    at their first use, so no load waits for another: the gates go first, and memory waits
    //    being in issue order, the decay scan below waits only for them while the rows are in
    //    flight. The k and q rows move to LDS as whole cache lines (a fragment's pieces are
    //    half lines 4 KB apart), into the two 4 KB slices of the k planes that this wave alone
    //    writes in step 2, after it has read them back in fragment order.
    //    Wave 0 alone loads the gates (by hand, and waits for them by hand: as ordinary loads
    //    under a branch the compiler placed them, or the wait for them, after the row
    //    transfers) and computes the decay for the block.
    const int tl = t0 + lane;
    float g_raw = 0.f;
    uint32_t b_bits = 0, a_bits = 0, al_bits = 0, dt_bits = 0;
    if (wave == 0) {
        const int tlc = min(tl, T - 1);
        if constexpr (GATED) {
            asm volatile("global_load_ushort %0, %1, off" : "=v"(b_bits) : "v"(gt.b + (size_t)tlc * gt.ld + h));
            asm volatile("global_load_ushort %0, %1, off" : "=v"(a_bits) : "v"(gt.a + (size_t)tlc * gt.ld + h));
            asm volatile("global_load_ushort %0, %1, off" : "=v"(al_bits) : "v"(gt.A_log + h));
            asm volatile("global_load_ushort %0, %1, off" : "=v"(dt_bits) : "v"(gt.dt_bias + h));
        } else {
            asm volatile("global_load_dword %0, %1, off" : "=v"(g_raw) : "v"(gt.g + (size_t)tlc * H + h));
            asm volatile("global_load_ushort %0, %1, off" : "=v"(b_bits) : "v"(gt.beta + (size_t)tlc * H + h));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    const int qb = 3 - wave;
    const int krow = 16 * wave + col, qrow = 16 * qb + col;
    unsigned char* const stg_k = sm + R0;                             // row r at r * 256
    unsigned char* const stg_q = sm + R0 + PLANE + (wave - qb) * 4096;  // rows of block qb
    stage_rows(k + (size_t)hk * DK, HK * DK, t0, 16 * wave, T, stg_k, lane);
    stage_rows(q + (size_t)hk * DK, HK * DK, t0, 16 * qb, T, stg_q, lane);
    // the v rows 16 wave .. + 15 go to region 1 (A is written there from step 3 on); each wave
    // reads its dim step of all 64 rows after the next block barrier
    stage_rows(v + (size_t)h * DK, H * DK, t0, 16 * wave, T, sm + R1, lane);
    u32x4 kraw[4], qraw[4], vc[4];
    __builtin_amdgcn_sched_barrier(0);

    // 1. cumulative log-decay, in index order (wave 0, lane = token), published through LDS
    //    at the barrier below
    if (wave == 0) {
        float gv, bv;
        if constexpr (GATED) {
            asm volatile("s_waitcnt vmcnt(12)" : "+v"(b_bits), "+v"(a_bits), "+v"(al_bits), "+v"(dt_bits));  // the 12 row transfers may be in flight
            bf16 be;
            float gg;
            gate_values(f32((bf16)b_bits), f32((bf16)a_bits), -expf(f32((bf16)al_bits)), f32((bf16)dt_bits), be, gg);
            gv = tl < T ? gg : 0.f;
            bv = tl < T ? f32(be) : 0.f;
        } else {
            asm volatile("s_waitcnt vmcnt(12)" : "+v"(g_raw), "+v"(b_bits));
            gv = tl < T ? g_raw : 0.f;
            bv = tl < T ? __uint_as_float(b_bits << 16) : 0.f;
        }
        float cs = 0.f;
        for (int j = 0; j < C; j++) {
            const float gj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gv), j));
            if (j <= lane) cs = cs + gj;
        }
        const float last = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cs), C - 1));
        cum[lane] = cs;
        bet[lane] = bv;
        ecum[lane] = expf(cs);
        erem[lane] = expf(last - cs);
    }
    // the staged rows; rows past T are zero from here on
    wait_vm_all();
#pragma unroll
    for (int s = 0; s < 4; s++) {
        kraw[s] = staged_perm(stg_k, krow, s, grp);
        qraw[s] = staged_perm(stg_q, qrow, s, grp);
    }
    __syncthreads();
#pragma unroll
    for (int tb_ = 0; tb_ < 4; tb_++) vc[tb_] = staged_perm(sm + R1, 16 * tb_ + col, wave, grp);
    const u32x4 zero4 = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int s = 0; s < 4; s++) {
        if (t0 + krow >= T) kraw[s] = zero4;
        if (t0 + qrow >= T) qraw[s] = zero4;
    }
#pragma unroll
    for (int tb_ = 0; tb_ < 4; tb_++)
        if (t0 + 16 * tb_ + col >= T) vc[tb_] = zero4;
    Q35_PHASE(1);

    // 2. L2 norms (row sums over the 4 lane groups), TF32 split of k^, q^ and qd
    float ks = 0.f, qs = 0.f;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        float kf[8], qf[8];
        unpack8v(kraw[s], kf);
        unpack8v(qraw[s], qf);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            ks += kf[e] * kf[e];
            qs += qf[e] * qf[e];
        }
    }
    ks += __shfl_xor(ks, 16, 64);
    ks += __shfl_xor(ks, 32, 64);
    qs += __shfl_xor(qs, 16, 64);
    qs += __shfl_xor(qs, 32, 64);
    const float kinv = rsqrtf(ks + 1e-6f), qinv = rsqrtf(qs + 1e-6f) * scale;
    if (grp == 0) kinv_s[krow] = kinv;
    const float ecq = ecum[qrow];
    u32x4 khi[4], klo[4], qhi[4], qlo[4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        float kt_[8], qt_[8], qd_[8], kf[8], qf[8];
        unpack8v(kraw[s], kf);
        unpack8v(qraw[s], qf);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            kt_[e] = tf32_rna(kf[e] * kinv);
            const float qx = qf[e] * qinv;
            qt_[e] = tf32_rna(qx);
            qd_[e] = qx * ecq;
        }
        split_tf32(kt_, khi[s], klo[s]);
        split_tf32(qt_, qhi[s], qlo[s]);
        khi_pl[(wave * 4 + s) * FRAG + lane] = khi[s];
        klo_pl[(wave * 4 + s) * FRAG + lane] = klo[s];
        ws.qd[(rec * 16 + qb * 4 + s) * FRAG + lane] = pack8v(qd_);
    }
    __syncthreads();
    Q35_PHASE(2);

    // 3. pair products. A tiles (wave, jt <= wave): rows i of this wave's k^, columns j.
    //    The decay and beta of the lane's rows are read once, as vectors, and each tile's decay
    //    factors are formed for every element and masked by a select: per-element reads inside
    //    the j <= i branches each waited for the LDS.
    const f32x4 cum_i = *reinterpret_cast<const f32x4*>(cum + 16 * wave + 4 * grp);
    const f32x4 bet_i = *reinterpret_cast<const f32x4*>(bet + 16 * wave + 4 * grp);
#pragma unroll
    for (int jt = 0; jt < 4; jt++) {
        if (jt > wave) continue;
        const float cum_j = cum[16 * jt + col];
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const u32x4 bh = khi_pl[(jt * 4 + s) * FRAG + lane], bl = klo_pl[(jt * 4 + s) * FRAG + lane];
            acc = mfma16(klo[s], bl, acc);
            acc = mfma16(klo[s], bh, acc);
            acc = mfma16(khi[s], bl, acc);
            acc = mfma16(khi[s], bh, acc);
        }
        const int j = 16 * jt + col;
        float dec[4];
#pragma unroll
        for (int r = 0; r < 4; r++) dec[r] = expf(cum_i[r] - cum_j);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int i = 16 * wave + 4 * grp + r;
            am[i * FLD + j] = j < i ? bet_i[r] * acc[r] * dec[r] : 0.f;
        }
    }
    // P^T tiles (jt <= qb, qb): rows j of k^ (planes), columns i of this wave's q^ rows.
    // pb fragment (qb, s) = tiles 2s and 2s + 1, lane for lane.
    {
        f32x4 pt[4];
        const float cum_q = cum[qrow];
#pragma unroll
        for (int jt = 0; jt < 4; jt++) {
            pt[jt] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (jt > qb) continue;
            const f32x4 cum_j = *reinterpret_cast<const f32x4*>(cum + 16 * jt + 4 * grp);
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const u32x4 ah = khi_pl[(jt * 4 + s) * FRAG + lane], al = klo_pl[(jt * 4 + s) * FRAG + lane];
                pt[jt] = mfma16(al, qlo[s], pt[jt]);
                pt[jt] = mfma16(al, qhi[s], pt[jt]);
                pt[jt] = mfma16(ah, qlo[s], pt[jt]);
                pt[jt] = mfma16(ah, qhi[s], pt[jt]);
            }
            const int i = qrow;
            float dec[4];
#pragma unroll
            for (int r = 0; r < 4; r++) dec[r] = expf(cum_q - cum_j[r]);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int j = 16 * jt + 4 * grp + r;
                pt[jt][r] = j <= i ? round_bf16(pt[jt][r] * dec[r]) : 0.f;
            }
        }
        ws.pb[(rec * 8 + qb * 2 + 0) * FRAG + lane] = pack_pair(pt[0], pt[1]);
        // fragment (qb, 1) of row blocks 0 and 1 lies above the diagonal: all zero, neither
        // written nor read
        if (qb >= 2) ws.pb[(rec * 8 + qb * 2 + 1) * FRAG + lane] = pack_pair(pt[2], pt[3]);
    }
    __syncthreads();
    Q35_PHASE(3);

    // 4. T = (I + A)^-1. Upper off-diagonal blocks are zero; the diagonal blocks by forward
    //    substitution in the reference order (wave w, lanes 0..15: one column each).
    //    Each block of T is written with its Tb = bf16(T_ij beta_j) as it is produced.
    for (int x = tid; x < 6 * 256; x += PT) {
        const int blk = x / 256, r = (x % 256) / 16, cc = x % 16;
        const int bi = blk < 3 ? 0 : blk < 5 ? 1 : 2;
        const int bj = blk < 3 ? blk + 1 : blk < 5 ? blk - 1 : 3;
        tm[(16 * bi + r) * FLD + 16 * bj + cc] = 0.f;
        tb[(16 * bi + r) * TLD + 16 * bj + cc] = 0;
    }
    if (lane < 16) {
        const int base = 16 * wave, cc = lane;
        const float beta_c = bet[base + cc];
        float xs[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            float acc = r == cc ? 1.f : 0.f;
#pragma unroll
            for (int j = 0; j < r; j++) acc = fmaf(-am[(base + r) * FLD + base + j], xs[j], acc);
            xs[r] = acc;
        }
#pragma unroll
        for (int r = 0; r < 16; r++) {
            tm[(base + r) * FLD + base + cc] = xs[r];
            tb[(base + r) * TLD + base + cc] = to_bf16(xs[r] * beta_c);
        }
    }
    __syncthreads();
    Q35_PHASE(4);
    //    the off-diagonal levels, wave bi computing T_{bi, bi - lv}
    if (wave >= 1) inverse_level<1>(wave, am, tm, tb, bet, scr, col, grp);
    __syncthreads();
    if (wave >= 2) inverse_level<2>(wave, am, tm, tb, bet, scr, col, grp);
    __syncthreads();
    if (wave >= 3) inverse_level<3>(wave, am, tm, tb, bet, scr, col, grp);
    __syncthreads();
    Q35_PHASE(5);

    // 5. the raw k rows go to region 1 (A is dead) for step 6
#pragma unroll
    for (int s = 0; s < 4; s++) reinterpret_cast<u32x4*>(am)[(wave * 4 + s) * FRAG + lane] = kraw[s];
    __syncthreads();
    Q35_PHASE(6);

    // 6. dims 32 wave .. 32 wave + 31: kw, kd and v transposed on the MFMA (lane = dim,
    //    4 tokens per tile), then kd^T fragments, u = Tb v tiles and w^T = kw^T Tb^T tiles.
    //    Operand fk[s][half] = kw^T fragment (dims 16 (2 wave + half) + l%16, tokens step s);
    //    fv likewise for v.
    u32x4 fkw[2][2], fvt[2][2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        f32x4 tkw[2][2], tkd[2][2], tv[2][2];
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const int tb_ = 2 * s + p, row = 16 * tb_ + col;
            const float ki = kinv_s[row], e1 = ecum[row], e2 = erem[row];
            float kf[8], a1[8], a2[8];
            unpack8v(reinterpret_cast<const u32x4*>(am)[(tb_ * 4 + wave) * FRAG + lane], kf);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float kx = kf[e] * ki;
                a1[e] = kx * e1;
                a2[e] = kx * e2;
            }
            const u32x4 akw = pack8v(a1), akd = pack8v(a2);
#pragma unroll
            for (int half = 0; half < 2; half++) {
                const u32x4 sel = select_op(half, col, grp);
                const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                tkw[p][half] = mfma16(akw, sel, z);
                tkd[p][half] = mfma16(akd, sel, z);
                tv[p][half] = mfma16(vc[tb_], sel, z);
            }
        }
#pragma unroll
        for (int half = 0; half < 2; half++) {
            ws.kd[(rec * 16 + (2 * wave + half) * 2 + s) * FRAG + lane] = pack_pair(tkd[0][half], tkd[1][half]);
            fkw[s][half] = pack_pair(tkw[0][half], tkw[1][half]);
            fvt[s][half] = pack_pair(tv[0][half], tv[1][half]);
        }
    }
#pragma unroll
    for (int it = 0; it < 4; it++) {
        f32x4 wt[2];
#pragma unroll
        for (int half = 0; half < 2; half++) {
            f32x4 ua = {0.f, 0.f, 0.f, 0.f}, wa = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s <= it / 2; s++) {  // T is lower triangular
                const bf16* tr = tb + (16 * it + col) * TLD + 32 * s + 4 * grp;
                const u32x2 t_lo = *reinterpret_cast<const u32x2*>(tr);
                const u32x2 t_hi = *reinterpret_cast<const u32x2*>(tr + 16);
                const u32x4 tbf = u32x4{t_lo[0], t_lo[1], t_hi[0], t_hi[1]};
                ua = mfma16(tbf, fvt[s][half], ua);
                wa = mfma16(fkw[s][half], tbf, wa);
            }
            ws.u[(rec * 32 + it * 8 + 2 * wave + half) * FRAG + lane] = u32x2{pack2(ua[0], ua[1]), pack2(ua[2], ua[3])};
            wt[half] = wa;
        }
        ws.w[(rec * 16 + it * 4 + wave) * FRAG + lane] = pack_pair(wt[0], wt[1]);
    }
    // the chunk's decay, stored last: a store before a block barrier is waited for there
    if (wave == 0 && lane == C - 1) ws.decay[rec] = ecum[C - 1];
    Q35_PHASE(7);
}

// gdn_prep8: the same per-item arithmetic as gdn_prep on eight waves, for launches whose items
// all fit on the device at once (one block per CU), where a block's latency sets the time:
//   * waves 0-3 load and normalise k row block `wave`, waves 4-7 q row block `wave - 4` (and the
//     v columns of dim step `wave - 4`); both sides write their TF32 planes to LDS;
//   * the cumulative log-decay runs on wave 3 alone and reaches the others through LDS; the q
//     side forms qd after the barrier that publishes it;
//   * the ten A tiles and the six pb fragments (ten P tiles) go to the eight waves by a fixed
//     table, two or three tiles each, both operands from the LDS planes;
//   * the inverse runs on waves 0-3 as in gdn_prep;
//   * step 6 splits by product: waves 4-7 transpose v and kd (and store the kd fragments)
//     while waves 0-3 work through the inverse's off-diagonal levels, then form u = Tb v;
//     waves 0-3 transpose kw and form w^T, each for dim step `wave & 3`. The raw k rows for
//     the transposes go to the q-plane region, free after the pair products;
//   * an inverse level's partial product passes through the wave's own LDS scratch without
//     a block barrier.
// Every tile, fragment and store is computed by the same instruction sequence on the same
// values as in gdn_prep, so the records are bit for bit the same.
constexpr int PT8 = 512;
constexpr int QPL = PREP_SMEM;                         // q^ planes: hi then lo, [4 blocks][4 steps]
// input rows staged by LDS DMA: k, q and v of the chunk, [64 rows][256 B] each
constexpr int STG_K = QPL + 2 * PLANE;
constexpr int STG_Q = STG_K + C * STG_ROW;
constexpr int STG_V = STG_Q + C * STG_ROW;
constexpr int PREP8_SMEM = STG_V + C * STG_ROW;
static_assert(PREP8_SMEM <= 160 * 1024, "gdn_prep8 fits the LDS");

// One fragment (64 lanes x 16 or 8 bytes at frag, a wave-uniform address) stored at device
// scope (the SC1 cache-policy bit): the line is written through the XCD's L2 instead of being
// left dirty there. A kernel's end writes back every dirty L2 line before the next kernel can
// start, and for the 8-wave prep, whose records (72 KB per item) are all written in the last
// microseconds of the launch, that flush was the largest part of the gap before the scan
// (config 0: 5.4 us with ~9 MB of records, 1.9 us with them written through). The 4-wave prep
// keeps ordinary stores: its records are re-read by the scan of the same segment from L2.
template <typename V>
__device__ __forceinline__ void store_through(V* frag, int lane, V v) {
    const auto r = __builtin_amdgcn_make_buffer_rsrc(frag, (short)0, 0x7fffffff, 0x00020000);
    constexpr int SC1 = 0x10;
    if constexpr (sizeof(V) == 16) __builtin_amdgcn_raw_buffer_store_b128(v, r, lane * 16, 0, SC1);
    else __builtin_amdgcn_raw_buffer_store_b64(v, r, lane * 8, 0, SC1);
}

// A tile (i, j) of the chunk: A_ij for the rows of k block i and the columns of k block j
__device__ __forceinline__ void prep8_a_tile(int bi, int bj, const u32x4* khi_pl, const u32x4* klo_pl, float* am,
                                             const float* cum, const float* bet, int lane) {
    const int col = lane & 15, grp = lane >> 4;
    // decay and beta as vectors up front, decay factors masked by a select (see gdn_prep)
    const f32x4 cum_i = *reinterpret_cast<const f32x4*>(cum + 16 * bi + 4 * grp);
    const f32x4 bet_i = *reinterpret_cast<const f32x4*>(bet + 16 * bi + 4 * grp);
    const float cum_j = cum[16 * bj + col];
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const u32x4 ah = khi_pl[(bi * 4 + s) * FRAG + lane], al = klo_pl[(bi * 4 + s) * FRAG + lane];
        const u32x4 bh = khi_pl[(bj * 4 + s) * FRAG + lane], bl = klo_pl[(bj * 4 + s) * FRAG + lane];
        acc = mfma16(al, bl, acc);
        acc = mfma16(al, bh, acc);
        acc = mfma16(ah, bl, acc);
        acc = mfma16(ah, bh, acc);
    }
    const int j = 16 * bj + col;
    float dec[4];
#pragma unroll
    for (int r = 0; r < 4; r++) dec[r] = expf(cum_i[r] - cum_j);
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int i = 16 * bi + 4 * grp + r;
        am[i * FLD + j] = j < i ? bet_i[r] * acc[r] * dec[r] : 0.f;
    }
}

// pb fragment (qb, s): P^T tiles 2 s and 2 s + 1 of q block qb (zero past the diagonal)
__device__ __forceinline__ void prep8_p_frag(int qb, int s2, const u32x4* khi_pl, const u32x4* klo_pl,
                                             const u32x4* qhi_pl, const u32x4* qlo_pl, const float* cum,
                                             const Work& ws, size_t rec, int lane) {
    const int col = lane & 15, grp = lane >> 4;
    f32x4 pt[2];
    const float cum_q = cum[16 * qb + col];
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const int jt = 2 * s2 + p;
        pt[p] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (jt > qb) continue;
        const f32x4 cum_j = *reinterpret_cast<const f32x4*>(cum + 16 * jt + 4 * grp);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const u32x4 ah = khi_pl[(jt * 4 + s) * FRAG + lane], al = klo_pl[(jt * 4 + s) * FRAG + lane];
            const u32x4 qh = qhi_pl[(qb * 4 + s) * FRAG + lane], ql = qlo_pl[(qb * 4 + s) * FRAG + lane];
            pt[p] = mfma16(al, ql, pt[p]);
            pt[p] = mfma16(al, qh, pt[p]);
            pt[p] = mfma16(ah, ql, pt[p]);
            pt[p] = mfma16(ah, qh, pt[p]);
        }
        const int i = 16 * qb + col;
        float dec[4];
#pragma unroll
        for (int r = 0; r < 4; r++) dec[r] = expf(cum_q - cum_j[r]);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int j = 16 * jt + 4 * grp + r;
            pt[p][r] = j <= i ? round_bf16(pt[p][r] * dec[r]) : 0.f;
        }
    }
    store_through(&ws.pb[(rec * 8 + qb * 2 + s2) * FRAG], lane, pack_pair(pt[0], pt[1]));
}

// Diagonal block (base, base) of T = (I + A)^-1 (and of Tb) by forward substitution, column cc on lane cc,
// with the block's 120 strictly-lower entries of A read from LDS into registers before the
// first product, so the substitution does not wait on the LDS along its chain (the same
// products and sums, in the same order, as reading each entry where it is used).
__device__ __forceinline__ void diag_inverse_preloaded(const float* am, float* tm, bf16* tb, const float* bet, int base,
                                                       int cc) {
    float a[120];
#pragma unroll
    for (int r = 1, n = 0; r < 16; r++)
#pragma unroll
        for (int j = 0; j < r; j++, n++) a[n] = am[(base + r) * FLD + base + j];
    __builtin_amdgcn_sched_barrier(0);
    float xs[16];
#pragma unroll
    for (int r = 0, n = 0; r < 16; r++) {
        float acc = r == cc ? 1.f : 0.f;
#pragma unroll
        for (int j = 0; j < r; j++, n++) acc = fmaf(-a[n], xs[j], acc);
        xs[r] = acc;
    }
    const float beta_c = bet[base + cc];
#pragma unroll
    for (int r = 0; r < 16; r++) {
        tm[(base + r) * FLD + base + cc] = xs[r];
        tb[(base + r) * TLD + base + cc] = to_bf16(xs[r] * beta_c);
    }
}

template <bool GATED>
__global__ void __launch_bounds__(PT8)
    gdn_prep8(const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v, Gates gt, Work ws,
              int T, int H, int HK, float scale, const GSeqs gs) {
    extern __shared__ __align__(16) unsigned char sm[];
    u32x4* khi_pl = reinterpret_cast<u32x4*>(sm + R0);
    u32x4* klo_pl = reinterpret_cast<u32x4*>(sm + R0 + PLANE);
    u32x4* qhi_pl = reinterpret_cast<u32x4*>(sm + QPL);
    u32x4* qlo_pl = reinterpret_cast<u32x4*>(sm + QPL + PLANE);
    float* tm = reinterpret_cast<float*>(sm + R0_TM);
    bf16* tb = reinterpret_cast<bf16*>(sm + R0_TB);
    float* am = reinterpret_cast<float*>(sm + R1);
    float* cum = reinterpret_cast<float*>(sm + R2);
    float* bet = cum + C;
    float* ecum = bet + C;
    float* erem = ecum + C;
    float* kinv_s = erem + C;

    const int c = blockIdx.x, h = blockIdx.y, NC = gridDim.x;
    int cl = c;
    if (gs.n > 0) {
        int sq = 0;
        while (sq + 1 < gs.n && c >= gs.chk[sq + 1]) sq++;
        cl = c - gs.chk[sq];
        const int r0 = gs.tok[sq];
        T = gs.tok[sq + 1] - r0;
        q += (size_t)r0 * HK * DK;
        k += (size_t)r0 * HK * DK;
        v += (size_t)r0 * H * DK;
        gt = gt.from_row(r0, H);
    }
    const int hk = h / (H / HK);
    const int tid = threadIdx.x, lane = tid & 63, col = lane & 15, grp = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool kside = wave < 4;
    const int blk = wave & 3;  // k row block (k side) / q row block and v dim step (q side)
    // role: 0 = the whole item; split launches (gridDim.z = 2) give each item two blocks,
    // 1 = A, the inverse, w, u and kd (waves 4-7 move v instead of q), 2 = qd and pb
    const int role = gridDim.z == 1 ? 0 : 1 + (int)blockIdx.z;
    const bool has_q = role != 1, has_t = role != 2;
    const size_t rec = (size_t)h * NC + c;
    const int t0 = cl * C;
    Q35_PHASE_START();
    Q35_WSTART();

    // 0. loads, unconditional (rows past T read row T - 1 and are zeroed after step 1) so that
    //    none waits for another; wave 3's gates first, which its decay scan waits for alone.
    //    The k and q rows go to LDS as whole lines (a fragment's pieces are half lines 4 KB
    //    apart) and are read back in fragment order.
    const int row = 16 * blk + col;
    const int tl = t0 + lane;
    // (the gate loads are issued by hand and waited for by hand, together with the four row
    // transfers issued after them: as ordinary loads the compiler placed the wait for beta, or
    // the loads themselves, after the transfers were issued or before them)
    float g_raw = 0.f;
    uint32_t b_bits = 0, a_bits = 0, al_bits = 0, dt_bits = 0;
    if (wave == 3) {
        const int tlc = min(tl, T - 1);
        if constexpr (GATED) {
            asm volatile("global_load_ushort %0, %1, off" : "=v"(b_bits) : "v"(gt.b + (size_t)tlc * gt.ld + h));
            asm volatile("global_load_ushort %0, %1, off" : "=v"(a_bits) : "v"(gt.a + (size_t)tlc * gt.ld + h));
            asm volatile("global_load_ushort %0, %1, off" : "=v"(al_bits) : "v"(gt.A_log + h));
            asm volatile("global_load_ushort %0, %1, off" : "=v"(dt_bits) : "v"(gt.dt_bias + h));
        } else {
            asm volatile("global_load_dword %0, %1, off" : "=v"(g_raw) : "v"(gt.g + (size_t)tlc * H + h));
            asm volatile("global_load_ushort %0, %1, off" : "=v"(b_bits) : "v"(gt.beta + (size_t)tlc * H + h));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    unsigned char* const stg = sm + (kside ? STG_K : STG_Q);
    if (kside || has_q)
        stage_rows((kside ? k : q) + (size_t)hk * DK, HK * DK, t0, 16 * blk, T, stg, lane);
    else
        stage_rows(v + (size_t)h * DK, H * DK, t0, 16 * blk, T, sm + STG_V, lane);
    __builtin_amdgcn_sched_barrier(0);

    // 1. cumulative log-decay on wave 3 alone (lane = token), published through LDS for step
    //    3 on: one chain of 64 dependent adds in index order, lane j keeping the running sum
    //    after term j (the same additions in the same order as a per-lane prefix loop)
    Q35_WSTAMP(0);
    if (wave == 3) {
        float gv, bv;
        if constexpr (GATED) {
            asm volatile("s_waitcnt vmcnt(4)" : "+v"(b_bits), "+v"(a_bits), "+v"(al_bits), "+v"(dt_bits));
            bf16 be;
            float gg;
            gate_values(f32((bf16)b_bits), f32((bf16)a_bits), -expf(f32((bf16)al_bits)), f32((bf16)dt_bits), be, gg);
            gv = tl < T ? gg : 0.f;
            bv = tl < T ? f32(be) : 0.f;
        } else {
            asm volatile("s_waitcnt vmcnt(4)" : "+v"(g_raw), "+v"(b_bits));
            gv = tl < T ? g_raw : 0.f;
            bv = tl < T ? __uint_as_float(b_bits << 16) : 0.f;
        }
        float run = 0.f, cs = 0.f;
#pragma unroll
        for (int j = 0; j < C; j++) {
            run = run + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gv), j));
            cs = lane == j ? run : cs;
        }
        cum[lane] = cs;
        bet[lane] = bv;
        ecum[lane] = expf(cs);
        erem[lane] = expf(run - cs);
    }
#ifdef Q35_PHASE_TIMING
    if (wave == 3) asm volatile("" ::"v"(ecum[lane]));
#endif
    Q35_WSTAMP(1);
    // the wave's own rows from LDS; then the q side stages the v rows, read by dim step after
    // the next barrier. Rows past T are zero from here on.
    wait_vm_all();
    u32x4 raw[4], vc[4];
    const bool has_rows = kside || has_q;
    if (has_rows) {
#pragma unroll
        for (int s = 0; s < 4; s++) raw[s] = staged_perm(stg, row, s, grp);
    }
    if (!kside && role == 0) stage_rows(v + (size_t)h * DK, H * DK, t0, 16 * blk, T, sm + STG_V, lane);
#pragma unroll
    for (int s = 0; s < 4; s++)
        if (t0 + row >= T) raw[s] = u32x4{0u, 0u, 0u, 0u};

    // 2. L2 norms and TF32 splits: k side -> k planes, q side -> q planes
    float qinv = 0.f;
    if (has_rows) {
        float ss = 0.f;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            float xf[8];
            unpack8v(raw[s], xf);
#pragma unroll
            for (int e = 0; e < 8; e++) ss += xf[e] * xf[e];
        }
        asm volatile("" ::"v"(ss));
        Q35_WSTAMP(2);
        ss += __shfl_xor(ss, 16, 64);
        ss += __shfl_xor(ss, 32, 64);
        if (kside) {
            const float kinv = rsqrtf(ss + 1e-6f);
            if (grp == 0) kinv_s[row] = kinv;
#pragma unroll
            for (int s = 0; s < 4; s++) {
                float kt_[8], kf[8];
                unpack8v(raw[s], kf);
#pragma unroll
                for (int e = 0; e < 8; e++) kt_[e] = tf32_rna(kf[e] * kinv);
                u32x4 h, l;
                split_tf32(kt_, h, l);
                khi_pl[(blk * 4 + s) * FRAG + lane] = h;
                klo_pl[(blk * 4 + s) * FRAG + lane] = l;
            }
        } else {
            qinv = rsqrtf(ss + 1e-6f) * scale;
#pragma unroll
            for (int s = 0; s < 4; s++) {
                float qt_[8], qf[8];
                unpack8v(raw[s], qf);
#pragma unroll
                for (int e = 0; e < 8; e++) qt_[e] = tf32_rna(qf[e] * qinv);
                u32x4 h, l;
                split_tf32(qt_, h, l);
                qhi_pl[(blk * 4 + s) * FRAG + lane] = h;
                qlo_pl[(blk * 4 + s) * FRAG + lane] = l;
            }
        }
    }
    Q35_WSTAMP(3);
    if (!kside && has_t) wait_vm_all();  // the staged v rows
    __syncthreads();
    Q35_PHASE(2);
    Q35_WSTAMP(4);
    // qd = (q^ scale) e^cum once the cumulative decay is in LDS
    if (!kside && has_t) {
#pragma unroll
        for (int tb_ = 0; tb_ < 4; tb_++) {
            vc[tb_] = staged_perm(sm + STG_V, 16 * tb_ + col, blk, grp);
            if (t0 + 16 * tb_ + col >= T) vc[tb_] = u32x4{0u, 0u, 0u, 0u};
        }
    }
    if (!kside && has_q) {
        const float ecq = ecum[row];
#pragma unroll
        for (int s = 0; s < 4; s++) {
            float qd_[8], qf[8];
            unpack8v(raw[s], qf);
#pragma unroll
            for (int e = 0; e < 8; e++) qd_[e] = qf[e] * qinv * ecq;
            store_through(&ws.qd[(rec * 16 + blk * 4 + s) * FRAG], lane, pack8v(qd_));
        }
    }

    // 3. pair products by table: 10 A tiles and the 6 pb fragments that are not all zero (the
    //    scan never reads fragment 1 of row blocks 0 and 1) over 8 waves, or each set over the
    //    8 waves of its own block in a split launch
    if (role == 0) {
        switch (wave) {
            case 0:
                prep8_a_tile(3, 3, khi_pl, klo_pl, am, cum, bet, lane);
                prep8_a_tile(3, 2, khi_pl, klo_pl, am, cum, bet, lane);
                prep8_a_tile(0, 0, khi_pl, klo_pl, am, cum, bet, lane);
                break;
            case 1:
                prep8_a_tile(3, 1, khi_pl, klo_pl, am, cum, bet, lane);
                prep8_a_tile(3, 0, khi_pl, klo_pl, am, cum, bet, lane);
                prep8_a_tile(1, 1, khi_pl, klo_pl, am, cum, bet, lane);
                break;
            case 2:
                prep8_a_tile(2, 2, khi_pl, klo_pl, am, cum, bet, lane);
                prep8_a_tile(2, 1, khi_pl, klo_pl, am, cum, bet, lane);
                prep8_a_tile(2, 0, khi_pl, klo_pl, am, cum, bet, lane);
                break;
            case 3:
                prep8_a_tile(1, 0, khi_pl, klo_pl, am, cum, bet, lane);
                prep8_p_frag(0, 0, khi_pl, klo_pl, qhi_pl, qlo_pl, cum, ws, rec, lane);
                prep8_p_frag(2, 1, khi_pl, klo_pl, qhi_pl, qlo_pl, cum, ws, rec, lane);
                break;
            case 4:
                prep8_p_frag(3, 0, khi_pl, klo_pl, qhi_pl, qlo_pl, cum, ws, rec, lane);
                break;
            case 5:
                prep8_p_frag(3, 1, khi_pl, klo_pl, qhi_pl, qlo_pl, cum, ws, rec, lane);
                break;
            case 6:
                prep8_p_frag(2, 0, khi_pl, klo_pl, qhi_pl, qlo_pl, cum, ws, rec, lane);
                break;
            default:
                prep8_p_frag(1, 0, khi_pl, klo_pl, qhi_pl, qlo_pl, cum, ws, rec, lane);
                break;
        }
    } else if (role == 1) {
        // the 10 A tiles over the 8 waves
        switch (wave) {
            case 0:
                prep8_a_tile(3, 3, khi_pl, klo_pl, am, cum, bet, lane);
                prep8_a_tile(0, 0, khi_pl, klo_pl, am, cum, bet, lane);
                break;
            case 1:
                prep8_a_tile(3, 2, khi_pl, klo_pl, am, cum, bet, lane);
                prep8_a_tile(1, 1, khi_pl, klo_pl, am, cum, bet, lane);
                break;
            case 2:
                prep8_a_tile(3, 1, khi_pl, klo_pl, am, cum, bet, lane);
                break;
            case 3:
                prep8_a_tile(3, 0, khi_pl, klo_pl, am, cum, bet, lane);
                break;
            case 4:
                prep8_a_tile(2, 2, khi_pl, klo_pl, am, cum, bet, lane);
                break;
            case 5:
                prep8_a_tile(2, 1, khi_pl, klo_pl, am, cum, bet, lane);
                break;
            case 6:
                prep8_a_tile(2, 0, khi_pl, klo_pl, am, cum, bet, lane);
                break;
            default:
                prep8_a_tile(1, 0, khi_pl, klo_pl, am, cum, bet, lane);
                break;
        }
    } else {
        // the 6 pb fragments, one per wave; this block's work ends here
        switch (wave) {
            case 0:
                prep8_p_frag(0, 0, khi_pl, klo_pl, qhi_pl, qlo_pl, cum, ws, rec, lane);
                break;
            case 1:
                prep8_p_frag(1, 0, khi_pl, klo_pl, qhi_pl, qlo_pl, cum, ws, rec, lane);
                break;
            case 2:
                prep8_p_frag(2, 0, khi_pl, klo_pl, qhi_pl, qlo_pl, cum, ws, rec, lane);
                break;
            case 3:
                prep8_p_frag(2, 1, khi_pl, klo_pl, qhi_pl, qlo_pl, cum, ws, rec, lane);
                break;
            case 4:
                prep8_p_frag(3, 0, khi_pl, klo_pl, qhi_pl, qlo_pl, cum, ws, rec, lane);
                break;
            case 5:
                prep8_p_frag(3, 1, khi_pl, klo_pl, qhi_pl, qlo_pl, cum, ws, rec, lane);
                break;
            default: break;
        }
        return;
    }
    Q35_WSTAMP(5);
    __syncthreads();
    Q35_PHASE(3);

    // 4. T = (I + A)^-1: zero upper blocks (all threads), diagonal blocks on waves 0-3. The raw
    //    k rows go to the q-plane region (dead after step 3) for step 6's transposes, which the
    //    q side runs while waves 0-3 work through the off-diagonal levels.
    u32x4* const kraw_pl = reinterpret_cast<u32x4*>(sm + QPL);
    if (kside) {
#pragma unroll
        for (int s = 0; s < 4; s++) kraw_pl[(blk * 4 + s) * FRAG + lane] = raw[s];
    }
    for (int x = tid; x < 6 * 256; x += PT8) {
        const int blk_ = x / 256, r = (x % 256) / 16, cc = x % 16;
        const int bi = blk_ < 3 ? 0 : blk_ < 5 ? 1 : 2;
        const int bj = blk_ < 3 ? blk_ + 1 : blk_ < 5 ? blk_ - 1 : 3;
        tm[(16 * bi + r) * FLD + 16 * bj + cc] = 0.f;
        tb[(16 * bi + r) * TLD + 16 * bj + cc] = 0;
    }
    // step 6's transposes of dim step ds = wave & 3: q side the kd fragments (stored) and v,
    // k side kw, into f[token step][half] (fvt or fkw)
    const int ds = blk;
    u32x4 f[2][2];
    auto transposes = [&]() {
#pragma unroll
        for (int s = 0; s < 2; s++) {
            f32x4 ta[2][2], tk[2][2];
#pragma unroll
            for (int p = 0; p < 2; p++) {
                const int tb_ = 2 * s + p, rw = 16 * tb_ + col;
                const float ki = kinv_s[rw], e = kside ? ecum[rw] : erem[rw];
                float kf[8], a[8];
                unpack8v(kraw_pl[(tb_ * 4 + ds) * FRAG + lane], kf);
#pragma unroll
                for (int x = 0; x < 8; x++) a[x] = kf[x] * ki * e;
                const u32x4 ak = pack8v(a);
#pragma unroll
                for (int half = 0; half < 2; half++) {
                    const u32x4 sel = select_op(half, col, grp);
                    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                    tk[p][half] = mfma16(ak, sel, z);
                    if (!kside) ta[p][half] = mfma16(vc[tb_], sel, z);
                }
            }
#pragma unroll
            for (int half = 0; half < 2; half++) {
                if (kside) {
                    f[s][half] = pack_pair(tk[0][half], tk[1][half]);
                } else {
                    store_through(&ws.kd[(rec * 16 + (2 * ds + half) * 2 + s) * FRAG], lane,
                                  pack_pair(tk[0][half], tk[1][half]));
                    f[s][half] = pack_pair(ta[0][half], ta[1][half]);
                }
            }
        }
    };
    if (kside && lane < 16) diag_inverse_preloaded(am, tm, tb, bet, 16 * blk, lane);
    __syncthreads();
    Q35_PHASE(4);
    if (!kside) transposes();
    float* scr = reinterpret_cast<float*>(sm + R0_SC) + blk * 256;
    if (kside && blk >= 1) inverse_level<1>(blk, am, tm, tb, bet, scr, col, grp);
    __syncthreads();
    if (kside && blk >= 2) inverse_level<2>(blk, am, tm, tb, bet, scr, col, grp);
    __syncthreads();
    if (kside && blk >= 3) inverse_level<3>(blk, am, tm, tb, bet, scr, col, grp);
    __syncthreads();
    Q35_PHASE(5);

    Q35_PHASE(6);

    // 6. (Tb was written with T in step 4) u = Tb v on the q side (its transposes ran in step 4);
    //    on the k side the kw transpose and w^T = kw^T Tb^T
    if (kside) transposes();
#pragma unroll
    for (int it = 0; it < 4; it++) {
        f32x4 wt[2];
#pragma unroll
        for (int half = 0; half < 2; half++) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s <= it / 2; s++) {  // T is lower triangular
                const bf16* tr = tb + (16 * it + col) * TLD + 32 * s + 4 * grp;
                const u32x2 t_lo = *reinterpret_cast<const u32x2*>(tr);
                const u32x2 t_hi = *reinterpret_cast<const u32x2*>(tr + 16);
                const u32x4 tbf = u32x4{t_lo[0], t_lo[1], t_hi[0], t_hi[1]};
                acc = kside ? mfma16(f[s][half], tbf, acc) : mfma16(tbf, f[s][half], acc);
            }
            if (!kside)
                store_through(&ws.u[(rec * 32 + it * 8 + 2 * ds + half) * FRAG], lane,
                              u32x2{pack2(acc[0], acc[1]), pack2(acc[2], acc[3])});
            wt[half] = acc;
        }
        if (kside) store_through(&ws.w[(rec * 16 + it * 4 + ds) * FRAG], lane, pack_pair(wt[0], wt[1]));
    }
    // the chunk's decay, stored last: a store before a block barrier is waited for there
    if (wave == 3 && lane == C - 1) ws.decay[rec] = ecum[C - 1];  // (role 0 or 1)
    Q35_PHASE(7);
    Q35_WSTAMP(6);
    Q35_WFLUSH();
}

// ------------------------------------------------------------------ gdn_scan

constexpr int BV = 16;    // value columns per MFMA tile; a block owns NSUB such halves
constexpr int SLD = DK + 8;  // bf16 stride of Sb^T [16 NSUB][128]
constexpr int VLD = C + 8;   // bf16 stride of v_new^T [16 NSUB][64]

template <int NSUB>
struct ChainOps {
    u32x4 w[4];        // w fragments (row block = wave, dim steps)
    u32x4 kd[2][2];    // kd^T fragments (dim blocks 2 wave + i, token steps)
    u32x2 u[NSUB];     // u tiles (row block = wave, dim blocks NSUB slice + half)
    float decay;
};

struct OutOps {
    u32x4 qd[4];    // qd fragments (row block = wave - 4, dim steps)
    u32x4 pb[2];    // pb fragments (row block, token steps)
};

// Fragment streams of one head as raw buffer loads: the descriptor (scalar registers) points
// at the head's first record, the per-chunk byte offset is a scalar soffset and the lane
// offset is one fixed vector register, so the loads need no vector address arithmetic
// (vector address temporaries would alias the destinations of loads still in flight).
struct Streams {
    __amdgpu_buffer_rsrc_t w, kd, qd, pb, u;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t stream_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}

// The o rows of chunk c for one head and column slice (base = o + h * 128 + first column): a
// buffer over the chunk's rows below T, so a lane stores with its fixed in-chunk offset and a
// row past T falls outside the buffer and is dropped by the hardware (no per-row test).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t out_rows(bf16* base, int c, int T, int H) {
    // every value is wave-uniform; readfirstlane keeps the descriptor in scalar registers
    const int rows = __builtin_amdgcn_readfirstlane(max(0, min(C, T - c * C)));
    const uint64_t a = (uint64_t)(base + (size_t)c * C * H * DK);
    const uint64_t au = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)) << 32) |
                        (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(au), (short)0, rows * H * DK * 2, 0x00020000);
}

__device__ __forceinline__ u32x4 bload16(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

template <int NSUB>
__device__ __forceinline__ void load_chain(ChainOps<NSUB>& op, const Streams& sr, const float* decay, int c, int rb,
                                           int lane, int slice) {
    const int v16 = lane * 16;
    const int rec_w = c * 16 * 1024 + rb * 4 * 1024;
#pragma unroll
    for (int s = 0; s < 4; s++) op.w[s] = bload16(sr.w, v16 + s * 1024, rec_w);
#pragma unroll
    for (int i = 0; i < 4; i++) op.kd[i >> 1][i & 1] = bload16(sr.kd, v16 + i * 1024, rec_w);
#pragma unroll
    for (int hf = 0; hf < NSUB; hf++)
        op.u[hf] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                                 sr.u, lane * 8, c * 32 * 512 + (rb * 8 + NSUB * slice + hf) * 512, 0));
    op.decay = decay[c];
}

__device__ __forceinline__ void load_out(OutOps& op, const Streams& sr, int c, int rb, int lane) {
    const int v16 = lane * 16;
#pragma unroll
    for (int s = 0; s < 4; s++) op.qd[s] = bload16(sr.qd, v16 + s * 1024, c * 16 * 1024 + rb * 4 * 1024);
    op.pb[0] = bload16(sr.pb, v16, c * 8 * 1024 + rb * 2 * 1024);
    // token step 1 of row blocks 0 and 1 lies above the diagonal (all zero, not stored)
    if (rb >= 2) op.pb[1] = bload16(sr.pb, v16 + 1024, c * 8 * 1024 + rb * 2 * 1024);
}

// B operand from a [16][ld] bf16 LDS array: row `col`, k step s in perm order
__device__ __forceinline__ u32x4 lds_perm(const bf16* base, int ld, int col, int s, int grp) {
    const bf16* p = base + col * ld + 32 * s + 4 * grp;
    const u32x2 a = *reinterpret_cast<const u32x2*>(p);
    const u32x2 b = *reinterpret_cast<const u32x2*>(p + 16);
    return u32x4{a[0], a[1], b[0], b[1]};
}

// Per chunk, two barriers:  [chain: write bf16(S)^T]  A  [chain: v_new = u - w Sb -> LDS;
// output: acc = qd Sb]  B  [chain: S = S decay + kd^T v_new; output: o = acc + pb v_new].
// Chain waves read Sb only between A and B; output waves read v_new after B and are done
// before the next A, when v_new is rewritten.
//
// A block owns NSUB 16-column halves of one head's value columns (NSUB = 1: 16 columns, eight
// slice blocks per head; NSUB = 2: 32 columns, four). Every half runs the same instructions
// on the same operand fragments as a one-half block would, so both forms give the same bits;
// the two-half form fetches each chunk's shared w / kd / qd / pb fragments once for two halves
// and is used when it needs fewer rounds of blocks on the device (gdn_launch).
//
// OS = 2: two sets of four output waves (12 waves), set X taking the chunks c with c % 2 == X.
// bf16(S) and v_new are double-buffered by chunk parity, so a set reads chunk c's copies after
// barriers A and B of chunk c and has the two barrier windows of chunk c + 1 for its o stores
// and operand prefetches, which no longer hold the chain waves at the next barrier A. The
// products are the same instructions on the same operands, so the output is the same bits.
template <int NSUB, int OS>
__global__ void __launch_bounds__(256 + 256 * OS)
    gdn_scan(Work ws, const float* __restrict__ decay_all, bf16* __restrict__ o, int T, int H, int NC,
             const float* __restrict__ s_in, size_t s_in_stride, float* __restrict__ s_out, size_t s_out_stride,
             const GSeqs gs) {
    constexpr int BVB = BV * NSUB, NSB = DK / BVB;
    __shared__ __align__(16) bf16 sbt_[OS][BVB * SLD];
    __shared__ __align__(16) bf16 vnt_[OS][BVB * VLD];
    const int h = blockIdx.x % H, slice = (blockIdx.x / H) % NSB, v0 = slice * BVB;
    size_t rec0 = (size_t)h * NC;
    if (gs.n > 0) {
        // packed sequences: blocks (sequence, slice, head); each sequence is scanned alone
        // from its own (or the shared) initial state over its own chunks
        const int sq = blockIdx.x / (H * NSB);
        rec0 += gs.chk[sq];
        NC = gs.chk[sq + 1] - gs.chk[sq];
        T = gs.tok[sq + 1] - gs.tok[sq];
        o += (size_t)gs.tok[sq] * H * DK;
        if (s_in) s_in += sq * s_in_stride;
        if (s_out) s_out += sq * s_out_stride;
        if (NC == 0) {
            // an empty sequence: its final state is its initial state (the whole block leaves
            // here, before any barrier)
            if (s_out != nullptr && tid_of_block() < 128)
                for (int x = tid_of_block(); x < DK * BVB; x += 128) {
                    const size_t at_ = ((size_t)h * DK + x / BVB) * DK + v0 + x % BVB;
                    s_out[at_] = s_in ? s_in[at_] : 0.f;
                }
            return;
        }
    }
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 15, grp = lane >> 4;
    const int uwave = __builtin_amdgcn_readfirstlane(wave);  // wave-uniform for the compiler
    const bool chain = uwave < 4;
    const int rb = uwave & 3;  // row block: state rows 32 rb .. (chain) / output rows 16 rb .. (output)
    auto at = [&](int c) { return min(c, NC - 1); };
    const Streams sr{stream_rsrc(ws.w + rec0 * 16 * FRAG), stream_rsrc(ws.kd + rec0 * 16 * FRAG),
                     stream_rsrc(ws.qd + rec0 * 16 * FRAG), stream_rsrc(ws.pb + rec0 * 8 * FRAG),
                     stream_rsrc(ws.u + rec0 * 32 * FRAG)};
    const float* decay = decay_all + rec0;  // read-only kernel argument: scalar loads

    if (chain) {
        // state rows 32 rb + 16 i + 4 grp + r, column v0 + 16 hf + col
        f32x4 st[NSUB][2];
#pragma unroll
        for (int hf = 0; hf < NSUB; hf++)
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    st[hf][i][r] = s_in ? s_in[((size_t)h * DK + 32 * rb + 16 * i + 4 * grp + r) * DK + v0 + 16 * hf + col]
                                        : 0.f;
        Q35_LPHASE_START();
        auto step = [&](const ChainOps<NSUB>& cur, int par) {
            bf16* sbt = sbt_[OS == 2 ? par : 0];
            bf16* vnt = vnt_[OS == 2 ? par : 0];
#pragma unroll
            for (int hf = 0; hf < NSUB; hf++)
#pragma unroll
                for (int i = 0; i < 2; i++)
                    *reinterpret_cast<u32x2*>(sbt + (16 * hf + col) * SLD + 32 * rb + 16 * i + 4 * grp) =
                        u32x2{pack2(st[hf][i][0], st[hf][i][1]), pack2(st[hf][i][2], st[hf][i][3])};
            Q35_LPHASE(8);
            __syncthreads();  // A
            Q35_LPHASE(9);
            u32x4 sb[NSUB][4];
#pragma unroll
            for (int hf = 0; hf < NSUB; hf++)
#pragma unroll
                for (int s = 0; s < 4; s++) sb[hf][s] = lds_perm(sbt + 16 * hf * SLD, SLD, col, s, grp);
            __builtin_amdgcn_sched_barrier(0);  // all the reads in flight before the first MFMA
#pragma unroll
            for (int hf = 0; hf < NSUB; hf++) {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < 4; s++) acc = mfma16(cur.w[s], sb[hf][s], acc);
                const float vn0 = lo_f32(cur.u[hf][0]) - acc[0], vn1 = hi_f32(cur.u[hf][0]) - acc[1];
                const float vn2 = lo_f32(cur.u[hf][1]) - acc[2], vn3 = hi_f32(cur.u[hf][1]) - acc[3];
                *reinterpret_cast<u32x2*>(vnt + (16 * hf + col) * VLD + 16 * rb + 4 * grp) =
                    u32x2{pack2(vn0, vn1), pack2(vn2, vn3)};
            }
            Q35_LPHASE(10);
            __syncthreads();  // B
            Q35_LPHASE(11);
            u32x4 vb[NSUB][2];
#pragma unroll
            for (int hf = 0; hf < NSUB; hf++) {
                vb[hf][0] = lds_perm(vnt + 16 * hf * VLD, VLD, col, 0, grp);
                vb[hf][1] = lds_perm(vnt + 16 * hf * VLD, VLD, col, 1, grp);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int hf = 0; hf < NSUB; hf++)
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    st[hf][i] *= cur.decay;
                    st[hf][i] = mfma16(cur.kd[i][0], vb[hf][0], st[hf][i]);
                    st[hf][i] = mfma16(cur.kd[i][1], vb[hf][1], st[hf][i]);
                }
            Q35_LPHASE(12);
        };
        if constexpr (OS == 2) {
            // three rotating operand sets (chunk c + 2 requested while chunk c is processed), so
            // the chain fits the twelve-wave block's registers
            ChainOps<NSUB> opa, opb, opc;
            load_chain(opa, sr, decay, at(0), rb, lane, slice);
            __builtin_amdgcn_sched_barrier(0);
            load_chain(opb, sr, decay, at(1), rb, lane, slice);
            const int NC3 = NC - NC % 3;
            for (int c = 0; c < NC3; c += 3) {
                load_chain(opc, sr, decay, at(c + 2), rb, lane, slice);
                step(opa, c & 1);
                load_chain(opa, sr, decay, at(c + 3), rb, lane, slice);
                step(opb, (c + 1) & 1);
                load_chain(opb, sr, decay, at(c + 4), rb, lane, slice);
                step(opc, (c + 2) & 1);
            }
            if (NC3 < NC) step(opa, NC3 & 1);
            if (NC3 + 1 < NC) step(opb, (NC3 + 1) & 1);
        } else {
            // four rotating operand sets: chunk c + 3 is requested while chunk c is processed
            ChainOps<NSUB> opa, opb, opc, opd;
            load_chain(opa, sr, decay, at(0), rb, lane, slice);
            __builtin_amdgcn_sched_barrier(0);  // the sets in order: the loop's waits count whole sets
            load_chain(opb, sr, decay, at(1), rb, lane, slice);
            __builtin_amdgcn_sched_barrier(0);  // the sets in order: the loop's waits count whole sets
            load_chain(opc, sr, decay, at(2), rb, lane, slice);
            // Whole groups of four chunks, then a tail of at most three. The main loop has no
            // early exit, so its only back edge follows the fourth step and the compiler's memory
            // waits stay per operand set (an exit after the first step would merge into the loop
            // header and make every group wait for the loads of the two newest sets).
            const int NC4 = NC & ~3;
            for (int c = 0; c < NC4; c += 4) {
                load_chain(opd, sr, decay, at(c + 3), rb, lane, slice);
                step(opa, 0);
                load_chain(opa, sr, decay, at(c + 4), rb, lane, slice);
                step(opb, 1);
                load_chain(opb, sr, decay, at(c + 5), rb, lane, slice);
                step(opc, 0);
                load_chain(opc, sr, decay, at(c + 6), rb, lane, slice);
                step(opd, 1);
            }
            if (NC4 < NC) step(opa, 0);
            if (NC4 + 1 < NC) step(opb, 1);
            if (NC4 + 2 < NC) step(opc, 0);
        }
        Q35_LPHASE_FLUSH();
        if (s_out) {
#pragma unroll
            for (int hf = 0; hf < NSUB; hf++)
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        s_out[((size_t)h * DK + 32 * rb + 16 * i + 4 * grp + r) * DK + v0 + 16 * hf + col] = st[hf][i][r];
        }
    } else if constexpr (OS == 2) {
        // output set X = (wave - 4) / 4; its own chunks are X, X + 2, ...; own chunk k uses the
        // operand set sp (k even) or sq (k odd), reloaded for own chunk k + 2 in the window after
        // it is consumed
        const int X = (uwave - 4) >> 2;
        f32x4 acc[NSUB];
        int pend = -1;  // the own chunk whose o waits to be stored
        auto store_rows = [&](int r0) {
            const auto ro = out_rows(o + (size_t)h * DK + v0, pend, T, H);
#pragma unroll
            for (int hf = 0; hf < NSUB; hf++)
#pragma unroll
                for (int r = r0; r < r0 + 2; r++)
                    __builtin_amdgcn_raw_buffer_store_b16(to_bf16(acc[hf][r]), ro,
                                                          ((16 * rb + 4 * grp + r) * H * DK + 16 * hf + col) * 2, 0, 0);
        };
        auto own = [&](const OutOps& cur, int c) {
            const bf16* sbt = sbt_[c & 1];
            const bf16* vnt = vnt_[c & 1];
            __syncthreads();  // A
            u32x4 sb[NSUB][4];
#pragma unroll
            for (int hf = 0; hf < NSUB; hf++)
#pragma unroll
                for (int s = 0; s < 4; s++) sb[hf][s] = lds_perm(sbt + 16 * hf * SLD, SLD, col, s, grp);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int hf = 0; hf < NSUB; hf++) {
                acc[hf] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < 4; s++) acc[hf] = mfma16(cur.qd[s], sb[hf][s], acc[hf]);
            }
            __syncthreads();  // B
            u32x4 vb[NSUB][2];
#pragma unroll
            for (int hf = 0; hf < NSUB; hf++) {
                vb[hf][0] = lds_perm(vnt + 16 * hf * VLD, VLD, col, 0, grp);
                vb[hf][1] = lds_perm(vnt + 16 * hf * VLD, VLD, col, 1, grp);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int hf = 0; hf < NSUB; hf++) {
                acc[hf] = mfma16(cur.pb[0], vb[hf][0], acc[hf]);
                if (rb >= 2) acc[hf] = mfma16(cur.pb[1], vb[hf][1], acc[hf]);
            }
            pend = c;
        };
        // a chunk of the other set: the pending stores, half in each barrier window, and the
        // reload of the operand set just consumed
        auto other = [&](OutOps& reload, int c_load) {
            __syncthreads();  // A
            if (pend >= 0) store_rows(0);
            load_out(reload, sr, at(c_load), rb, lane);
            __syncthreads();  // B
            if (pend >= 0) store_rows(2);
        };
        OutOps sp, sq;
        load_out(sp, sr, at(X), rb, lane);
        __builtin_amdgcn_sched_barrier(0);
        load_out(sq, sr, at(X + 2), rb, lane);
        // groups of four chunks g .. g + 3: own chunks g + X (sp) and g + 2 + X (sq)
        auto group = [&](int g, int lim) {
            if (X == 0) {
                if (0 < lim) own(sp, g);
                if (1 < lim) other(sp, g + 4);
                if (2 < lim) own(sq, g + 2);
                if (3 < lim) other(sq, g + 6);
            } else {
                if (0 < lim) other(sq, g + 3);  // own chunk g - 1 used sq
                if (1 < lim) own(sp, g + 1);
                if (2 < lim) other(sp, g + 5);
                if (3 < lim) own(sq, g + 3);
            }
        };
        const int NC4 = NC & ~3;
        for (int g = 0; g < NC4; g += 4) group(g, 4);
        if (NC4 < NC) group(NC4, NC - NC4);
        if (pend == NC - 1) {
            // the last chunk was this set's, with no later window for its stores (a set's own
            // chunk before that was stored in the windows of the chunk after it)
            store_rows(0);
            store_rows(2);
        }
    } else {
        bf16* sbt = sbt_[0];
        bf16* vnt = vnt_[0];
        auto step = [&](const OutOps& cur, int c) {
            __syncthreads();  // A
            u32x4 sb[NSUB][4];
#pragma unroll
            for (int hf = 0; hf < NSUB; hf++)
#pragma unroll
                for (int s = 0; s < 4; s++) sb[hf][s] = lds_perm(sbt + 16 * hf * SLD, SLD, col, s, grp);
            __builtin_amdgcn_sched_barrier(0);
            f32x4 acc[NSUB];
#pragma unroll
            for (int hf = 0; hf < NSUB; hf++) {
                acc[hf] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < 4; s++) acc[hf] = mfma16(cur.qd[s], sb[hf][s], acc[hf]);
            }
            __syncthreads();  // B
            u32x4 vb[NSUB][2];
#pragma unroll
            for (int hf = 0; hf < NSUB; hf++) {
                vb[hf][0] = lds_perm(vnt + 16 * hf * VLD, VLD, col, 0, grp);
                vb[hf][1] = lds_perm(vnt + 16 * hf * VLD, VLD, col, 1, grp);
            }
            __builtin_amdgcn_sched_barrier(0);
            const auto ro = out_rows(o + (size_t)h * DK + v0, c, T, H);
#pragma unroll
            for (int hf = 0; hf < NSUB; hf++) {
                acc[hf] = mfma16(cur.pb[0], vb[hf][0], acc[hf]);
                if (rb >= 2) acc[hf] = mfma16(cur.pb[1], vb[hf][1], acc[hf]);
#pragma unroll
                for (int r = 0; r < 4; r++)
                    __builtin_amdgcn_raw_buffer_store_b16(to_bf16(acc[hf][r]), ro,
                                                          ((16 * rb + 4 * grp + r) * H * DK + 16 * hf + col) * 2, 0, 0);
            }
        };
        OutOps opa, opb, opc, opd;
        load_out(opa, sr, at(0), rb, lane);
        __builtin_amdgcn_sched_barrier(0);  // the sets in order: the loop's waits count whole sets
        load_out(opb, sr, at(1), rb, lane);
        __builtin_amdgcn_sched_barrier(0);  // the sets in order: the loop's waits count whole sets
        load_out(opc, sr, at(2), rb, lane);
        const int NC4 = NC & ~3;  // the same group / tail split as the chain waves
        for (int c = 0; c < NC4; c += 4) {
            load_out(opd, sr, at(c + 3), rb, lane);
            step(opa, c);
            load_out(opa, sr, at(c + 4), rb, lane);
            step(opb, c + 1);
            load_out(opb, sr, at(c + 5), rb, lane);
            step(opc, c + 2);
            load_out(opc, sr, at(c + 6), rb, lane);
            step(opd, c + 3);
        }
        if (NC4 < NC) step(opa, NC4);
        if (NC4 + 1 < NC) step(opb, NC4 + 1);
        if (NC4 + 2 < NC) step(opc, NC4 + 2);
    }
}

// T == 0: s_out = s_in, or zero (a kernel rather than a memset/memcpy node, so that a
// captured graph re-executes it).
__global__ void __launch_bounds__(256) state_pass(const float4* __restrict__ s_in, float4* __restrict__ s_out, size_t n4) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n4) s_out[i] = s_in ? s_in[i] : float4{0.f, 0.f, 0.f, 0.f};
}

// Long single sequences run as consecutive segments of at most SEG_BYTES of records each:
// prep and scan of segment j, then of segment j + 1 from the state segment j left, all on
// the caller's stream. A segment's records are then still in the 256 MB memory-side
// (Infinity) cache when the scan reads them back, instead of coming from HBM (measured at
// T = 8192, 32 heads: the scan's chunk step takes 0.84 us with 4096-token segments and
// about 1.4 us over the whole sequence). The segments split at chunk boundaries and the
// float32 state passes between them unrounded, so the result is bit for bit the one-shot
// result (the reference's two-phase == one-shot invariant). Segments reuse the start of the
// workspace; two float32 [H, 128, 128] states after the records alternate between them.
#ifndef Q35_SEG_MB
#define Q35_SEG_MB 200
#endif
constexpr size_t SEG_BYTES = (size_t)Q35_SEG_MB << 20;
constexpr size_t REC_BYTES = 72 * 1024;

struct Plan {
    int NC;         // chunks of the sequence
    int seg;        // chunks per segment (== NC: one segment)
    size_t states;  // byte offset of the two segment states in the workspace (seg > 0 only)
    size_t total;   // workspace bytes
};

Plan plan_segments(int T, int H) {
    Plan p;
    p.NC = (T + C - 1) / C;
    const size_t max_chunks = std::max<size_t>(1, SEG_BYTES / (REC_BYTES * (size_t)std::max(H, 1)));
    const int nseg = (int)((p.NC + max_chunks - 1) / max_chunks);
    p.seg = nseg <= 1 ? p.NC : (p.NC + nseg - 1) / nseg;
    // The size stays that of all NC chunks' records (so a buffer sized for T also serves a
    // packed launch of T rows), plus the two states when the sequence is segmented.
    const size_t recs = Layout((size_t)p.NC, H).total;
    p.states = (recs + 255) / 256 * 256;
    p.total = nseg <= 1 ? recs : p.states + 2 * (size_t)H * DK * DK * 4;
    return p;
}

// Form choices a test can force (-1: chosen by the launch shape). They are process-wide and
// set only through q35_gdn_force_forms, a test hook outside the op ABI; the op entry points
// never read the environment.
std::atomic<int> force_prep_wide{-1}, force_prep_split{-1}, force_scan_halves{-1}, force_scan_osets{-1};

// gdn_prep8 when every item gets a CU of its own (the launch is latency-bound); gdn_prep (three
// 4-wave blocks per CU) otherwise.
bool prep_wide(long items) {
    const int f = force_prep_wide.load(std::memory_order_relaxed);
    if (f >= 0) return f != 0;
    const int cus = device_cus();
    return cus > 0 && items <= cus;
}

// gdn_prep8 as two blocks per item (the inverse path and the q side on CUs of their own) when
// twice the items still fit the device.
bool prep_split(long items) {
    const int f = force_prep_split.load(std::memory_order_relaxed);
    if (f >= 0) return f != 0;
    const int cus = device_cus();
    return cus > 0 && 2 * items <= cus;
}

// Halves per scan block: one 8-wave scan block fits a CU, so `units` (heads x sequences)
// blocks of NSUB halves run in ceil(units * 8 / NSUB / CUs) rounds. The two-half block's chunk
// step is ~1.46x the one-half block's (measured alone on the device: 1.24 vs 0.85 us), so it
// is chosen when it saves enough rounds (config 2's 32 heads: one round either way, one half;
// 48 heads: two rounds against one, two halves).
int scan_halves(int units) {
    const int f = force_scan_halves.load(std::memory_order_relaxed);
    if (f == 1 || f == 2) return f;
    const long cus = device_cus();
    if (cus <= 0) return 1;
    const long r1 = ((long)units * 8 + cus - 1) / cus, r2 = ((long)units * 4 + cus - 1) / cus;
    return 146 * r2 < 100 * r1 ? 2 : 1;
}

// Output-wave sets of the one-half scan block (gdn_scan's OS); both give the same bits.
int scan_output_sets() {
    const int f = force_scan_osets.load(std::memory_order_relaxed);
    return f == 1 ? 1 : 2;
}

// One launch pair over packed sequences (gs.n > 0: T is the total row count and gs
// describes the sequences, their chunk offsets filled here) or over one sequence (or one
// segment of it) of T rows.
// The prep kernel's dynamic LDS limit, set once per process for each of its forms.
template <typename K>
hipError_t allow_smem(K kernel, int bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                               bytes);
}

int gdn_launch(const void* q, const void* k, const void* v, const Gates& gt, void* o, float* workspace, int T, int H,
               int HK, float scale, const void* s_in, size_t s_in_stride, void* s_out, size_t s_out_stride, GSeqs gs,
               hipStream_t st) {
    static const hipError_t configured = [] {
        hipError_t e = allow_smem(gdn_prep<false>, PREP_SMEM);
        if (e == hipSuccess) e = allow_smem(gdn_prep<true>, PREP_SMEM);
        if (e == hipSuccess) e = allow_smem(gdn_prep8<false>, PREP8_SMEM);
        if (e == hipSuccess) e = allow_smem(gdn_prep8<true>, PREP8_SMEM);
        return e;
    }();
    if (configured != hipSuccess) return configured;
    int NC = (T + C - 1) / C, nseq = 1;
    if (gs.n > 0) {
        nseq = gs.n;
        gs.chk[0] = 0;
        for (int i = 0; i < gs.n; i++) gs.chk[i + 1] = gs.chk[i] + (gs.tok[i + 1] - gs.tok[i] + C - 1) / C;
        NC = gs.chk[gs.n];
    }
    if (NC == 0) return hipSuccess;
    const Work ws = split(workspace, NC, H);
    const bf16 *qb = static_cast<const bf16*>(q), *kb = static_cast<const bf16*>(k), *vb = static_cast<const bf16*>(v);
    const bool gated = gt.b != nullptr;
    if (prep_wide((long)NC * H)) {
        const dim3 grid(NC, H, prep_split((long)NC * H) ? 2 : 1);
        if (gated) gdn_prep8<true><<<grid, PT8, PREP8_SMEM, st>>>(qb, kb, vb, gt, ws, T, H, HK, scale, gs);
        else gdn_prep8<false><<<grid, PT8, PREP8_SMEM, st>>>(qb, kb, vb, gt, ws, T, H, HK, scale, gs);
    } else {
        if (gated) gdn_prep<true><<<dim3(NC, H), PT, PREP_SMEM, st>>>(qb, kb, vb, gt, ws, T, H, HK, scale, gs);
        else gdn_prep<false><<<dim3(NC, H), PT, PREP_SMEM, st>>>(qb, kb, vb, gt, ws, T, H, HK, scale, gs);
    }
    const int halves = scan_halves(H * nseq);
    const int osets = halves == 1 ? scan_output_sets() : 1;
    auto scan = halves == 2 ? gdn_scan<2, 1> : osets == 2 ? gdn_scan<1, 2> : gdn_scan<1, 1>;
    scan<<<H * (DK / (BV * halves)) * nseq, 256 + 256 * osets, 0, st>>>(ws, ws.decay, static_cast<bf16*>(o), T, H, NC,
                                                        static_cast<const float*>(s_in), s_in_stride,
                                                        static_cast<float*>(s_out), s_out_stride, gs);
    return hipGetLastError();
}

int gdn_run(const void* q, const void* k, const void* v, const Gates& gt, void* o, float* workspace,
            int T, int H, int HK, float scale, const void* s_in, size_t s_in_stride, void* s_out,
            size_t s_out_stride, GSeqs gs, void* stream) {
    if (T < 0 || H <= 0 || HK <= 0 || H % HK != 0) return hipErrorInvalidValue;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const float* si = static_cast<const float*>(s_in);
    float* so = static_cast<float*>(s_out);
    if (gs.n == 0 && T == 0) {
        if (so == nullptr) return hipSuccess;
        const size_t n4 = (size_t)H * DK * DK / 4;
        state_pass<<<cdiv(n4, 256), 256, 0, st>>>(reinterpret_cast<const float4*>(si), reinterpret_cast<float4*>(so),
                                                  n4);
        return hipGetLastError();
    }
    if (T > 0 && (!all_set({q, k, v, o, workspace}) || (gt.b == nullptr && !all_set({gt.g, gt.beta}))))
        return hipErrorInvalidValue;
    if (((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
          reinterpret_cast<uintptr_t>(workspace)) & 15) != 0)
        return hipErrorInvalidValue;
    if (gs.n > 0)
        return gdn_launch(q, k, v, gt, o, workspace, T, H, HK, scale, s_in, s_in_stride, s_out, s_out_stride, gs,
                          st);
    const Plan p = plan_segments(T, H);
    if (p.seg >= p.NC)
        return gdn_launch(q, k, v, gt, o, workspace, T, H, HK, scale, s_in, 0, s_out, 0, gs, st);
    float* states[2] = {reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(workspace) + p.states),
                        reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(workspace) + p.states) +
                            (size_t)H * DK * DK};
    const float* cur_in = si;
    for (int c0 = 0, j = 0; c0 < p.NC; c0 += p.seg, j++) {
        const int t0 = c0 * C, len = std::min(T - t0, p.seg * C);
        const bool last = c0 + p.seg >= p.NC;
        float* out = last ? so : states[j & 1];
        const int rc = gdn_launch(static_cast<const bf16*>(q) + (size_t)t0 * HK * DK,
                                  static_cast<const bf16*>(k) + (size_t)t0 * HK * DK,
                                  static_cast<const bf16*>(v) + (size_t)t0 * H * DK, gt.from_row(t0, H),
                                  static_cast<bf16*>(o) + (size_t)t0 * H * DK, workspace, len, H, HK, scale, cur_in, 0,
                                  out, 0, gs, st);
        if (rc != 0) return rc;
        cur_in = out;
    }
    return hipSuccess;
}

}  // namespace
}  // namespace q35

using namespace q35;

#ifdef Q35_PHASE_TIMING
extern "C" int q35_debug_phase_ticks(unsigned long long* out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(q35_phase_ticks), sizeof(q35_phase_ticks));
}
extern "C" int q35_debug_wave_ticks(unsigned long long* out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(q35_wave_ticks), sizeof(q35_wave_ticks));
}
#endif

// Test hook (no reference counterpart, not part of the op ABI): forces the prep and scan forms
// that the bit-identity tests compare. -1 restores the shape-based choice. Every form gives the
// same bits, so the hook changes only which kernels run.
extern "C" int q35_gdn_force_forms(int prep_wide_, int prep_split_, int scan_halves_, int scan_osets_) {
    force_prep_wide.store(prep_wide_, std::memory_order_relaxed);
    force_prep_split.store(prep_split_, std::memory_order_relaxed);
    force_scan_halves.store(scan_halves_, std::memory_order_relaxed);
    force_scan_osets.store(scan_osets_, std::memory_order_relaxed);
    return 0;
}

namespace {
// precomputed gates (the reference's entry points)
Gates given(const float* g, const void* beta) {
    return Gates{g, static_cast<const bf16*>(beta), nullptr, nullptr, 0, nullptr, nullptr};
}
}  // namespace

extern "C" size_t cs1_gdn_workspace_floats(int T, int H) {
    if (T < 0 || H < 0) return 0;
    return (plan_segments(T, std::max(H, 1)).total + 3) / 4;
}

extern "C" int cs1_gdn_prefill(const void* q, const void* k, const void* v, const float* g, const void* beta, void* o,
                               float* workspace, int T, int H, int HK, float scale, void* stream) {
    return gdn_run(q, k, v, given(g, beta), o, workspace, T, H, HK, scale, nullptr, 0, nullptr, 0, GSeqs{0, {}, {}},
                   stream);
}

extern "C" int cs1_gdn_prefill_x(const void* q, const void* k, const void* v, const float* g, const void* beta,
                                 void* o, float* workspace, int T, int H, int HK, float scale, const void* s_in,
                                 void* s_out, void* stream) {
    return gdn_run(q, k, v, given(g, beta), o, workspace, T, H, HK, scale, s_in, 0, s_out, 0, GSeqs{0, {}, {}},
                   stream);
}

// ---- cs1_gdn_prefill_x_static: the same launch pair with a library-owned workspace ----
//
// For callers that cannot allocate (code under graph capture, tight serving loops): the
// workspace is this file-scope device array, one copy per GPU, held until the process ends.
// Host code never passes `scratch` itself to a kernel (its host-side name is only a stand-in
// for the symbol); it passes the device address that hipGetSymbolAddress returns, looked up
// once per device with that device current. The prep kernel writes every workspace byte the
// scan reads, so nothing has to be cleared between calls. Calls that overlap on one GPU share
// the array and race; a caller serialises them (one stream, or events).
constexpr size_t STATIC_SCRATCH_BYTES = (size_t)64 << 20;
__device__ __align__(256) unsigned char scratch[STATIC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex scratch_mutex;
void* scratch_ptr[MAX_DEVICES];

// The current device's address of `scratch`, looked up on the first call on that device.
hipError_t device_scratch(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (!scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        scratch_ptr[dev] = p;
    }
    *out = scratch_ptr[dev];
    return hipSuccess;
}
}  // namespace

extern "C" int cs1_gdn_prefill_x_static(const void* q, const void* k, const void* v, const float* g, const void* beta,
                                        void* o, int T, int H, int HK, float scale, const void* s_in, void* s_out,
                                        void* stream) {
    if (T < 0 || H <= 0) return hipErrorInvalidValue;
    if (plan_segments(T, H).total > STATIC_SCRATCH_BYTES) return hipErrorInvalidValue;
    void* ws = nullptr;
    const hipError_t e = device_scratch(&ws);
    if (e != hipSuccess) return e;
    return gdn_run(q, k, v, given(g, beta), o, static_cast<float*>(ws), T, H, HK, scale, s_in, 0, s_out, 0,
                   GSeqs{0, {}, {}}, stream);
}

namespace {
int varlen_run(const void* q, const void* k, const void* v, const Gates& gt, void* o, float* workspace,
               const int32_t* cu_seqlens, int nseq, int H, int HK, float scale, const void* s_in, size_t s_in_stride,
               void* s_out, size_t s_out_stride, void* stream) {
    if (nseq < 0 || nseq > GSEQS_MAX) return hipErrorInvalidValue;
    if (nseq == 0) return hipSuccess;
    if (!cu_seqlens || cu_seqlens[0] != 0) return hipErrorInvalidValue;
    GSeqs gs;
    gs.n = nseq;
    for (int i = 0; i <= nseq; i++) {
        if (i > 0 && cu_seqlens[i] < cu_seqlens[i - 1]) return hipErrorInvalidValue;
        gs.tok[i] = cu_seqlens[i];
    }
    return gdn_run(q, k, v, gt, o, workspace, cu_seqlens[nseq], H, HK, scale, s_in, s_in_stride, s_out, s_out_stride,
                   gs, stream);
}

// The raw gate projections of the gated entry points; null when the arguments are invalid.
bool raw_gates(const void* b, const void* a, int ld, const void* A_log, const void* dt_bias, int H, Gates* out) {
    if (!b || !a || !A_log || !dt_bias || ld < H) return false;
    *out = Gates{nullptr,
                 nullptr,
                 static_cast<const bf16*>(b),
                 static_cast<const bf16*>(a),
                 ld,
                 static_cast<const bf16*>(A_log),
                 static_cast<const bf16*>(dt_bias)};
    return true;
}
}  // namespace

extern "C" int cs1_gdn_prefill_varlen(const void* q, const void* k, const void* v, const float* g, const void* beta,
                                      void* o, float* workspace, const int32_t* cu_seqlens, int nseq, int H, int HK,
                                      float scale, const void* s_in, size_t s_in_stride, void* s_out,
                                      size_t s_out_stride, void* stream) {
    return varlen_run(q, k, v, given(g, beta), o, workspace, cu_seqlens, nseq, H, HK, scale, s_in, s_in_stride, s_out,
                      s_out_stride, stream);
}

extern "C" int cs1_gdn_prefill_gated_x(const void* q, const void* k, const void* v, const void* b, const void* a,
                                       int ld, const void* A_log, const void* dt_bias, void* o, float* workspace,
                                       int T, int H, int HK, float scale, const void* s_in, void* s_out,
                                       void* stream) {
    Gates gt{};
    if (T > 0 && !raw_gates(b, a, ld, A_log, dt_bias, H, &gt)) return hipErrorInvalidValue;
    return gdn_run(q, k, v, gt, o, workspace, T, H, HK, scale, s_in, 0, s_out, 0, GSeqs{0, {}, {}}, stream);
}

extern "C" int cs1_gdn_prefill_gated_varlen(const void* q, const void* k, const void* v, const void* b,
                                            const void* a, int ld, const void* A_log, const void* dt_bias, void* o,
                                            float* workspace, const int32_t* cu_seqlens, int nseq, int H, int HK,
                                            float scale, const void* s_in, size_t s_in_stride, void* s_out,
                                            size_t s_out_stride, void* stream) {
    Gates gt{};
    if (nseq > 0 && !raw_gates(b, a, ld, A_log, dt_bias, H, &gt)) return hipErrorInvalidValue;
    return varlen_run(q, k, v, gt, o, workspace, cu_seqlens, nseq, H, HK, scale, s_in, s_in_stride, s_out,
                      s_out_stride, stream);
}
