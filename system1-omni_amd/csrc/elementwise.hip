// HBM-bound elementwise kernels of the prefill: the GDN causal conv1d + SiLU, the GDN
// gates, the attention output gate, SwiGLU and the embedding gather.
//
// Rounding points follow the reference kernels (elementwise.cu:11-87): conv taps
// accumulate with fmaf in tap order then round to bf16 before SiLU, SiLU/sigmoid are
// x/(1+expf(-x)) and 1/(1+expf(-x)) in float32, and each bf16 op result is rounded.
// The layouts are the reference's; the work split is MI355X's: 16-byte accesses per
// lane, and the conv slides a 4-row window down a run of tokens in registers so every
// input row is fetched from HBM once.
#include <algorithm>

#include "common.h"

namespace q35 {
namespace {

constexpr int THREADS = 256;

// Embedding gather: the grid is flattened over (token, 16-byte chunk of a row), so
// consecutive lanes copy consecutive chunks of one row and a row's chunks are spread over
// as many lanes as it has; each lane copies `per` chunks strided by the grid width.
__global__ void __launch_bounds__(THREADS) embed_rows(const int32_t* __restrict__ ids, const Pack8* __restrict__ table,
                                                      Pack8* __restrict__ out, unsigned row_packs, size_t total) {
    const size_t stride = (size_t)gridDim.x * THREADS;
    for (size_t i = (size_t)blockIdx.x * THREADS + threadIdx.x; i < total; i += stride) {
        const size_t row = i / row_packs, col = i - row * row_packs;
        out[i] = table[(size_t)ids[row] * row_packs + col];
    }
}

// ---- causal depthwise conv1d (k = 4) + SiLU ----

constexpr int CONV_RUN = 16;       // tokens per thread (each run also reads the 3 rows before it)
constexpr int CONV_RUN_LONG = 32;  // for launches with threads to spare: less history re-read
constexpr size_t CONV_LONG_MIN_THREADS = 65536;
constexpr int CONV_BATCH = 8;      // rows loaded ahead, a batch before the previous one's stores

__device__ __forceinline__ void conv_store(bf16* q, bf16* k, bf16* v, int key_dim, int value_dim, int t, int c,
                                           const Pack8& y) {
    bf16* dst;
    if (c < key_dim)
        dst = q + (size_t)t * key_dim + c;
    else if (c < 2 * key_dim)
        dst = k + (size_t)t * key_dim + (c - key_dim);
    else
        dst = v + (size_t)t * value_dim + (c - 2 * key_dim);
    *reinterpret_cast<Pack8*>(dst) = y;
}

// Packed sequences of one conv launch (up to CONV_SEQS_MAX): sequence s is rows tok[s] ..
// tok[s + 1] - 1 and runs run[s] .. run[s + 1] - 1; every sequence starts from the same three
// history rows (hist, rows of ld; null: zeros). n == 0: one sequence of T rows, zero history.
constexpr int CONV_SEQS_MAX = 64;
struct ConvSeqs {
    int n;
    int tok[CONV_SEQS_MAX + 1], run[CONV_SEQS_MAX + 1];
    const bf16* hist;
};

// One thread owns 8 consecutive channels for RUN consecutive tokens. Requires
// 8 | key_dim, 8 | value_dim, 8 | ld and 16-byte aligned buffers (checked by the host).
template <int RUN>
__global__ void __launch_bounds__(THREADS)
    gdn_conv_vec_kernel(const bf16* __restrict__ qkv, int ld, const bf16* __restrict__ w, bf16* __restrict__ q,
                        bf16* __restrict__ k, bf16* __restrict__ v, int T, int key_dim, int value_dim,
                        const ConvSeqs sq) {
    const int packs = (2 * key_dim + value_dim) / 8;
    const int idx = blockIdx.x * THREADS + threadIdx.x;
    const int runs = sq.n > 0 ? sq.run[sq.n] : (T + RUN - 1) / RUN;
    if (idx >= packs * runs) return;
    const int cp = idx % packs;
    int run = idx / packs;
    const bf16* hist = nullptr;
    if (sq.n > 0) {
        // packed sequences: this run's sequence (a scan over at most 64) addressed alone
        int s = 0;
        while (s + 1 < sq.n && run >= sq.run[s + 1]) s++;
        run -= sq.run[s];
        const int r0 = sq.tok[s];
        T = sq.tok[s + 1] - r0;
        qkv += (size_t)r0 * ld;
        q += (size_t)r0 * key_dim;
        k += (size_t)r0 * key_dim;
        v += (size_t)r0 * value_dim;
        hist = sq.hist;
    }
    const int c = cp * 8, t0 = run * RUN;
    float wt[8][4];
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        // taps of channels c+i and c+i+1: 8 consecutive bf16 = 16 bytes
        const Pack8 p = *reinterpret_cast<const Pack8*>(w + (size_t)(c + i) * 4);
        float f[8];
        unpack8(p, f);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            wt[i][j] = f[j];
            wt[i + 1][j] = f[4 + j];
        }
    }
    float win[3][8];  // rows t-3, t-2, t-1
#pragma unroll
    for (int r = 0; r < 3; r++) {
        const int s = t0 - 3 + r;
        if (s >= 0) {
            unpack8(*reinterpret_cast<const Pack8*>(qkv + (size_t)s * ld + c), win[r]);
        } else if (hist != nullptr) {
            unpack8(*reinterpret_cast<const Pack8*>(hist + (size_t)(3 + s) * ld + c), win[r]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) win[r][i] = 0.f;
        }
    }
    const int t_end = min(T, t0 + RUN);
    auto one_row = [&](int t, const Pack8& raw) {
        float cur[8];
        unpack8(raw, cur);
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float acc = 0.f;
            // zero history rows leave acc unchanged: fmaf(w, 0, acc) == acc
            acc = fmaf(wt[i][0], win[0][i], acc);
            acc = fmaf(wt[i][1], win[1][i], acc);
            acc = fmaf(wt[i][2], win[2][i], acc);
            acc = fmaf(wt[i][3], cur[i], acc);
            y[i] = conv_silu(round_bf16(acc));
        }
        conv_store(q, k, v, key_dim, value_dim, t, c, pack8(y));
#pragma unroll
        for (int i = 0; i < 8; i++) {
            win[0][i] = win[1][i];
            win[1][i] = win[2][i];
            win[2][i] = cur[i];
        }
    };
    // a whole run: batch b + 1's loads are issued before batch b's stores (a fixed schedule,
    // fully unrolled), so a thread keeps a batch of loads in flight instead of one row
    int t = t0;
    if (t0 + RUN <= t_end) {
        Pack8 cur_b[CONV_BATCH], next_b[CONV_BATCH];
#pragma unroll
        for (int u = 0; u < CONV_BATCH; u++) cur_b[u] = *reinterpret_cast<const Pack8*>(qkv + (size_t)(t0 + u) * ld + c);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int bt = 0; bt < RUN / CONV_BATCH; bt++) {
            if (bt + 1 < RUN / CONV_BATCH) {
#pragma unroll
                for (int u = 0; u < CONV_BATCH; u++)
                    next_b[u] = *reinterpret_cast<const Pack8*>(qkv + (size_t)(t0 + (bt + 1) * CONV_BATCH + u) * ld + c);
            }
            __builtin_amdgcn_sched_barrier(0);  // the batch's loads stay ahead of this batch's rows
#pragma unroll
            for (int u = 0; u < CONV_BATCH; u++) one_row(t0 + bt * CONV_BATCH + u, cur_b[u]);
#pragma unroll
            for (int u = 0; u < CONV_BATCH; u++) cur_b[u] = next_b[u];
        }
        t = t_end;
    }
    for (; t < t_end; t++) one_row(t, *reinterpret_cast<const Pack8*>(qkv + (size_t)t * ld + c));
}

// Any shape (unaligned buffers or channel counts not a multiple of 8): one thread per
// channel and run of CONV_RUN tokens, sliding the same 3-row window as the vector kernel, one
// bf16 at a time.
__global__ void __launch_bounds__(THREADS)
    gdn_conv_any_kernel(const bf16* __restrict__ qkv, int ld, const bf16* __restrict__ w, bf16* __restrict__ q,
                        bf16* __restrict__ k, bf16* __restrict__ v, int T, int key_dim, int value_dim) {
    const int channels = 2 * key_dim + value_dim;
    const int runs = (T + CONV_RUN - 1) / CONV_RUN;
    const size_t idx = (size_t)blockIdx.x * THREADS + threadIdx.x;
    if (idx >= (size_t)runs * channels) return;
    const int c = (int)(idx % channels), t0 = (int)(idx / channels) * CONV_RUN;
    bf16* dst;
    int dld;
    if (c < key_dim) {
        dst = q + c;
        dld = key_dim;
    } else if (c < 2 * key_dim) {
        dst = k + (c - key_dim);
        dld = key_dim;
    } else {
        dst = v + (c - 2 * key_dim);
        dld = value_dim;
    }
    const float w0 = f32(w[c * 4]), w1 = f32(w[c * 4 + 1]), w2 = f32(w[c * 4 + 2]), w3 = f32(w[c * 4 + 3]);
    float h0 = t0 >= 3 ? f32(qkv[(size_t)(t0 - 3) * ld + c]) : 0.f;
    float h1 = t0 >= 2 ? f32(qkv[(size_t)(t0 - 2) * ld + c]) : 0.f;
    float h2 = t0 >= 1 ? f32(qkv[(size_t)(t0 - 1) * ld + c]) : 0.f;
    const int t_end = min(T, t0 + CONV_RUN);
    for (int t = t0; t < t_end; t++) {
        const float x = f32(qkv[(size_t)t * ld + c]);
        // taps in order; a zero (padding) row leaves the sum unchanged
        const float acc = fmaf(w3, x, fmaf(w2, h2, fmaf(w1, h1, fmaf(w0, h0, 0.f))));
        dst[(size_t)t * dld] = to_bf16(conv_silu(round_bf16(acc)));
        h0 = h1;
        h1 = h2;
        h2 = x;
    }
}

// ---- gates ----

// Rows of H heads with H % 8 == 0 and 16-byte aligned operands: a thread takes 8 heads of
// one token (one 16-byte load of b and of a, one 16-byte beta store, two of g). The head
// constants are loaded once per thread; threads of a block walk tokens with a grid stride.
__global__ void __launch_bounds__(THREADS)
    gdn_gates_vec_kernel(const bf16* __restrict__ b, const bf16* __restrict__ a, int ld,
                         const bf16* __restrict__ A_log, const bf16* __restrict__ dt_bias, bf16* __restrict__ beta,
                         float* __restrict__ g, int T, int H) {
    const int groups = H / 8;
    const size_t total = (size_t)T * groups;
    const size_t stride = (size_t)gridDim.x * THREADS;
    for (size_t i = (size_t)blockIdx.x * THREADS + threadIdx.x; i < total; i += stride) {
        const size_t t = i / groups;
        const int h0 = (int)(i - t * groups) * 8;
        float bv[8], av[8], al[8], dt[8], gv[8];
        unpack8(*reinterpret_cast<const Pack8*>(b + t * ld + h0), bv);
        unpack8(*reinterpret_cast<const Pack8*>(a + t * ld + h0), av);
        unpack8(*reinterpret_cast<const Pack8*>(A_log + h0), al);
        unpack8(*reinterpret_cast<const Pack8*>(dt_bias + h0), dt);
        Pack8 out;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            bf16 lo, hi;
            gate_values(bv[e], av[e], -expf(al[e]), dt[e], lo, gv[e]);
            gate_values(bv[e + 1], av[e + 1], -expf(al[e + 1]), dt[e + 1], hi, gv[e + 1]);
            out.w[e / 2] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        *reinterpret_cast<Pack8*>(beta + t * H + h0) = out;
        f32x4* gp = reinterpret_cast<f32x4*>(g + t * H + h0);
        gp[0] = f32x4{gv[0], gv[1], gv[2], gv[3]};
        gp[1] = f32x4{gv[4], gv[5], gv[6], gv[7]};
    }
}

// Any H or alignment: one thread per (token, head).
__global__ void __launch_bounds__(THREADS)
    gdn_gates_any_kernel(const bf16* __restrict__ b, const bf16* __restrict__ a, int ld,
                         const bf16* __restrict__ A_log, const bf16* __restrict__ dt_bias, bf16* __restrict__ beta,
                         float* __restrict__ g, int T, int H) {
    const size_t i = (size_t)blockIdx.x * THREADS + threadIdx.x;
    if (i >= (size_t)T * H) return;
    const size_t t = i / H;
    const int h = (int)(i - t * H);
    gate_values(f32(b[t * ld + h]), f32(a[t * ld + h]), -expf(f32(A_log[h])), f32(dt_bias[h]), beta[i], g[i]);
}

// ---- sigmoid gate and SwiGLU ----

__device__ __forceinline__ float gate_factor(bf16 g) { return round_bf16(gate_sigmoid(f32(g))); }

__global__ void __launch_bounds__(THREADS) sigmoid_gate_vec_kernel(Pack8* __restrict__ x, const Pack8* __restrict__ gate,
                                                                   size_t n8) {
    const size_t i = (size_t)blockIdx.x * THREADS + threadIdx.x;
    if (i >= n8) return;
    float xv[8], gv[8];
    unpack8(x[i], xv);
    const Pack8 gp = gate[i];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        gv[2 * e] = round_bf16(gate_sigmoid(lo_f32(gp.w[e])));
        gv[2 * e + 1] = round_bf16(gate_sigmoid(hi_f32(gp.w[e])));
    }
#pragma unroll
    for (int e = 0; e < 8; e++) xv[e] *= gv[e];
    x[i] = pack8(xv);
}

__global__ void __launch_bounds__(THREADS) sigmoid_gate_kernel(bf16* __restrict__ x, const bf16* __restrict__ gate,
                                                               size_t n) {
    const size_t i = (size_t)blockIdx.x * THREADS + threadIdx.x;
    if (i >= n) return;
    x[i] = to_bf16(f32(x[i]) * gate_factor(gate[i]));
}

__global__ void __launch_bounds__(THREADS) silu_mul_vec_kernel(const Pack8* __restrict__ gate_up, int ld8,
                                                               Pack8* __restrict__ out, int I8, size_t n8) {
    const size_t i = (size_t)blockIdx.x * THREADS + threadIdx.x;
    if (i >= n8) return;
    const size_t t = i / I8, j = i % I8;
    const Pack8* row = gate_up + t * ld8;
    float g[8], u[8];
    unpack8(row[j], g);
    unpack8(row[I8 + j], u);
#pragma unroll
    for (int e = 0; e < 8; e++) g[e] = round_bf16(silu(g[e])) * u[e];
    out[i] = pack8(g);
}

__global__ void __launch_bounds__(THREADS) silu_mul_kernel(const bf16* __restrict__ gate_up, int ld,
                                                           bf16* __restrict__ out, int I, size_t n) {
    const size_t i = (size_t)blockIdx.x * THREADS + threadIdx.x;
    if (i >= n) return;
    const size_t t = i / I, j = i % I;
    const bf16* row = gate_up + t * ld;
    out[i] = to_bf16(round_bf16(silu(f32(row[j]))) * f32(row[I + j]));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace q35

using namespace q35;

extern "C" int cs1_embed(const int32_t* ids, const void* table, void* out, int T, int D, void* stream) {
    if (D % 8 != 0 || D < 0 || T < 0) return hipErrorInvalidValue;
    if (T == 0 || D == 0) return hipSuccess;
    if (!all_set({ids, table, out}) || !aligned16(table) || !aligned16(out)) return hipErrorInvalidValue;
    const size_t total = (size_t)T * (D / 8);
    const unsigned blocks = (unsigned)std::min<size_t>(cdiv(total, THREADS), 2048);
    embed_rows<<<blocks, THREADS, 0, static_cast<hipStream_t>(stream)>>>(ids, static_cast<const Pack8*>(table),
                                                                        static_cast<Pack8*>(out), D / 8, total);
    return hipGetLastError();
}

extern "C" int cs1_gdn_conv(const void* qkv, int ld, const void* w, void* q, void* k, void* v, int T, int key_dim,
                            int value_dim, void* stream) {
    if (T < 0 || key_dim < 0 || value_dim < 0 || ld < 2 * key_dim + value_dim) return hipErrorInvalidValue;
    const int channels = 2 * key_dim + value_dim;
    const size_t n = (size_t)T * channels;
    if (n == 0) return hipSuccess;
    if (!all_set({qkv, w, q, k, v})) return hipErrorInvalidValue;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const bool vec = key_dim % 8 == 0 && value_dim % 8 == 0 && ld % 8 == 0 && aligned16(qkv) && aligned16(w) &&
                     aligned16(q) && aligned16(k) && aligned16(v);
    if (vec) {
        ConvSeqs one;
        one.n = 0;
        one.hist = nullptr;
        const size_t threads_long = (size_t)(channels / 8) * ((T + CONV_RUN_LONG - 1) / CONV_RUN_LONG);
        if (threads_long >= CONV_LONG_MIN_THREADS) {
            gdn_conv_vec_kernel<CONV_RUN_LONG><<<cdiv(threads_long, THREADS), THREADS, 0, st>>>(
                static_cast<const bf16*>(qkv), ld, static_cast<const bf16*>(w), static_cast<bf16*>(q),
                static_cast<bf16*>(k), static_cast<bf16*>(v), T, key_dim, value_dim, one);
        } else {
            const size_t threads = (size_t)(channels / 8) * ((T + CONV_RUN - 1) / CONV_RUN);
            gdn_conv_vec_kernel<CONV_RUN><<<cdiv(threads, THREADS), THREADS, 0, st>>>(
                static_cast<const bf16*>(qkv), ld, static_cast<const bf16*>(w), static_cast<bf16*>(q),
                static_cast<bf16*>(k), static_cast<bf16*>(v), T, key_dim, value_dim, one);
        }
    } else {
        const size_t threads = (size_t)channels * ((T + CONV_RUN - 1) / CONV_RUN);
        gdn_conv_any_kernel<<<cdiv(threads, THREADS), THREADS, 0, st>>>(
            static_cast<const bf16*>(qkv), ld, static_cast<const bf16*>(w), static_cast<bf16*>(q),
            static_cast<bf16*>(k), static_cast<bf16*>(v), T, key_dim, value_dim);
    }
    return hipGetLastError();
}

extern "C" int cs1_gdn_conv_varlen(const void* qkv, int ld, const void* w, void* q, void* k, void* v,
                                   const int32_t* cu_seqlens, int nseq, const void* hist, int key_dim, int value_dim,
                                   void* stream) {
    if (nseq < 0 || nseq > CONV_SEQS_MAX || key_dim < 0 || value_dim < 0 || ld < 2 * key_dim + value_dim)
        return hipErrorInvalidValue;
    if (nseq == 0) return hipSuccess;
    if (!cu_seqlens || cu_seqlens[0] != 0 || !all_set({qkv, w, q, k, v})) return hipErrorInvalidValue;
    if (key_dim % 8 != 0 || value_dim % 8 != 0 || ld % 8 != 0 || !aligned16(qkv) || !aligned16(w) || !aligned16(q) ||
        !aligned16(k) || !aligned16(v) || (hist && !aligned16(hist)))
        return hipErrorInvalidValue;
    ConvSeqs sq;
    sq.n = nseq;
    sq.hist = static_cast<const bf16*>(hist);
    sq.tok[0] = 0;
    sq.run[0] = 0;
    for (int i = 0; i < nseq; i++) {
        if (cu_seqlens[i + 1] < cu_seqlens[i]) return hipErrorInvalidValue;
        sq.tok[i + 1] = cu_seqlens[i + 1];
        sq.run[i + 1] = sq.run[i] + (cu_seqlens[i + 1] - cu_seqlens[i] + CONV_RUN - 1) / CONV_RUN;
    }
    const size_t threads = (size_t)((2 * key_dim + value_dim) / 8) * sq.run[nseq];
    if (threads == 0) return hipSuccess;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    gdn_conv_vec_kernel<CONV_RUN><<<cdiv(threads, THREADS), THREADS, 0, st>>>(
        static_cast<const bf16*>(qkv), ld, static_cast<const bf16*>(w), static_cast<bf16*>(q), static_cast<bf16*>(k),
        static_cast<bf16*>(v), cu_seqlens[nseq], key_dim, value_dim, sq);
    return hipGetLastError();
}

extern "C" int cs1_gdn_gates(const void* b, const void* a, int ld, const void* A_log, const void* dt_bias, void* beta,
                             float* g, int T, int H, void* stream) {
    if (T < 0 || H < 0 || ld < H) return hipErrorInvalidValue;
    const size_t n = (size_t)T * H;
    if (n == 0) return hipSuccess;
    if (!all_set({b, a, A_log, dt_bias, beta, g})) return hipErrorInvalidValue;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const bf16 *pb = static_cast<const bf16*>(b), *pa = static_cast<const bf16*>(a);
    const bf16 *pl = static_cast<const bf16*>(A_log), *pd = static_cast<const bf16*>(dt_bias);
    if (H % 8 == 0 && ld % 8 == 0 && aligned16(b) && aligned16(a) && aligned16(A_log) && aligned16(dt_bias) &&
        aligned16(beta) && aligned16(g)) {
        const unsigned blocks = (unsigned)std::min<size_t>(cdiv(n / 8, THREADS), 1024);
        gdn_gates_vec_kernel<<<blocks, THREADS, 0, st>>>(pb, pa, ld, pl, pd, static_cast<bf16*>(beta), g, T, H);
    } else {
        gdn_gates_any_kernel<<<cdiv(n, THREADS), THREADS, 0, st>>>(pb, pa, ld, pl, pd, static_cast<bf16*>(beta), g, T,
                                                                   H);
    }
    return hipGetLastError();
}

extern "C" int cs1_sigmoid_gate(void* x, const void* gate, size_t n, void* stream) {
    if (n == 0) return hipSuccess;
    if (!all_set({x, gate})) return hipErrorInvalidValue;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (n % 8 == 0 && aligned16(x) && aligned16(gate))
        sigmoid_gate_vec_kernel<<<cdiv(n / 8, THREADS), THREADS, 0, st>>>(static_cast<Pack8*>(x),
                                                                          static_cast<const Pack8*>(gate), n / 8);
    else
        sigmoid_gate_kernel<<<cdiv(n, THREADS), THREADS, 0, st>>>(static_cast<bf16*>(x), static_cast<const bf16*>(gate),
                                                                  n);
    return hipGetLastError();
}

extern "C" int cs1_silu_mul(const void* gate_up, int ld, void* out, int T, int I, void* stream) {
    if (T < 0 || I < 0 || ld < 2 * I) return hipErrorInvalidValue;
    const size_t n = (size_t)T * I;
    if (n == 0) return hipSuccess;
    if (!all_set({gate_up, out})) return hipErrorInvalidValue;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (I % 8 == 0 && ld % 8 == 0 && aligned16(gate_up) && aligned16(out))
        silu_mul_vec_kernel<<<cdiv(n / 8, THREADS), THREADS, 0, st>>>(static_cast<const Pack8*>(gate_up), ld / 8,
                                                                      static_cast<Pack8*>(out), I / 8, n / 8);
    else
        silu_mul_kernel<<<cdiv(n, THREADS), THREADS, 0, st>>>(static_cast<const bf16*>(gate_up), ld,
                                                              static_cast<bf16*>(out), I, n);
    return hipGetLastError();
}
