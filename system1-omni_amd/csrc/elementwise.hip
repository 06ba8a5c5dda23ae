// HBM-bound elementwise kernels of the prefill: the GDN causal conv1d + SiLU, the GDN
// gates, the attention output gate, SwiGLU and the embedding gather.
//
// Rounding points follow the reference kernels (elementwise.cu:11-87): conv taps
// accumulate with fmaf in tap order then round to bf16 before SiLU, SiLU/sigmoid are
// x/(1+expf(-x)) and 1/(1+expf(-x)) in float32, and each bf16 op result is rounded.
// The layouts are the reference's; the work split is MI355X's: 16-byte accesses per
// lane, and the conv slides a 4-row window down a run of tokens in registers so every
// input row is fetched from HBM once.
#include "common.h"

namespace q35 {
namespace {

constexpr int THREADS = 256;

__global__ void __launch_bounds__(THREADS) embed_kernel(const int32_t* __restrict__ ids, const Pack8* __restrict__ table,
                                                        Pack8* __restrict__ out, int packs) {
    const size_t t = blockIdx.x;
    const size_t id = (size_t)ids[t];
    for (int i = threadIdx.x; i < packs; i += blockDim.x) out[t * packs + i] = table[id * packs + i];
}

// ---- causal depthwise conv1d (k = 4) + SiLU ----

constexpr int CONV_RUN = 16;  // tokens per thread

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

// One thread owns 8 consecutive channels for CONV_RUN consecutive tokens. Requires
// 8 | key_dim, 8 | value_dim, 8 | ld and 16-byte aligned buffers (checked by the host).
__global__ void __launch_bounds__(THREADS)
    gdn_conv_vec_kernel(const bf16* __restrict__ qkv, int ld, const bf16* __restrict__ w, bf16* __restrict__ q,
                        bf16* __restrict__ k, bf16* __restrict__ v, int T, int key_dim, int value_dim,
                        const ConvSeqs sq) {
    const int packs = (2 * key_dim + value_dim) / 8;
    const int idx = blockIdx.x * THREADS + threadIdx.x;
    const int runs = sq.n > 0 ? sq.run[sq.n] : (T + CONV_RUN - 1) / CONV_RUN;
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
    const int c = cp * 8, t0 = run * CONV_RUN;
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
    const int t_end = min(T, t0 + CONV_RUN);
    for (int t = t0; t < t_end; t++) {
        float cur[8];
        unpack8(*reinterpret_cast<const Pack8*>(qkv + (size_t)t * ld + c), cur);
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
    }
}

// Any shape: one thread per (t, channel).
__global__ void __launch_bounds__(THREADS)
    gdn_conv_scalar_kernel(const bf16* __restrict__ qkv, int ld, const bf16* __restrict__ w, bf16* __restrict__ q,
                           bf16* __restrict__ k, bf16* __restrict__ v, int T, int key_dim, int value_dim) {
    const int channels = 2 * key_dim + value_dim;
    const size_t idx = (size_t)blockIdx.x * THREADS + threadIdx.x;
    if (idx >= (size_t)T * channels) return;
    const int t = (int)(idx / channels), c = (int)(idx % channels);
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int s = t - 3 + j;
        if (s >= 0) acc = fmaf(f32(w[c * 4 + j]), f32(qkv[(size_t)s * ld + c]), acc);
    }
    const bf16 y = to_bf16(conv_silu(round_bf16(acc)));
    if (c < key_dim)
        q[(size_t)t * key_dim + c] = y;
    else if (c < 2 * key_dim)
        k[(size_t)t * key_dim + c - key_dim] = y;
    else
        v[(size_t)t * value_dim + c - 2 * key_dim] = y;
}

// ---- gates ----

__global__ void __launch_bounds__(THREADS)
    gdn_gates_kernel(const bf16* __restrict__ b, const bf16* __restrict__ a, int ld, const bf16* __restrict__ A_log,
                     const bf16* __restrict__ dt_bias, bf16* __restrict__ beta, float* __restrict__ g, int n, int H) {
    const int i = blockIdx.x * THREADS + threadIdx.x;
    if (i >= n) return;
    const int h = i % H;
    const size_t src = (size_t)(i / H) * ld + h;
    beta[i] = to_bf16(sigmoid(f32(b[src])));
    const float x = f32(a[src]) + f32(dt_bias[h]);
    const float sp = x > 20.f ? x : log1pf(expf(x));
    g[i] = -expf(f32(A_log[h])) * sp;
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
    if (D % 8 != 0 || D < 0) return hipErrorInvalidValue;
    if (T <= 0 || D == 0) return hipSuccess;
    embed_kernel<<<T, THREADS, 0, static_cast<hipStream_t>(stream)>>>(ids, static_cast<const Pack8*>(table),
                                                                      static_cast<Pack8*>(out), D / 8);
    return hipGetLastError();
}

extern "C" int cs1_gdn_conv(const void* qkv, int ld, const void* w, void* q, void* k, void* v, int T, int key_dim,
                            int value_dim, void* stream) {
    if (T < 0 || key_dim < 0 || value_dim < 0 || ld < 2 * key_dim + value_dim) return hipErrorInvalidValue;
    const int channels = 2 * key_dim + value_dim;
    const size_t n = (size_t)T * channels;
    if (n == 0) return hipSuccess;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const bool vec = key_dim % 8 == 0 && value_dim % 8 == 0 && ld % 8 == 0 && aligned16(qkv) && aligned16(w) &&
                     aligned16(q) && aligned16(k) && aligned16(v);
    if (vec) {
        const size_t threads = (size_t)(channels / 8) * ((T + CONV_RUN - 1) / CONV_RUN);
        ConvSeqs one;
        one.n = 0;
        one.hist = nullptr;
        gdn_conv_vec_kernel<<<cdiv(threads, THREADS), THREADS, 0, st>>>(
            static_cast<const bf16*>(qkv), ld, static_cast<const bf16*>(w), static_cast<bf16*>(q),
            static_cast<bf16*>(k), static_cast<bf16*>(v), T, key_dim, value_dim, one);
    } else {
        gdn_conv_scalar_kernel<<<cdiv(n, THREADS), THREADS, 0, st>>>(
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
    if (!cu_seqlens || cu_seqlens[0] != 0) return hipErrorInvalidValue;
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
    gdn_conv_vec_kernel<<<cdiv(threads, THREADS), THREADS, 0, st>>>(
        static_cast<const bf16*>(qkv), ld, static_cast<const bf16*>(w), static_cast<bf16*>(q), static_cast<bf16*>(k),
        static_cast<bf16*>(v), cu_seqlens[nseq], key_dim, value_dim, sq);
    return hipGetLastError();
}

extern "C" int cs1_gdn_gates(const void* b, const void* a, int ld, const void* A_log, const void* dt_bias, void* beta,
                             float* g, int T, int H, void* stream) {
    if (T < 0 || H < 0 || ld < H) return hipErrorInvalidValue;
    const int n = T * H;
    if (n == 0) return hipSuccess;
    gdn_gates_kernel<<<cdiv(n, THREADS), THREADS, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const bf16*>(b), static_cast<const bf16*>(a), ld, static_cast<const bf16*>(A_log),
        static_cast<const bf16*>(dt_bias), static_cast<bf16*>(beta), g, n, H);
    return hipGetLastError();
}

extern "C" int cs1_sigmoid_gate(void* x, const void* gate, size_t n, void* stream) {
    if (n == 0) return hipSuccess;
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
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (I % 8 == 0 && ld % 8 == 0 && aligned16(gate_up) && aligned16(out))
        silu_mul_vec_kernel<<<cdiv(n / 8, THREADS), THREADS, 0, st>>>(static_cast<const Pack8*>(gate_up), ld / 8,
                                                                      static_cast<Pack8*>(out), I / 8, n / 8);
    else
        silu_mul_kernel<<<cdiv(n, THREADS), THREADS, 0, st>>>(static_cast<const bf16*>(gate_up), ld,
                                                              static_cast<bf16*>(out), I, n);
    return hipGetLastError();
}
