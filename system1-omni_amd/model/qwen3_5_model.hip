// Native host runner of the Qwen3.5-style hybrid decoder prefill over the cs1_* ABI.
//
// The op sequence is the reference executor's (src/models/qwen3_5/native/src/model.rs):
//   embed ids -> res; x = rms_norm(res, input_norm[0])                     (1075-1098, 1143-1156)
//   per layer:
//     Gated DeltaNet: gdn_in = x W_in^T; conv1d + SiLU -> q, k, v;
//       o = gdn_prefill(q, k, v, gates(b, a)) (the gates computed inside the prefill: one launch
//       pair instead of the reference's separate gates kernel); ln = gated_rms_norm(o, z);
//       delta = ln W_out^T
//                                                                          (1159-1233)
//     full attention: attn_in = x W_qkv^T; attn_prep (q/k norm, RoPE, gate split);
//       ao = attention_gated(q, k, v in place, gate); delta = ao W_o^T     (1234-1285)
//     res += delta, x = rms_norm(res, post_norm)                            (1287-1300)
//     gate_up = x W_gu^T; act = silu(gate) up; delta = act W_down^T        (1301-1315)
//     res += delta, x = rms_norm(res, next layer's input_norm or final_norm) (1316-1332)
//   last hidden = x[T - 1] as float32                                       (1100-1115)
// the decision head of src/models/cua_s1/native/src/executor.rs:61-78 (float64 dot
// products of embedding rows with the last hidden state), and prefix branching: capture of a
// prompt prefix and the continuation of several candidates from it (run_window 1352-1571),
// scored by summed token log-probabilities (src/models/lfm2/engine.py:128-146).
//
// Memory: the weights live in one device allocation (about 8 GB for the 4B-class and 54 GB
// for the 27B-class configuration), the per-prompt buffers in a second one sized for
// max_tokens, a captured prefix in a third.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <new>
#include <set>
#include <tuple>
#include <vector>

#include "qwen3_5_model.h"
#include "qwen3_5_ops.h"

namespace {

constexpr size_t BF16 = 2;

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// ---------------------------------------------------------------- device kernels

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// uniform in (0, 1] from the top 24 bits
__device__ __forceinline__ float unit(uint64_t bits) { return ((float)(bits >> 40) + 1.f) * (1.f / 16777216.f); }

__device__ __forceinline__ uint16_t bf16_rne(float x) {
    const uint32_t u = __float_as_uint(x);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float bf16_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

enum Fill { FILL_NORMAL = 0, FILL_CONST = 1, FILL_LOG_UNIFORM16 = 2 };

// Element i of a tensor keyed `key`: N(0, 1) * value (Box-Muller on two counter-based
// uniforms), or the constant `value`, or log(U(0, 16)).
__global__ void fill_kernel(uint16_t* p, size_t n, uint64_t key, int kind, float value) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        float x;
        if (kind == FILL_CONST) {
            x = value;
        } else {
            const uint64_t r = mix64(key ^ mix64(i));
            if (kind == FILL_NORMAL) {
                const float u1 = unit(r), u2 = unit(mix64(r));
                x = sqrtf(-2.f * logf(u1)) * cospif(2.f * u2) * value;
            } else {
                x = logf(16.f * unit(r));
            }
        }
        p[i] = bf16_rne(x);
    }
}

template <int OP>
__device__ __forceinline__ float block_reduce(float v, float* red) {
    for (int o = 32; o > 0; o >>= 1) {
        const float w = __shfl_xor(v, o, 64);
        v = OP == 0 ? fmaxf(v, w) : v + w;
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    v = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) v = OP == 0 ? fmaxf(v, red[i]) : v + red[i];
    return v;
}

// out[r] = log softmax(logits[r, :])[target[r]] in float32 from bfloat16 logits (the
// reference scores `logits.float().log_softmax(-1)` gathered at the target). One block per
// row; V a multiple of 8 (16-byte loads).
__global__ void __launch_bounds__(256) logprob_kernel(const uint16_t* __restrict__ logits, int V,
                                                      const int32_t* __restrict__ target, float* __restrict__ out) {
    __shared__ float red[4];
    const uint4* row = reinterpret_cast<const uint4*>(logits + (size_t)blockIdx.x * V);
    const int n8 = V / 8;
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < n8; i += 256) {
        const uint4 p = row[i];
        const uint32_t w[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
        for (int e = 0; e < 4; e++)
            mx = fmaxf(mx, fmaxf(__uint_as_float(w[e] << 16), __uint_as_float(w[e] & 0xffff0000u)));
    }
    mx = block_reduce<0>(mx, red);
    float s = 0.f;
    for (int i = threadIdx.x; i < n8; i += 256) {
        const uint4 p = row[i];
        const uint32_t w[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
        for (int e = 0; e < 4; e++)
            s += expf(__uint_as_float(w[e] << 16) - mx) + expf(__uint_as_float(w[e] & 0xffff0000u) - mx);
    }
    s = block_reduce<1>(s, red);
    if (threadIdx.x == 0) {
        const float t = bf16_f32(logits[(size_t)blockIdx.x * V + target[blockIdx.x]]);
        out[blockIdx.x] = t - mx - logf(s);
    }
}

// ---------------------------------------------------------------- model

struct Tensor {
    size_t off = 0, numel = 0;
};

struct Layer {
    bool full = false;
    Tensor input_norm, post_norm;
    Tensor gdn_in, conv, a_log, dt_bias, gnorm, gout;  // Gated DeltaNet
    Tensor qkv, q_norm, k_norm, o;                      // full attention
    Tensor gate_up, down;
};

struct Widths {
    size_t kd, vd, conv, gdn_in, attn_q, attn_in, kv;
};

struct Scratch {
    size_t ids, res, x, delta, gdn_in, lq, lk, lv, lo, ln, ws, attn_in, aq, agate, ak, ao, gate_up, act,
        cos, sin, ccos, csin, hs, tgt, logits, lp, total;
};

// Per-layer state of a captured prompt prefix (offsets into the prefix allocation).
struct Prefix {
    int len = 0;
    unsigned char* mem = nullptr;
    std::vector<size_t> k, v;        // per attention layer: [len, Hk Dh] post-prep K, raw V
    std::vector<size_t> state, tail; // per GDN layer: float32 [Hv, 128, 128], 3 pre-conv rows
    size_t last = 0;                 // final-norm hidden state of row len - 1
};

struct Model {
    Q35ModelConfig cfg{};
    Widths w{};
    int max_tokens = 0;
    void* stream = nullptr;
    void* gemm = nullptr;
    unsigned char* weights = nullptr;
    unsigned char* scratch = nullptr;
    Scratch s{};
    Tensor embed, final_norm, lm_head;
    std::vector<Layer> layers;
    bool graph_enabled = false;
    bool tune_gemm = false;                         // time hipBLASLt candidates per shape
    std::set<std::tuple<int, int, int>> tuned;      // shapes (M, N, K) already tuned
    std::map<int, void*> graphs;  // prompt length -> executable graph
    int cos_len = 0;              // positions held by the rotary tables
    Prefix pre;
};

// The packed candidates of a scoring pass: rows off[c] .. off[c] + len[c] - 1.
struct Cands {
    std::vector<int> off, len;
};

enum Mode { PLAIN = 0, CAPTURE = 1, CANDIDATES = 2 };

void* at(Model& m, const Tensor& t) { return m.weights + t.off; }
unsigned char* sc(Model& m, size_t off) { return m.scratch + off; }

#define TRY(x)                          \
    do {                                \
        const int rc_ = (x);            \
        if (rc_ != 0) return rc_;       \
    } while (0)

bool valid(const Q35ModelConfig& c) {
    return c.layers > 0 && c.hidden > 0 && c.hidden % 8 == 0 && c.intermediate > 0 && c.intermediate % 8 == 0 &&
           c.vocab > 0 && c.vocab % 8 == 0 && c.heads > 0 && c.kv_heads > 0 && c.heads % c.kv_heads == 0 &&
           c.head_dim == 256 && c.rotary_half > 0 && 2 * c.rotary_half <= c.head_dim && c.lin_k_heads > 0 &&
           c.lin_v_heads > 0 && c.lin_v_heads % c.lin_k_heads == 0 && c.lin_k_dim == 128 && c.lin_v_dim == 128 &&
           c.full_attention_interval > 0 && c.eps > 0.f && c.rope_theta > 0.0 && (c.lm_head == 0 || c.lm_head == 1);
}

int fill(Model& m, const Tensor& t, uint64_t key, int kind, float value) {
    if (t.numel == 0) return 0;
    const unsigned blocks = (unsigned)std::min<size_t>((t.numel + 255) / 256, 65536);
    fill_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(m.stream)>>>(
        reinterpret_cast<uint16_t*>(at(m, t)), t.numel, key, kind, value);
    return hipGetLastError();
}

uint16_t host_bf16(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// Rotary tables for the given positions as the reference computes them on the host
// (src/models/qwen3_5/native/src/inputs.rs:75-93, all three position axes equal for text):
// float32 inverse frequencies theta^(-2i / (2 half)), float32 angle, float64 cos / sin,
// rounded to bfloat16.
int rotary_rows(Model& m, const std::vector<int>& pos, size_t cos_off, size_t sin_off) {
    const int half = m.cfg.rotary_half;
    std::vector<float> inv(half);
    for (int i = 0; i < half; i++)
        inv[i] = 1.f / powf((float)m.cfg.rope_theta, (float)(2 * i) / (float)(2 * half));
    std::vector<uint16_t> c(pos.size() * half), s(pos.size() * half);
    for (size_t t = 0; t < pos.size(); t++)
        for (int i = 0; i < half; i++) {
            const double a = (double)(inv[i] * (float)pos[t]);
            c[t * half + i] = host_bf16((float)std::cos(a));
            s[t * half + i] = host_bf16((float)std::sin(a));
        }
    TRY(cs1_upload(sc(m, cos_off), c.data(), c.size() * 2, m.stream));
    TRY(cs1_upload(sc(m, sin_off), s.data(), s.size() * 2, m.stream));
    return 0;
}

int rotary(Model& m) {
    if (m.cos_len >= m.max_tokens) return 0;
    std::vector<int> pos(m.max_tokens);
    for (int t = 0; t < m.max_tokens; t++) pos[t] = t;
    TRY(rotary_rows(m, pos, m.s.cos, m.s.sin));
    m.cos_len = m.max_tokens;
    return 0;
}

// y [T, N] = x [T, K] W^T with W [N, K]
// (the first call at a shape re-chooses its plan by timing when tuning is on; never under
// capture, where cs1_gemm keeps the deterministic plan)
int gemm(Model& m, size_t x, const Tensor& wt, size_t y, int T, int N, int K) {
    if (m.tune_gemm && T > 0 && !m.tuned.count({T, N, K})) {
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        TRY(hipStreamIsCapturing(static_cast<hipStream_t>(m.stream), &cap));
        if (cap == hipStreamCaptureStatusNone) {
            TRY(cs1_gemm_tune(m.gemm, sc(m, x), at(m, wt), sc(m, y), T, N, K, N, m.stream));
            m.tuned.insert({T, N, K});
            return 0;
        }
    }
    return cs1_gemm(m.gemm, sc(m, x), at(m, wt), sc(m, y), T, N, K, N, m.stream);
}

// Calls f(first packed row, cu_seqlens) for each group of up to 64 candidates (the packed
// launches take at most 64 sequences).
template <class F>
int for_groups(const Cands* cd, F&& f) {
    const size_t n = cd->off.size();
    for (size_t g0 = 0; g0 < n; g0 += 64) {
        const size_t g1 = std::min(n, g0 + 64);
        std::vector<int32_t> cu(g1 - g0 + 1);
        cu[0] = 0;
        for (size_t i = g0; i < g1; i++) cu[i - g0 + 1] = cu[i - g0] + cd->len[i];
        TRY(f(cd->off[g0], cu));
    }
    return 0;
}

// Packed Gated DeltaNet over the candidates, every candidate starting from the same captured
// state; the gates (b, a: rows of ld) are computed inside the prefill.
int gdn_candidates(Model& m, const Cands* cd, const void* q, const void* k, const void* v, const unsigned char* b,
                   const unsigned char* a, int ld, const Layer& L, const void* s0, float scale) {
    const Q35ModelConfig& c = m.cfg;
    const size_t kd = m.w.kd * BF16, vd = m.w.vd * BF16, row = (size_t)ld * BF16;
    return for_groups(cd, [&](int r0, const std::vector<int32_t>& cu) {
        return cs1_gdn_prefill_gated_varlen(static_cast<const unsigned char*>(q) + r0 * kd,
                                            static_cast<const unsigned char*>(k) + r0 * kd,
                                            static_cast<const unsigned char*>(v) + r0 * vd, b + r0 * row,
                                            a + r0 * row, ld, at(m, L.a_log), at(m, L.dt_bias),
                                            sc(m, m.s.lo) + r0 * vd, reinterpret_cast<float*>(sc(m, m.s.ws)),
                                            cu.data(), (int)cu.size() - 1, c.lin_v_heads, c.lin_k_heads, scale, s0, 0,
                                            nullptr, 0, m.stream);
    });
}

// The layer stack on T embedded rows (res holds the embeddings). PLAIN: one prompt from
// position 0. CAPTURE: the same, keeping the per-layer prefix state in m.pre. CANDIDATES:
// rows are the packed candidates, each continuing the captured prefix at position pre.len.
int run(Model& m, int T, Mode mode, const Cands* cd) {
    const Q35ModelConfig& c = m.cfg;
    const Widths& w = m.w;
    const Scratch& s = m.s;
    const int hv = c.lin_v_heads, hq = c.heads, hk = c.kv_heads, hd = c.head_dim;
    const size_t gw = w.gdn_in * BF16, aw = w.attn_in * BF16, qrow = (size_t)hq * hd * BF16, kvb = w.kv * BF16;
    const int P = m.pre.len;
    void* st = m.stream;
    const float gdn_scale = powf((float)c.lin_k_dim, -0.5f), att_scale = powf((float)hd, -0.5f);
    TRY(cs1_rms_norm(sc(m, s.res), at(m, m.layers[0].input_norm), sc(m, s.x), T, c.hidden, c.eps, st));
    int ai = 0, li = 0;
    for (size_t i = 0; i < m.layers.size(); i++) {
        const Layer& L = m.layers[i];
        if (!L.full) {
            const int ld = (int)w.gdn_in;
            TRY(gemm(m, s.x, L.gdn_in, s.gdn_in, T, (int)w.gdn_in, c.hidden));
            unsigned char* base = sc(m, s.gdn_in);
            unsigned char* z = base + w.conv * BF16;
            unsigned char* b = z + w.vd * BF16;
            unsigned char* a = b + hv * BF16;
            if (mode == CANDIDATES) {
                // every candidate's convolution sees the prefix's last three pre-conv rows as
                // its history, then the delta rule runs from the prefix's final state, each in
                // one packed launch per 64 candidates (model.rs:1421-1470)
                TRY(for_groups(cd, [&](int r0, const std::vector<int32_t>& cu) {
                    return cs1_gdn_conv_varlen(base + (size_t)r0 * gw, ld, at(m, L.conv),
                                               sc(m, s.lq) + (size_t)r0 * w.kd * BF16,
                                               sc(m, s.lk) + (size_t)r0 * w.kd * BF16,
                                               sc(m, s.lv) + (size_t)r0 * w.vd * BF16, cu.data(), (int)cu.size() - 1,
                                               m.pre.mem + m.pre.tail[li], (int)w.kd, (int)w.vd, st);
                }));
                TRY(gdn_candidates(m, cd, sc(m, s.lq), sc(m, s.lk), sc(m, s.lv), b, a, ld, L,
                                   m.pre.mem + m.pre.state[li], gdn_scale));
            } else {
                TRY(cs1_gdn_conv(base, ld, at(m, L.conv), sc(m, s.lq), sc(m, s.lk), sc(m, s.lv), T, (int)w.kd,
                                 (int)w.vd, st));
                // the gates are computed inside the prefill (no separate cs1_gdn_gates launch)
                TRY(cs1_gdn_prefill_gated_x(sc(m, s.lq), sc(m, s.lk), sc(m, s.lv), b, a, ld, at(m, L.a_log),
                                            at(m, L.dt_bias), sc(m, s.lo), reinterpret_cast<float*>(sc(m, s.ws)), T,
                                            hv, c.lin_k_heads, gdn_scale, nullptr,
                                            mode == CAPTURE ? m.pre.mem + m.pre.state[li] : nullptr, st));
                if (mode == CAPTURE)  // the last three pre-conv rows (model.rs:1427-1434)
                    TRY(cs1_copy_dd(m.pre.mem + m.pre.tail[li], base + (size_t)(T - 3) * gw, 3 * gw, st));
            }
            TRY(cs1_gated_rms_norm(sc(m, s.lo), z, ld, at(m, L.gnorm), sc(m, s.ln), T, hv, c.lin_v_dim, c.eps, st));
            TRY(gemm(m, s.ln, L.gout, s.delta, T, c.hidden, (int)w.vd));
            li++;
        } else {
            const int ld = (int)w.attn_in;
            TRY(gemm(m, s.x, L.qkv, s.attn_in, T, (int)w.attn_in, c.hidden));
            unsigned char* base = sc(m, s.attn_in);
            unsigned char* k = base + w.attn_q * BF16;
            unsigned char* v = k + kvb;
            const size_t co = mode == CANDIDATES ? s.ccos : s.cos, so = mode == CANDIDATES ? s.csin : s.sin;
            TRY(cs1_attn_prep(base, k, ld, at(m, L.q_norm), at(m, L.k_norm), sc(m, co), sc(m, so), sc(m, s.aq),
                              sc(m, s.agate), sc(m, s.ak), T, hq, hk, hd, c.rotary_half, c.eps, st));
            if (mode == CANDIDATES) {
                // every candidate attends to the cached prefix K/V and, causally, its own rows,
                // in one packed launch per 64 candidates (model.rs:1495-1554)
                TRY(for_groups(cd, [&](int r0, const std::vector<int32_t>& cu) {
                    return cs1_attention_prefix_varlen(sc(m, s.aq) + r0 * qrow, sc(m, s.ak) + (size_t)r0 * kvb,
                                                       v + (size_t)r0 * aw, ld, m.pre.mem + m.pre.k[ai],
                                                       m.pre.mem + m.pre.v[ai], (int)w.kv, P,
                                                       sc(m, s.agate) + r0 * qrow, sc(m, s.ao) + r0 * qrow, nullptr,
                                                       cu.data(), (int)cu.size() - 1, hq, hk, hd, att_scale, st);
                }));
            } else {
                if (mode == CAPTURE) {  // post-prep K, raw V (model.rs:1527-1531)
                    TRY(cs1_copy_dd(m.pre.mem + m.pre.k[ai], sc(m, s.ak), (size_t)T * kvb, st));
                    TRY(cs1_copy2d(m.pre.mem + m.pre.v[ai], kvb, v, aw, kvb, T, st));
                }
                TRY(cs1_attention_gated(sc(m, s.aq), sc(m, s.ak), v, ld, sc(m, s.agate), sc(m, s.ao), T, hq, hk, hd,
                                        att_scale, st));
            }
            TRY(gemm(m, s.ao, L.o, s.delta, T, c.hidden, hq * hd));
            ai++;
        }
        TRY(cs1_add_rms_norm(sc(m, s.res), sc(m, s.delta), at(m, L.post_norm), sc(m, s.x), T, c.hidden, c.eps, st));
        TRY(gemm(m, s.x, L.gate_up, s.gate_up, T, 2 * c.intermediate, c.hidden));
        TRY(cs1_silu_mul(sc(m, s.gate_up), 2 * c.intermediate, sc(m, s.act), T, c.intermediate, st));
        TRY(gemm(m, s.act, L.down, s.delta, T, c.hidden, c.intermediate));
        const Tensor& next = i + 1 < m.layers.size() ? m.layers[i + 1].input_norm : m.final_norm;
        TRY(cs1_add_rms_norm(sc(m, s.res), sc(m, s.delta), at(m, next), sc(m, s.x), T, c.hidden, c.eps, st));
    }
    return 0;
}

bool ids_ok(const Model& m, const int32_t* ids, int T) {
    for (int t = 0; t < T; t++)
        if (ids[t] < 0 || ids[t] >= m.cfg.vocab) return false;
    return true;
}

int embed(Model& m, const int32_t* ids, int T) {
    if (!ids_ok(m, ids, T)) return hipErrorInvalidValue;
    TRY(cs1_upload(sc(m, m.s.ids), ids, (size_t)T * 4, m.stream));
    return cs1_embed(reinterpret_cast<const int32_t*>(sc(m, m.s.ids)), at(m, m.embed), sc(m, m.s.res), T,
                     m.cfg.hidden, m.stream);
}

int forward_rows(Model& m, const int32_t* ids, int T) {
    if (T <= 0 || T > m.max_tokens || !ids) return hipErrorInvalidValue;
    TRY(rotary(m));
    TRY(embed(m, ids, T));
    if (!m.graph_enabled) return run(m, T, PLAIN, nullptr);
    auto it = m.graphs.find(T);
    if (it != m.graphs.end()) return cs1_graph_launch(it->second, m.stream);
    // Run eagerly once (builds the GEMM plans and gives this call's result; run() advances
    // the residual in place, so the captured graph is not replayed now).
    TRY(run(m, T, PLAIN, nullptr));
    TRY(cs1_stream_sync(m.stream));
    TRY(cs1_graph_begin(m.stream));
    const int rc = run(m, T, PLAIN, nullptr);
    void* exec = nullptr;
    const int rc2 = cs1_graph_end(m.stream, &exec);
    if (rc != 0) return rc;
    if (rc2 != 0) return rc2;
    m.graphs[T] = exec;
    return 0;
}

int forward(Model& m, const int32_t* ids, int T, float* last) {
    if (!last) return hipErrorInvalidValue;
    TRY(forward_rows(m, ids, T));
    std::vector<uint16_t> row(m.cfg.hidden);
    TRY(cs1_download(row.data(), sc(m, m.s.x) + (size_t)(T - 1) * m.cfg.hidden * BF16, row.size() * BF16, m.stream));
    for (int i = 0; i < m.cfg.hidden; i++) {
        const uint32_t u = (uint32_t)row[i] << 16;
        std::memcpy(&last[i], &u, 4);
    }
    return 0;
}

// lp[r] = log softmax(lm_head h_r)[target[r]] for rows r < R of the hidden rows at `hs`.
int token_logprobs(Model& m, size_t hs, const int32_t* targets, int R, float* lp) {
    TRY(cs1_upload(sc(m, m.s.tgt), targets, (size_t)R * 4, m.stream));
    TRY(gemm(m, hs, m.lm_head, m.s.logits, R, m.cfg.vocab, m.cfg.hidden));
    logprob_kernel<<<R, 256, 0, static_cast<hipStream_t>(m.stream)>>>(
        reinterpret_cast<const uint16_t*>(sc(m, m.s.logits)), m.cfg.vocab,
        reinterpret_cast<const int32_t*>(sc(m, m.s.tgt)), reinterpret_cast<float*>(sc(m, m.s.lp)));
    TRY(hipGetLastError());
    return cs1_download(lp, sc(m, m.s.lp), (size_t)R * 4, m.stream);
}

void free_prefix(Prefix& p) {
    if (p.mem) cs1_free(p.mem);
    p = Prefix{};
}

int capture(Model& m, const int32_t* ids, int P) {
    // every argument is checked before the previous prefix is released or any work is queued
    if (!ids || P < 64 || P % 64 != 0 || P > m.max_tokens || !ids_ok(m, ids, P)) return hipErrorInvalidValue;
    free_prefix(m.pre);
    const Q35ModelConfig& c = m.cfg;
    Prefix& p = m.pre;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += align256(bytes);
        return o;
    };
    for (const Layer& L : m.layers) {
        if (L.full) {
            p.k.push_back(take((size_t)P * m.w.kv * BF16));
            p.v.push_back(take((size_t)P * m.w.kv * BF16));
        } else {
            p.state.push_back(take((size_t)c.lin_v_heads * c.lin_k_dim * c.lin_v_dim * 4));
            p.tail.push_back(take(3 * m.w.gdn_in * BF16));
        }
    }
    p.last = take((size_t)c.hidden * BF16);
    TRY(cs1_malloc(reinterpret_cast<void**>(&p.mem), off));
    TRY(rotary(m));
    TRY(embed(m, ids, P));
    TRY(run(m, P, CAPTURE, nullptr));
    TRY(cs1_copy_dd(p.mem + p.last, sc(m, m.s.x) + (size_t)(P - 1) * c.hidden * BF16, (size_t)c.hidden * BF16,
                    m.stream));
    TRY(cs1_stream_sync(m.stream));
    p.len = P;
    return 0;
}

int score(Model& m, const int32_t* ids, const int32_t* lens, int n, double* scores) {
    if (!ids || !lens || n <= 0 || !scores || !m.cfg.lm_head || m.pre.len == 0) return hipErrorInvalidValue;
    const int P = m.pre.len;
    Cands cd;
    int R = 0;
    for (int c = 0; c < n; c++) {
        if (lens[c] <= 0 || P + lens[c] > m.max_tokens) return hipErrorInvalidValue;
        cd.off.push_back(R);
        cd.len.push_back(lens[c]);
        R += lens[c];
        if (R > m.max_tokens) return hipErrorInvalidValue;
    }
    if (!ids_ok(m, ids, R)) return hipErrorInvalidValue;
    std::vector<int> pos(R);
    for (int c = 0; c < n; c++)
        for (int j = 0; j < lens[c]; j++) pos[cd.off[c] + j] = P + j;
    TRY(rotary_rows(m, pos, m.s.ccos, m.s.csin));
    TRY(embed(m, ids, R));
    TRY(run(m, R, CANDIDATES, &cd));
    // the row predicting token j of candidate c: the prefix's last row for j = 0, else the
    // candidate's row j - 1
    const size_t hb = (size_t)m.cfg.hidden * BF16;
    for (int c = 0; c < n; c++) {
        TRY(cs1_copy_dd(sc(m, m.s.hs) + cd.off[c] * hb, m.pre.mem + m.pre.last, hb, m.stream));
        if (cd.len[c] > 1)
            TRY(cs1_copy_dd(sc(m, m.s.hs) + (cd.off[c] + 1) * hb, sc(m, m.s.x) + cd.off[c] * hb, (cd.len[c] - 1) * hb,
                            m.stream));
    }
    std::vector<float> lp(R);
    TRY(token_logprobs(m, m.s.hs, ids, R, lp.data()));
    for (int c = 0; c < n; c++) {
        double acc = 0.0;
        for (int j = 0; j < cd.len[c]; j++) acc += lp[cd.off[c] + j];
        scores[c] = acc;
    }
    return 0;
}

void release(Model* m) {
    for (auto& kv : m->graphs) cs1_graph_destroy(kv.second);
    free_prefix(m->pre);
    if (m->gemm) cs1_gemm_destroy(m->gemm);
    if (m->weights) cs1_free(m->weights);
    if (m->scratch) cs1_free(m->scratch);
    if (m->stream) cs1_stream_destroy(m->stream);
    delete m;
}

}  // namespace

extern "C" {

int q35m_create(const Q35ModelConfig* cfg, uint64_t seed, int max_tokens, void** out) {
    if (!cfg || !out || max_tokens <= 0 || !valid(*cfg)) return hipErrorInvalidValue;
    *out = nullptr;
    Model* m = new (std::nothrow) Model();
    if (!m) return hipErrorOutOfMemory;
    m->cfg = *cfg;
    m->max_tokens = max_tokens;
    const Q35ModelConfig& c = *cfg;
    Widths& w = m->w;
    w.kd = (size_t)c.lin_k_heads * c.lin_k_dim;
    w.vd = (size_t)c.lin_v_heads * c.lin_v_dim;
    w.conv = 2 * w.kd + w.vd;
    w.gdn_in = w.conv + w.vd + 2 * (size_t)c.lin_v_heads;
    w.attn_q = (size_t)c.heads * c.head_dim * 2;
    w.kv = (size_t)c.kv_heads * c.head_dim;
    w.attn_in = w.attn_q + 2 * w.kv;

    // weight arena
    size_t off = 0;
    auto take = [&](size_t numel) {
        Tensor t{off, numel};
        off += align256(numel * BF16);
        return t;
    };
    m->embed = take((size_t)c.vocab * c.hidden);
    m->final_norm = take(c.hidden);
    if (c.lm_head) m->lm_head = take((size_t)c.vocab * c.hidden);
    m->layers.resize(c.layers);
    for (int i = 0; i < c.layers; i++) {
        Layer& L = m->layers[i];
        L.full = (i + 1) % c.full_attention_interval == 0;
        L.input_norm = take(c.hidden);
        L.post_norm = take(c.hidden);
        if (L.full) {
            L.qkv = take(w.attn_in * c.hidden);
            L.q_norm = take(c.head_dim);
            L.k_norm = take(c.head_dim);
            L.o = take((size_t)c.hidden * c.heads * c.head_dim);
        } else {
            L.gdn_in = take(w.gdn_in * c.hidden);
            L.conv = take(w.conv * 4);
            L.a_log = take(c.lin_v_heads);
            L.dt_bias = take(c.lin_v_heads);
            L.gnorm = take(c.lin_v_dim);
            L.gout = take((size_t)c.hidden * w.vd);
        }
        L.gate_up = take((size_t)2 * c.intermediate * c.hidden);
        L.down = take((size_t)c.hidden * c.intermediate);
    }
    const size_t weight_bytes = off;

    // per-prompt buffers
    const size_t T = (size_t)max_tokens;
    Scratch& s = m->s;
    off = 0;
    auto buf = [&](size_t bytes) {
        const size_t o = off;
        off += align256(bytes);
        return o;
    };
    s.ids = buf(T * 4);
    s.res = buf(T * c.hidden * BF16);
    s.x = buf(T * c.hidden * BF16);
    s.delta = buf(T * c.hidden * BF16);
    s.gdn_in = buf(T * w.gdn_in * BF16);
    s.lq = buf(T * w.kd * BF16);
    s.lk = buf(T * w.kd * BF16);
    s.lv = buf(T * w.vd * BF16);
    s.lo = buf(T * w.vd * BF16);
    s.ln = buf(T * w.vd * BF16);
    // (packed candidates restart chunks per sequence: up to 64 more chunks per launch)
    s.ws = buf(cs1_gdn_workspace_floats(max_tokens + 64 * 64, c.lin_v_heads) * 4);
    s.attn_in = buf(T * w.attn_in * BF16);
    s.aq = buf(T * c.heads * c.head_dim * BF16);
    s.agate = buf(T * c.heads * c.head_dim * BF16);
    s.ak = buf(T * w.kv * BF16);
    s.ao = buf(T * c.heads * c.head_dim * BF16);
    s.gate_up = buf(T * 2 * c.intermediate * BF16);
    s.act = buf(T * c.intermediate * BF16);
    s.cos = buf(T * c.rotary_half * BF16);
    s.sin = buf(T * c.rotary_half * BF16);
    // candidate scoring: packed rotary rows, the scored hidden rows, targets, logits and
    // log-probabilities
    s.ccos = buf(T * c.rotary_half * BF16);
    s.csin = buf(T * c.rotary_half * BF16);
    s.hs = buf(T * c.hidden * BF16);
    s.tgt = buf(T * 4);
    s.logits = buf(c.lm_head ? T * c.vocab * BF16 : 0);
    s.lp = buf(T * 4);
    s.total = off;

    int rc = cs1_stream_create(&m->stream);
    if (rc == 0) rc = cs1_malloc(reinterpret_cast<void**>(&m->weights), weight_bytes);
    if (rc == 0) rc = cs1_malloc(reinterpret_cast<void**>(&m->scratch), s.total);
    if (rc == 0) {
        m->gemm = cs1_gemm_create(32u << 20);
        if (!m->gemm) rc = hipErrorOutOfMemory;
    }
    // initialisation (modeling_qwen3_5.py 812-820 and the N(0, 0.02) linears)
    uint64_t key = seed * 0x100000001b3ull;
    auto next = [&]() { return key = (key + 0x9e3779b97f4a7c15ull) * 0xd1342543de82ef95ull; };
    auto normal = [&](const Tensor& t) { return rc ? rc : (rc = fill(*m, t, next(), FILL_NORMAL, 0.02f)); };
    auto constant = [&](const Tensor& t, float v) { return rc ? rc : (rc = fill(*m, t, next(), FILL_CONST, v)); };
    normal(m->embed);
    constant(m->final_norm, 0.f);
    for (Layer& L : m->layers) {
        constant(L.input_norm, 0.f);
        constant(L.post_norm, 0.f);
        if (L.full) {
            normal(L.qkv);
            constant(L.q_norm, 0.f);
            constant(L.k_norm, 0.f);
            normal(L.o);
        } else {
            normal(L.gdn_in);
            normal(L.conv);
            if (rc == 0) rc = fill(*m, L.a_log, next(), FILL_LOG_UNIFORM16, 0.f);
            constant(L.dt_bias, 1.f);
            constant(L.gnorm, 1.f);
            normal(L.gout);
        }
        normal(L.gate_up);
        normal(L.down);
    }
    if (c.lm_head) normal(m->lm_head);
    if (rc == 0) rc = cs1_stream_sync(m->stream);
    if (rc != 0) {
        release(m);
        return rc;
    }
    *out = m;
    return 0;
}

void q35m_destroy(void* model) {
    if (model) release(static_cast<Model*>(model));
}

int q35m_set_graph(void* model, int enabled) {
    if (!model) return hipErrorInvalidValue;
    static_cast<Model*>(model)->graph_enabled = enabled != 0;
    return 0;
}

int q35m_set_gemm_tuning(void* model, int enabled) {
    if (!model) return hipErrorInvalidValue;
    static_cast<Model*>(model)->tune_gemm = enabled != 0;
    return 0;
}

int q35m_forward(void* model, const int32_t* ids, int T, float* last_hidden) {
    if (!model) return hipErrorInvalidValue;
    return forward(*static_cast<Model*>(model), ids, T, last_hidden);
}

// executor.rs:61-78 letter_logits: logit i = (float) sum_j (double) letters[i H + j] (double) last[j]
// in index order, rows i < n only; every logit is computed before any is checked, and a
// non-finite one fails the call.
int q35m_letter_logits(const float* letters, const float* last, int H, int n, float* logits) {
    if (!letters || !last || !logits || H <= 0 || n <= 0) return hipErrorInvalidValue;
    for (int i = 0; i < n; i++) {
        double acc = 0.0;
        for (int j = 0; j < H; j++) acc += (double)letters[(size_t)i * H + j] * (double)last[j];
        logits[i] = (float)acc;
    }
    for (int i = 0; i < n; i++)
        if (!std::isfinite(logits[i])) return hipErrorInvalidValue;
    return 0;
}

int q35m_decide(void* model, const int32_t* ids, int T, const int32_t* label_ids, int n_labels, float* logits) {
    if (!model || !label_ids || n_labels <= 0 || !logits) return hipErrorInvalidValue;
    Model& m = *static_cast<Model*>(model);
    for (int i = 0; i < n_labels; i++)
        if (label_ids[i] < 0 || label_ids[i] >= m.cfg.vocab) return hipErrorInvalidValue;
    const int H = m.cfg.hidden;
    std::vector<float> last(H);
    TRY(forward(m, ids, T, last.data()));
    // the label rows of the bf16 embedding, as float32 (exact)
    std::vector<uint16_t> row(H);
    std::vector<float> letters((size_t)n_labels * H);
    for (int i = 0; i < n_labels; i++) {
        TRY(cs1_download(row.data(), static_cast<unsigned char*>(at(m, m.embed)) + (size_t)label_ids[i] * H * BF16,
                         (size_t)H * BF16, m.stream));
        for (int j = 0; j < H; j++) {
            const uint32_t u = (uint32_t)row[j] << 16;
            std::memcpy(&letters[(size_t)i * H + j], &u, 4);
        }
    }
    return q35m_letter_logits(letters.data(), last.data(), H, n_labels, logits);
}

int q35m_capture(void* model, const int32_t* ids, int P) {
    if (!model) return hipErrorInvalidValue;
    return capture(*static_cast<Model*>(model), ids, P);
}

int q35m_score(void* model, const int32_t* ids, const int32_t* lens, int n, double* scores) {
    if (!model) return hipErrorInvalidValue;
    return score(*static_cast<Model*>(model), ids, lens, n, scores);
}

int q35m_logprobs(void* model, const int32_t* ids, int T, float* logprobs) {
    if (!model || !logprobs || T < 2) return hipErrorInvalidValue;
    Model& m = *static_cast<Model*>(model);
    if (!m.cfg.lm_head) return hipErrorInvalidValue;
    TRY(forward_rows(m, ids, T));
    return token_logprobs(m, m.s.x, ids + 1, T - 1, logprobs);
}

int q35m_tensor(void* model, int layer, int which, void** ptr, size_t* numel) {
    if (!model || !ptr || !numel) return hipErrorInvalidValue;
    Model& m = *static_cast<Model*>(model);
    const Tensor* t = nullptr;
    if (which == Q35M_EMBED) t = &m.embed;
    else if (which == Q35M_FINAL_NORM) t = &m.final_norm;
    else if (which == Q35M_LM_HEAD) t = &m.lm_head;
    else {
        if (layer < 0 || layer >= (int)m.layers.size()) return hipErrorInvalidValue;
        const Layer& L = m.layers[layer];
        const Tensor* table[] = {nullptr,     nullptr,  &L.input_norm, &L.post_norm, &L.gdn_in,  &L.conv,
                                 &L.a_log,    &L.dt_bias, &L.gnorm,    &L.gout,      &L.qkv,     &L.q_norm,
                                 &L.k_norm,   &L.o,       &L.gate_up,  &L.down};
        if (which < 0 || which > Q35M_MLP_DOWN) return hipErrorInvalidValue;
        t = table[which];
    }
    if (!t || t->numel == 0) return hipErrorInvalidValue;
    *ptr = at(m, *t);
    *numel = t->numel;
    return 0;
}

void* q35m_stream(void* model) { return model ? static_cast<Model*>(model)->stream : nullptr; }

}  // extern "C"
