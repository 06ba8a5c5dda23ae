// Native host runner of the Qwen3.5-style hybrid decoder prefill over the cs1_* ABI.
//
// The op sequence is the reference executor's (src/models/qwen3_5/native/src/model.rs):
//   embed ids -> res; x = rms_norm(res, input_norm[0])                     (1075-1098, 1143-1156)
//   per layer:
//     Gated DeltaNet: gdn_in = x W_in^T; conv1d + SiLU -> q, k, v; gates (b, a) -> beta, g;
//       o = gdn_prefill(q, k, v, g, beta); ln = gated_rms_norm(o, z); delta = ln W_out^T
//                                                                          (1159-1233)
//     full attention: attn_in = x W_qkv^T; attn_prep (q/k norm, RoPE, gate split);
//       ao = attention_gated(q, k, v in place, gate); delta = ao W_o^T     (1234-1285)
//     res += delta, x = rms_norm(res, post_norm)                            (1287-1300)
//     gate_up = x W_gu^T; act = silu(gate) up; delta = act W_down^T        (1301-1315)
//     res += delta, x = rms_norm(res, next layer's input_norm or final_norm) (1316-1332)
//   last hidden = x[T - 1] as float32                                       (1100-1115)
// and the decision head of src/models/cua_s1/native/src/executor.rs:61-78 (float64 dot
// products of embedding rows with the last hidden state).
//
// Memory: the weights live in one device allocation (about 8 GB for the 4B-class
// configuration), the per-prompt buffers in a second one sized for max_tokens.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <map>
#include <new>
#include <vector>

#include "qwen3_5_model.h"
#include "qwen3_5_ops.h"

namespace {

constexpr size_t BF16 = 2;

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// ---------------------------------------------------------------- device initialisation

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
    size_t kd, vd, conv, gdn_in, attn_q, attn_in;
};

struct Scratch {
    size_t ids, res, x, delta, gdn_in, lq, lk, lv, lo, ln, beta, g, ws, attn_in, aq, agate, ak, ao, gate_up, act,
        cos, sin, total;
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
    Tensor embed, final_norm;
    std::vector<Layer> layers;
    bool graph_enabled = false;
    std::map<int, void*> graphs;  // prompt length -> executable graph
    int cos_len = 0;              // positions held by the rotary tables
};

void* at(Model& m, const Tensor& t) { return m.weights + t.off; }
void* sc(Model& m, size_t off, size_t row_bytes = 0, size_t row = 0) { return m.scratch + off + row * row_bytes; }

#define TRY(x)                          \
    do {                                \
        const int rc_ = (x);            \
        if (rc_ != 0) return rc_;       \
    } while (0)

bool valid(const Q35ModelConfig& c) {
    return c.layers > 0 && c.hidden > 0 && c.hidden % 8 == 0 && c.intermediate > 0 && c.intermediate % 8 == 0 &&
           c.vocab > 0 && c.heads > 0 && c.kv_heads > 0 && c.heads % c.kv_heads == 0 && c.head_dim == 256 &&
           c.rotary_half > 0 && 2 * c.rotary_half <= c.head_dim && c.lin_k_heads > 0 && c.lin_v_heads > 0 &&
           c.lin_v_heads % c.lin_k_heads == 0 && c.lin_k_dim == 128 && c.lin_v_dim == 128 &&
           c.full_attention_interval > 0 && c.eps > 0.f && c.rope_theta > 0.0;
}

int fill(Model& m, const Tensor& t, uint64_t key, int kind, float value) {
    if (t.numel == 0) return 0;
    const unsigned blocks = (unsigned)std::min<size_t>((t.numel + 255) / 256, 65536);
    fill_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(m.stream)>>>(
        reinterpret_cast<uint16_t*>(at(m, t)), t.numel, key, kind, value);
    return hipGetLastError();
}

// Rotary tables for positions 0 .. T-1 as the reference computes them on the host
// (src/models/qwen3_5/native/src/inputs.rs:75-93, all three position axes equal for text):
// float32 inverse frequencies theta^(-2i / (2 half)), float32 angle, float64 cos / sin,
// rounded to bfloat16.
int rotary(Model& m, int T) {
    const int half = m.cfg.rotary_half;
    std::vector<float> inv(half);
    for (int i = 0; i < half; i++)
        inv[i] = 1.f / powf((float)m.cfg.rope_theta, (float)(2 * i) / (float)(2 * half));
    std::vector<uint16_t> c((size_t)T * half), s((size_t)T * half);
    auto rne = [](float x) {
        uint32_t u;
        std::memcpy(&u, &x, 4);
        return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    };
    for (int t = 0; t < T; t++)
        for (int i = 0; i < half; i++) {
            const double a = (double)(inv[i] * (float)t);
            c[(size_t)t * half + i] = rne((float)std::cos(a));
            s[(size_t)t * half + i] = rne((float)std::sin(a));
        }
    TRY(cs1_upload(sc(m, m.s.cos), c.data(), c.size() * 2, m.stream));
    TRY(cs1_upload(sc(m, m.s.sin), s.data(), s.size() * 2, m.stream));
    m.cos_len = T;
    return 0;
}

// y [T, N] = x [T, K] W^T with W [N, K]
int gemm(Model& m, size_t x, const Tensor& wt, size_t y, int T, int N, int K) {
    return cs1_gemm(m.gemm, sc(m, x), at(m, wt), sc(m, y), T, N, K, N, m.stream);
}

// The layer stack on embedded rows (res already holds the embeddings).
int run(Model& m, int T) {
    const Q35ModelConfig& c = m.cfg;
    const Widths& w = m.w;
    const int hv = c.lin_v_heads, hq = c.heads, hk = c.kv_heads, hd = c.head_dim;
    void* st = m.stream;
    TRY(cs1_rms_norm(sc(m, m.s.res), at(m, m.layers[0].input_norm), sc(m, m.s.x), T, c.hidden, c.eps, st));
    for (size_t i = 0; i < m.layers.size(); i++) {
        const Layer& L = m.layers[i];
        if (!L.full) {
            const int ld = (int)w.gdn_in;
            TRY(gemm(m, m.s.x, L.gdn_in, m.s.gdn_in, T, (int)w.gdn_in, c.hidden));
            unsigned char* base = static_cast<unsigned char*>(sc(m, m.s.gdn_in));
            unsigned char* z = base + w.conv * BF16;
            unsigned char* b = z + w.vd * BF16;
            unsigned char* a = b + hv * BF16;
            TRY(cs1_gdn_conv(base, ld, at(m, L.conv), sc(m, m.s.lq), sc(m, m.s.lk), sc(m, m.s.lv), T, (int)w.kd,
                             (int)w.vd, st));
            TRY(cs1_gdn_gates(b, a, ld, at(m, L.a_log), at(m, L.dt_bias), sc(m, m.s.beta),
                              static_cast<float*>(sc(m, m.s.g)), T, hv, st));
            TRY(cs1_gdn_prefill(sc(m, m.s.lq), sc(m, m.s.lk), sc(m, m.s.lv), static_cast<const float*>(sc(m, m.s.g)),
                                sc(m, m.s.beta), sc(m, m.s.lo), static_cast<float*>(sc(m, m.s.ws)), T, hv,
                                c.lin_k_heads, powf((float)c.lin_k_dim, -0.5f), st));
            TRY(cs1_gated_rms_norm(sc(m, m.s.lo), z, ld, at(m, L.gnorm), sc(m, m.s.ln), T, hv, c.lin_v_dim, c.eps,
                                   st));
            TRY(gemm(m, m.s.ln, L.gout, m.s.delta, T, c.hidden, (int)w.vd));
        } else {
            const int ld = (int)w.attn_in;
            TRY(gemm(m, m.s.x, L.qkv, m.s.attn_in, T, (int)w.attn_in, c.hidden));
            unsigned char* base = static_cast<unsigned char*>(sc(m, m.s.attn_in));
            unsigned char* k = base + w.attn_q * BF16;
            unsigned char* v = k + (size_t)hk * hd * BF16;
            TRY(cs1_attn_prep(base, k, ld, at(m, L.q_norm), at(m, L.k_norm), sc(m, m.s.cos), sc(m, m.s.sin),
                              sc(m, m.s.aq), sc(m, m.s.agate), sc(m, m.s.ak), T, hq, hk, hd, c.rotary_half, c.eps,
                              st));
            TRY(cs1_attention_gated(sc(m, m.s.aq), sc(m, m.s.ak), v, ld, sc(m, m.s.agate), sc(m, m.s.ao), T, hq, hk,
                                    hd, powf((float)hd, -0.5f), st));
            TRY(gemm(m, m.s.ao, L.o, m.s.delta, T, c.hidden, hq * hd));
        }
        TRY(cs1_add_rms_norm(sc(m, m.s.res), sc(m, m.s.delta), at(m, L.post_norm), sc(m, m.s.x), T, c.hidden, c.eps,
                             st));
        TRY(gemm(m, m.s.x, L.gate_up, m.s.gate_up, T, 2 * c.intermediate, c.hidden));
        TRY(cs1_silu_mul(sc(m, m.s.gate_up), 2 * c.intermediate, sc(m, m.s.act), T, c.intermediate, st));
        TRY(gemm(m, m.s.act, L.down, m.s.delta, T, c.hidden, c.intermediate));
        const Tensor& next = i + 1 < m.layers.size() ? m.layers[i + 1].input_norm : m.final_norm;
        TRY(cs1_add_rms_norm(sc(m, m.s.res), sc(m, m.s.delta), at(m, next), sc(m, m.s.x), T, c.hidden, c.eps, st));
    }
    return 0;
}

int forward(Model& m, const int32_t* ids, int T, float* last) {
    if (T <= 0 || T > m.max_tokens || !ids || !last) return hipErrorInvalidValue;
    for (int t = 0; t < T; t++)
        if (ids[t] < 0 || ids[t] >= m.cfg.vocab) return hipErrorInvalidValue;
    if (m.cos_len < T) TRY(rotary(m, m.max_tokens));
    TRY(cs1_upload(sc(m, m.s.ids), ids, (size_t)T * 4, m.stream));
    TRY(cs1_embed(static_cast<const int32_t*>(sc(m, m.s.ids)), at(m, m.embed), sc(m, m.s.res), T, m.cfg.hidden,
                  m.stream));
    if (m.graph_enabled) {
        auto it = m.graphs.find(T);
        if (it != m.graphs.end()) {
            TRY(cs1_graph_launch(it->second, m.stream));
        } else {
            // Run eagerly once (builds the GEMM plans and gives this call's result; run()
            // advances the residual in place, so the captured graph is not replayed now).
            TRY(run(m, T));
            TRY(cs1_stream_sync(m.stream));
            TRY(cs1_graph_begin(m.stream));
            const int rc = run(m, T);
            void* exec = nullptr;
            const int rc2 = cs1_graph_end(m.stream, &exec);
            if (rc != 0) return rc;
            if (rc2 != 0) return rc2;
            m.graphs[T] = exec;
        }
    } else {
        TRY(run(m, T));
    }
    std::vector<uint16_t> row(m.cfg.hidden);
    TRY(cs1_download(row.data(), static_cast<unsigned char*>(sc(m, m.s.x)) + (size_t)(T - 1) * m.cfg.hidden * BF16,
                     row.size() * BF16, m.stream));
    for (int i = 0; i < m.cfg.hidden; i++) {
        const uint32_t u = (uint32_t)row[i] << 16;
        std::memcpy(&last[i], &u, 4);
    }
    return 0;
}

void release(Model* m) {
    for (auto& kv : m->graphs) cs1_graph_destroy(kv.second);
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
    w.attn_in = w.attn_q + 2 * (size_t)c.kv_heads * c.head_dim;

    // weight arena
    size_t off = 0;
    auto take = [&](size_t numel) {
        Tensor t{off, numel};
        off += align256(numel * BF16);
        return t;
    };
    m->embed = take((size_t)c.vocab * c.hidden);
    m->final_norm = take(c.hidden);
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
    s.beta = buf(T * c.lin_v_heads * BF16);
    s.g = buf(T * c.lin_v_heads * 4);
    s.ws = buf(cs1_gdn_workspace_floats(max_tokens, c.lin_v_heads) * 4);
    s.attn_in = buf(T * w.attn_in * BF16);
    s.aq = buf(T * c.heads * c.head_dim * BF16);
    s.agate = buf(T * c.heads * c.head_dim * BF16);
    s.ak = buf(T * c.kv_heads * c.head_dim * BF16);
    s.ao = buf(T * c.heads * c.head_dim * BF16);
    s.gate_up = buf(T * 2 * c.intermediate * BF16);
    s.act = buf(T * c.intermediate * BF16);
    s.cos = buf(T * c.rotary_half * BF16);
    s.sin = buf(T * c.rotary_half * BF16);
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

int q35m_forward(void* model, const int32_t* ids, int T, float* last_hidden) {
    if (!model) return hipErrorInvalidValue;
    return forward(*static_cast<Model*>(model), ids, T, last_hidden);
}

int q35m_decide(void* model, const int32_t* ids, int T, const int32_t* label_ids, int n_labels, float* logits) {
    if (!model || !label_ids || n_labels <= 0 || !logits) return hipErrorInvalidValue;
    Model& m = *static_cast<Model*>(model);
    for (int i = 0; i < n_labels; i++)
        if (label_ids[i] < 0 || label_ids[i] >= m.cfg.vocab) return hipErrorInvalidValue;
    const int H = m.cfg.hidden;
    std::vector<float> last(H);
    TRY(forward(m, ids, T, last.data()));
    std::vector<uint16_t> row(H);
    for (int i = 0; i < n_labels; i++) {
        TRY(cs1_download(row.data(), static_cast<unsigned char*>(at(m, m.embed)) + (size_t)label_ids[i] * H * BF16,
                         (size_t)H * BF16, m.stream));
        double acc = 0.0;
        for (int j = 0; j < H; j++) {
            const uint32_t u = (uint32_t)row[j] << 16;
            float f;
            std::memcpy(&f, &u, 4);
            acc += (double)f * (double)last[j];
        }
        logits[i] = (float)acc;
        if (!std::isfinite(logits[i])) return hipErrorInvalidValue;
    }
    return 0;
}

int q35m_tensor(void* model, int layer, int which, void** ptr, size_t* numel) {
    if (!model || !ptr || !numel) return hipErrorInvalidValue;
    Model& m = *static_cast<Model*>(model);
    const Tensor* t = nullptr;
    if (which == Q35M_EMBED) t = &m.embed;
    else if (which == Q35M_FINAL_NORM) t = &m.final_norm;
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
