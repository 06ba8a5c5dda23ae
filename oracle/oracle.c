/*
 * CPU oracle for the Qwen3.5 hybrid prefill hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links, loads or calls
 * this file; it is the checker that tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg compare the HIP kernels against.
 *
 * Every function restates the arithmetic of one reference item, cited file:line
 * relative to the reference checkout (src/backends/cuda/qwen3_5/...,
 * tests/qwen3_5/kernels.rs, src/models/qwen3_5/native/src/inputs.rs).  Three kinds
 * of functions live here:
 *   - float64 references, the ones the reference's own GPU tests use
 *     (kernels.rs:436-469 attention, kernels.rs:479-525 gated delta rule);
 *   - emulators of the reference CUDA kernels' rounding points: bfloat16 stores,
 *     TF32 pair products, the blocked float32 triangular inverse, the flash
 *     attention tile order (gdn_prefill.cu, attention.cu, elementwise.cu, norm.cu);
 *   - the input generator of the reference tests (xorshift, kernels.rs:26-36).
 *
 * Built with -ffp-contract=off so that a*b+c is never silently fused: fmaf() is
 * written out exactly where the reference kernels use it.
 *
 * Pinning (what makes each function trustworthy) is listed per function in the
 * repository's design notes and exercised by tests/test_oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- numerics */

static inline float bf(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* float -> bfloat16, round to nearest even (NaN kept quiet), as __float2bfloat16
 * and the `half` crate's bf16::from_f32 both do. */
static inline uint16_t f2bf(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static inline float rbf(float x) { return bf(f2bf(x)); }

/* cvt.rna.tf32.f32 (PTX ISA): keep 10 explicit mantissa bits, round to nearest with
 * ties away from zero. Inf/NaN pass through. */
static inline float tf32_rna(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) return x;
    u += 0x1000u;
    u &= 0xffffe000u;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline float silu_f(float x) { return x / (1.f + expf(-x)); }      /* common.cuh:40 */
static inline float sigmoid_f(float x) { return 1.f / (1.f + expf(-x)); } /* common.cuh:41 */

void orc_f32_to_bf16(const float* x, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = f2bf(x[i]);
}
void orc_f32_to_tf32(const float* x, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = tf32_rna(x[i]);
}

/* ------------------------------------------------------------- generator */

/* kernels.rs:26-36: uniform values in [-amp, amp) from a xorshift64 stream,
 * rounded to bfloat16. */
void orc_xorshift_bf16(uint16_t* out, size_t n, uint64_t seed, float amp) {
    uint64_t x = (seed * 0x9e3779b97f4a7c15ull) | 1ull;
    for (size_t i = 0; i < n; i++) {
        x ^= x << 13;
        x ^= x >> 7;
        x ^= x << 17;
        const float u = (float)(x >> 40) / (float)(1ull << 24);
        out[i] = f2bf((u * 2.0f - 1.0f) * amp);
    }
}

/* ------------------------------------------------- gated delta rule, f64 */

/* kernels.rs:479-525 (transformers' torch_recurrent_gated_delta_rule in float64,
 * TF:331-380): per head, per token, L2-normalise q and k (eps 1e-6 inside the
 * sqrt), scale q, decay the state, apply the delta rule, read out.  `scale` is the
 * q scale (the reference test uses d^-1/2).  s_in/s_out are [H, d, d] (K-major)
 * or null. */
void orc_gdn_recurrent_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                           const uint16_t* beta, int T, int H, int HK, int d, double scale,
                           const float* s_in, double* out, double* s_out) {
    const int group = H / HK;
#pragma omp parallel for schedule(dynamic)
    for (int head = 0; head < H; head++) {
        const int kh = head / group;
        double* s = (double*)calloc((size_t)d * d, sizeof(double));
        double* qv = (double*)malloc(sizeof(double) * d);
        double* kv = (double*)malloc(sizeof(double) * d);
        double* vv = (double*)malloc(sizeof(double) * d);
        if (s_in)
            for (size_t i = 0; i < (size_t)d * d; i++) s[i] = s_in[(size_t)head * d * d + i];
        for (int t = 0; t < T; t++) {
            double qs = 0, ks = 0;
            for (int i = 0; i < d; i++) {
                qv[i] = bf(q[((size_t)t * HK + kh) * d + i]);
                kv[i] = bf(k[((size_t)t * HK + kh) * d + i]);
                qs += qv[i] * qv[i];
                ks += kv[i] * kv[i];
            }
            const double qi = 1.0 / sqrt(qs + 1e-6), ki = 1.0 / sqrt(ks + 1e-6);
            for (int i = 0; i < d; i++) {
                qv[i] = qv[i] * qi * scale;
                kv[i] *= ki;
                vv[i] = bf(v[((size_t)t * H + head) * d + i]);
            }
            const double decay = exp((double)g[(size_t)t * H + head]);
            const double b = bf(beta[(size_t)t * H + head]);
            for (size_t i = 0; i < (size_t)d * d; i++) s[i] *= decay;
            for (int j = 0; j < d; j++) {
                double mem = 0;
                for (int i = 0; i < d; i++) mem += kv[i] * s[(size_t)i * d + j];
                const double delta = (vv[j] - mem) * b;
                for (int i = 0; i < d; i++) s[(size_t)i * d + j] += kv[i] * delta;
            }
            for (int j = 0; j < d; j++) {
                double acc = 0;
                for (int i = 0; i < d; i++) acc += qv[i] * s[(size_t)i * d + j];
                out[((size_t)t * H + head) * d + j] = acc;
            }
        }
        if (s_out)
            for (size_t i = 0; i < (size_t)d * d; i++) s_out[(size_t)head * d * d + i] = s[i];
        free(s);
        free(qv);
        free(kv);
        free(vv);
    }
}

/* ------------------------------ gated delta rule, CUDA-kernel emulation */

enum { GC = 64, GK = 128, GV = 128 };

/* Blocked T = (I + A)^-1 of a strictly lower triangular 64x64 A (row stride 64),
 * in the order of gdn_prefill.cu:250-287: 16x16 diagonal blocks by forward
 * substitution with fmaf, then three levels of off-diagonal blocks, each block
 * T_ij = -T_ii * sum_{kb=j}^{i-1} A_ik T_kj with the inner sums in fmaf order. */
static void tri_inverse_blocked(const float* am, float* tm) {
    memset(tm, 0, sizeof(float) * GC * GC);
    for (int base = 0; base < GC; base += 16)
        for (int col = 0; col < 16; col++) {
            float xs[16];
            for (int r = 0; r < 16; r++) {
                float acc = r == col ? 1.f : 0.f;
                for (int j = 0; j < r; j++) acc = fmaf(-am[(base + r) * GC + base + j], xs[j], acc);
                xs[r] = acc;
            }
            for (int r = 0; r < 16; r++) tm[(base + r) * GC + base + col] = xs[r];
        }
    float sc[3 * 256];
    for (int lv = 1; lv < 4; lv++) {
        const int nb = 4 - lv;
        for (int x = 0; x < nb * 256; x++) {
            const int bi = lv + x / 256, bj = bi - lv, r = (x % 256) / 16, cc = x % 16;
            float acc = 0.f;
            for (int kb = bj; kb < bi; kb++)
                for (int m = 0; m < 16; m++)
                    acc = fmaf(am[(16 * bi + r) * GC + 16 * kb + m], tm[(16 * kb + m) * GC + 16 * bj + cc], acc);
            sc[x] = acc;
        }
        for (int x = 0; x < nb * 256; x++) {
            const int bi = lv + x / 256, bj = bi - lv, r = (x % 256) / 16, cc = x % 16;
            const float* s0 = sc + (x / 256) * 256 + cc;
            float acc = 0.f;
            for (int m = 0; m <= r; m++) acc = fmaf(tm[(16 * bi + r) * GC + 16 * bi + m], s0[m * 16], acc);
            tm[(16 * bi + r) * GC + 16 * bj + cc] = -acc;
        }
    }
}

void orc_tri_inverse_blocked(const float* am, float* tm) { tri_inverse_blocked(am, tm); }

/* One head of cs1_gdn_prefill_x, following the rounding points of
 * gdn_prefill.cu (prep 133-328, state 382-456, out 507-543):
 *   cum: sequential float32 sum over the chunk (140-158), decay = expf(total);
 *   q,k: float32 L2 norms with rsqrt(sum + 1e-6), q times `scale` (168-188);
 *   qd = bf16(q^ * e^cum), kd = bf16(k^ * e^(cum_last - cum)) (201-202);
 *   A, P: TF32 operands (cvt.rna), float32 accumulation in 4-term groups (207-239);
 *   A_ij = (beta_i A_ij) e^(cum_i-cum_j) for j < i; pb = bf16(P e^(cum_i-cum_j)) j <= i (242-247);
 *   T blocked inverse (250-287); tb = bf16(T_ij beta_j); kw = bf16(k^ e^cum) (291-300);
 *   u = bf16(tb v), w = bf16(tb kw) (308-328);
 *   per chunk: Sb = bf16(S); vn = bf16(u - w Sb); o = bf16(qd Sb + pb vn);
 *   S = S * decay + kd^T vn, all float32 (388-455, 507-543).
 * Padding rows of the last chunk have g = 0, beta = 0, q = k = v = 0 (134-138). */
static void gdn_emul_head(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                          const uint16_t* beta, int T, int H, int HK, float scale, int head,
                          const float* s_in, uint16_t* o, float* s_out) {
    const int hk = head / (H / HK);
    const int NC = (T + GC - 1) / GC;
    float* S = (float*)malloc(sizeof(float) * GK * GV);
    float* Sb = (float*)malloc(sizeof(float) * GK * GV);
    float* kx = (float*)malloc(sizeof(float) * GC * GK);
    float* qx = (float*)malloc(sizeof(float) * GC * GK);
    float* kt = (float*)malloc(sizeof(float) * GC * GK);
    float* qt = (float*)malloc(sizeof(float) * GC * GK);
    float* qd = (float*)malloc(sizeof(float) * GC * GK);
    float* kd = (float*)malloc(sizeof(float) * GC * GK);
    float* kw = (float*)malloc(sizeof(float) * GC * GK);
    float* vb = (float*)malloc(sizeof(float) * GC * GV);
    float* u = (float*)malloc(sizeof(float) * GC * GV);
    float* w = (float*)malloc(sizeof(float) * GC * GK);
    float* vn = (float*)malloc(sizeof(float) * GC * GV);
    float* am = (float*)malloc(sizeof(float) * GC * GC);
    float* pr = (float*)malloc(sizeof(float) * GC * GC);
    float* pb = (float*)malloc(sizeof(float) * GC * GC);
    float* tm = (float*)malloc(sizeof(float) * GC * GC);
    float* tb = (float*)malloc(sizeof(float) * GC * GC);
    float cum[GC], bet[GC], ecum[GC], erem[GC];
    if (s_in)
        memcpy(S, s_in + (size_t)head * GK * GV, sizeof(float) * GK * GV);
    else
        memset(S, 0, sizeof(float) * GK * GV);

    for (int c = 0; c < NC; c++) {
        for (int r = 0; r < GC; r++) {
            const int t = c * GC + r;
            cum[r] = t < T ? g[(size_t)t * H + head] : 0.f;
            bet[r] = t < T ? bf(beta[(size_t)t * H + head]) : 0.f;
        }
        float s = 0.f;
        for (int r = 0; r < GC; r++) {
            s = s + cum[r];
            cum[r] = s;
        }
        const float decay = expf(s);
        for (int r = 0; r < GC; r++) {
            ecum[r] = expf(cum[r]);
            erem[r] = expf(cum[GC - 1] - cum[r]);
        }
        for (int r = 0; r < GC; r++) {
            const int t = c * GC + r;
            float ks = 0.f, qs = 0.f;
            float kr[GK], qr[GK];
            for (int d = 0; d < GK; d++) {
                kr[d] = t < T ? bf(k[((size_t)t * HK + hk) * GK + d]) : 0.f;
                qr[d] = t < T ? bf(q[((size_t)t * HK + hk) * GK + d]) : 0.f;
            }
            /* warp_sum over 32 lanes of 4 strided partials (lane + 32 e) */
            float pk[32], pq[32];
            for (int l = 0; l < 32; l++) {
                pk[l] = pq[l] = 0.f;
                for (int e = 0; e < 4; e++) {
                    pk[l] += kr[l + 32 * e] * kr[l + 32 * e];
                    pq[l] += qr[l + 32 * e] * qr[l + 32 * e];
                }
            }
            for (int off = 16; off > 0; off >>= 1)
                for (int l = 0; l < off; l++) {
                    pk[l] += pk[l + off];
                    pq[l] += pq[l + off];
                }
            ks = pk[0];
            qs = pq[0];
            const float kinv = 1.f / sqrtf(ks + 1e-6f), qinv = 1.f / sqrtf(qs + 1e-6f) * scale;
            for (int d = 0; d < GK; d++) {
                const float a = kr[d] * kinv, b = qr[d] * qinv;
                kx[r * GK + d] = a;
                qx[r * GK + d] = b;
                kt[r * GK + d] = tf32_rna(a);
                qt[r * GK + d] = tf32_rna(b);
                qd[r * GK + d] = rbf(b * ecum[r]);
                kd[r * GK + d] = rbf(a * erem[r]);
                kw[r * GK + d] = rbf(a * ecum[r]);
            }
        }
        for (int i = 0; i < GC; i++)
            for (int j = 0; j <= i; j++) {
                float accA = 0.f, accP = 0.f;
                for (int k0 = 0; k0 < GK; k0 += 4) {
                    float sa = 0.f, sp = 0.f;
                    for (int e = 0; e < 4; e++) {
                        sa += kt[i * GK + k0 + e] * kt[j * GK + k0 + e];
                        sp += qt[i * GK + k0 + e] * kt[j * GK + k0 + e];
                    }
                    accA += sa;
                    accP += sp;
                }
                am[i * GC + j] = accA;
                pr[i * GC + j] = accP;
            }
        for (int i = 0; i < GC; i++)
            for (int j = 0; j < GC; j++) {
                const float dec = j <= i ? expf(cum[i] - cum[j]) : 0.f;
                am[i * GC + j] = j < i ? bet[i] * am[i * GC + j] * dec : 0.f;
                pb[i * GC + j] = j <= i ? rbf(pr[i * GC + j] * dec) : 0.f;
            }
        tri_inverse_blocked(am, tm);
        for (int i = 0; i < GC; i++)
            for (int j = 0; j < GC; j++) tb[i * GC + j] = rbf(tm[i * GC + j] * bet[j]);
        for (int r = 0; r < GC; r++) {
            const int t = c * GC + r;
            for (int d = 0; d < GV; d++) vb[r * GV + d] = t < T ? bf(v[((size_t)t * H + head) * GV + d]) : 0.f;
        }
        for (int i = 0; i < GC; i++) {
            for (int d = 0; d < GV; d++) {
                float au = 0.f, aw = 0.f;
                for (int j = 0; j <= i; j++) {
                    au += tb[i * GC + j] * vb[j * GV + d];
                    aw += tb[i * GC + j] * kw[j * GK + d];
                }
                u[i * GV + d] = rbf(au);
                w[i * GK + d] = rbf(aw);
            }
        }
        /* state and output */
        for (int x = 0; x < GK * GV; x++) Sb[x] = rbf(S[x]);
        for (int i = 0; i < GC; i++)
            for (int d = 0; d < GV; d++) {
                float acc = 0.f;
                for (int kk = 0; kk < GK; kk++) acc += w[i * GK + kk] * Sb[kk * GV + d];
                vn[i * GV + d] = rbf(u[i * GV + d] - acc);
            }
        for (int i = 0; i < GC; i++) {
            const int t = c * GC + i;
            if (t >= T) continue;
            for (int d = 0; d < GV; d++) {
                float acc = 0.f;
                for (int kk = 0; kk < GK; kk++) acc += qd[i * GK + kk] * Sb[kk * GV + d];
                for (int j = 0; j <= i; j++) acc += pb[i * GC + j] * vn[j * GV + d];
                o[((size_t)t * H + head) * GV + d] = f2bf(acc);
            }
        }
        for (int x = 0; x < GK * GV; x++) S[x] *= decay;
        for (int kk = 0; kk < GK; kk++)
            for (int d = 0; d < GV; d++) {
                float acc = S[kk * GV + d];
                for (int j = 0; j < GC; j++) acc += kd[j * GK + kk] * vn[j * GV + d];
                S[kk * GV + d] = acc;
            }
    }
    if (s_out) memcpy(s_out + (size_t)head * GK * GV, S, sizeof(float) * GK * GV);
    free(S); free(Sb); free(kx); free(qx); free(kt); free(qt); free(qd); free(kd); free(kw);
    free(vb); free(u); free(w); free(vn); free(am); free(pr); free(pb); free(tm); free(tb);
}

/* cs1_gdn_prefill_x (gdn_prefill.cu:568-615) on the CPU: T == 0 passes the state
 * through (or zeroes s_out when s_in is null). Returns 0, or -1 on bad shapes. */
int orc_gdn_chunk_emul(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                       const uint16_t* beta, int T, int H, int HK, float scale, const float* s_in,
                       uint16_t* o, float* s_out) {
    if (T < 0 || HK <= 0 || H % HK != 0) return -1;
    if (T == 0) {
        if (s_out) {
            if (s_in)
                memcpy(s_out, s_in, sizeof(float) * (size_t)H * GK * GV);
            else
                memset(s_out, 0, sizeof(float) * (size_t)H * GK * GV);
        }
        return 0;
    }
#pragma omp parallel for schedule(dynamic)
    for (int head = 0; head < H; head++) gdn_emul_head(q, k, v, g, beta, T, H, HK, scale, head, s_in, o, s_out);
    return 0;
}

/* ------------------------------------------------ flash attention, f64 */

/* kernels.rs:436-469: causal softmax(q k^T * scale) v in float64 for query rows
 * [q_base, T) (or the listed rows), GQA head h -> kv head h / (Hq / Hk); v is read
 * in rows of ldv.
 * out [T, Hq, Dh] (rows below q_base untouched), lse [Hq, T] natural log. */
void orc_attention_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v, int ldv, int T, int Hq,
                       int Hk, int Dh, double scale, int q_base, const int* rows, int nrows, double* out,
                       double* lse) {
    const int group = Hq / Hk;
    /* rows (optional): only these query rows are computed */
    const int n = rows ? nrows : T - q_base;
#pragma omp parallel for schedule(dynamic)
    for (int ri = 0; ri < n; ri++) {
        const int i = rows ? rows[ri] : q_base + ri;
        double* s = (double*)malloc(sizeof(double) * (size_t)(i + 1));
        for (int h = 0; h < Hq; h++) {
            const int gk = h / group;
            const uint16_t* qi = q + ((size_t)i * Hq + h) * Dh;
            double m = -INFINITY;
            for (int j = 0; j <= i; j++) {
                const uint16_t* kj = k + ((size_t)j * Hk + gk) * Dh;
                double acc = 0;
                for (int d = 0; d < Dh; d++) acc += (double)bf(qi[d]) * (double)bf(kj[d]);
                s[j] = acc * scale;
                if (s[j] > m) m = s[j];
            }
            double z = 0;
            for (int j = 0; j <= i; j++) {
                s[j] = exp(s[j] - m);
                z += s[j];
            }
            for (int d = 0; d < Dh; d++) {
                double acc = 0;
                for (int j = 0; j <= i; j++) acc += s[j] * (double)bf(v[(size_t)j * ldv + (size_t)gk * Dh + d]);
                out[((size_t)i * Hq + h) * Dh + d] = acc / z;
            }
            if (lse) lse[(size_t)h * T + i] = m + log(z);
        }
        free(s);
    }
}

/* ---------------------------------------- flash attention, CUDA emulation */

/* flash_kernel (attention.cu:84-234) for one query row: keys in tiles of 32
 * (BN), scores scaled by scale*log2(e) in float32, running max/sum in base 2,
 * P rounded to bf16 for the P*V product while the running sum l keeps the float32
 * p; out = o / l, rounded to bf16, or with the gate
 * bf16(round_bf16(o / l) * round_bf16(sigmoid(gate))) (attention.cu:221-231).
 * lse (optional, [Hq, T]) = (m + log2 l) * ln 2, natural log. */
/* One query row i of orc_attention_emul (all heads): the row depends only on itself and the
 * fixed key-tile order, so any subset of rows can be emulated on its own. */
static void attention_emul_row(const uint16_t* q, const uint16_t* k, const uint16_t* v, int ldv, const uint16_t* gate,
                               int T, int Hq, int Hk, int Dh, float scale, int i, float* o, uint16_t* out, float* lse) {
    const int group = Hq / Hk;
    const float sl2 = scale * 1.4426950408889634f;
    float sc[32];
    for (int h = 0; h < Hq; h++) {
        const int gk = h / group;
        const uint16_t* qi = q + ((size_t)i * Hq + h) * Dh;
        float m = -INFINITY, l = 0.f;
        for (int d = 0; d < Dh; d++) o[d] = 0.f;
        for (int k0 = 0; k0 <= i; k0 += 32) {
            float mx = -INFINITY;
            for (int e = 0; e < 32; e++) {
                const int key = k0 + e;
                if (key <= i) {
                    const uint16_t* kj = k + ((size_t)key * Hk + gk) * Dh;
                    float acc = 0.f;
                    for (int d = 0; d < Dh; d++) acc += bf(qi[d]) * bf(kj[d]);
                    sc[e] = acc * sl2;
                } else {
                    sc[e] = -INFINITY;
                }
                mx = fmaxf(mx, sc[e]);
            }
            const float mn = fmaxf(m, mx);
            const float base = mn == -INFINITY ? 0.f : mn;
            const float alpha = exp2f(m - base);
            m = mn;
            l *= alpha;
            for (int d = 0; d < Dh; d++) o[d] *= alpha;
            for (int e = 0; e < 32; e++) {
                const float p = exp2f(sc[e] - base);
                l += p;
                const float pr = rbf(p);
                if (pr != 0.f) {
                    const int key = k0 + e;
                    for (int d = 0; d < Dh; d++) o[d] += pr * bf(v[(size_t)key * ldv + (size_t)gk * Dh + d]);
                }
            }
        }
        const float inv = 1.f / l;
        for (int d = 0; d < Dh; d++) {
            float a = o[d] * inv;
            if (gate) a = rbf(a) * rbf(sigmoid_f(bf(gate[((size_t)i * Hq + h) * Dh + d])));
            out[((size_t)i * Hq + h) * Dh + d] = f2bf(a);
        }
        if (lse) lse[(size_t)h * T + i] = (m + log2f(l)) * 0.6931471805599453f;
    }
}

void orc_attention_emul(const uint16_t* q, const uint16_t* k, const uint16_t* v, int ldv, const uint16_t* gate,
                        int T, int Hq, int Hk, int Dh, float scale, int q_base, uint16_t* out, float* lse) {
#pragma omp parallel for schedule(dynamic)
    for (int i = q_base; i < T; i++) {
        float* o = (float*)malloc(sizeof(float) * Dh);
        attention_emul_row(q, k, v, ldv, gate, T, Hq, Hk, Dh, scale, i, o, out, lse);
        free(o);
    }
}

/* The same emulation restricted to the listed query rows (each in [0, T)); other rows of out
 * and lse are left as they are. Long sequences are checked on sampled rows this way, as the
 * reference's own test does for its float64 reference (kernels.rs:436-469). */
void orc_attention_emul_rows(const uint16_t* q, const uint16_t* k, const uint16_t* v, int ldv, const uint16_t* gate,
                             int T, int Hq, int Hk, int Dh, float scale, const int* rows, int nrows, uint16_t* out,
                             float* lse) {
#pragma omp parallel for schedule(dynamic)
    for (int r = 0; r < nrows; r++) {
        float* o = (float*)malloc(sizeof(float) * Dh);
        attention_emul_row(q, k, v, ldv, gate, T, Hq, Hk, Dh, scale, rows[r], o, out, lse);
        free(o);
    }
}

/* ------------------------------------------------------- elementwise ops */

/* gdn_conv_kernel (elementwise.cu:20-40): per channel c and token t,
 * acc = fmaf chain over taps j = 0..3 of w[c,j] * x[t-3+j, c] (zero left pad),
 * y = bf16(silu(round_bf16(acc))), split into q | k | v. */
void orc_gdn_conv(const uint16_t* qkv, int ld, const uint16_t* w, uint16_t* q, uint16_t* k, uint16_t* v, int T,
                  int key_dim, int value_dim) {
    const int ch = 2 * key_dim + value_dim;
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++)
        for (int c = 0; c < ch; c++) {
            float acc = 0.f;
            for (int j = 0; j < 4; j++) {
                const int s = t - 3 + j;
                if (s >= 0) acc = fmaf(bf(w[c * 4 + j]), bf(qkv[(size_t)s * ld + c]), acc);
            }
            const uint16_t y = f2bf(silu_f(rbf(acc)));
            if (c < key_dim)
                q[(size_t)t * key_dim + c] = y;
            else if (c < 2 * key_dim)
                k[(size_t)t * key_dim + c - key_dim] = y;
            else
                v[(size_t)t * value_dim + c - 2 * key_dim] = y;
        }
}

/* gdn_gates_kernel (elementwise.cu:44-55): beta = bf16(sigmoid(b));
 * g = -expf(A_log) * softplus(a + dt_bias), softplus threshold 20. */
void orc_gdn_gates(const uint16_t* b, const uint16_t* a, int ld, const uint16_t* A_log, const uint16_t* dt_bias,
                   uint16_t* beta, float* g, int T, int H) {
    for (int t = 0; t < T; t++)
        for (int h = 0; h < H; h++) {
            const size_t src = (size_t)t * ld + h, i = (size_t)t * H + h;
            beta[i] = f2bf(sigmoid_f(bf(b[src])));
            const float x = bf(a[src]) + bf(dt_bias[h]);
            const float sp = x > 20.f ? x : log1pf(expf(x));
            g[i] = -expf(bf(A_log[h])) * sp;
        }
}

/* gated_rms_norm_kernel (norm.cu:223-245), D = 128: the sum of squares as 32
 * lanes of 4 consecutive values then a butterfly; normed = round_bf16(x * inv),
 * scaled = round_bf16(w * normed), out = bf16(scaled * silu(z)). */
void orc_gated_rms_norm(const uint16_t* x, const uint16_t* z, int ldz, const uint16_t* w, uint16_t* out, int T,
                        int H, int D, float eps) {
    const int rows = T * H, per = D / 32;
#pragma omp parallel for schedule(static)
    for (int row = 0; row < rows; row++) {
        const size_t base = (size_t)row * D, zbase = (size_t)(row / H) * ldz + (size_t)(row % H) * D;
        float part[32];
        for (int l = 0; l < 32; l++) {
            part[l] = 0.f;
            for (int i = 0; i < per; i++) {
                const float vx = bf(x[base + l * per + i]);
                part[l] += vx * vx;
            }
        }
        for (int off = 16; off > 0; off >>= 1)
            for (int l = 0; l < off; l++) part[l] += part[l + off];
        const float inv = 1.f / sqrtf(part[0] / D + eps);
        for (int d = 0; d < D; d++) {
            const float normed = rbf(bf(x[base + d]) * inv);
            const float scaled = rbf(bf(w[d]) * normed);
            out[base + d] = f2bf(scaled * silu_f(bf(z[zbase + d])));
        }
    }
}

/* attn_prep_kernel (attention.cu:21-71): per (t, head), zero-centred RMSNorm
 * x = round_bf16(x * rsqrt(mean x^2 + eps) * (1 + w)), then rotate_half RoPE on
 * the first 2*half dims, y = round_bf16(round_bf16(x cos) + round_bf16(r sin)) with
 * r = -x[d+half] (d < half) or x[d-half]; the gate half of each q row is copied. */
void orc_attn_prep(const uint16_t* qg, const uint16_t* kr, int ld, const uint16_t* qw, const uint16_t* kw,
                   const uint16_t* cs, const uint16_t* sn, uint16_t* q, uint16_t* gate, uint16_t* k, int T, int Hq,
                   int Hk, int Dh, int half, float eps) {
    const int heads = Hq + Hk;
#pragma omp parallel for schedule(static)
    for (int wi = 0; wi < T * heads; wi++) {
        const int t = wi / heads, hh = wi % heads;
        const int is_q = hh < Hq, h = is_q ? hh : hh - Hq;
        const uint16_t* src = is_q ? qg + (size_t)t * ld + (size_t)h * 2 * Dh : kr + (size_t)t * ld + (size_t)h * Dh;
        const uint16_t* w = is_q ? qw : kw;
        float x[512], y[512];
        const int per = Dh / 32;
        float part[32];
        for (int l = 0; l < 32; l++) {
            part[l] = 0.f;
            for (int i = 0; i < per; i++) {
                x[l * per + i] = bf(src[l * per + i]);
                part[l] += x[l * per + i] * x[l * per + i];
            }
        }
        for (int off = 16; off > 0; off >>= 1)
            for (int l = 0; l < off; l++) part[l] += part[l + off];
        const float inv = 1.f / sqrtf(part[0] / Dh + eps);
        for (int d = 0; d < Dh; d++) x[d] = rbf(x[d] * inv * (1.f + bf(w[d])));
        for (int d = 0; d < Dh; d++) {
            y[d] = x[d];
            if (d < 2 * half) {
                const int fi = d % half;
                const float c = bf(cs[(size_t)t * half + fi]), s = bf(sn[(size_t)t * half + fi]);
                const float r = d < half ? -x[d + half] : x[d - half];
                y[d] = rbf(rbf(x[d] * c) + rbf(r * s));
            }
        }
        if (is_q) {
            for (int d = 0; d < Dh; d++) {
                q[((size_t)t * Hq + h) * Dh + d] = f2bf(y[d]);
                gate[((size_t)t * Hq + h) * Dh + d] = src[Dh + d];
            }
        } else {
            for (int d = 0; d < Dh; d++) k[((size_t)t * Hk + h) * Dh + d] = f2bf(y[d]);
        }
    }
}

/* sigmoid_gate_kernel (elementwise.cu:58-62): x = bf16(x * round_bf16(sigmoid(gate))). */
void orc_sigmoid_gate(uint16_t* x, const uint16_t* gate, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] = f2bf(bf(x[i]) * rbf(sigmoid_f(bf(gate[i]))));
}

/* silu_mul_kernel (elementwise.cu:66-73): out = bf16(round_bf16(silu(gate)) * up). */
void orc_silu_mul(const uint16_t* gate_up, int ld, uint16_t* out, int T, int I) {
    for (int t = 0; t < T; t++)
        for (int j = 0; j < I; j++) {
            const uint16_t* row = gate_up + (size_t)t * ld;
            out[(size_t)t * I + j] = f2bf(rbf(silu_f(bf(row[j]))) * bf(row[I + j]));
        }
}

/* Block sum of 256 threads as block_sum (common.cuh:313-327): per-thread strided
 * partials (i = tid + 256 m), 32-lane butterflies within 8 warps, then a butterfly
 * over the 8 warp sums. */
static float block_sum256(const float* part) {
    float wsum[8];
    for (int wp = 0; wp < 8; wp++) {
        float lanes[32];
        for (int l = 0; l < 32; l++) lanes[l] = part[wp * 32 + l];
        for (int off = 16; off > 0; off >>= 1)
            for (int l = 0; l < off; l++) lanes[l] += lanes[l + off];
        wsum[wp] = lanes[0];
    }
    float lanes[32];
    for (int l = 0; l < 32; l++) lanes[l] = l < 8 ? wsum[l] : 0.f;
    for (int off = 16; off > 0; off >>= 1)
        for (int l = 0; l < off; l++) lanes[l] += lanes[l + off];
    return lanes[0];
}

/* rms_norm_kernel (norm.cu:157-171): out = bf16(x * rsqrt(mean x^2 + eps) * (1 + w)). */
void orc_rms_norm(const uint16_t* x, const uint16_t* w, uint16_t* out, int rows, int D, float eps) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        float part[256];
        for (int t = 0; t < 256; t++) {
            part[t] = 0.f;
            for (int i = t; i < D; i += 256) {
                const float v = bf(x[(size_t)r * D + i]);
                part[t] += v * v;
            }
        }
        const float inv = 1.f / sqrtf(block_sum256(part) / D + eps);
        for (int i = 0; i < D; i++) out[(size_t)r * D + i] = f2bf(bf(x[(size_t)r * D + i]) * inv * (1.f + bf(w[i])));
    }
}

/* add_rms_norm_kernel (norm.cu:175-193): residual = bf16(residual + delta), then
 * rms_norm of the new residual. */
void orc_add_rms_norm(uint16_t* residual, const uint16_t* delta, const uint16_t* w, uint16_t* out, int rows, int D,
                      float eps) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        float part[256];
        uint16_t* res = residual + (size_t)r * D;
        for (int i = 0; i < D; i++) res[i] = f2bf(bf(res[i]) + bf(delta[(size_t)r * D + i]));
        for (int t = 0; t < 256; t++) {
            part[t] = 0.f;
            for (int i = t; i < D; i += 256) part[t] += bf(res[i]) * bf(res[i]);
        }
        const float inv = 1.f / sqrtf(block_sum256(part) / D + eps);
        for (int i = 0; i < D; i++) out[(size_t)r * D + i] = f2bf(bf(res[i]) * inv * (1.f + bf(w[i])));
    }
}

/* rotary_tables (inputs.rs:69-95) for text positions (all three rope axes equal):
 * inv_i = 1 / theta^(2i / (2 half)) in float32, angle = (float)(inv_i * pos) taken
 * to float64 for cos/sin, each rounded float32 -> bf16. cos/sin are [T, half]. */
void orc_rotary_tables(const int64_t* positions, int T, int half, double theta, uint16_t* cs, uint16_t* sn) {
    for (int t = 0; t < T; t++)
        for (int i = 0; i < half; i++) {
            const float inv = 1.f / powf((float)theta, (float)(2 * i) / (float)(2 * half));
            const double angle = (double)(inv * (float)positions[t]);
            cs[(size_t)t * half + i] = f2bf((float)cos(angle));
            sn[(size_t)t * half + i] = f2bf((float)sin(angle));
        }
}
