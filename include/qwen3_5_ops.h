/*
 * C interface of libqwen3_5_hip.so: the Qwen3.5 hybrid-decoder prefill operations for
 * AMD Instinct MI355X (gfx950), plus the few HIP runtime calls a caller needs so that
 * it loads this one library at run time and never links HIP itself.
 *
 * Drop-in boundary: every declaration in the "reference interface" sections has the
 * name, argument order, argument meaning, return convention and ABI version of the
 * reference's src/backends/cuda/qwen3_5/ops.h (ABI v6, ops.h:16-138), which its Rust
 * executor resolves by name (src/models/qwen3_5/native/src/cuda.rs:50-133). Each is
 * cited below with the ops.h line it replaces.  Declarations in the "additions"
 * section are new symbols; the reference has no counterpart and existing symbols keep
 * their semantics.
 *
 * Conventions (ops.h:1-9): tensors are row-major and bfloat16 unless a pointer is
 * float; token-major [T, heads, dim]; GQA head h reads kv head h / (H / HK).  Every
 * operation queues work on `stream` (a hipStream_t passed as void*), allocates
 * nothing, never waits on the host, and returns 0 or a hipError_t code (hipBLASLt
 * failures of the GEMMs are returned as 1000 + hipblasStatus_t).  Argument errors
 * return hipErrorInvalidValue.  Only cs1_upload / cs1_download synchronize.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>

/* ops.h:16 -- the interface version the Rust loader checks (cuda.rs:12, 160-165). */
#define CS1_ABI_VERSION 6

#ifdef __cplusplus
extern "C" {
#endif

/* ---- reference interface: runtime (ops.h:22-44, runtime.cu:7-74) ---- */

uint32_t cs1_abi_version(void);                                            /* ops.h:24 */
const char* cs1_error_string(int code);                                    /* ops.h:25 */
int cs1_set_device(int device);                                            /* ops.h:26 */
int cs1_malloc(void** ptr, size_t bytes);                                  /* ops.h:27 */
int cs1_free(void* ptr);                                                   /* ops.h:28 */
int cs1_stream_create(void** stream);                                      /* ops.h:29 */
int cs1_stream_sync(void* stream);                                         /* ops.h:30 */
int cs1_stream_destroy(void* stream);                                      /* ops.h:31 */
int cs1_graph_begin(void* stream);                                         /* ops.h:32 */
int cs1_graph_end(void* stream, void** exec);                              /* ops.h:33 */
int cs1_graph_launch(void* exec, void* stream);                            /* ops.h:34 */
int cs1_graph_destroy(void* exec);                                         /* ops.h:35 */
/* Copy and wait for the copy. */
int cs1_upload(void* dst, const void* src, size_t bytes, void* stream);   /* ops.h:37 */
int cs1_download(void* dst, const void* src, size_t bytes, void* stream); /* ops.h:38 */
/* Device-to-device copy, queued only. */
int cs1_copy_dd(void* dst, const void* src, size_t bytes, void* stream);  /* ops.h:40 */
/* Pitched device-to-device copy: height rows of width bytes. */
int cs1_copy2d(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width, size_t height,
               void* stream);                                              /* ops.h:43 */

/* ---- reference interface: operations (ops.h:46-126) ---- */

/* out[t] = table[ids[t]], rows of D (D % 8 == 0).                            ops.h:48 */
int cs1_embed(const int32_t* ids, const void* table, void* out, int T, int D, void* stream);

/* Zero-centred RMSNorm over rows of D: out = x * rsqrt(mean x^2 + eps) * (1 + w).  ops.h:51 */
int cs1_rms_norm(const void* x, const void* w, void* out, int rows, int D, float eps, void* stream);

/* residual = bf16(residual + delta); out = cs1_rms_norm(residual).             ops.h:54 */
int cs1_add_rms_norm(void* residual, const void* delta, const void* w, void* out, int rows, int D, float eps,
                     void* stream);

/* Gated RMSNorm of the GDN output x [T, H, 128] with z [T, H*128] in rows of ldz:
 * out = bf16(round(w * round(x * rsqrt(mean x^2 + eps))) * silu(z)).          ops.h:59 */
int cs1_gated_rms_norm(const void* x, const void* z, int ldz, const void* w, void* out, int T, int H, int D,
                       float eps, void* stream);

/* Depthwise causal conv1d (kernel 4, no bias, zero left padding) + SiLU over qkv [T, ld],
 * split into q [T, key_dim], k [T, key_dim], v [T, value_dim]; w is [2*key_dim+value_dim, 4].
 *                                                                               ops.h:64 */
int cs1_gdn_conv(const void* qkv, int ld, const void* w, void* q, void* k, void* v, int T, int key_dim,
                 int value_dim, void* stream);

/* beta = bf16(sigmoid(b)); g = -exp(A_log) * softplus(a + dt_bias) (float32); b, a are
 * [T, H] in rows of ld.                                                         ops.h:69 */
int cs1_gdn_gates(const void* b, const void* a, int ld, const void* A_log, const void* dt_bias, void* beta,
                  float* g, int T, int H, void* stream);

/* Chunked gated delta rule (chunk 64, dk = dv = 128), q and k L2-normalised inside, q
 * scaled by `scale`: q, k [T, HK, 128], v [T, H, 128], g float [T, H], beta [T, H],
 * o [T, H, 128].  The caller owns the workspace of cs1_gdn_workspace_floats(T, H) floats.
 *                                                                            ops.h:73-75 */
size_t cs1_gdn_workspace_floats(int T, int H);
int cs1_gdn_prefill(const void* q, const void* k, const void* v, const float* g, const void* beta, void* o,
                    float* workspace, int T, int H, int HK, float scale, void* stream);

/* Same scan with an explicit float32 state: s_in [H, 128, 128] (K-major) before the
 * window, or null for zero; s_out receives the state after it, or null.  T == 0 copies
 * s_in to s_out (zeroes s_out when s_in is null).  A continuation that starts at a
 * multiple of 64 repeats the one-pass arithmetic bit for bit.                ops.h:82-84 */
int cs1_gdn_prefill_x(const void* q, const void* k, const void* v, const float* g, const void* beta, void* o,
                      float* workspace, int T, int H, int HK, float scale, const void* s_in, void* s_out,
                      void* stream);

/* Attention inputs: q and gate from qg [T, Hq, 2*Dh], k from kr [T, Hk, Dh], both in
 * rows of ld; per-head zero-centred RMSNorm, then rotate_half RoPE on the first 2*half
 * dims with cos/sin [T, half] (bf16).  Writes q [T, Hq, Dh], gate [T, Hq*Dh], k [T, Hk, Dh].
 * The reference accepts Dh = 256 only; this build also accepts Dh = 128.      ops.h:89 */
int cs1_attn_prep(const void* qg, const void* kr, int ld, const void* qw, const void* kw, const void* cos,
                  const void* sin, void* q, void* gate, void* k, int T, int Hq, int Hk, int Dh, int half, float eps,
                  void* stream);

/* Causal GQA attention, Dh = 256: q [T, Hq, Dh], k [T, Hk, Dh], v [T, Hk, Dh] in rows of
 * ldv; out [T, Hq, Dh].                                                        ops.h:95 */
int cs1_attention(const void* q, const void* k, const void* v, int ldv, void* out, int T, int Hq, int Hk, int Dh,
                  float scale, void* stream);

/* Same, with the sigmoid gate [T, Hq, Dh] fused into the epilogue: out =
 * bf16(round(attn) * round(sigmoid(gate))), bit-identical to cs1_attention followed by
 * cs1_sigmoid_gate.  gate must be non-null when T > 0.                        ops.h:101 */
int cs1_attention_gated(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out, int T,
                        int Hq, int Hk, int Dh, float scale, void* stream);

/* Windowed variant: k and v cover rows [0, T); q, gate and out rows [q_base, T) of
 * buffers indexed from row 0.  q_base % 64 == 0.                               ops.h:108 */
int cs1_attention_gated_prefix(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out,
                               int T, int Hq, int Hk, int Dh, float scale, int q_base, void* stream);

/* x = bf16(x * round(sigmoid(gate))), n elements.                              ops.h:113 */
int cs1_sigmoid_gate(void* x, const void* gate, size_t n, void* stream);

/* out [T, I] = bf16(round(silu(gate)) * up) from gate_up [T, 2I] (gate first), rows of ld.
 *                                                                              ops.h:116 */
int cs1_silu_mul(const void* gate_up, int ld, void* out, int T, int I, void* stream);

/* y [M, N] (rows of ldy) = x [M, K] * w [N, K]^T, bf16 in and out, float32 accumulation,
 * through hipBLASLt with one fixed algorithm per shape (the first heuristic choice without
 * atomic split-K accumulation; never waits on the host).                   ops.h:120-124 */
void* cs1_gemm_create(size_t workspace_bytes);
void cs1_gemm_destroy(void* gemm);
int cs1_gemm(void* gemm, const void* x, const void* w, void* y, int M, int N, int K, int ldy, void* stream);

/* Additive (no counterpart in ops.h): cs1_gemm with the shape's plan re-chosen by timing up
 * to 16 of hipBLASLt's heuristic candidates on these operands, fastest kept (y holds the
 * kept kernel's result on return). Unlike cs1_gemm it synchronises the stream, so it must
 * not be called under stream capture (returns hipErrorStreamCaptureUnsupported). The
 * choice follows measured times, so two processes may keep different kernels for a shape;
 * without this call every plan is the deterministic first heuristic choice. */
int cs1_gemm_tune(void* gemm, const void* x, const void* w, void* y, int M, int N, int K, int ldy, void* stream);

/* ---- reference interface: vision tower (ops.h:127-138) ----
 * Out of scope for this build (the vision tower is not on the text prefill path).  The
 * symbols exist so that the reference loader, which resolves every name, can load the
 * library (cuda.rs:33-46); each returns hipErrorNotSupported. */
int cs1_vision_linear(void* gemm, const void* x, const void* w, const void* bias, void* y, int M, int N, int K,
                      void* stream);
int cs1_gemm_f32(void* gemm, const float* x, const float* w, float* y, int M, int N, int K, void* stream);
int cs1_vision_norm(const void* x, const void* w, const void* b, void* y, int rows, int d, void* stream);
int cs1_vision_position(void* x, const void* table, const int* indices, const float* weights, int n, void* stream);
int cs1_vision_rope(const void* qkv, const float* co, const float* si, void* q, void* k, int n, void* stream);
int cs1_vision_attention(const void* q, const void* k, const void* v, void* out, int n, void* stream);
int cs1_vision_bias(void* x, const void* bias, size_t n, int d, void* stream);
int cs1_vision_gelu(void* x, size_t n, int exact, void* stream);
int cs1_vision_add(void* x, const void* delta, size_t n, void* stream);
int cs1_vision_to_float(const void* x, float* out, size_t n, void* stream);
int cs1_vision_lora_add(void* x, const float* delta, size_t n, float scale, void* stream);

/* ---- additions (no counterpart in the reference) ---- */

/* Causal GQA attention for Dh = 128 or 256 with everything optional: gate (null = no
 * gate), lse [Hq, T] float32 natural-log log-sum-exp of each query row's scaled scores
 * (null = not written), q_base as in cs1_attention_gated_prefix.  With Dh = 256 and a
 * gate it is cs1_attention_gated_prefix bit for bit. */
int cs1_attention_ex(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out, float* lse,
                     int T, int Hq, int Hk, int Dh, float scale, int q_base, void* stream);

/* Varlen form of cs1_attention_ex for packed sequences (replaces the per-sequence launch
 * loop of the reference executor, model.rs:1242-1282): cu_seqlens is a HOST array of
 * nseq + 1 nondecreasing row offsets with cu_seqlens[0] = 0; sequence s is rows
 * [cu_seqlens[s], cu_seqlens[s + 1]) of q, k, v (rows of ldv), gate and out, causal within
 * itself; lse is [Hq, cu_seqlens[nseq]].  Each sequence's result equals a cs1_attention_ex
 * call on its rows bit for bit.  One launch per 64 sequences. */
int cs1_attention_varlen(const void* q, const void* k, const void* v, int ldv, const void* gate, void* out,
                         float* lse, const int32_t* cu_seqlens, int nseq, int Hq, int Hk, int Dh, float scale,
                         void* stream);

/* Varlen form of cs1_gdn_conv for packed sequences that all continue one history (the
 * per-candidate conv of the reference's scoring path, model.rs:1427-1434 and 1421-1470):
 * cu_seqlens is a HOST array of nseq + 1 (at most 64) nondecreasing row offsets with
 * cu_seqlens[0] = 0; sequence s is rows [cu_seqlens[s], cu_seqlens[s + 1]) of qkv (rows of
 * ld) and of q, k, v.  Each sequence's first outputs see the three rows of hist (rows of ld:
 * the three pre-conv rows before position 0; null: zeros) as their history, so each result
 * equals cs1_gdn_conv on [hist | its rows] bit for bit.  Requires 8 | key_dim, value_dim and
 * ld and 16-byte aligned buffers.  One launch. */
int cs1_gdn_conv_varlen(const void* qkv, int ld, const void* w, void* q, void* k, void* v, const int32_t* cu_seqlens,
                        int nseq, const void* hist, int key_dim, int value_dim, void* stream);

/* cs1_attention_varlen for packed sequences that all continue one shared prefix (the
 * candidate scoring of the reference executor, model.rs:1495-1554, which attends each
 * candidate to the cached prefix K/V): pre (a multiple of 64) prefix rows whose post-prep K
 * is kp (rows of Hk * Dh) and V is vp (rows of ldvp).  Sequence s is rows [cu_seqlens[s],
 * cu_seqlens[s + 1]) of q, k, v, gate and out at positions pre, pre + 1, ...: its queries
 * attend to the prefix keys and, causally, its own; lse is [Hq, cu_seqlens[nseq]].  Each
 * sequence's result equals cs1_attention_ex on [prefix K/V | its K/V] with q_base = pre bit
 * for bit.  No K/V copies; one launch per 64 sequences. */
int cs1_attention_prefix_varlen(const void* q, const void* k, const void* v, int ldv, const void* kp, const void* vp,
                                int ldvp, int pre, const void* gate, void* out, float* lse, const int32_t* cu_seqlens,
                                int nseq, int Hq, int Hk, int Dh, float scale, void* stream);

/* No counterpart in the reference: cs1_gdn_prefill_x without the workspace argument, for
 * callers that cannot allocate device memory (code under graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The workspace is a 64 MiB array inside the library, one
 * per GPU, kept until the process ends; the call itself allocates nothing.  Limit: the
 * workspace of (T, H) must fit, i.e. ceil(T / 64) * H <= 910 (e.g. T <= 1792 at H = 32,
 * T <= 58,240 at H = 1); larger shapes return hipErrorInvalidValue.  Every call on a GPU
 * shares that GPU's array, so calls that overlap in time on one GPU race: serialise them.
 * Results are bit for bit those of cs1_gdn_prefill_x. */
int cs1_gdn_prefill_x_static(const void* q, const void* k, const void* v, const float* g, const void* beta, void* o,
                             int T, int H, int HK, float scale, const void* s_in, void* s_out, void* stream);

/* Varlen form of cs1_gdn_prefill_x for packed sequences (the candidate-packed prefill of the
 * reference's scoring path, model.rs:1421-1470, which runs the delta rule per candidate):
 * cu_seqlens is a HOST array of nseq + 1 (at most 64) nondecreasing row offsets with
 * cu_seqlens[0] = 0; sequence s is rows [cu_seqlens[s], cu_seqlens[s + 1]) of q, k (rows of
 * HK * 128), v and o (rows of H * 128), g and beta (rows of H).  Sequence s starts from the
 * float32 state s_in + s * s_in_stride ([H, 128, 128]; stride 0: one state shared by all,
 * s_in null: zeros) and, when s_out is non-null, leaves its final state at
 * s_out + s * s_out_stride.  Chunks restart at each sequence (each result equals a
 * cs1_gdn_prefill_x call on the sequence's rows bit for bit).  The workspace must hold
 * cs1_gdn_workspace_floats(64 * sum_s ceil(len_s / 64), H) floats.  One launch pair. */
int cs1_gdn_prefill_varlen(const void* q, const void* k, const void* v, const float* g, const void* beta, void* o,
                           float* workspace, const int32_t* cu_seqlens, int nseq, int H, int HK, float scale,
                           const void* s_in, size_t s_in_stride, void* s_out, size_t s_out_stride, void* stream);

/* Gated forms of cs1_gdn_prefill_x and cs1_gdn_prefill_varlen (no reference counterpart:
 * they fold the reference's separate gates launch, cs1_gdn_gates / gdn_gates_kernel at
 * elementwise.cu:42-55 and 115-124, into the GDN prep).  Instead of g and beta they take the
 * raw projections b and a (bf16; token t, head h at b[t * ld + h], a[t * ld + h], ld >= H)
 * and the per-head A_log and dt_bias (bf16 [H]); beta = bf16(sigmoid(b)) and
 * g = -exp(A_log) * softplus(a + dt_bias) are computed in the prep with cs1_gdn_gates'
 * arithmetic, so each result equals cs1_gdn_gates followed by cs1_gdn_prefill_x (or _varlen)
 * bit for bit, without the g / beta buffers or the extra launch.  Everything else (workspace,
 * states, varlen rules, T = 0 pass-through) is that of the ungated form. */
int cs1_gdn_prefill_gated_x(const void* q, const void* k, const void* v, const void* b, const void* a, int ld,
                            const void* A_log, const void* dt_bias, void* o, float* workspace, int T, int H, int HK,
                            float scale, const void* s_in, void* s_out, void* stream);
int cs1_gdn_prefill_gated_varlen(const void* q, const void* k, const void* v, const void* b, const void* a, int ld,
                                 const void* A_log, const void* dt_bias, void* o, float* workspace,
                                 const int32_t* cu_seqlens, int nseq, int H, int HK, float scale, const void* s_in,
                                 size_t s_in_stride, void* s_out, size_t s_out_stride, void* stream);

#ifdef __cplusplus
}
#endif
