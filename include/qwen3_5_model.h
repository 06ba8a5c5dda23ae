/*
 * C interface of libqwen3_5_model.so: a native host runner for the Qwen3.5-style hybrid
 * decoder prefill, built on the cs1_* operations of libqwen3_5_hip.so.
 *
 * It replays the reference executor's text prefill (src/models/qwen3_5/native/src/model.rs:
 * Model::forward_batch 769-826 for one prompt, run 1119-1318, gemm 702-721, last_hidden
 * 1100-1115) and the decision head of src/models/cua_s1/native/src/executor.rs:61-78
 * (float64 dot products of label rows of the embedding with the final-norm hidden state
 * of the last token).  There is no checkpoint loader: weights are initialised on the
 * device from a seed with the random-init conventions of transformers' Qwen3.5
 * (modeling_qwen3_5.py 812-820): linear, embedding and conv weights N(0, 0.02), zero
 * RMSNorm weights (the norms scale by 1 + w), gated-norm weights one, dt_bias one,
 * A_log = log U(0, 16).
 *
 * Every function returns 0 or an error code of the op library (hipError_t, or 1000 +
 * hipBLASLt status); argument errors return hipErrorInvalidValue (1).
 */
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct Q35ModelConfig {
    int layers;                  /* decoder layers */
    int hidden;                  /* model width */
    int intermediate;            /* SwiGLU width */
    int vocab;                   /* embedding rows */
    int heads, kv_heads;         /* full-attention q / kv heads */
    int head_dim;                /* full-attention head dim (256: the reference attention's only size) */
    int rotary_half;             /* rotary frequencies per head (rotated dims = 2 * rotary_half) */
    double rope_theta;
    int lin_k_heads, lin_v_heads;  /* Gated DeltaNet q/k and v heads */
    int lin_k_dim, lin_v_dim;      /* Gated DeltaNet head dims (128) */
    int full_attention_interval; /* layer i is full attention when (i + 1) % interval == 0 */
    float eps;                   /* RMSNorm epsilon */
    int lm_head;                 /* 1: a separate [vocab, hidden] LM head for token log-probabilities */
} Q35ModelConfig;

/* Weight tensors, for tests that rebuild the forward on the host. */
enum {
    Q35M_EMBED = 0,       /* [vocab, hidden] */
    Q35M_FINAL_NORM = 1,  /* [hidden] */
    Q35M_INPUT_NORM = 2,  /* [hidden] per layer */
    Q35M_POST_NORM = 3,   /* [hidden] per layer */
    Q35M_GDN_IN = 4,      /* [2 kd + 2 vd + 2 Hv, hidden]: q | k | v | z | b | a rows */
    Q35M_GDN_CONV = 5,    /* [2 kd + vd, 4] */
    Q35M_GDN_A_LOG = 6,   /* [Hv] */
    Q35M_GDN_DT_BIAS = 7, /* [Hv] */
    Q35M_GDN_NORM = 8,    /* [lin_v_dim] */
    Q35M_GDN_OUT = 9,     /* [hidden, vd] */
    Q35M_ATTN_QKV = 10,   /* [2 Hq Dh + 2 Hk Dh, hidden]: per q head (q | gate), then k, v */
    Q35M_ATTN_Q_NORM = 11, /* [Dh] */
    Q35M_ATTN_K_NORM = 12, /* [Dh] */
    Q35M_ATTN_O = 13,     /* [hidden, Hq Dh] */
    Q35M_MLP_GATE_UP = 14, /* [2 I, hidden]: gate rows then up rows */
    Q35M_MLP_DOWN = 15,   /* [hidden, I] */
    Q35M_LM_HEAD = 16     /* [vocab, hidden] (lm_head = 1) */
};

/* Allocate and initialise a model for prompts of up to max_tokens tokens. */
int q35m_create(const Q35ModelConfig* cfg, uint64_t seed, int max_tokens, void** model);
void q35m_destroy(void* model);

/* Use a captured hipGraph of the layer stack for repeated prompt lengths (the first call
 * at a length runs eagerly, then captures; later calls at that length replay). */
int q35m_set_graph(void* model, int enabled);

/* Off by default: every GEMM runs the deterministic plan of cs1_gemm, so results are
 * bitwise repeatable across processes. When enabled, the first call at each GEMM shape
 * (outside capture) re-chooses that shape's plan with cs1_gemm_tune: faster on some shapes,
 * but the kept kernel, and with it the float32 summation order, can differ between processes. */
int q35m_set_gemm_tuning(void* model, int enabled);

/* Prefill one prompt; writes the final-norm hidden state of the last token (hidden floats).
 * Synchronous: returns after the state is on the host. */
int q35m_forward(void* model, const int32_t* ids, int T, float* last_hidden);

/* forward, then logits[i] = float64 dot(embedding row label_ids[i], last hidden). */
int q35m_decide(void* model, const int32_t* ids, int T, const int32_t* label_ids, int n_labels, float* logits);

/* The decision head's arithmetic alone (host only, no device work), replacing
 * src/models/cua_s1/native/src/executor.rs:61-78 letter_logits: logits[i] = (float) of the
 * float64 sum over j of (double) letters[i * H + j] * (double) last[j], for rows i < n only
 * (later rows are never read); hipErrorInvalidValue if any of the n logits is not finite. */
int q35m_letter_logits(const float* letters, const float* last, int H, int n, float* logits);

/* Prefix branching (the reference executor's capture / continue pair, model.rs:952-1073 and
 * run_window 1352-1571, with the candidate scoring of src/models/lfm2/engine.py:128-146).
 *
 * q35m_capture runs prompt rows [0, P) (P a positive multiple of 64) and keeps, per layer,
 * the state a continuation needs: post-prep K and raw V rows of each attention layer, the
 * float32 final state and the last three pre-conv rows of each Gated DeltaNet layer, and the
 * final-norm hidden state of row P - 1.
 *
 * q35m_score continues that prefix with n candidates packed into one pass (the GEMMs,
 * norms and MLP over all candidate rows; conv, the delta rule and attention per candidate
 * from the shared prefix state), and returns per candidate the summed log-probability of
 * its tokens: scores[c] = sum_j log softmax(lm_head h_{P-1+j})[ids_c[j]], h_{P-1} being the
 * prefix's last row. Requires lm_head = 1 and a preceding capture on this model. */
int q35m_capture(void* model, const int32_t* ids, int P);
int q35m_score(void* model, const int32_t* ids, const int32_t* lens, int n, double* scores);

/* Full forward of one prompt and the log-probability of each next token:
 * logprobs[t] = log softmax(lm_head h_t)[ids[t + 1]] for t < T - 1 (requires lm_head = 1). */
int q35m_logprobs(void* model, const int32_t* ids, int T, float* logprobs);

/* Device address and element count of a weight tensor (layer ignored for model-wide ones);
 * returns hipErrorInvalidValue if the layer has no such tensor. */
int q35m_tensor(void* model, int layer, int which, void** ptr, size_t* numel);

/* The stream the model queues its work on. */
void* q35m_stream(void* model);

#ifdef __cplusplus
}
#endif
