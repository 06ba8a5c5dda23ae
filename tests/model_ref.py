"""Host restatement of the hybrid decoder prefill for the model-runner parity tests.

The op sequence is the reference executor's (src/models/qwen3_5/native/src/model.rs:1119-1318);
each op is the oracle's emulation of the corresponding reference kernel, and each GEMM is the
float64 product of the bf16 operands rounded once to bf16 (cuBLASLt / hipBLASLt accumulate
in float32, so single results may differ by one bf16 step). For full-size models the GEMMs can
run as float32 products (BLAS sgemm, float32 accumulation like the device's) rounded once to
bf16, which keeps a 4B-class 4096-token forward within a minute or two of host time."""
import functools

import numpy as np

import oracle as O
from qwen3_5_native import model as QM


def gemm(x, w, M, N, K, fp32=False):
    """fp32=False: float64 product; True: float32 BLAS product; either rounded once to bf16."""
    xf = O.bf16_to_f32(x).reshape(M, K)
    wf = O.bf16_to_f32(w).reshape(N, K)
    if fp32:
        return O.f32_to_bf16(np.ascontiguousarray(xf @ wf.T, np.float32)).reshape(-1)
    return O.f32_to_bf16((xf.astype(np.float64) @ wf.T.astype(np.float64)).astype(np.float32)).reshape(-1)


def forward(m: QM.Model, ids, fp32_gemm=False, progress=None) -> np.ndarray:
    """Final-norm hidden state of the last row, float."""
    T = len(ids)
    return O.bf16_to_f32(forward_rows(m, ids, fp32_gemm, progress).reshape(T, m.cfg.hidden)[T - 1])


def forward_rows(m: QM.Model, ids, fp32_gemm=False, progress=None) -> np.ndarray:
    """Final-norm hidden states of every row, bf16 bits [T * hidden]. progress(i), if given,
    is called after each layer."""
    gemm_ = functools.partial(gemm, fp32=fp32_gemm)
    c = m.cfg
    T = len(ids)
    kd, vd = c.lin_k_heads * c.lin_k_dim, c.lin_v_heads * c.lin_v_dim
    conv = 2 * kd + vd
    gdn_w = conv + vd + 2 * c.lin_v_heads
    attn_q = c.heads * c.head_dim * 2
    attn_w = attn_q + 2 * c.kv_heads * c.head_dim
    H, D, I = c.hidden, c.head_dim, c.intermediate
    emb = m.tensor(QM.EMBED).reshape(c.vocab, H)
    res = emb[np.asarray(ids)].reshape(-1).copy()
    cs, sn = O.rotary_tables(np.arange(T, dtype=np.int64), c.rotary_half, c.rope_theta)
    x = O.rms_norm(res, m.tensor(QM.INPUT_NORM, 0), T, H, c.eps)
    for i in range(c.layers):
        if not c.is_full(i):
            gi = gemm_(x, m.tensor(QM.GDN_IN, i), T, gdn_w, H)
            q, k, v = O.gdn_conv(gi, gdn_w, m.tensor(QM.GDN_CONV, i), T, kd, vd)
            beta, g = O.gdn_gates(gi[conv + vd:], gi[conv + vd + c.lin_v_heads:], gdn_w, m.tensor(QM.GDN_A_LOG, i),
                                  m.tensor(QM.GDN_DT_BIAS, i), T, c.lin_v_heads)
            o, _ = O.gdn_chunk_emul(q.reshape(-1), k.reshape(-1), v.reshape(-1), g.reshape(-1), beta.reshape(-1), T,
                                    c.lin_v_heads, c.lin_k_heads, scale=c.lin_k_dim ** -0.5, want_state=False)
            ln = O.gated_rms_norm(o.reshape(-1), gi[conv:], gdn_w, m.tensor(QM.GDN_NORM, i), T, c.lin_v_heads,
                                  c.lin_v_dim, c.eps)
            delta = gemm_(ln, m.tensor(QM.GDN_OUT, i), T, H, vd)
        else:
            ai = gemm_(x, m.tensor(QM.ATTN_QKV, i), T, attn_w, H)
            q, gate, k = O.attn_prep(ai, ai[attn_q:], attn_w, m.tensor(QM.ATTN_Q_NORM, i),
                                     m.tensor(QM.ATTN_K_NORM, i), cs, sn, T, c.heads, c.kv_heads, D,
                                     c.rotary_half, c.eps)
            ao = O.attention_emul(q.reshape(-1), k.reshape(-1), ai[attn_q + c.kv_heads * D:], attn_w,
                                  gate.reshape(-1), T, c.heads, c.kv_heads, D, D ** -0.5)
            delta = gemm_(ao.reshape(-1), m.tensor(QM.ATTN_O, i), T, H, c.heads * D)
        res, x = O.add_rms_norm(res, delta, m.tensor(QM.POST_NORM, i), T, H, c.eps)
        gu = gemm_(x, m.tensor(QM.MLP_GATE_UP, i), T, 2 * I, H)
        act = O.silu_mul(gu, 2 * I, T, I)
        delta = gemm_(act.reshape(-1), m.tensor(QM.MLP_DOWN, i), T, H, I)
        nxt = m.tensor(QM.INPUT_NORM, i + 1) if i + 1 < c.layers else m.tensor(QM.FINAL_NORM)
        res, x = O.add_rms_norm(res, delta, nxt, T, H, c.eps)
        if progress is not None:
            progress(i)
    return np.asarray(x).reshape(-1)


def logprobs(m: QM.Model, ids) -> np.ndarray:
    """log p(ids[t + 1] | ids[:t + 1]): bf16 logits from the LM head (one bf16 rounding of
    the float64 product), then a float64 log-softmax (src/models/lfm2/engine.py:141-143 takes
    `logits.float().log_softmax(-1)`)."""
    T, H = len(ids), m.cfg.hidden
    x = forward_rows(m, ids)[: (T - 1) * H]
    logits = O.bf16_to_f32(gemm(x, m.tensor(QM.LM_HEAD), T - 1, m.cfg.vocab, H)).reshape(T - 1, -1).astype(np.float64)
    mx = logits.max(1, keepdims=True)
    lse = mx[:, 0] + np.log(np.exp(logits - mx).sum(1))
    return logits[np.arange(T - 1), np.asarray(ids[1:])] - lse


def decide(m: QM.Model, last, labels) -> np.ndarray:
    """cua_s1 executor.rs:61-78: float64 dots of embedding rows with the last hidden state."""
    emb = m.tensor(QM.EMBED).reshape(m.cfg.vocab, m.cfg.hidden)
    rows = O.bf16_to_f32(emb[np.asarray(labels)]).astype(np.float64)
    return (rows @ np.asarray(last, np.float64)).astype(np.float32)
