"""Writes tests/golden/transformers_fixtures.npz: input/output vectors of the spec-of-record
arithmetic in transformers' Qwen3.5 modelling code (transformers 5.15.0, installed in the build
container; the reference pins 5.17.0, whose GDN and attention code paths read the same).

Run once, in the build container only (the GPU box has no need for it and the tests read only
the .npz):   python tests/golden/make_transformers_fixtures.py

Hub kernels stay off: HF_HUB_OFFLINE is set, and neither the `kernels` package nor `fla` is
installed, so transformers' decorators resolve to the torch functions below.

Cases (all inputs are bf16 values, stored as uint16 bit patterns):
- gdn_a: torch_chunk_gated_delta_rule (modeling_qwen3_5.py 246-327), T=130 (3 chunks, ragged),
  H=2 v-heads over HK=1 qk-head (GQA by repeat_interleave, 500-502), L2-normalised q/k in the
  kernel, a random float32 initial state, float32 math; outputs o [T,H,128] and the final state.
- gdn_b: the same at T=70, H=2, HK=2, zero initial state, faster decay; output o only.
- gates: beta = sigmoid(b) in bf16, g = -exp(A_log) * softplus(a + dt_bias) in float32 (495-497).
- attn128 / attn256: eager_attention_forward (601-621) in bf16 with a causal mask, then the
  output gate attn * sigmoid(gate) (698), at Dh=128 (T=80, Hq=4, Hk=1) and Dh=256 (T=40,
  Hq=2, Hk=1); output bf16 [T, Hq*Dh].
"""
import os
import sys

os.environ["HF_HUB_OFFLINE"] = "1"
os.environ.setdefault("TRANSFORMERS_NO_ADVISORY_WARNINGS", "1")

import numpy as np
import torch
import torch.nn.functional as F
import transformers
from transformers.models.qwen3_5 import modeling_qwen3_5 as m

HERE = os.path.dirname(os.path.abspath(__file__))


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16).copy()


def unwrap(f):
    while hasattr(f, "__wrapped__"):
        f = f.__wrapped__
    return f


def bf16_randn(rng, shape, amp):
    return torch.from_numpy((rng.standard_normal(shape) * amp).astype(np.float32)).to(torch.bfloat16)


def gdn_case(rng, T, H, HK, decay, with_state):
    D = 128
    q = bf16_randn(rng, (T, HK, D), 1.0)
    k = bf16_randn(rng, (T, HK, D), 1.0)
    v = bf16_randn(rng, (T, H, D), 1.0)
    g = torch.from_numpy((-np.abs(rng.standard_normal((T, H))) * decay).astype(np.float32))
    beta = torch.sigmoid(bf16_randn(rng, (T, H), 1.0).float()).to(torch.bfloat16)
    s_in = torch.from_numpy((rng.standard_normal((H, D, D)) * 0.05).astype(np.float32)) if with_state else None
    rep = H // HK
    qf = q.float().repeat_interleave(rep, dim=1)[None]
    kf = k.float().repeat_interleave(rep, dim=1)[None]
    fn = unwrap(m.torch_chunk_gated_delta_rule)
    o, s_out = fn(qf, kf, v.float()[None], g[None], beta.float()[None], chunk_size=64,
                  initial_state=None if s_in is None else s_in[None], output_final_state=True,
                  use_qk_l2norm_in_kernel=True)
    out = {"q": bits(q), "k": bits(k), "v": bits(v), "g": g.numpy(), "beta": bits(beta),
           "o": o[0].float().numpy(), "dims": np.array([T, H, HK], np.int32)}
    if s_in is not None:
        out["s_in"] = s_in.numpy()
        out["s_out"] = s_out[0].float().numpy()
    return out


def gates_case(rng, T, H):
    b = bf16_randn(rng, (T, H), 2.0)
    a = bf16_randn(rng, (T, H), 4.0)  # a + dt_bias reaches past the softplus threshold (20) rarely; see below
    a[0, 0] = 30.0  # softplus linear branch
    A_log = torch.log(torch.from_numpy(rng.uniform(1, 16, H).astype(np.float32))).to(torch.bfloat16)
    dt_bias = bf16_randn(rng, (H,), 1.0)
    beta = b.sigmoid()
    g = -A_log.float().exp() * F.softplus(a.float() + dt_bias)
    return {"b": bits(b), "a": bits(a), "A_log": bits(A_log), "dt_bias": bits(dt_bias),
            "beta": bits(beta), "g": g.float().numpy(), "dims": np.array([T, H], np.int32)}


class _Module:
    training = False

    def __init__(self, groups):
        self.num_key_value_groups = groups


def attn_case(rng, T, Hq, Hk, Dh):
    q = bf16_randn(rng, (T, Hq, Dh), 1.0)
    k = bf16_randn(rng, (T, Hk, Dh), 1.0)
    v = bf16_randn(rng, (T, Hk, Dh), 1.0)
    gate = bf16_randn(rng, (T, Hq * Dh), 2.0)
    scale = Dh ** -0.5
    mask = torch.full((T, T), float("-inf")).triu(1).to(torch.bfloat16)[None, None]
    o, _ = m.eager_attention_forward(_Module(Hq // Hk), q.transpose(0, 1)[None], k.transpose(0, 1)[None],
                                     v.transpose(0, 1)[None], mask, scaling=scale)
    o = o.reshape(T, Hq * Dh)
    out = o * torch.sigmoid(gate)
    return {"q": bits(q), "k": bits(k), "v": bits(v), "gate": bits(gate), "out": bits(out),
            "dims": np.array([T, Hq, Hk, Dh], np.int32)}


def main():
    torch.manual_seed(0)
    rng = np.random.default_rng(20261202)
    cases = {
        "gdn_a": gdn_case(rng, 130, 2, 1, 0.05, True),
        "gdn_b": gdn_case(rng, 70, 2, 2, 0.3, False),
        "gates": gates_case(rng, 64, 8),
        "attn128": attn_case(rng, 80, 4, 1, 128),
        "attn256": attn_case(rng, 40, 2, 1, 256),
    }
    flat = {f"{c}/{k}": v for c, d in cases.items() for k, v in d.items()}
    flat["transformers_version"] = np.array(transformers.__version__)
    path = os.path.join(HERE, "transformers_fixtures.npz")
    np.savez_compressed(path, **flat)
    print(path, os.path.getsize(path), "bytes", file=sys.stderr)


if __name__ == "__main__":
    main()
