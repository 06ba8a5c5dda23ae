"""The oracle and the HIP path against transformers' own Qwen3.5 arithmetic (the spec of record,
modeling_qwen3_5.py), through fixtures written by tests/golden/make_transformers_fixtures.py.

The reference's CUDA kernels round at bf16 points that transformers' float32 chunked GDN and
bf16 eager attention do not share, so these are tolerance checks, with bars a dropped term, a
wrong scale, sign or head mapping would exceed by orders of magnitude:
  * GDN (float32 chunked rule, L2-normalised q/k, GQA, initial state): output max-abs
    <= 2e-2 * max|ref| and mean-abs <= 2e-3 * max|ref|; final state relative <= 1e-2
    (measured for the emulated reference kernel: 4.8e-3 * max|ref|, 5.4e-4, 3.0e-3);
  * gates: beta bit-equal; g within 4 float32 ulps (torch's exp/softplus vs expf/log1pf);
  * gated attention (bf16 eager softmax, then attn * sigmoid(gate)): max-abs <= 2e-2 (about one
    bf16 step at |out| < 4) and mean-abs <= 1e-3 (measured 1.56e-2 and 3.8e-4).
The float64 recurrence of the reference's tests (kernels.rs:479-525) agrees with transformers'
float32 chunked rule to 3e-8, which pins that restatement to the spec as well.
"""
import os

import numpy as np
import pytest

import oracle as O

FIX = np.load(os.path.join(os.path.dirname(__file__), "golden", "transformers_fixtures.npz"))


def case(name):
    return {k.split("/", 1)[1]: FIX[k] for k in FIX.files if k.startswith(name + "/")}


def flat(x):
    return np.ascontiguousarray(x).reshape(-1)


def gdn_bars(o, z, s=None):
    ref = z["o"]
    scale = float(np.abs(ref).max())
    d = np.abs(O.bf16_to_f32(o).reshape(ref.shape) - ref)
    assert d.max() <= 2e-2 * scale and d.mean() <= 2e-3 * scale, (d.max(), d.mean(), scale)
    if s is not None:
        rel = np.linalg.norm(s - z["s_out"]) / np.linalg.norm(z["s_out"])
        assert rel <= 1e-2, rel


def attn_bars(out, z):
    ref = O.bf16_to_f32(z["out"]).reshape(-1)
    d = np.abs(O.bf16_to_f32(flat(out)) - ref)
    assert d.max() <= 2e-2 and d.mean() <= 1e-3, (d.max(), d.mean())


@pytest.mark.parametrize("name", ["gdn_a", "gdn_b"])
def test_oracle_gdn_matches_transformers(name):
    z = case(name)
    T, H, HK = (int(x) for x in z["dims"])
    s_in = z.get("s_in")
    o, s = O.gdn_chunk_emul(flat(z["q"]), flat(z["k"]), flat(z["v"]), flat(z["g"]), flat(z["beta"]), T, H, HK,
                            s_in=s_in)
    gdn_bars(o, z, s if s_in is not None else None)
    f = O.gdn_recurrent_f64(flat(z["q"]), flat(z["k"]), flat(z["v"]), flat(z["g"]), flat(z["beta"]), T, H, HK,
                            s_in=s_in)
    assert np.abs(f - z["o"]).max() <= 1e-6 * np.abs(z["o"]).max() + 1e-7


def test_oracle_gates_match_transformers():
    z = case("gates")
    T, H = (int(x) for x in z["dims"])
    beta, g = O.gdn_gates(flat(z["b"]), flat(z["a"]), H, flat(z["A_log"]), flat(z["dt_bias"]), T, H)
    assert np.array_equal(beta, flat(z["beta"]))
    np.testing.assert_allclose(g, flat(z["g"]), rtol=4 * 2.0 ** -23, atol=0)


@pytest.mark.parametrize("name", ["attn128", "attn256"])
def test_oracle_gated_attention_matches_transformers(name):
    z = case(name)
    T, Hq, Hk, Dh = (int(x) for x in z["dims"])
    out = O.attention_emul(flat(z["q"]), flat(z["k"]), flat(z["v"]), Hk * Dh, flat(z["gate"]), T, Hq, Hk, Dh,
                           Dh ** -0.5)
    attn_bars(out, z)


# ------------------------------------------------------------------ the HIP path


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["gdn_a", "gdn_b"])
def test_gpu_gdn_matches_transformers(name):
    from test_gpu_gdn import run_gdn
    from gpu_helpers import say
    z = case(name)
    T, H, HK = (int(x) for x in z["dims"])
    say(f"gdn vs transformers fixture {name} T={T} H={H} HK={HK}")
    s_in = z.get("s_in")
    o, s = run_gdn(flat(z["q"]), flat(z["k"]), flat(z["v"]), flat(z["g"]), flat(z["beta"]), T, H, HK, s_in=s_in,
                   want_state=s_in is not None)
    gdn_bars(o, z, s)


@pytest.mark.gpu
def test_gpu_gates_match_transformers():
    from gpu_helpers import dev, empty, get, get_bf16, say, stream
    from qwen3_5_native import hip
    z = case("gates")
    T, H = (int(x) for x in z["dims"])
    say(f"gates vs transformers fixture T={T} H={H}")
    api, st = hip.api(), stream()
    db, da, dA, ddt = dev(flat(z["b"])), dev(flat(z["a"])), dev(flat(z["A_log"])), dev(flat(z["dt_bias"]))
    beta, g = empty(T * H * 2), empty(T * H * 4)
    hip.check(api.cs1_gdn_gates(db.at(0), da.at(0), H, dA.at(0), ddt.at(0), beta.at(0), g.at(0), T, H, st.handle),
              "gates")
    assert np.array_equal(get_bf16(beta, T * H), flat(z["beta"]))
    np.testing.assert_allclose(get(g, np.float32, T * H), flat(z["g"]), rtol=4 * 2.0 ** -23, atol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["attn128", "attn256"])
def test_gpu_gated_attention_matches_transformers(name):
    from test_gpu_attention import attn
    from gpu_helpers import dev, say
    z = case(name)
    T, Hq, Hk, Dh = (int(x) for x in z["dims"])
    say(f"gated attention vs transformers fixture {name} T={T} Hq={Hq} Hk={Hk} Dh={Dh}")
    out = attn(dev(flat(z["q"])), dev(flat(z["k"])), dev(flat(z["v"])), Hk * Dh, dev(flat(z["gate"])), T, Hq, Hk, Dh,
               Dh ** -0.5)
    attn_bars(out, z)
