"""GPU parity of the model runner at the benchmark configurations' real sizes.

* Config 3 (4B-class, 32 layers, T = 4096): the decision prefill against the host
  restatement (tests/model_ref.py: each op the oracle's emulation of the reference kernel, GEMMs
  as float32 BLAS products rounded once to bf16), the reference executor's layer loop
  (src/models/qwen3_5/native/src/model.rs:1119-1338) and decision head
  (src/models/cua_s1/native/src/executor.rs:61-78). One layer of each kind at the full shape
  within the north-star bars; the 32-layer last hidden state within 2x the distance between two
  host restatements that differ only in GEMM summation order, and the 8-label argmax
  identical, asserted unconditionally.
* The same decision in two fresh processes: bitwise identical logits (every GEMM plan is the
  deterministic first heuristic choice).
* Config 4 (27B-class, 64 layers): capture of a 2048-token prefix and scoring of 8 packed
  candidates against full forwards of prefix + candidate (model.rs:1352-1571,
  src/models/lfm2/engine.py:128-146), and the two path kernels at the config's layer shapes
  (GDN 16 qk / 48 v heads, attention 24 / 4 x 256 over the cached prefix) against the oracle.
"""
import os
import subprocess
import sys
import time

import numpy as np
import pytest

import oracle as O
from gpu_helpers import bf16_errors, dev, empty, get, get_bf16, say, stream
import model_ref
from qwen3_5_native import hip
from qwen3_5_native import model as QM

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
T3 = 4096
LABELS3 = (np.arange(8) * 997 + 151).astype(np.int32)


def cfg3_ids():
    return np.random.default_rng(4).integers(0, QM.CFG3_4B.vocab, T3).astype(np.int32)


def cfg4_job():
    """The benchmark's config-4 job: a 2048-token prefix and 8 candidates of U[64, 256] tokens."""
    rng = np.random.default_rng(6)
    prefix = rng.integers(0, QM.CFG4_27B.vocab, 2048).astype(np.int32)
    lens = rng.integers(64, 257, 8)
    cands = [rng.integers(0, QM.CFG4_27B.vocab, int(k)).astype(np.int32) for k in lens]
    return prefix, cands


_CFG3_LOGITS = {}


@pytest.mark.parametrize("kind", ["gdn", "attention"])
def test_cfg3_single_layer_at_full_shape_matches_host_restatement(kind):
    """One config-3 decoder layer of each kind (hidden 2560, SwiGLU 9728, GDN 16/32 x 128 or
    attention 16/4 x 256, both norms) at T = 4096 against the host restatement: the final-norm
    last hidden state within max-abs 2e-2 / mean-abs 2e-3 of its scale."""
    stream()
    cfg = QM.Config(**{**QM.CFG3_4B.__dict__, "layers": 1,
                       "full_attention_interval": 1 if kind == "attention" else 4})
    say(f"model cfg3 single {kind} layer T={T3}")
    m = QM.Model(cfg, seed=2, max_tokens=T3)
    try:
        ids = cfg3_ids()
        got = m.forward(ids)
        want = model_ref.forward(m, ids, fp32_gemm=True)
    finally:
        m.close()
    d = np.abs(got.astype(np.float64) - want)
    scale = float(np.abs(want).max())
    say(f"  max diff {d.max():.3e} mean {d.mean():.3e} scale {scale:.3e}")
    assert d.max() <= 2e-2 * scale and d.mean() <= 2e-3 * scale, (d.max(), d.mean(), scale)


@pytest.mark.timeout(900)
def test_cfg3_decision_prefill_matches_host_restatement():
    """The full 32-layer decision prefill. Every GEMM result may differ from another float32
    summation order by one bf16 step, and over 32 random-init layers those differences grow
    (two host restatements that differ only in GEMM accumulation drift apart by about 1e-2 of
    the scale on the mean). So the bar is that noise floor, measured here between two host
    restatements (float32 GEMMs and float64 GEMMs, each rounded once to bf16): the device may
    differ from the first by at most 2x their distance (max and mean), and the 8-label argmax
    is identical in all three, asserted unconditionally."""
    stream()
    ids = cfg3_ids()
    say(f"model cfg3 4B-class T={T3}: device forward")
    m = QM.Model(QM.CFG3_4B, seed=0, max_tokens=T3)
    try:
        got = m.forward(ids)
        logits = m.decide(ids, LABELS3)
        _CFG3_LOGITS["in_process"] = logits.copy()
        hosts = []
        for mode in (True, False):
            t0 = time.time()
            hosts.append(model_ref.forward(m, ids, fp32_gemm=mode, progress=lambda i: say(
                f"  host ({mode}) layer {i} done ({time.time() - t0:.0f} s)") if i % 8 == 7 else None))
        want, alt = hosts
        want_l, alt_l = model_ref.decide(m, want, LABELS3), model_ref.decide(m, alt, LABELS3)
        np.testing.assert_allclose(logits, model_ref.decide(m, got, LABELS3), rtol=1e-6, atol=1e-6)
    finally:
        m.close()
    d = np.abs(got.astype(np.float64) - want)
    floor = np.abs(alt.astype(np.float64) - want)
    scale = float(np.abs(want).max())
    top2 = np.sort(want_l)[-2:]
    say(f"  device vs host: max {d.max():.3e} mean {d.mean():.3e}; host vs host (noise floor): max "
        f"{floor.max():.3e} mean {floor.mean():.3e}; scale {scale:.3e}")
    say(f"  logits {np.round(logits, 4)}\n  host   {np.round(want_l, 4)}\n  host'  {np.round(alt_l, 4)}\n"
        f"  top-2 margin {top2[1] - top2[0]:.4f}, max logit diff {np.abs(logits - want_l).max():.4f}")
    assert np.isfinite(got).all()
    assert d.mean() <= 2 * floor.mean() and d.max() <= 2 * floor.max(), (d.mean(), floor.mean())
    assert d.mean() <= 2e-2 * scale
    assert int(np.argmax(logits)) == int(np.argmax(want_l)) == int(np.argmax(alt_l))


_CHILD = r"""
import sys
import numpy as np
sys.path[:0] = [{root!r}, {pkg!r}]
from qwen3_5_native import hip, model as QM
hip.load(); hip.set_device(0)
ids = np.random.default_rng(4).integers(0, QM.CFG3_4B.vocab, {T}).astype(np.int32)
m = QM.Model(QM.CFG3_4B, seed=0, max_tokens={T})
m.set_graph(True)
a = m.decide(ids, (np.arange(8) * 997 + 151).astype(np.int32))
b = m.decide(ids, (np.arange(8) * 997 + 151).astype(np.int32))
assert np.array_equal(a, b)
print("LOGITS", a.astype(np.float32).tobytes().hex(), flush=True)
m.close()
"""


@pytest.mark.timeout(300)
def test_cfg3_decision_is_bitwise_repeatable_across_processes():
    """Two fresh processes (each with its own GEMM handle and plans, graph replay on) give the
    same logits bit for bit, equal to this process's eager decision."""
    code = _CHILD.format(root=ROOT, pkg=os.path.join(ROOT, "system1-omni_amd"), T=T3)
    outs = []
    for i in range(2):
        say(f"model cfg3 decision in child process {i}")
        r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=240)
        assert r.returncode == 0, r.stderr[-2000:]
        line = [x for x in r.stdout.splitlines() if x.startswith("LOGITS ")][0]
        outs.append(np.frombuffer(bytes.fromhex(line.split()[1]), np.float32))
        say(f"  logits {np.round(outs[-1], 4)}")
    np.testing.assert_array_equal(outs[0], outs[1])
    if "in_process" in _CFG3_LOGITS:
        np.testing.assert_array_equal(outs[0], _CFG3_LOGITS["in_process"])


@pytest.mark.timeout(600)
def test_cfg4_candidate_scores_match_full_forwards():
    """27B-class model: scores from the captured 2048-token prefix equal the same sums from a
    full forward of prefix + candidate (the continuation repeats the one-shot arithmetic up to
    GEMM summation order, model.rs:1358-1367); scoring twice from one capture is identical."""
    stream()
    prefix, cands = cfg4_job()
    P = len(prefix)
    say(f"model cfg4 27B-class: capture P={P}, score {len(cands)} candidates {[len(c) for c in cands]}")
    m = QM.Model(QM.CFG4_27B, seed=0, max_tokens=P + 256)
    try:
        m.capture(prefix)
        got = m.score(cands)
        again = m.score(cands)
        full = []
        for i, c in enumerate(cands):
            full.append(float(m.logprobs(np.concatenate([prefix, c]))[P - 1:].sum()))
            say(f"  candidate {i}: score {got[i]:.3f}, full forward {full[-1]:.3f}")
    finally:
        m.close()
    np.testing.assert_array_equal(again, got)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, np.array(full), rtol=2e-3, atol=0.3)
    assert int(np.argmax(got)) == int(np.argmax(full))


def test_cfg4_gdn_varlen_layer_shape_matches_oracle():
    """cs1_gdn_prefill_varlen at the 27B layer shape (16 qk / 48 v heads) over the config-4
    candidate lengths, all starting from one shared prefix state (stride 0), against the
    emulated reference kernel per candidate: outputs within max-abs 2e-2 / mean-abs 2e-3,
    final states within rel 1e-3."""
    api, st = hip.api(), stream()
    H, HK, D = 48, 16, 128
    _, cands = cfg4_job()
    lens = [len(c) for c in cands]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    rng = np.random.default_rng(31)

    def unit(x):
        return x / np.sqrt((x * x).sum(-1, keepdims=True))

    q = O.f32_to_bf16(unit(rng.standard_normal((T, HK, D))).astype(np.float32)).reshape(-1)
    k = O.f32_to_bf16(unit(rng.standard_normal((T, HK, D))).astype(np.float32)).reshape(-1)
    v = O.f32_to_bf16(rng.standard_normal((T, H, D)).astype(np.float32)).reshape(-1)
    beta = O.f32_to_bf16((1 / (1 + np.exp(-rng.standard_normal(T * H)))).astype(np.float32))
    g = (-np.log1p(np.exp(rng.standard_normal(T * H))) * 0.1).astype(np.float32)
    s0 = (rng.standard_normal((H, D, D)) * 0.05).astype(np.float32)
    say(f"gdn varlen 27B shape H={H} HK={HK} lens={lens}")
    bufs = (dev(q), dev(k), dev(v), dev(g), dev(beta))
    o = empty(T * H * D * 2)
    nch = int(sum((x + 63) // 64 for x in lens))
    ws = empty(api.cs1_gdn_workspace_floats(64 * nch, H) * 4)
    si = dev(s0.reshape(-1))
    so = empty(len(lens) * H * D * D * 4)
    hip.check(api.cs1_gdn_prefill_varlen(*(b.at(0) for b in bufs), o.at(0), ws.at(0), cu.ctypes.data, len(lens), H,
                                         HK, D ** -0.5, si.at(0), 0, so.at(0), H * D * D, st.handle), "varlen")
    got_o = get_bf16(o, T * H * D).reshape(T, H, D)
    got_s = get(so, np.float32, len(lens) * H * D * D).reshape(len(lens), H, D, D)
    for i, L in enumerate(lens):
        r = slice(int(cu[i]), int(cu[i]) + L)
        eo, es = O.gdn_chunk_emul(q.reshape(T, HK, D)[r].reshape(-1), k.reshape(T, HK, D)[r].reshape(-1),
                                  v.reshape(T, H, D)[r].reshape(-1), g.reshape(T, H)[r].reshape(-1),
                                  beta.reshape(T, H)[r].reshape(-1), L, H, HK, s_in=s0)
        mx, mean = bf16_errors(got_o[r], O.bf16_to_f32(eo))
        rel = float(np.linalg.norm(got_s[i] - es) / np.linalg.norm(es))
        say(f"  candidate {i} (L={L}): max-abs {mx:.2e} mean-abs {mean:.2e} state rel {rel:.2e}")
        assert mx <= 2e-2 and mean <= 2e-3 and rel <= 1e-3


def test_cfg4_prefix_attention_layer_shape_matches_oracle():
    """cs1_attention_prefix_varlen at the 27B layer shape (24 q / 4 kv heads, Dh 256, gated,
    LSE) over the config-4 candidates continuing a 2048-row cached prefix, against the
    emulated reference kernel on each candidate's window [prefix | candidate] with
    q_base = 2048 (attention.cu:279-295, cs1_attention_gated_prefix)."""
    api, st = hip.api(), stream()
    Hq, Hk, Dh, P = 24, 4, 256, 2048
    _, cands = cfg4_job()
    lens = [len(c) for c in cands]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    rng = np.random.default_rng(41)

    def bf(n):
        return O.f32_to_bf16(rng.standard_normal(n).astype(np.float32))

    q, gate = bf(T * Hq * Dh), bf(T * Hq * Dh)
    k, v = bf(T * Hk * Dh), bf(T * Hk * Dh)
    kp, vp = bf(P * Hk * Dh), bf(P * Hk * Dh)
    say(f"attention prefix varlen 27B shape Hq={Hq} Hk={Hk} Dh={Dh} P={P} lens={lens}")
    out, lse = empty(T * Hq * Dh * 2), empty(Hq * T * 4)
    dq, dk, dv, dkp, dvp, dg = (dev(x) for x in (q, k, v, kp, vp, gate))
    hip.check(api.cs1_attention_prefix_varlen(dq.at(0), dk.at(0), dv.at(0), Hk * Dh, dkp.at(0), dvp.at(0), Hk * Dh, P,
                                              dg.at(0), out.at(0), lse.at(0), cu.ctypes.data, len(lens), Hq, Hk, Dh,
                                              Dh ** -0.5, st.handle), "prefix varlen")
    got = get_bf16(out, T * Hq * Dh).reshape(T, Hq, Dh)
    got_lse = get(lse, np.float32, Hq * T).reshape(Hq, T)
    rq, rk = Hq * Dh, Hk * Dh
    for i, L in enumerate(lens):
        r0 = int(cu[i])
        W = P + L
        kw = np.concatenate([kp, k[r0 * rk:(r0 + L) * rk]])
        vw = np.concatenate([vp, v[r0 * rk:(r0 + L) * rk]])
        qw = np.concatenate([np.zeros(P * rq, np.uint16), q[r0 * rq:(r0 + L) * rq]])
        gw = np.concatenate([np.zeros(P * rq, np.uint16), gate[r0 * rq:(r0 + L) * rq]])
        eo, el = O.attention_emul(qw, kw, vw, rk, gw, W, Hq, Hk, Dh, Dh ** -0.5, q_base=P, want_lse=True)
        mx, mean = bf16_errors(got[r0:r0 + L], O.bf16_to_f32(eo[P:]))
        lerr = float(np.abs(got_lse[:, r0:r0 + L] - el[:, P:]).max())
        say(f"  candidate {i} (L={L}): max-abs {mx:.2e} mean-abs {mean:.2e} lse {lerr:.2e}")
        assert mx <= 2e-2 and mean <= 2e-3 and lerr <= 1e-3
