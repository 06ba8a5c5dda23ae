"""GPU parity of the chunked Gated DeltaNet prefill (cs1_gdn_prefill{,_x}).

Mirrors tests/qwen3_5/kernels.rs:476-622, 692-742, 931-1088 and adds the benchmark
configurations. Bars:
  * vs the float64 recurrent reference: max |diff| <= 2e-2 * max |ref| (kernels.rs:620);
  * vs the emulated reference kernel (same rounding points, oracle/oracle.c): bf16 output
    max-abs <= 2e-2 and mean-abs <= 2e-3, float32 final state relative (Frobenius) <= 1e-3;
  * bit-for-bit: two-phase == one-shot, T = 0 state pass-through under graph capture.
"""
import json
import os

import numpy as np
import pytest

import oracle as O
from gpu_helpers import bf16_errors, dev, empty, get, get_bf16, say, stream
from qwen3_5_native import hip

pytestmark = pytest.mark.gpu
GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kernel_tests_log.json")))
D = 128


def run_gdn(q, k, v, g, beta, T, H, HK, scale=D ** -0.5, s_in=None, want_state=False, bufs=None):
    """One cs1_gdn_prefill_x call through the C ABI; returns (o bf16 [T,H,D], state or None)."""
    api, st = hip.api(), stream()
    dq, dk, dv, dg, db = bufs or (dev(q), dev(k), dev(v), dev(np.asarray(g, np.float32)), dev(beta))
    o = empty(max(T, 1) * H * D * 2)
    ws = empty(max(api.cs1_gdn_workspace_floats(T, H), 1) * 4)
    si = dev(np.asarray(s_in, np.float32)) if s_in is not None else None
    so = empty(H * D * D * 4) if want_state else None
    hip.check(api.cs1_gdn_prefill_x(dq.at(0), dk.at(0), dv.at(0), dg.at(0), db.at(0), o.at(0), ws.at(0), T, H, HK,
                                    scale, si.at(0) if si else None, so.at(0) if so else None, st.handle),
              "gdn prefill")
    out = get_bf16(o, T * H * D).reshape(T, H, D)
    state = get(so, np.float32, H * D * D).reshape(H, D, D) if want_state else None
    return out, state


def cfg0_inputs(T, H, HK, seed=0, s0_std=0.0):
    """Configs 0 and 2: q, k ~ N(0,1) -> bf16, L2-normalised per head; v ~ N(0,1);
    beta = sigmoid(N(0,1)); g = -softplus(N(0,1)) * 0.1; optional S0 ~ N(0, s0_std)."""
    rng = np.random.default_rng(seed)

    def unit(x):
        return x / np.sqrt((x * x).sum(-1, keepdims=True))

    q = O.f32_to_bf16(unit(rng.standard_normal((T, HK, D))).astype(np.float32)).reshape(-1)
    k = O.f32_to_bf16(unit(rng.standard_normal((T, HK, D))).astype(np.float32)).reshape(-1)
    v = O.f32_to_bf16(rng.standard_normal((T, H, D)).astype(np.float32)).reshape(-1)
    beta = O.f32_to_bf16((1 / (1 + np.exp(-rng.standard_normal(T * H)))).astype(np.float32))
    g = (-np.log1p(np.exp(rng.standard_normal(T * H))) * 0.1).astype(np.float32)
    s0 = (rng.standard_normal((H, D, D)) * s0_std).astype(np.float32) if s0_std else None
    return q, k, v, g, beta, s0


def check_vs_emulator(o, s, q, k, v, g, beta, T, H, HK, s0=None, label="", state_bar=True):
    eo, es = O.gdn_chunk_emul(q, k, v, g, beta, T, H, HK, s_in=s0)
    mx, mean = bf16_errors(o, O.bf16_to_f32(eo))
    say(f"  {label} vs emulated reference kernel: max-abs {mx:.2e} mean-abs {mean:.2e}")
    assert mx <= 2e-2 and mean <= 2e-3, (mx, mean)
    if s is not None and state_bar:
        rel = float(np.linalg.norm(s - es) / max(np.linalg.norm(es), 1e-30))
        say(f"  {label} final state relative error {rel:.2e}")
        assert rel <= 1e-3, rel
    return eo, es


@pytest.mark.parametrize("case", GOLDEN["gated_delta"], ids=lambda c: f"t{c['t']}h{c['h']}hk{c['hk']}a{c['qk_amp']}")
def test_gated_delta_rule_matches_recurrent_reference(case):
    t, h, hk = case["t"], case["h"], case["hk"]
    say(f"gdn recurrent case t={t} h={h} hk={hk} decay={case['decay_scale']} amp={case['qk_amp']}")
    q, k, v, g, b = O.gdn_test_inputs(t, h, hk, case["decay_scale"], case["qk_amp"])
    o, s = run_gdn(q, k, v, g, b, t, h, hk, want_state=True)
    got = O.bf16_to_f32(o).astype(np.float64)
    assert np.isfinite(got).all()
    want, s_want = O.gdn_recurrent_f64(q, k, v, g, b, t, h, hk, want_state=True)
    scale = np.abs(want).max()
    worst = np.abs(got - want).max()
    say(f"  largest difference {worst:.2e}, largest |reference| {scale:.2e} (reference kernel: {case['kernel_max_diff']:.2e})")
    assert worst <= 2e-2 * scale
    # no worse than the reference kernel's recorded error, with room for summation order
    assert worst <= 1.5 * case["kernel_max_diff"] + 1e-30
    _, es = check_vs_emulator(o, s, q, k, v, g, b, t, h, hk, label=f"t={t}", state_bar=False)
    # the float32 state is graded against float64: no worse than the emulated reference kernel's
    if np.abs(s_want).max() > 0:
        ours = np.linalg.norm(s - s_want) / np.linalg.norm(s_want)
        theirs = np.linalg.norm(es - s_want) / np.linalg.norm(s_want)
        say(f"  state vs float64: ours {ours:.2e}, emulated reference kernel {theirs:.2e}")
        assert ours <= 1.5 * theirs + 1e-6


def test_config0_gdn_layer():
    T, H, HK = 512, 16, 16
    say(f"gdn config0 T={T} H={H} HK={HK}")
    q, k, v, g, b, _ = cfg0_inputs(T, H, HK, seed=0)
    o, s = run_gdn(q, k, v, g, b, T, H, HK, want_state=True)
    check_vs_emulator(o, s, q, k, v, g, b, T, H, HK, label="config0")
    want, s_want = O.gdn_recurrent_f64(q, k, v, g, b, T, H, HK, want_state=True)
    worst = np.abs(O.bf16_to_f32(o) - want).max()
    say(f"  vs float64: {worst:.2e} of max {np.abs(want).max():.2e}")
    assert worst <= 2e-2 * np.abs(want).max()
    assert np.linalg.norm(s - s_want) / np.linalg.norm(s_want) < 1e-2


def test_config2_gdn_at_full_size():
    T, H, HK = 8192, 32, 16
    say(f"gdn config2 T={T} H={H} HK={HK} with S0 ~ N(0, 0.01)")
    q, k, v, g, b, s0 = cfg0_inputs(T, H, HK, seed=2, s0_std=0.01)
    o, s = run_gdn(q, k, v, g, b, T, H, HK, s_in=s0, want_state=True)
    assert np.isfinite(O.bf16_to_f32(o)).all() and np.isfinite(s).all()
    check_vs_emulator(o, s, q, k, v, g, b, T, H, HK, s0=s0, label="config2")


def test_gdn_prefill_two_phase_matches_one_shot_bit_for_bit():
    """kernels.rs:1049-1054; the 8192- and 8229-token cases run in segments (records over 200
    MiB), so they also check that segmentation is invisible in the result; the 22045-token case
    runs as four segments, so the two ping-pong segment states are each written twice."""
    api, st = hip.api(), stream()
    for t, h, hk, amp, decay in [(107, 4, 2, 1.0, 1.0), (936, 4, 2, 0.01, 1.0), (3399, 3, 1, 0.01, 1.0),
                                 (65, 4, 2, 0.01, 1e-9), (8192, 32, 16, 1.0, 0.01), (8229, 32, 16, 1.0, 0.01),
                                 (22045, 32, 16, 1.0, 0.01)]:
        say(f"gdn two-phase t={t} h={h} hk={hk}")
        q, k, v, g, b = O.gdn_test_inputs(t, h, hk, decay, amp)
        full, s_full = run_gdn(q, k, v, g, b, t, h, hk, want_state=True)
        p = max(int(t * 0.6) // 64 * 64, 64)
        o1, s1 = run_gdn(q[: p * hk * D], k[: p * hk * D], v[: p * h * D], g[: p * h], b[: p * h], p, h, hk,
                         want_state=True)
        o2, s2 = run_gdn(q[p * hk * D:], k[p * hk * D:], v[p * h * D:], g[p * h:], b[p * h:], t - p, h, hk, s_in=s1,
                         want_state=True)
        np.testing.assert_array_equal(o1, full[:p])
        np.testing.assert_array_equal(o2, full[p:])
        np.testing.assert_array_equal(s2, s_full)
        # T = 0: the state passes through untouched
        sin = dev(s1)
        so = empty(h * D * D * 4)
        hip.check(api.cs1_gdn_prefill_x(None, None, None, None, None, None, None, 0, h, hk, 1.0, sin.at(0), so.at(0),
                                        st.handle), "state passthrough")
        np.testing.assert_array_equal(get(so, np.float32, h * D * D).reshape(h, D, D), s1)


@pytest.mark.parametrize("t,h,hk,varlen", [(1000, 48, 16, False), (3399, 48, 16, False), (300, 32, 16, False),
                                            (0, 48, 16, True)])
def test_gdn_scan_block_forms_are_bit_identical(t, h, hk, varlen, forms):
    """The scan runs one or two 16-column halves per block (chosen by how many rounds of
    blocks the device needs: two halves at 48 heads, one at 32). Both forms must give the same
    bits, for single sequences with an initial state and for packed sequences."""
    api, st = hip.api(), stream()
    say(f"gdn scan block forms t={t} h={h} hk={hk} varlen={varlen}")
    if not varlen:
        q, k, v, g, b, s0 = cfg0_inputs(t, h, hk, seed=5, s0_std=0.01)
        runs = []
        for halves in ("1", "2"):
            forms(scan_halves=int(halves))
            runs.append(run_gdn(q, k, v, g, b, t, h, hk, s_in=s0, want_state=True))
        np.testing.assert_array_equal(runs[0][0], runs[1][0])
        np.testing.assert_array_equal(runs[0][1], runs[1][1])
        return
    lens = [64, 1, 0, 200, 129]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    q, k, v, g, b, _ = cfg0_inputs(T, h, hk, seed=6)
    s0 = (np.random.default_rng(7).standard_normal((h, D, D)) * 0.01).astype(np.float32)
    dq, dk, dv, dg, db, si = dev(q), dev(k), dev(v), dev(g), dev(b), dev(s0)
    outs = []
    for halves in ("1", "2"):
        forms(scan_halves=int(halves))
        o = empty(T * h * D * 2)
        so = empty(len(lens) * h * D * D * 4)
        ws = empty(api.cs1_gdn_workspace_floats(T + 64 * len(lens), h) * 4)
        hip.check(api.cs1_gdn_prefill_varlen(dq.at(0), dk.at(0), dv.at(0), dg.at(0), db.at(0), o.at(0), ws.at(0),
                                             cu.ctypes.data, len(lens), h, hk, D ** -0.5, si.at(0), 0, so.at(0),
                                             h * D * D, st.handle), "varlen")
        outs.append((get_bf16(o, T * h * D), get(so, np.float32, len(lens) * h * D * D)))
    np.testing.assert_array_equal(outs[0][0], outs[1][0])
    np.testing.assert_array_equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("t,h,hk,varlen", [(64, 8, 4, False), (65, 8, 4, False), (130, 6, 3, False),
                                            (192, 16, 16, False), (300, 32, 16, False), (450, 8, 2, False),
                                            (8229, 32, 16, False), (0, 16, 8, True)])
def test_gdn_scan_output_sets_are_bit_identical(t, h, hk, varlen, forms):
    """The one-half scan block runs its output with one set of four waves or with two sets
    taking alternate chunks (bf16(S) and v_new double-buffered, the o stores in the next
    chunk's barrier windows). Both must give the same output and final state: chunk counts
    1 to 5 (each tail of the set and chain loops), a segmented long sequence, and packed
    sequences including empty and one-row ones."""
    api, st = hip.api(), stream()
    say(f"gdn scan output sets t={t} h={h} hk={hk} varlen={varlen}")
    forms(scan_halves=1)
    if not varlen:
        q, k, v, g, b, s0 = cfg0_inputs(t, h, hk, seed=9, s0_std=0.01)
        runs = []
        for osets in ("1", "2"):
            forms(scan_halves=1, scan_osets=int(osets))
            runs.append(run_gdn(q, k, v, g, b, t, h, hk, s_in=s0, want_state=True))
        np.testing.assert_array_equal(runs[0][0], runs[1][0])
        np.testing.assert_array_equal(runs[0][1], runs[1][1])
        return
    lens = [64, 1, 0, 200, 129, 65, 128, 3]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    q, k, v, g, b, _ = cfg0_inputs(T, h, hk, seed=10)
    s0 = (np.random.default_rng(11).standard_normal((len(lens), h, D, D)) * 0.01).astype(np.float32)
    dq, dk, dv, dg, db, si = dev(q), dev(k), dev(v), dev(g), dev(b), dev(s0)
    outs = []
    for osets in ("1", "2"):
        forms(scan_halves=1, scan_osets=int(osets))
        o = empty(T * h * D * 2)
        so = empty(len(lens) * h * D * D * 4)
        ws = empty(api.cs1_gdn_workspace_floats(T + 64 * len(lens), h) * 4)
        hip.check(api.cs1_gdn_prefill_varlen(dq.at(0), dk.at(0), dv.at(0), dg.at(0), db.at(0), o.at(0), ws.at(0),
                                             cu.ctypes.data, len(lens), h, hk, D ** -0.5, si.at(0), h * D * D,
                                             so.at(0), h * D * D, st.handle), "varlen")
        outs.append((get_bf16(o, T * h * D), get(so, np.float32, len(lens) * h * D * D)))
    np.testing.assert_array_equal(outs[0][0], outs[1][0])
    np.testing.assert_array_equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("t,h,hk", [(512, 16, 16), (130, 6, 3), (107, 48, 16), (64, 8, 4)])
def test_gdn_prep_forms_are_bit_identical(t, h, hk, forms):
    """Launches whose chunks all fit on the device at once run the 8-wave prep (gdn_prep8),
    as two blocks per chunk when twice as many fit, the others the 4-wave one; every form must
    write the same records. The workspace starts as NaN bytes each time, so a record one form
    leaves unwritten shows up as a difference."""
    api, st = hip.api(), stream()
    say(f"gdn prep forms t={t} h={h} hk={hk}")
    q, k, v, g, b, s0 = cfg0_inputs(t, h, hk, seed=8, s0_std=0.01)
    bufs = (dev(q), dev(k), dev(v), dev(g), dev(b))
    si = dev(s0)
    nws = api.cs1_gdn_workspace_floats(t, h)
    runs = []
    for wide, split in (("0", "0"), ("1", "0"), ("1", "1")):
        forms(prep_wide=int(wide), prep_split=int(split))
        ws = dev(np.full(nws, 0xFFFFFFFF, np.uint32))
        o, so = empty(t * h * D * 2), empty(h * D * D * 4)
        hip.check(api.cs1_gdn_prefill_x(*(x.at(0) for x in bufs), o.at(0), ws.at(0), t, h, hk, D ** -0.5, si.at(0),
                                        so.at(0), st.handle), "gdn prefill")
        runs.append((get_bf16(o, t * h * D), get(so, np.float32, h * D * D), get(ws, np.uint32, nws)))
    for other in runs[1:]:
        np.testing.assert_array_equal(runs[0][0], other[0])
        np.testing.assert_array_equal(runs[0][1], other[1])
        np.testing.assert_array_equal(runs[0][2], other[2])  # every record byte


def test_gdn_empty_window_captures_state_copy_and_zero_initial_state():
    # kernels.rs:692-742: T = 0 under graph capture must re-run the copy / zero on replay
    api, st = hip.api(), stream()
    h, n = 2, 2 * D * D
    state = dev(np.ones(n, np.float32))
    output = dev(np.full(n, 2.0, np.float32))

    def window(inp):
        hip.check(api.cs1_gdn_prefill_x(None, None, None, None, None, None, None, 0, h, 1, 1.0, inp, output.at(0),
                                        st.handle), "empty gdn window")

    say("gdn empty window graph capture")
    copy = hip.Graph(st, lambda: window(state.at(0)))
    hip.upload(state, np.full(n, 3.0, np.float32), st)
    for _ in range(3):
        copy.launch(st)
        np.testing.assert_array_equal(get(output, np.float32, n), np.full(n, 3.0, np.float32))
    zero = hip.Graph(st, lambda: window(None))
    for _ in range(3):
        hip.upload(output, np.full(n, 3.0, np.float32), st)
        zero.launch(st)
        assert not get(output, np.float32, n).any()


def test_gdn_graph_replay_matches_eager():
    # the prefill is capturable: replays (with eager work in between) repeat the eager result
    api, st = hip.api(), stream()
    T, H, HK = 300, 4, 2
    say(f"gdn graph replay T={T}")
    q, k, v, g, b, s0 = cfg0_inputs(T, H, HK, seed=5, s0_std=0.01)
    bufs = (dev(q), dev(k), dev(v), dev(g), dev(b))
    eager, s_eager = run_gdn(q, k, v, g, b, T, H, HK, s_in=s0, want_state=True, bufs=bufs)
    o = empty(T * H * D * 2)
    ws = empty(api.cs1_gdn_workspace_floats(T, H) * 4)
    si, so = dev(s0), empty(H * D * D * 4)

    def record():
        hip.check(api.cs1_gdn_prefill_x(*(x.at(0) for x in bufs), o.at(0), ws.at(0), T, H, HK, D ** -0.5, si.at(0),
                                        so.at(0), st.handle), "captured gdn")

    graph = hip.Graph(st, record)
    for i in range(3):
        hip.upload(o, np.zeros(T * H * D, np.uint16), st)
        graph.launch(st)
        np.testing.assert_array_equal(get_bf16(o, T * H * D).reshape(T, H, D), eager)
        np.testing.assert_array_equal(get(so, np.float32, H * D * D).reshape(H, D, D), s_eager)
        run_gdn(q, k, v, g, b, 64, H, HK, bufs=bufs)  # unrelated eager work between replays


def test_gdn_zero_inputs_and_tiny_amplitudes_are_finite():
    for amp in (0.0, 1e-18):
        say(f"gdn amplitude {amp}")
        q, k, v, g, b = O.gdn_test_inputs(65, 4, 2, 0.01, amp)
        o, s = run_gdn(q, k, v, g, b, 65, 4, 2, want_state=True)
        f = O.bf16_to_f32(o)
        assert np.isfinite(f).all() and np.isfinite(s).all()
        if amp == 0.0:
            assert not f.any()


@pytest.mark.parametrize("shared_state", [True, False])
def test_gdn_varlen_matches_per_sequence_calls(shared_state):
    """cs1_gdn_prefill_varlen over packed sequences (empty, partial-chunk and multi-chunk ones)
    equals one cs1_gdn_prefill_x call per sequence bit for bit, outputs and final states, with
    one initial state shared by all sequences (the candidate-scoring case) or one each."""
    api, st = hip.api(), stream()
    H, HK = 8, 4
    lens = [0, 1, 63, 64, 65, 200, 129, 0, 7]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    q, k, v, g, beta, _ = cfg0_inputs(T, H, HK, seed=11)
    rng = np.random.default_rng(12)
    n = len(lens)
    states = (rng.standard_normal((1 if shared_state else n, H, D, D)) * 0.05).astype(np.float32)
    say(f"gdn varlen lens={lens} shared_state={shared_state}")
    bufs = (dev(q), dev(k), dev(v), dev(g), dev(beta))
    o = empty(T * H * D * 2)
    nch = int(sum((x + 63) // 64 for x in lens))
    ws = empty(api.cs1_gdn_workspace_floats(64 * nch, H) * 4)
    si = dev(states.reshape(-1))
    so = empty(n * H * D * D * 4)
    stride = 0 if shared_state else H * D * D
    hip.check(api.cs1_gdn_prefill_varlen(*(b.at(0) for b in bufs), o.at(0), ws.at(0), cu.ctypes.data, n, H, HK,
                                         D ** -0.5, si.at(0), stride, so.at(0), H * D * D, st.handle), "varlen")
    got_o = get_bf16(o, T * H * D).reshape(T, H, D)
    got_s = get(so, np.float32, n * H * D * D).reshape(n, H, D, D)
    for i, L in enumerate(lens):
        r0 = int(cu[i])
        s0 = states[0 if shared_state else i]
        if L == 0:
            np.testing.assert_array_equal(got_s[i], s0)
            continue
        rows = slice(r0, r0 + L)
        one_o, one_s = run_gdn(q.reshape(T, HK, D)[rows].reshape(-1), k.reshape(T, HK, D)[rows].reshape(-1),
                               v.reshape(T, H, D)[rows].reshape(-1), g.reshape(T, H)[rows].reshape(-1),
                               beta.reshape(T, H)[rows].reshape(-1), L, H, HK, s_in=s0, want_state=True)
        np.testing.assert_array_equal(got_o[rows], one_o)
        np.testing.assert_array_equal(got_s[i], one_s)


def test_gdn_varlen_arguments():
    api, st = hip.api(), stream()
    cu = np.array([0, 64, 32], np.int32)  # decreasing
    assert api.cs1_gdn_prefill_varlen(None, None, None, None, None, None, None, cu.ctypes.data, 2, 8, 4, 1.0, None, 0,
                                      None, 0, st.handle) != 0
    cu = np.zeros(66, np.int32)
    assert api.cs1_gdn_prefill_varlen(None, None, None, None, None, None, None, cu.ctypes.data, 65, 8, 4, 1.0, None, 0,
                                      None, 0, st.handle) != 0
    assert api.cs1_gdn_prefill_varlen(None, None, None, None, None, None, None, None, 0, 8, 4, 1.0, None, 0, None, 0,
                                      st.handle) == 0


def gate_projections(T, H, ld, seed):
    """Model-like raw gate inputs: rows of ld bf16 holding b at columns [0, H) and a at
    [H, 2H) (the reference's projection layout), A_log = log U(0, 16) and dt_bias ~ 1 + N(0, 0.1)
    (transformers' init, TF:816-820), with a spread that reaches the softplus threshold (x > 20)."""
    rng = np.random.default_rng(seed)
    rows = O.f32_to_bf16((rng.standard_normal((T, ld)) * 2.0).astype(np.float32)).reshape(T, ld)
    rows[::7, H] = O.f32_to_bf16(np.float32([25.0]))[0]  # a + dt_bias above 20 on some tokens
    A_log = O.f32_to_bf16(np.log(rng.uniform(1e-3, 16.0, H)).astype(np.float32))
    dt = O.f32_to_bf16((1.0 + rng.standard_normal(H) * 0.1).astype(np.float32))
    return rows.reshape(-1), A_log, dt


@pytest.mark.parametrize("t,h,hk,prep", [(2000, 16, 8, "4-wave"), (130, 6, 3, "8-wave"), (107, 48, 16, "8-wave"),
                                         (64, 8, 4, "split"), (8229, 32, 16, "segmented")])
def test_gated_prefill_equals_gates_then_prefill(t, h, hk, prep, forms):
    """cs1_gdn_prefill_gated_x (beta and g computed inside the prep from the raw projections)
    equals cs1_gdn_gates followed by cs1_gdn_prefill_x bit for bit, outputs and final state, on
    every prep form (4-wave, 8-wave, split 8-wave, and a segmented long sequence)."""
    api, st = hip.api(), stream()
    say(f"gated gdn prefill t={t} h={h} hk={hk} prep={prep}")
    if prep == "split":
        forms(prep_wide=1, prep_split=1)
    elif prep == "8-wave":
        forms(prep_wide=1, prep_split=0)
    q, k, v, _, _, s0 = cfg0_inputs(t, h, hk, seed=31, s0_std=0.01)
    ld = 2 * h + 24
    rows, A_log, dt = gate_projections(t, h, ld, seed=32)
    drows, dA, ddt = dev(rows), dev(A_log), dev(dt)
    beta, g = empty(t * h * 2), empty(t * h * 4)
    hip.check(api.cs1_gdn_gates(drows.at(0), drows.at(2 * h), ld, dA.at(0), ddt.at(0), beta.at(0), g.at(0), t, h,
                                st.handle), "gates")
    dq, dk, dv, si = dev(q), dev(k), dev(v), dev(s0)
    ws = empty(api.cs1_gdn_workspace_floats(t, h) * 4)
    o1, o2 = empty(t * h * D * 2), empty(t * h * D * 2)
    so1, so2 = empty(h * D * D * 4), empty(h * D * D * 4)
    hip.check(api.cs1_gdn_prefill_x(dq.at(0), dk.at(0), dv.at(0), g.at(0), beta.at(0), o1.at(0), ws.at(0), t, h, hk,
                                    D ** -0.5, si.at(0), so1.at(0), st.handle), "ungated")
    hip.check(api.cs1_gdn_prefill_gated_x(dq.at(0), dk.at(0), dv.at(0), drows.at(0), drows.at(2 * h), ld, dA.at(0),
                                          ddt.at(0), o2.at(0), ws.at(0), t, h, hk, D ** -0.5, si.at(0), so2.at(0),
                                          st.handle), "gated")
    a_o, b_o = get_bf16(o1, t * h * D), get_bf16(o2, t * h * D)
    assert np.isfinite(O.bf16_to_f32(b_o)).all()
    np.testing.assert_array_equal(b_o, a_o)
    np.testing.assert_array_equal(get(so2, np.float32, h * D * D), get(so1, np.float32, h * D * D))


def test_gated_varlen_equals_gates_then_varlen():
    """cs1_gdn_prefill_gated_varlen equals cs1_gdn_gates + cs1_gdn_prefill_varlen bit for bit
    over packed sequences (empty and partial-chunk ones) from a shared initial state; argument
    errors for missing gate inputs or ld < H."""
    api, st = hip.api(), stream()
    H, HK = 8, 4
    lens = [0, 1, 63, 64, 65, 200, 7]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    say(f"gated gdn varlen lens={lens}")
    q, k, v, _, _, _ = cfg0_inputs(T, H, HK, seed=33)
    s0 = (np.random.default_rng(34).standard_normal((H, D, D)) * 0.05).astype(np.float32)
    ld = 40
    rows, A_log, dt = gate_projections(T, H, ld, seed=35)
    drows, dA, ddt = dev(rows), dev(A_log), dev(dt)
    beta, g = empty(T * H * 2), empty(T * H * 4)
    hip.check(api.cs1_gdn_gates(drows.at(0), drows.at(2 * H), ld, dA.at(0), ddt.at(0), beta.at(0), g.at(0), T, H,
                                st.handle), "gates")
    dq, dk, dv, si = dev(q), dev(k), dev(v), dev(s0)
    nch = int(sum((x + 63) // 64 for x in lens))
    ws = empty(api.cs1_gdn_workspace_floats(64 * nch, H) * 4)
    n = len(lens)
    outs = []
    for gated in (False, True):
        o, so = empty(T * H * D * 2), empty(n * H * D * D * 4)
        if gated:
            rc = api.cs1_gdn_prefill_gated_varlen(dq.at(0), dk.at(0), dv.at(0), drows.at(0), drows.at(2 * H), ld,
                                                  dA.at(0), ddt.at(0), o.at(0), ws.at(0), cu.ctypes.data, n, H, HK,
                                                  D ** -0.5, si.at(0), 0, so.at(0), H * D * D, st.handle)
        else:
            rc = api.cs1_gdn_prefill_varlen(dq.at(0), dk.at(0), dv.at(0), g.at(0), beta.at(0), o.at(0), ws.at(0),
                                            cu.ctypes.data, n, H, HK, D ** -0.5, si.at(0), 0, so.at(0), H * D * D,
                                            st.handle)
        hip.check(rc, f"varlen gated={gated}")
        outs.append((get_bf16(o, T * H * D), get(so, np.float32, n * H * D * D)))
    np.testing.assert_array_equal(outs[1][0], outs[0][0])
    np.testing.assert_array_equal(outs[1][1], outs[0][1])
    # argument errors: missing gate inputs, ld < H
    assert api.cs1_gdn_prefill_gated_x(dq.at(0), dk.at(0), dv.at(0), None, drows.at(0), ld, dA.at(0), ddt.at(0),
                                       None, ws.at(0), 64, H, HK, 1.0, None, None,
                                       st.handle) == hip.HIP_ERROR_INVALID_VALUE
    assert api.cs1_gdn_prefill_gated_x(dq.at(0), dk.at(0), dv.at(0), drows.at(0), drows.at(0), H - 1, dA.at(0),
                                       ddt.at(0), None, ws.at(0), 64, H, HK, 1.0, None, None,
                                       st.handle) == hip.HIP_ERROR_INVALID_VALUE
    assert api.cs1_gdn_prefill_gated_varlen(dq.at(0), dk.at(0), dv.at(0), drows.at(0), drows.at(0), ld, None,
                                            ddt.at(0), None, ws.at(0), cu.ctypes.data, n, H, HK, 1.0, None, 0, None,
                                            0, st.handle) == hip.HIP_ERROR_INVALID_VALUE
