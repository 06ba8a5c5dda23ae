"""GPU parity of the causal GQA flash attention (cs1_attention*, cs1_attention_ex).

Mirrors tests/qwen3_5/kernels.rs:273-474 and 852-929 and adds benchmark config 1
(Dh = 128, sigmoid gate, float32 log-sum-exp), which the reference kernel does not
support. Bars:
  * vs float64 (kernels.rs:436-472): per (row, head) max|diff| / max(max|ref|, 1e-3) < 1.6e-2;
  * vs the emulated reference kernel: bf16 max-abs <= 2e-2, mean-abs <= 2e-3;
  * LSE vs float64 within 1e-3 absolute;
  * bit-for-bit: fused gate == attention + cs1_sigmoid_gate; windowed == full pass.
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


def attn(q, k, v, ldv, gate, T, Hq, Hk, Dh, scale, q_base=0, lse=False, v_off=0):
    api, st = hip.api(), stream()
    out = empty(T * Hq * Dh * 2)
    lse_buf = empty(Hq * T * 4) if lse else None
    hip.check(api.cs1_attention_ex(q.at(0), k.at(0), v.at(v_off * 2), ldv, gate.at(0) if gate else None, out.at(0),
                                   lse_buf.at(0) if lse else None, T, Hq, Hk, Dh, scale, q_base, st.handle),
              "attention_ex")
    o = get_bf16(out, T * Hq * Dh).reshape(T, Hq, Dh)
    return (o, get(lse_buf, np.float32, Hq * T).reshape(Hq, T)) if lse else o


@pytest.mark.parametrize("case", GOLDEN["attention"], ids=lambda c: f"t{c['t']}")
def test_flash_attention_matches_float64_reference(case):
    api, st = hip.api(), stream()
    t, amp = case["t"], case["amp"]
    hq, hk, dh = 16, 4, 256
    say(f"attention f64 case t={t} amp={amp}")
    qh, kh = O.xorshift_bf16(t * hq * dh, 1, amp), O.xorshift_bf16(t * hk * dh, 2, amp)
    ldv, v_at = 10240, (hq * 2 + hk) * dh
    qkvh = O.xorshift_bf16(t * ldv, 3, 1.0)
    q, k, qkv = dev(qh), dev(kh), dev(qkvh)
    out = empty(t * hq * dh * 2)
    hip.check(api.cs1_attention(q.at(0), k.at(0), qkv.at(v_at * 2), ldv, out.at(0), t, hq, hk, dh, 0.0625, st.handle),
              "attention")
    got = get_bf16(out, t * hq * dh).reshape(t, hq, dh)
    gf = O.bf16_to_f32(got).astype(np.float64)
    assert np.isfinite(gf).all()
    vh = np.concatenate([qkvh[v_at:], np.zeros(v_at, np.uint16)])
    rows = sorted(set(range(0, t, -(-t // 64))) | {t - 1})
    want = O.attention_f64(qh, kh, vh, ldv, t, hq, hk, dh, 0.0625, rows=rows)
    worst = max(np.abs(gf[i, h] - want[i, h]).max() / max(1e-3, np.abs(want[i, h]).max()) for i in rows
                for h in range(hq))
    say(f"  largest relative difference {worst:.2e} (reference kernel {case['kernel_max_rel_diff']:.2e})")
    assert worst < 1.6e-2
    emu = O.attention_emul(qh, kh, vh, ldv, None, t, hq, hk, dh, 0.0625)
    mx, mean = bf16_errors(got, O.bf16_to_f32(emu))
    say(f"  vs emulated reference kernel: max-abs {mx:.2e} mean-abs {mean:.2e}")
    assert mx <= 2e-2 and mean <= 2e-3


def test_fused_attention_gate_matches_separate_pass():
    api, st = hip.api(), stream()
    dh = 256
    for hq, hk in [(24, 4), (16, 4), (4, 4), (16, 1)]:
        for t in [1, 63, 64, 65, 139, 712, 2048]:
            say(f"fused gate hq={hq} hk={hk} t={t}")
            ldv = hk * dh + 16
            q = dev(O.xorshift_bf16(t * hq * dh, 1, 2.0))
            k = dev(O.xorshift_bf16(t * hk * dh, 2, 2.0))
            v = dev(O.xorshift_bf16(t * ldv, 3, 1.0))
            n = t * hq * dh
            gates = O.xorshift_bf16(n, 4, 12.0).reshape(-1, dh)
            gates[:, 0] = O.f32_to_bf16(np.float32([-40.0]))[0]
            gates[:, 1] = O.f32_to_bf16(np.float32([40.0]))[0]
            gates[:, 2] = 0
            gate = dev(gates)
            sep, fused = empty(n * 2), empty(n * 2)
            hip.check(api.cs1_attention(q.at(0), k.at(0), v.at(0), ldv, sep.at(0), t, hq, hk, dh, 0.0625, st.handle),
                      "separate attention")
            hip.check(api.cs1_sigmoid_gate(sep.at(0), gate.at(0), n, st.handle), "separate gate")
            hip.check(api.cs1_attention_gated(q.at(0), k.at(0), v.at(0), ldv, gate.at(0), fused.at(0), t, hq, hk, dh,
                                              0.0625, st.handle), "fused gate")
            want, got = get_bf16(sep, n), get_bf16(fused, n)
            assert np.isfinite(O.bf16_to_f32(got)).all()
            np.testing.assert_array_equal(got, want)


def test_windowed_attention_matches_full_pass_bit_for_bit():
    api, st = hip.api(), stream()
    hq, hk, dh = 24, 4, 256
    for t, bases in [(139, [64]), (712, [64, 128]), (972, [64, 896]), (2048, [64, 1024])]:
        ldv = hk * dh + 16
        q = dev(O.xorshift_bf16(t * hq * dh, 1, 2.0))
        k = dev(O.xorshift_bf16(t * hk * dh, 2, 2.0))
        v = dev(O.xorshift_bf16(t * ldv, 3, 1.0))
        gate = dev(O.xorshift_bf16(t * hq * dh, 4, 3.0))
        full = empty(t * hq * dh * 2)
        say(f"windowed attention t={t}")
        hip.check(api.cs1_attention_gated(q.at(0), k.at(0), v.at(0), ldv, gate.at(0), full.at(0), t, hq, hk, dh,
                                          0.0625, st.handle), "full pass")
        full_rows = get_bf16(full, t * hq * dh).reshape(t, -1)
        for qb in bases:
            win = empty(t * hq * dh * 2)
            hip.check(api.cs1_attention_gated_prefix(q.at(0), k.at(0), v.at(0), ldv, gate.at(0), win.at(0), t, hq, hk,
                                                     dh, 0.0625, qb, st.handle), "windowed pass")
            np.testing.assert_array_equal(get_bf16(win, t * hq * dh).reshape(t, -1)[qb:], full_rows[qb:])


def cfg1_inputs(T=2048, Hq=16, Hk=4, Dh=128, seed=1):
    rng = np.random.default_rng(seed)
    q = O.f32_to_bf16(rng.standard_normal(T * Hq * Dh).astype(np.float32))
    k = O.f32_to_bf16(rng.standard_normal(T * Hk * Dh).astype(np.float32))
    v = O.f32_to_bf16(rng.standard_normal(T * Hk * Dh).astype(np.float32))
    gate = O.f32_to_bf16(rng.standard_normal(T * Hq * Dh).astype(np.float32))
    return q, k, v, gate


@pytest.mark.parametrize("T", [2048, 1, 63, 65, 300])
def test_config1_dh128_gated_with_lse(T):
    Hq, Hk, Dh = 16, 4, 128
    scale = Dh ** -0.5
    say(f"attention config1 Dh=128 T={T}")
    q, k, v, gate = cfg1_inputs(T, Hq, Hk, Dh)
    out, lse = attn(dev(q), dev(k), dev(v), Hk * Dh, dev(gate), T, Hq, Hk, Dh, scale, lse=True)
    emu, else_ = O.attention_emul(q, k, v, Hk * Dh, gate, T, Hq, Hk, Dh, scale, want_lse=True)
    mx, mean = bf16_errors(out, O.bf16_to_f32(emu))
    say(f"  vs emulated reference kernel: max-abs {mx:.2e} mean-abs {mean:.2e}")
    assert mx <= 2e-2 and mean <= 2e-3
    rows = sorted(set(range(0, T, max(1, T // 64))) | {T - 1})
    want, wlse = O.attention_f64(q, k, v, Hk * Dh, T, Hq, Hk, Dh, scale, want_lse=True, rows=rows)
    gl = lse[:, rows]
    say(f"  lse vs float64: {np.abs(gl - wlse[:, rows]).max():.2e}")
    np.testing.assert_allclose(gl, wlse[:, rows], atol=1e-3, rtol=0)
    np.testing.assert_allclose(lse, else_, atol=1e-3, rtol=0)
    # the ungated output against float64 (reference relative bar)
    plain = attn(dev(q), dev(k), dev(v), Hk * Dh, None, T, Hq, Hk, Dh, scale)
    pf = O.bf16_to_f32(plain).astype(np.float64)
    worst = max(np.abs(pf[i, h] - want[i, h]).max() / max(1e-3, np.abs(want[i, h]).max()) for i in rows
                for h in range(Hq))
    say(f"  ungated vs float64 relative {worst:.2e}")
    assert worst < 1.6e-2


def test_north_star_shape_t8192_sampled_rows():
    """The north-star attention shape (T = 8192, 16/4 heads, Dh 128, gated, LSE): 1024 row
    blocks run longest-first over several rounds of the device. Checked on sampled rows, as
    the reference checks long sequences (kernels.rs:393-474): the ungated output against
    float64 (relative bar 1.6e-2), the LSE against float64 (1e-3), and the gated output and LSE
    against the emulated reference kernel (bf16 max-abs 2e-2 / mean-abs 2e-3, LSE 1e-3)."""
    T, Hq, Hk, Dh = 8192, 16, 4, 128
    scale = Dh ** -0.5
    say(f"attention north-star shape T={T} {Hq}/{Hk} Dh={Dh}, sampled rows")
    q, k, v, gate = cfg1_inputs(T, Hq, Hk, Dh, seed=21)
    rng = np.random.default_rng(22)
    # the first and last rows of several row blocks (longest and shortest work items), the
    # block boundaries around the middle, and random rows
    rows = {0, 1, 31, 32, 63, 64, 4095, 4096, 8127, 8128, 8190, T - 1}
    rows |= set(int(x) for x in rng.choice(T, 52, replace=False))
    rows = sorted(rows)
    dq, dk, dv, dg = dev(q), dev(k), dev(v), dev(gate)
    out, lse = attn(dq, dk, dv, Hk * Dh, dg, T, Hq, Hk, Dh, scale, lse=True)
    plain = attn(dq, dk, dv, Hk * Dh, None, T, Hq, Hk, Dh, scale)
    assert np.isfinite(O.bf16_to_f32(out)).all() and np.isfinite(lse).all()
    want, wlse = O.attention_f64(q, k, v, Hk * Dh, T, Hq, Hk, Dh, scale, want_lse=True, rows=rows)
    pf = O.bf16_to_f32(plain).astype(np.float64)
    worst = max(np.abs(pf[i, h] - want[i, h]).max() / max(1e-3, np.abs(want[i, h]).max()) for i in rows
                for h in range(Hq))
    say(f"  {len(rows)} rows: ungated vs float64 relative {worst:.2e}, "
        f"lse vs float64 {np.abs(lse[:, rows] - wlse[:, rows]).max():.2e}")
    assert worst < 1.6e-2
    np.testing.assert_allclose(lse[:, rows], wlse[:, rows], atol=1e-3, rtol=0)
    emu, else_ = O.attention_emul(q, k, v, Hk * Dh, gate, T, Hq, Hk, Dh, scale, want_lse=True, rows=rows)
    mx, mean = bf16_errors(out[rows], O.bf16_to_f32(emu[rows]))
    say(f"  gated vs emulated reference kernel: max-abs {mx:.2e} mean-abs {mean:.2e}")
    assert mx <= 2e-2 and mean <= 2e-3
    np.testing.assert_allclose(lse[:, rows], else_[:, rows], atol=1e-3, rtol=0)


def test_t32768_sampled_rows():
    """A long single sequence (T = 32768, 16/4 heads, Dh 128, gated, LSE): 4096 row blocks, rows
    of up to 1024 steps per key group, many lazy rescales. Same checks and bars as the
    north-star shape, on sampled rows."""
    T, Hq, Hk, Dh = 32768, 16, 4, 128
    scale = Dh ** -0.5
    say(f"attention T={T} {Hq}/{Hk} Dh={Dh}, sampled rows")
    q, k, v, gate = cfg1_inputs(T, Hq, Hk, Dh, seed=25)
    rng = np.random.default_rng(26)
    rows = sorted({0, 31, 32, 16383, 16384, 32735, 32736, T - 1} | set(int(x) for x in rng.choice(T, 16, replace=False)))
    dq, dk, dv, dg = dev(q), dev(k), dev(v), dev(gate)
    out, lse = attn(dq, dk, dv, Hk * Dh, dg, T, Hq, Hk, Dh, scale, lse=True)
    plain = attn(dq, dk, dv, Hk * Dh, None, T, Hq, Hk, Dh, scale)
    want, wlse = O.attention_f64(q, k, v, Hk * Dh, T, Hq, Hk, Dh, scale, want_lse=True, rows=rows)
    pf = O.bf16_to_f32(plain).astype(np.float64)
    worst = max(np.abs(pf[i, h] - want[i, h]).max() / max(1e-3, np.abs(want[i, h]).max()) for i in rows
                for h in range(Hq))
    say(f"  {len(rows)} rows: ungated vs float64 relative {worst:.2e}, "
        f"lse vs float64 {np.abs(lse[:, rows] - wlse[:, rows]).max():.2e}")
    assert worst < 1.6e-2
    np.testing.assert_allclose(lse[:, rows], wlse[:, rows], atol=1e-3, rtol=0)
    emu, else_ = O.attention_emul(q, k, v, Hk * Dh, gate, T, Hq, Hk, Dh, scale, want_lse=True, rows=rows)
    mx, mean = bf16_errors(out[rows], O.bf16_to_f32(emu[rows]))
    say(f"  gated vs emulated reference kernel: max-abs {mx:.2e} mean-abs {mean:.2e}")
    assert mx <= 2e-2 and mean <= 2e-3
    np.testing.assert_allclose(lse[:, rows], else_[:, rows], atol=1e-3, rtol=0)


def test_dh256_t8192_sampled_rows():
    """The config-3 attention shape (16/4 heads, Dh 256, gated, LSE) at T = 8192: 1024 blocks of
    flash256_kernel over several rounds of the device. Sampled rows against float64 (ungated,
    relative bar 1.6e-2; LSE 1e-3) and against the emulated reference kernel (gated, bf16
    max-abs 2e-2 / mean-abs 2e-3)."""
    T, Hq, Hk, Dh = 8192, 16, 4, 256
    scale = Dh ** -0.5
    say(f"attention T={T} {Hq}/{Hk} Dh={Dh}, sampled rows")
    q, k, v, gate = cfg1_inputs(T, Hq, Hk, Dh, seed=23)
    rng = np.random.default_rng(24)
    rows = sorted({0, 63, 64, 4095, 8127, 8128, T - 1} | set(int(x) for x in rng.choice(T, 40, replace=False)))
    dq, dk, dv, dg = dev(q), dev(k), dev(v), dev(gate)
    out, lse = attn(dq, dk, dv, Hk * Dh, dg, T, Hq, Hk, Dh, scale, lse=True)
    plain = attn(dq, dk, dv, Hk * Dh, None, T, Hq, Hk, Dh, scale)
    want, wlse = O.attention_f64(q, k, v, Hk * Dh, T, Hq, Hk, Dh, scale, want_lse=True, rows=rows)
    pf = O.bf16_to_f32(plain).astype(np.float64)
    worst = max(np.abs(pf[i, h] - want[i, h]).max() / max(1e-3, np.abs(want[i, h]).max()) for i in rows
                for h in range(Hq))
    say(f"  {len(rows)} rows: ungated vs float64 relative {worst:.2e}, "
        f"lse vs float64 {np.abs(lse[:, rows] - wlse[:, rows]).max():.2e}")
    assert worst < 1.6e-2
    np.testing.assert_allclose(lse[:, rows], wlse[:, rows], atol=1e-3, rtol=0)
    emu = O.attention_emul(q, k, v, Hk * Dh, gate, T, Hq, Hk, Dh, scale, rows=rows)
    mx, mean = bf16_errors(out[rows], O.bf16_to_f32(emu[rows]))
    say(f"  gated vs emulated reference kernel: max-abs {mx:.2e} mean-abs {mean:.2e}")
    assert mx <= 2e-2 and mean <= 2e-3


@pytest.mark.parametrize("hq,hk", [(32, 4), (8, 1), (12, 3)])
def test_dh128_head_ratios_vs_emulator(hq, hk):
    """GQA ratios beyond 4 q heads per kv head and odd kv-head counts on the Dh=128 path."""
    T, Dh = 257, 128
    say(f"attention Dh=128 hq={hq} hk={hk} T={T}")
    q, k, v, gate = cfg1_inputs(T, hq, hk, Dh, seed=5)
    out, lse = attn(dev(q), dev(k), dev(v), hk * Dh, dev(gate), T, hq, hk, Dh, Dh ** -0.5, lse=True)
    emu, else_ = O.attention_emul(q, k, v, hk * Dh, gate, T, hq, hk, Dh, Dh ** -0.5, want_lse=True)
    mx, mean = bf16_errors(out, O.bf16_to_f32(emu))
    say(f"  vs emulated reference kernel: max-abs {mx:.2e} mean-abs {mean:.2e}")
    assert mx <= 2e-2 and mean <= 2e-3
    np.testing.assert_allclose(lse, else_, atol=1e-3, rtol=0)


def test_dh128_window_and_strided_v_bit_for_bit():
    T, Hq, Hk, Dh = 700, 8, 2, 128
    q, k, _, gate = cfg1_inputs(T, Hq, Hk, Dh, seed=3)
    ldv = 3 * Hk * Dh + 8
    vbig = O.xorshift_bf16(T * ldv, 7, 1.0)
    dq, dk, dv, dg = dev(q), dev(k), dev(vbig), dev(gate)
    say("attention Dh=128 strided V, windows")
    full = attn(dq, dk, dv, ldv, dg, T, Hq, Hk, Dh, 0.09, v_off=2 * Hk * Dh)
    for qb in (64, 320, 640):
        win = attn(dq, dk, dv, ldv, dg, T, Hq, Hk, Dh, 0.09, q_base=qb, v_off=2 * Hk * Dh)
        np.testing.assert_array_equal(win[qb:], full[qb:])
    vv = np.ascontiguousarray(vbig.reshape(T, ldv)[:, 2 * Hk * Dh: 3 * Hk * Dh]).reshape(-1)
    emu = O.attention_emul(q, k, vv, Hk * Dh, gate, T, Hq, Hk, Dh, 0.09)
    mx, mean = bf16_errors(full, O.bf16_to_f32(emu))
    assert mx <= 2e-2 and mean <= 2e-3


@pytest.mark.parametrize("Dh,hq,hk,gated", [(128, 16, 4, True), (128, 6, 2, False), (256, 16, 4, True),
                                            (256, 8, 8, False)])
def test_varlen_matches_per_sequence_calls(Dh, hq, hk, gated):
    """cs1_attention_varlen over packed sequences equals cs1_attention_ex on each sequence's
    rows bit for bit (outputs and LSE); 70 sequences exercise the multi-launch path."""
    rng = np.random.default_rng(Dh + hq)
    lens = [1, 16, 17, 64, 300, 0, 129] + list(rng.integers(1, 40, 63))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    say(f"attention varlen Dh={Dh} {hq}/{hk} gated={gated} nseq={len(lens)} total={T}")
    api, st = hip.api(), stream()
    q, k, v, g = (O.f32_to_bf16(rng.standard_normal(T * h * Dh).astype(np.float32)) for h in (hq, hk, hk, hq))
    dq, dk, dv, dg = dev(q), dev(k), dev(v), dev(g)
    out, lse = empty(T * hq * Dh * 2), empty(hq * T * 4)
    hip.check(api.cs1_attention_varlen(dq.at(0), dk.at(0), dv.at(0), hk * Dh, dg.at(0) if gated else None, out.at(0),
                                       lse.at(0), cu.ctypes.data, len(lens), hq, hk, Dh, Dh ** -0.5, st.handle),
              "varlen")
    got = get_bf16(out, T * hq * Dh).reshape(T, hq, Dh)
    got_lse = get(lse, np.float32, hq * T).reshape(hq, T)
    for s in range(len(lens)):
        a, n = int(cu[s]), int(lens[s])
        if n == 0:
            continue
        sq, sk, sv, sg = (dev(x.reshape(T, -1)[a:a + n].reshape(-1)) for x in (q, k, v, g))
        o1, l1 = empty(n * hq * Dh * 2), empty(hq * n * 4)
        hip.check(api.cs1_attention_ex(sq.at(0), sk.at(0), sv.at(0), hk * Dh, sg.at(0) if gated else None, o1.at(0),
                                       l1.at(0), n, hq, hk, Dh, Dh ** -0.5, 0, st.handle), "ex")
        np.testing.assert_array_equal(got[a:a + n], get_bf16(o1, n * hq * Dh).reshape(n, hq, Dh))
        np.testing.assert_array_equal(got_lse[:, a:a + n], get(l1, np.float32, hq * n).reshape(hq, n))


def test_varlen_arguments():
    api, st = hip.api(), stream()
    say("attention varlen argument checks")
    bad = np.array([1, 5], np.int32)
    assert api.cs1_attention_varlen(None, None, None, 512, None, None, None, bad.ctypes.data, 1, 16, 4, 128, 0.1,
                                    st.handle) == hip.HIP_ERROR_INVALID_VALUE
    assert api.cs1_attention_varlen(None, None, None, 512, None, None, None, None, 0, 16, 4, 128, 0.1,
                                    st.handle) == 0


@pytest.mark.parametrize("Dh,hq,hk,gated", [(256, 16, 4, True), (256, 24, 4, True), (128, 16, 4, True),
                                            (128, 8, 8, False)])
def test_prefix_varlen_matches_windowed_calls(Dh, hq, hk, gated):
    """cs1_attention_prefix_varlen (packed candidates continuing one cached prefix) equals, per
    candidate, cs1_attention_ex over [prefix K/V | candidate K/V] with q_base = prefix length,
    bit for bit: the candidate-scoring attention without window copies."""
    api, st = hip.api(), stream()
    P = 128
    lens = [1, 40, 64, 100, 0, 33]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    rng = np.random.default_rng(21)

    def bf(n):
        return O.f32_to_bf16(rng.standard_normal(n).astype(np.float32))

    q, gate = bf(T * hq * Dh), bf(T * hq * Dh)
    k, v = bf(T * hk * Dh), bf(T * hk * Dh)
    kp, vp = bf(P * hk * Dh), bf(P * hk * Dh)
    say(f"attention prefix varlen Dh={Dh} hq={hq} hk={hk} P={P} lens={lens}")
    out = empty(T * hq * Dh * 2)
    lse = empty(hq * T * 4)
    dq, dk, dv, dkp, dvp, dg = (dev(x) for x in (q, k, v, kp, vp, gate))  # held until the results are read
    hip.check(api.cs1_attention_prefix_varlen(dq.at(0), dk.at(0), dv.at(0), hk * Dh, dkp.at(0), dvp.at(0), hk * Dh, P,
                                              dg.at(0) if gated else None, out.at(0), lse.at(0), cu.ctypes.data,
                                              len(lens), hq, hk, Dh, Dh ** -0.5, st.handle), "prefix varlen")
    got = get_bf16(out, T * hq * Dh).reshape(T, hq, Dh)
    got_lse = get(lse, np.float32, hq * T).reshape(hq, T)
    rq, rg = hq * Dh, hk * Dh
    for i, L in enumerate(lens):
        if L == 0:
            continue
        r0 = int(cu[i])
        W = P + L
        kw = np.concatenate([kp, k[r0 * rg:(r0 + L) * rg]])
        vw = np.concatenate([vp, v[r0 * rg:(r0 + L) * rg]])
        qw = np.concatenate([np.zeros(P * rq, np.uint16), q[r0 * rq:(r0 + L) * rq]])
        gw = np.concatenate([np.zeros(P * rq, np.uint16), gate[r0 * rq:(r0 + L) * rq]])
        one = empty(W * rq * 2)
        l1 = empty(hq * W * 4)
        wq, wk, wv, wg = (dev(x) for x in (qw, kw, vw, gw))
        hip.check(api.cs1_attention_ex(wq.at(0), wk.at(0), wv.at(0), rg, wg.at(0) if gated else None, one.at(0),
                                       l1.at(0), W, hq, hk, Dh, Dh ** -0.5, P, st.handle), "window")
        want = get_bf16(one, W * rq).reshape(W, hq, Dh)[P:]
        np.testing.assert_array_equal(got[r0:r0 + L], want)
        np.testing.assert_array_equal(got_lse[:, r0:r0 + L], get(l1, np.float32, hq * W).reshape(hq, W)[:, P:])


def test_prefix_varlen_arguments():
    api, st = hip.api(), stream()
    cu = np.array([0, 8], np.int32)
    buf = empty(1 << 20)
    # prefix length not a multiple of 64, missing prefix buffers
    assert api.cs1_attention_prefix_varlen(buf.at(0), buf.at(0), buf.at(0), 1024, buf.at(0), buf.at(0), 1024, 96, None,
                                           buf.at(0), None, cu.ctypes.data, 1, 16, 4, 256, 0.1, st.handle) != 0
    assert api.cs1_attention_prefix_varlen(buf.at(0), buf.at(0), buf.at(0), 1024, None, None, 1024, 64, None,
                                           buf.at(0), None, cu.ctypes.data, 1, 16, 4, 256, 0.1, st.handle) != 0
