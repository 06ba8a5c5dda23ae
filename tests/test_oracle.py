"""Pins the CPU oracle (no GPU needed).

The oracle is only trusted because these checks pass: the reference's own recorded
known answers (tests/golden/kernel_tests_log.json, transcribed from
benchmarks/gdn/artifacts/20261004/kernel-tests.log), closed forms, and independent
numpy restatements chosen so that a dropped term, a wrong sign or index, or a
transposed operand fails at least one of them.
"""
import json
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "kernel_tests_log.json")))


def sig3(x):
    return f"{x:.2e}"


# ----------------------------------------------------------- generator + GDN


def test_xorshift_matches_reference_recipe():
    # kernels.rs:26-36 by hand for the first values of seed 1, amp 1.
    x = (1 * 0x9E3779B97F4A7C15) & (2**64 - 1) | 1
    want = []
    for _ in range(8):
        x ^= (x << 13) & (2**64 - 1)
        x ^= x >> 7
        x ^= (x << 17) & (2**64 - 1)
        want.append(np.float32(np.float32(x >> 40) / np.float32(1 << 24) * np.float32(2.0) - np.float32(1.0)))
    got = O.bf16_to_f32(O.xorshift_bf16(8, 1, 1.0))
    np.testing.assert_array_equal(got, O.round_bf16(np.array(want, np.float32)))


@pytest.mark.parametrize("case", GOLDEN["gated_delta"], ids=lambda c: f"t{c['t']}h{c['h']}a{c['qk_amp']}")
def test_gdn_f64_and_emulator_reproduce_reference_log(case):
    t, h, hk = case["t"], case["h"], case["hk"]
    q, k, v, g, b = O.gdn_test_inputs(t, h, hk, case["decay_scale"], case["qk_amp"])
    want = O.gdn_recurrent_f64(q, k, v, g, b, t, h, hk)
    # the float64 reference's largest |value| depends only on the inputs: a known answer
    assert sig3(np.abs(want).max()) == sig3(case["max_abs_reference"])
    # the emulated CUDA kernel must show the recorded kernel's error (same rounding points)
    o, _ = O.gdn_chunk_emul(q, k, v, g, b, t, h, hk)
    err = np.abs(O.bf16_to_f32(o).astype(np.float64) - want).max()
    kat = case["kernel_max_diff"]
    if kat == 0:
        assert err == 0
    else:
        assert 0.85 * kat <= err <= 1.15 * kat, (err, kat)


def _normalize(x):
    x = x.astype(np.float64)
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + 1e-6)


def test_gdn_single_token_closed_form():
    # One token from a zero state: S = beta k^ v^T, o = scale (q^.k^) beta v.
    H, HK = 4, 2
    rng = np.random.default_rng(3)
    q = O.f32_to_bf16(rng.standard_normal((1, HK, 128)).astype(np.float32)).reshape(-1)
    k = O.f32_to_bf16(rng.standard_normal((1, HK, 128)).astype(np.float32)).reshape(-1)
    v = O.f32_to_bf16(rng.standard_normal((1, H, 128)).astype(np.float32)).reshape(-1)
    g = np.float32([-0.3, -0.1, -0.7, 0.0])
    beta = O.f32_to_bf16(np.float32([0.25, 0.5, 0.75, 1.0]))
    want = O.gdn_recurrent_f64(q, k, v, g, beta, 1, H, HK)
    qn = _normalize(O.bf16_to_f32(q).reshape(HK, 128))
    kn = _normalize(O.bf16_to_f32(k).reshape(HK, 128))
    vv = O.bf16_to_f32(v).reshape(H, 128).astype(np.float64)
    bb = O.bf16_to_f32(beta).astype(np.float64)
    for h in range(H):
        kh = h // 2
        closed = 128 ** -0.5 * (qn[kh] @ kn[kh]) * bb[h] * vv[h]
        np.testing.assert_allclose(want[0, h], closed, rtol=1e-12, atol=1e-14)
    o, s = O.gdn_chunk_emul(q, k, v, g, beta, 1, H, HK)
    np.testing.assert_allclose(O.bf16_to_f32(o).reshape(1, H, 128), want, atol=2e-2 * np.abs(want).max())
    for h in range(H):
        kh = h // 2
        np.testing.assert_allclose(s[h], bb[h] * np.outer(kn[kh], vv[h]), atol=2e-3)


def test_gdn_orthogonal_keys_reduce_to_linear_attention():
    # beta = 1, g = 0 and orthonormal keys: the delta rule never overwrites, so
    # o_t = scale * sum_{j<=t} (q^_t . k_j) v_j.
    T, H, HK = 100, 2, 1
    rng = np.random.default_rng(5)
    keys = np.zeros((T, 128), np.float32)
    keys[np.arange(T), np.arange(T)] = 1.0
    k = O.f32_to_bf16(keys).reshape(-1)
    q = O.f32_to_bf16(rng.standard_normal((T, 128)).astype(np.float32)).reshape(-1)
    v = O.f32_to_bf16(rng.standard_normal((T, H, 128)).astype(np.float32)).reshape(-1)
    g = np.zeros(T * H, np.float32)
    beta = O.f32_to_bf16(np.ones(T * H, np.float32))
    want = O.gdn_recurrent_f64(q, k, v, g, beta, T, H, HK)
    qn = _normalize(O.bf16_to_f32(q).reshape(T, 128))
    kn = _normalize(O.bf16_to_f32(k).reshape(T, 128))
    vv = O.bf16_to_f32(v).reshape(T, H, 128).astype(np.float64)
    scores = np.tril(qn @ kn.T) * 128 ** -0.5
    closed = np.einsum("tj,jhd->thd", scores, vv)
    np.testing.assert_allclose(want, closed, atol=1e-9)
    o, _ = O.gdn_chunk_emul(q, k, v, g, beta, T, H, HK)
    got = O.bf16_to_f32(o).astype(np.float64)
    assert np.abs(got - closed).max() <= 2e-2 * np.abs(closed).max()


def test_gdn_emulator_state_and_two_phase():
    T, H, HK = 200, 4, 2
    q, k, v, g, b = O.gdn_test_inputs(T, H, HK, 0.01, 1.0)
    rng = np.random.default_rng(9)
    s0 = (rng.standard_normal((H, 128, 128)) * 0.01).astype(np.float32)
    want, s_want = O.gdn_recurrent_f64(q, k, v, g, b, T, H, HK, s_in=s0, want_state=True)
    o, s = O.gdn_chunk_emul(q, k, v, g, b, T, H, HK, s_in=s0)
    assert np.abs(O.bf16_to_f32(o) - want).max() <= 2e-2 * np.abs(want).max()
    rel = np.linalg.norm(s - s_want) / np.linalg.norm(s_want)
    assert rel < 1e-2, rel
    # two phases split at a chunk boundary repeat the one-shot arithmetic bit for bit
    p = 128
    o1, s1 = O.gdn_chunk_emul(q[: p * HK * 128], k[: p * HK * 128], v[: p * H * 128], g[: p * H], b[: p * H], p, H,
                              HK, s_in=s0)
    o2, s2 = O.gdn_chunk_emul(q[p * HK * 128:], k[p * HK * 128:], v[p * H * 128:], g[p * H:], b[p * H:], T - p, H,
                              HK, s_in=s1)
    np.testing.assert_array_equal(np.concatenate([o1, o2]), o)
    np.testing.assert_array_equal(s2, s)
    # T = 0 passes the state through, or zeroes it without an input state
    e = np.zeros(0, np.uint16)
    _, sp = O.gdn_chunk_emul(e, e, e, np.zeros(0, np.float32), e, 0, H, HK, s_in=s0)
    np.testing.assert_array_equal(sp, s0)
    _, sz = O.gdn_chunk_emul(e, e, e, np.zeros(0, np.float32), e, 0, H, HK)
    assert not sz.any()


def test_blocked_triangular_inverse():
    rng = np.random.default_rng(1)
    a = np.tril(rng.uniform(-0.3, 0.3, (64, 64)), -1).astype(np.float32)
    t = O.tri_inverse_blocked(a)
    eye = np.eye(64)
    np.testing.assert_allclose((eye + a.astype(np.float64)) @ t, eye, atol=2e-5)
    np.testing.assert_allclose(t, np.linalg.inv(eye + a.astype(np.float64)), atol=2e-5)
    assert not np.triu(t, 1).any()


# ----------------------------------------------------------------- attention


@pytest.mark.parametrize("case", GOLDEN["attention"], ids=lambda c: f"t{c['t']}")
def test_attention_emulator_reproduces_reference_log(case):
    t, amp = case["t"], case["amp"]
    hq, hk, dh, ldv = 16, 4, 256, 10240
    v_at = (hq * 2 + hk) * dh
    q = O.xorshift_bf16(t * hq * dh, 1, amp)
    k = O.xorshift_bf16(t * hk * dh, 2, amp)
    qkv = O.xorshift_bf16(t * ldv, 3, 1.0)
    v = np.concatenate([qkv[v_at:], np.zeros(v_at, np.uint16)])
    rows = sorted(set(range(0, t, -(-t // 64))) | {t - 1})
    want = O.attention_f64(q, k, v, ldv, t, hq, hk, dh, 0.0625, rows=rows)
    got = O.bf16_to_f32(O.attention_emul(q, k, v, ldv, None, t, hq, hk, dh, 0.0625)).astype(np.float64)
    worst = 0.0
    for i in rows:
        for h in range(hq):
            w = want[i, h]
            worst = max(worst, np.abs(got[i, h] - w).max() / max(1e-3, np.abs(w).max()))
    assert sig3(worst) == sig3(case["kernel_max_rel_diff"])


def _np_attention(q, k, v, T, Hq, Hk, Dh, scale):
    qf = O.bf16_to_f32(q).reshape(T, Hq, Dh).astype(np.float64)
    kf = O.bf16_to_f32(k).reshape(T, Hk, Dh).astype(np.float64)
    vf = O.bf16_to_f32(v).reshape(T, Hk, Dh).astype(np.float64)
    out = np.empty((T, Hq, Dh))
    lse = np.empty((Hq, T))
    for h in range(Hq):
        g = h // (Hq // Hk)
        s = qf[:, h] @ kf[:, g].T * scale
        s[np.triu_indices(T, 1)] = -np.inf
        m = s.max(1, keepdims=True)
        p = np.exp(s - m)
        out[:, h] = p @ vf[:, g] / p.sum(1, keepdims=True)
        lse[h] = m[:, 0] + np.log(p.sum(1))
    return out, lse


def test_attention_f64_against_numpy_and_closed_forms():
    T, Hq, Hk, Dh = 70, 4, 2, 128
    rng = np.random.default_rng(2)
    q = O.f32_to_bf16(rng.standard_normal(T * Hq * Dh).astype(np.float32))
    k = O.f32_to_bf16(rng.standard_normal(T * Hk * Dh).astype(np.float32))
    v = O.f32_to_bf16(rng.standard_normal(T * Hk * Dh).astype(np.float32))
    out, lse = O.attention_f64(q, k, v, Hk * Dh, T, Hq, Hk, Dh, Dh ** -0.5, want_lse=True)
    want, wlse = _np_attention(q, k, v, T, Hq, Hk, Dh, Dh ** -0.5)
    np.testing.assert_allclose(out, want, atol=1e-10)
    np.testing.assert_allclose(lse, wlse, atol=1e-10)
    # uniform scores (q = 0): the running mean of V, and lse = log(i + 1)
    z = np.zeros_like(q)
    out0, lse0 = O.attention_f64(z, k, v, Hk * Dh, T, Hq, Hk, Dh, 0.1, want_lse=True)
    vf = O.bf16_to_f32(v).reshape(T, Hk, Dh).astype(np.float64)
    mean = np.cumsum(vf, 0) / np.arange(1, T + 1)[:, None, None]
    np.testing.assert_allclose(out0[:, 0], mean[:, 0], atol=1e-12)
    np.testing.assert_allclose(out0[:, 3], mean[:, 1], atol=1e-12)
    np.testing.assert_allclose(lse0[2], np.log(np.arange(1, T + 1)), atol=1e-12)
    # the emulator (float32, bf16 P) agrees within the reference's relative bound, and its lse
    eo, else_ = O.attention_emul(q, k, v, Hk * Dh, None, T, Hq, Hk, Dh, Dh ** -0.5, want_lse=True)
    assert np.abs(O.bf16_to_f32(eo) - want).max() <= 1.6e-2 * np.abs(want).max()
    np.testing.assert_allclose(else_, wlse, atol=1e-4)


def test_attention_emulator_gate_and_window():
    T, Hq, Hk, Dh = 150, 4, 1, 128
    rng = np.random.default_rng(4)
    q = O.f32_to_bf16(rng.standard_normal(T * Hq * Dh).astype(np.float32))
    k = O.f32_to_bf16(rng.standard_normal(T * Hk * Dh).astype(np.float32))
    v = O.f32_to_bf16(rng.standard_normal(T * Hk * Dh).astype(np.float32))
    gate = O.f32_to_bf16((rng.standard_normal(T * Hq * Dh) * 4).astype(np.float32))
    plain = O.attention_emul(q, k, v, Hk * Dh, None, T, Hq, Hk, Dh, 0.08).reshape(-1)
    fused = O.attention_emul(q, k, v, Hk * Dh, gate, T, Hq, Hk, Dh, 0.08).reshape(-1)
    np.testing.assert_array_equal(fused, O.sigmoid_gate(plain, gate))
    win = O.attention_emul(q, k, v, Hk * Dh, gate, T, Hq, Hk, Dh, 0.08, q_base=64).reshape(T, -1)
    np.testing.assert_array_equal(win[64:], fused.reshape(T, -1)[64:])
    # the row-restricted emulation equals the full one on those rows, and leaves the rest zero
    rows = [0, 5, 64, 149]
    out, lse = O.attention_emul(q, k, v, Hk * Dh, gate, T, Hq, Hk, Dh, 0.08, want_lse=True, rows=rows)
    full, flse = O.attention_emul(q, k, v, Hk * Dh, gate, T, Hq, Hk, Dh, 0.08, want_lse=True)
    np.testing.assert_array_equal(out[rows], full[rows])
    np.testing.assert_array_equal(lse[:, rows], flse[:, rows])
    others = np.setdiff1d(np.arange(T), rows)
    assert not out[others].any() and not lse[:, others].any()


# --------------------------------------------------------------- elementwise


def _fmaf(a, b, c):
    # exact in float64 for bf16 a, b and float32 c of this test's ranges, then one rounding
    return np.float32(np.float64(a) * np.float64(b) + np.float64(c))


def _bf16_ulp_close(a, b, ulps=1):
    a = a.astype(np.int32)
    b = b.astype(np.int32)
    return np.abs(a - b).max() <= ulps


def test_gdn_conv_against_numpy_restatement_and_history():
    T, kd, vd = 20, 64, 96
    ch = 2 * kd + vd
    ld = ch + 8
    rng = np.random.default_rng(6)
    x = O.f32_to_bf16(rng.standard_normal(T * ld).astype(np.float32))
    w = O.f32_to_bf16((rng.standard_normal(ch * 4) * 0.5).astype(np.float32))
    q, k, v = O.gdn_conv(x, ld, w, T, kd, vd)
    xf = O.bf16_to_f32(x).reshape(T, ld)
    wf = O.bf16_to_f32(w).reshape(ch, 4)
    acc = np.zeros((T, ch), np.float32)
    for j in range(4):
        for t in range(T):
            s = t - 3 + j
            if s >= 0:
                acc[t] = [_fmaf(wf[c, j], xf[s, c], acc[t, c]) for c in range(ch)]
    r = O.round_bf16(acc).astype(np.float64)
    y = O.f32_to_bf16((r / (1 + np.exp(-r))).astype(np.float32))
    assert _bf16_ulp_close(np.concatenate([q.reshape(T, kd), k.reshape(T, kd), v.reshape(T, vd)], 1), y)
    # continuation from three cached rows reproduces the full pass (kernels.rs:771-850)
    q2, k2, v2 = O.gdn_conv(x[(10 - 3) * ld:], ld, w, T - 7, kd, vd)
    np.testing.assert_array_equal(q2.reshape(-1, kd)[3:], q.reshape(T, kd)[10:])
    np.testing.assert_array_equal(v2.reshape(-1, vd)[3:], v.reshape(T, vd)[10:])


def test_gdn_gates_closed_form():
    T, H, ld = 33, 8, 24
    rng = np.random.default_rng(7)
    b = O.f32_to_bf16(rng.standard_normal(T * ld).astype(np.float32) * 3)
    a = O.f32_to_bf16(rng.standard_normal(T * ld).astype(np.float32) * 10)
    A_log = O.f32_to_bf16(np.log(rng.uniform(0.1, 16, H)).astype(np.float32))
    dt = O.f32_to_bf16(rng.standard_normal(H).astype(np.float32))
    beta, g = O.gdn_gates(b, a, ld, A_log, dt, T, H)
    bf = O.bf16_to_f32(b).reshape(T, ld)[:, :H].astype(np.float64)
    af = O.bf16_to_f32(a).reshape(T, ld)[:, :H].astype(np.float64)
    x = af + O.bf16_to_f32(dt).astype(np.float64)
    sp = np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20))))
    gw = -np.exp(O.bf16_to_f32(A_log).astype(np.float64)) * sp
    np.testing.assert_allclose(g.reshape(T, H), gw, rtol=1e-6, atol=1e-6)
    assert _bf16_ulp_close(beta.reshape(T, H), O.f32_to_bf16((1 / (1 + np.exp(-bf))).astype(np.float32)))


def test_norms_against_numpy():
    rng = np.random.default_rng(8)
    T, H, D = 9, 4, 128
    x = O.f32_to_bf16(rng.standard_normal(T * H * D).astype(np.float32))
    ldz = H * D + 64
    z = O.f32_to_bf16(rng.standard_normal(T * ldz).astype(np.float32))
    w = O.f32_to_bf16(rng.uniform(0.5, 1.5, D).astype(np.float32))
    out = O.gated_rms_norm(x, z, ldz, w, T, H, D, 1e-6)
    xf = O.bf16_to_f32(x).reshape(T * H, D).astype(np.float64)
    zf = O.bf16_to_f32(z).reshape(T, ldz)[:, : H * D].reshape(T * H, D).astype(np.float64)
    normed = O.round_bf16((xf / np.sqrt((xf ** 2).mean(1, keepdims=True) + 1e-6)).astype(np.float32))
    scaled = O.round_bf16(O.bf16_to_f32(w) * normed).astype(np.float64)
    want = O.f32_to_bf16((scaled * zf / (1 + np.exp(-zf))).astype(np.float32))
    assert _bf16_ulp_close(out.reshape(T * H, D), want)
    # zero-centred RMSNorm x (1 + w), and the residual add
    rows, Dm = 5, 2560
    xm = O.f32_to_bf16(rng.standard_normal(rows * Dm).astype(np.float32))
    dm = O.f32_to_bf16(rng.standard_normal(rows * Dm).astype(np.float32))
    wm = O.f32_to_bf16((rng.standard_normal(Dm) * 0.1).astype(np.float32))
    xf = O.bf16_to_f32(xm).reshape(rows, Dm).astype(np.float64)
    want = O.f32_to_bf16(xf / np.sqrt((xf ** 2).mean(1, keepdims=True) + 1e-6) * (1 + O.bf16_to_f32(wm)))
    assert _bf16_ulp_close(O.rms_norm(xm, wm, rows, Dm).reshape(rows, Dm), want)
    res, out = O.add_rms_norm(xm, dm, wm, rows, Dm)
    np.testing.assert_array_equal(res, O.f32_to_bf16(O.bf16_to_f32(xm) + O.bf16_to_f32(dm)))
    rf = O.bf16_to_f32(res).reshape(rows, Dm).astype(np.float64)
    want = O.f32_to_bf16(rf / np.sqrt((rf ** 2).mean(1, keepdims=True) + 1e-6) * (1 + O.bf16_to_f32(wm)))
    assert _bf16_ulp_close(out.reshape(rows, Dm), want)


def test_attn_prep_and_rotary_closed_forms():
    T, Hq, Hk, Dh, half = 6, 2, 1, 256, 32
    ld = Hq * 2 * Dh + 2 * Hk * Dh
    rng = np.random.default_rng(10)
    row = O.f32_to_bf16(rng.standard_normal(T * ld).astype(np.float32))
    qw = O.f32_to_bf16((rng.standard_normal(Dh) * 0.1).astype(np.float32))
    kw = O.f32_to_bf16((rng.standard_normal(Dh) * 0.1).astype(np.float32))
    pos = np.arange(T, dtype=np.int64) * 37
    cs, sn = O.rotary_tables(pos, half, 1e7)
    inv = 1.0 / (1e7 ** (np.arange(half) * 2 / (2 * half)))
    np.testing.assert_allclose(O.bf16_to_f32(cs).reshape(T, half), np.cos(np.outer(pos, inv)), atol=4e-3)
    np.testing.assert_allclose(O.bf16_to_f32(sn).reshape(T, half), np.sin(np.outer(pos, inv)), atol=4e-3)
    kr = row[Hq * 2 * Dh:]
    kr = np.concatenate([kr, np.zeros(Hq * 2 * Dh, np.uint16)])
    q, gate, k = O.attn_prep(row, kr, ld, qw, kw, cs, sn, T, Hq, Hk, Dh, half)
    rf = O.bf16_to_f32(row).reshape(T, ld).astype(np.float64)
    # the gate half of each q row is copied unchanged
    np.testing.assert_array_equal(gate.reshape(T, Hq, Dh), row.reshape(T, ld)[:, : Hq * 2 * Dh].reshape(T, Hq, 2, Dh)[:, :, 1])
    qin = rf[:, : Hq * 2 * Dh].reshape(T, Hq, 2, Dh)[:, :, 0]
    xn = qin / np.sqrt((qin ** 2).mean(-1, keepdims=True) + 1e-6) * (1 + O.bf16_to_f32(qw))
    c = np.cos(np.outer(pos, inv))[:, None, :]
    s = np.sin(np.outer(pos, inv))[:, None, :]
    rot = xn.copy()
    rot[..., :half] = xn[..., :half] * c - xn[..., half:2 * half] * s
    rot[..., half:2 * half] = xn[..., half:2 * half] * c + xn[..., :half] * s
    got = O.bf16_to_f32(q).reshape(T, Hq, Dh)
    np.testing.assert_allclose(got, rot, atol=0.05 * np.abs(rot).max())
    # dims past 2*half are the normalised values only
    np.testing.assert_array_equal(got[..., 2 * half:], O.round_bf16(O.round_bf16(xn[..., 2 * half:].astype(np.float32))))


def test_silu_mul_and_sigmoid_gate():
    rng = np.random.default_rng(11)
    T, I = 7, 40
    gu = O.f32_to_bf16(rng.standard_normal(T * 2 * I).astype(np.float32) * 4)
    out = O.silu_mul(gu, 2 * I, T, I)
    f = O.bf16_to_f32(gu).reshape(T, 2 * I).astype(np.float64)
    silu = O.round_bf16((f[:, :I] / (1 + np.exp(-f[:, :I]))).astype(np.float32)).astype(np.float64)
    assert _bf16_ulp_close(out.reshape(T, I), O.f32_to_bf16((silu * f[:, I:]).astype(np.float32)))
    x = O.f32_to_bf16(rng.standard_normal(100).astype(np.float32))
    gt = O.f32_to_bf16(np.concatenate([[-40, 40, 0], rng.standard_normal(97) * 5]).astype(np.float32))
    got = O.sigmoid_gate(x, gt)
    sg = O.round_bf16((1 / (1 + np.exp(-O.bf16_to_f32(gt).astype(np.float64)))).astype(np.float32))
    assert _bf16_ulp_close(got, O.f32_to_bf16(O.bf16_to_f32(x) * sg))
