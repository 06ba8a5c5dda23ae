"""Prefill throughput of the MI355X Qwen3.5 hot path, one JSON line on stdout.

Metric: "prefill tokens/s per layer type + ms per 4k-token hybrid
decision prefill".  A step is one prefill pass of one layer over one synthetic batch
with the inputs already resident in HBM:

  * headline (`value`): the gated GQA flash-attention layer of config 1
    (T = 2048, 16 q / 4 kv heads, Dh = 128, sigmoid gate, float32 LSE), tokens/s;
  * `layers`: the same measurement for the GDN layer of config 2 (causal conv1d + SiLU,
    then the chunked gated delta rule, T = 8192, 16 qk / 32 v heads, S0 ~ N(0, 0.01)) and
    of config 0 (T = 512, 16 / 16 heads), each with its kernels' roofline figures.

Timing: W untimed warm-up steps, then K steps bracketed by a stream sync on both sides;
per-kernel averages come from HIP events recorded on the stream the kernels run on
(hipEventElapsedTime over the K launches of the timed region).  Everything runs through
the library's C ABI; no torch in this process.

The CPU baseline is the repository's C restatement of the reference kernel (oracle/,
OpenMP) timed on this host on a bounded sample of the same workload.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "system1-omni_amd"))

from qwen3_5_native import hip  # noqa: E402

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E


class Events:
    """hipEvent_t pairs from the HIP runtime the library itself links."""

    def __init__(self):
        self.rt = ctypes.CDLL("libamdhip64.so.7")
        self.rt.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.rt.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.rt.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.rt.hipEventSynchronize.argtypes = [ctypes.c_void_p]

    def new(self):
        e = ctypes.c_void_p()
        hip.check(self.rt.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        return e.value

    def record(self, ev, stream):
        hip.check(self.rt.hipEventRecord(ev, stream.handle), "hipEventRecord")

    def ms(self, a, b):
        hip.check(self.rt.hipEventSynchronize(b), "hipEventSynchronize")
        out = ctypes.c_float()
        hip.check(self.rt.hipEventElapsedTime(ctypes.byref(out), a, b), "hipEventElapsedTime")
        return out.value


def bf16(rng, n, std=1.0):
    x = (rng.standard_normal(n) * std).astype(np.float32)
    u = x.view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def unit_rows_bf16(rng, rows, d):
    x = rng.standard_normal((rows, d))
    x /= np.sqrt((x * x).sum(-1, keepdims=True))
    u = x.astype(np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16).reshape(-1)


# The GPU raises its clock over the first tens of milliseconds of sustained load and lowers it
# again when idle: one T=8192 attention launch takes 356 us right after an idle second and
# settles at 293 us after about 50 ms of back-to-back launches (cfg1: 43.4 -> 38.2 us after
# about 30 ms). Every measured region is preceded by SETTLE_S seconds of the same launches
# (untimed, part of the warmup), so the figures are for the sustained clock.
SETTLE_S = 0.3


def settle(stream, launches, seconds=SETTLE_S):
    """Back-to-back launches for at least `seconds`, in batches that double until one takes
    20 ms, so the host synchronisations leave no idle gap long enough to drop the clock."""
    t0 = time.perf_counter()
    n = 1
    while True:
        tb = time.perf_counter()
        for _ in range(n):
            for _, fn in launches:
                fn()
        stream.sync()
        now = time.perf_counter()
        if now - t0 >= seconds:
            return
        if now - tb < 0.02:
            n *= 2


def timed(stream, ev, steps, warmup, launches):
    """Run `launches` (list of (name, fn)) per step.

    Returns the wall ms per step (host clock, stream synchronised on both sides of the K
    steps) and each launch's average GPU ms. The per-launch figure is one HIP event pair on
    the kernels' own stream around K back-to-back launches of that entry point alone (for a
    one-launch step this is the step region itself), so no event marker sits between two
    dispatches being timed. The warmup starts with `settle`."""
    settle(stream, launches)
    for _ in range(warmup):
        for _, fn in launches:
            fn()
    stream.sync()
    e0, e1 = ev.new(), ev.new()
    t0 = time.perf_counter()
    ev.record(e0, stream)
    for _ in range(steps):
        for _, fn in launches:
            fn()
    ev.record(e1, stream)
    stream.sync()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    if len(launches) == 1:
        return wall_ms, {launches[0][0]: ev.ms(e0, e1) / steps}
    per = {}
    for name, fn in launches:
        a, b = ev.new(), ev.new()
        ev.record(a, stream)
        for _ in range(steps):
            fn()
        ev.record(b, stream)
        per[name] = ev.ms(a, b) / steps
    return wall_ms, per


def bench_attention(api, st, ev, steps, warmup, T=2048, Hq=16, Hk=4, Dh=128, label="cfg1"):
    rng = np.random.default_rng(1)
    q, k, v, gate = (hip.to_device(bf16(rng, T * h * Dh), st) for h in (Hq, Hk, Hk, Hq))
    out, lse = hip.DeviceBuffer(T * Hq * Dh * 2), hip.DeviceBuffer(Hq * T * 4)

    def launch():
        hip.check(api.cs1_attention_ex(q.at(0), k.at(0), v.at(0), Hk * Dh, gate.at(0), out.at(0), lse.at(0), T, Hq, Hk,
                                       Dh, Dh ** -0.5, 0, st.handle), "attention")

    wall, per = timed(st, ev, steps, warmup, [("flash_attention", launch)])
    flops = 2.0 * T * T * Dh * Hq  # causal: half of 4 T^2 Dh Hq
    kern = per["flash_attention"]
    achieved = flops / (kern * 1e-3) / 1e12
    return {
        "workload": f"{label} gated GQA flash-attention prefill T={T} Hq={Hq} Hk={Hk} Dh={Dh} + fp32 LSE",
        "tokens_per_s": T / (wall * 1e-3), "ms_per_step": wall, "kernel_ms": per,
        "roofline": {"kernel": "flash32_kernel<gated>" if Dh == 128 else "flash256_kernel<gated>", "bound": "mfma",
                     "achieved": achieved,
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": achieved / PEAK_BF16_TFLOPS,
                     "algorithmic_flop": flops},
    }


def gdn_layer(api, st, T, H, HK, with_conv, s0_std, seed):
    D = 128
    rng = np.random.default_rng(seed)
    key_dim, value_dim = HK * D, H * D
    bufs = {}
    if with_conv:
        ch = 2 * key_dim + value_dim
        bufs["qkv"] = hip.to_device(bf16(rng, T * ch), st)
        bufs["w"] = hip.to_device(bf16(rng, ch * 4, 0.02), st)
        for n, w in (("q", key_dim), ("k", key_dim), ("v", value_dim)):
            bufs[n] = hip.DeviceBuffer(T * w * 2)
    else:
        bufs["q"] = hip.to_device(unit_rows_bf16(rng, T * HK, D), st)
        bufs["k"] = hip.to_device(unit_rows_bf16(rng, T * HK, D), st)
        bufs["v"] = hip.to_device(bf16(rng, T * H * D), st)
    beta = (1 / (1 + np.exp(-rng.standard_normal(T * H)))).astype(np.float32)
    bufs["beta"] = hip.to_device(((beta.view(np.uint32) + 0x7FFF + ((beta.view(np.uint32) >> 16) & 1)) >> 16)
                                 .astype(np.uint16), st)
    bufs["g"] = hip.to_device((-np.log1p(np.exp(rng.standard_normal(T * H))) * 0.1).astype(np.float32), st)
    bufs["s_in"] = hip.to_device((rng.standard_normal(H * D * D) * s0_std).astype(np.float32), st) if s0_std else None
    bufs["s_out"] = hip.DeviceBuffer(H * D * D * 4)
    bufs["o"] = hip.DeviceBuffer(T * H * D * 2)
    bufs["ws"] = hip.DeviceBuffer(api.cs1_gdn_workspace_floats(T, H) * 4)
    launches = []
    if with_conv:
        launches.append(("gdn_conv", lambda: hip.check(api.cs1_gdn_conv(
            bufs["qkv"].at(0), 2 * key_dim + value_dim, bufs["w"].at(0), bufs["q"].at(0), bufs["k"].at(0),
            bufs["v"].at(0), T, key_dim, value_dim, st.handle), "conv")))
    launches.append(("gdn_prefill", lambda: hip.check(api.cs1_gdn_prefill_x(
        bufs["q"].at(0), bufs["k"].at(0), bufs["v"].at(0), bufs["g"].at(0), bufs["beta"].at(0), bufs["o"].at(0),
        bufs["ws"].at(0), T, H, HK, D ** -0.5, bufs["s_in"].at(0) if bufs["s_in"] else None, bufs["s_out"].at(0),
        st.handle), "gdn")))
    return bufs, launches


def bench_gdn(api, st, ev, steps, warmup, T, H, HK, with_conv, s0_std, seed, label):
    D = 128
    bufs, launches = gdn_layer(api, st, T, H, HK, with_conv, s0_std, seed)
    wall, per = timed(st, ev, steps, warmup, launches)
    flops = 180224.0 * T * H  # dense-tile count per token per v-head: 10 C D + 6 D^2
    flops_tri = 139264.0 * T * H  # the same without the upper triangles of A, P and the T products
    io = 2 * T * HK * D * 2 + 2 * T * H * D * 2 + T * H * 6 + (2 if s0_std else 1) * H * D * D * 4
    g_ms = per["gdn_prefill"]
    res = {
        "workload": label, "tokens_per_s": T / (wall * 1e-3), "ms_per_step": wall, "kernel_ms": per,
        "gdn": {"bound": "mfma", "achieved": flops / (g_ms * 1e-3) / 1e12, "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": flops / (g_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                "algorithmic_flop": flops, "algorithmic_flop_triangular": flops_tri,
                "achieved_triangular": flops_tri / (g_ms * 1e-3) / 1e12, "algorithmic_io_bytes": io,
                "io_GBs": io / (g_ms * 1e-3) / 1e9},
    }
    if with_conv:
        cbytes = 2 * T * (2 * HK * D + H * D) * 2
        c_ms = per["gdn_conv"]
        res["conv"] = {"bound": "hbm", "achieved": cbytes / (c_ms * 1e-3) / 1e9, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                       "frac": cbytes / (c_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, "algorithmic_bytes": cbytes}
    return res


# The reference's only published timings for this path: its complete cs1_gdn_prefill call on
# one H200 (benchmarks/gdn/README.md:57-61, the "candidate" wall ms per call, passes 1 / 2).
H200_GDN_WALL_MS = {107: (0.050914, 0.050957), 936: (0.214176, 0.214178), 3399: (0.696768, 0.697262)}


def bench_gdn_reference_shapes(api, st, ev):
    """The reference harness's GDN benchmark (benchmarks/gdn/artifacts/20261003/kernel/harness/
    compare.py:76-135) on this GPU: T = 107, 936, 3399 tokens, 16 qk / 48 v heads, seed
    20261003, k ~ U(-1, 1), q = 0.8 k + 0.2 U, v ~ U, g = (U - 1) 0.01, beta = 0.5 U + 0.5 (numpy's
    generator, so the same distributions, not the same values). Its protocol: ten warm-up calls,
    then two passes of 100 complete cs1_gdn_prefill calls each; wall ms per call includes the
    host submission, the event span is the device time of the 100 calls."""
    H, HK, D = 48, 16, 128
    rng = np.random.default_rng(20261003)
    res = []
    for T in (107, 936, 3399):
        u = lambda *shape: rng.random(shape, dtype=np.float32) * 2 - 1  # noqa: E731
        k = O_bf16(u(T, HK, D))
        q = O_bf16(0.8 * bf16_f32(k) + 0.2 * bf16_f32(O_bf16(u(T, HK, D))))
        v = O_bf16(u(T, H, D))
        g = ((bf16_f32(O_bf16(u(T, H))) - 1) * 0.01).astype(np.float32)
        beta = O_bf16(bf16_f32(O_bf16(u(T, H))) * 0.5 + 0.5)
        dq, dk, dv, dg, db = (hip.to_device(np.ascontiguousarray(a).reshape(-1), st) for a in (q, k, v, g, beta))
        o = hip.DeviceBuffer(T * H * D * 2)
        ws = hip.DeviceBuffer(api.cs1_gdn_workspace_floats(T, H) * 4)

        def call():
            hip.check(api.cs1_gdn_prefill(dq.at(0), dk.at(0), dv.at(0), dg.at(0), db.at(0), o.at(0), ws.at(0), T, H,
                                          HK, D ** -0.5, st.handle), "gdn (reference shapes)")

        settle(st, [("gdn", call)])
        for _ in range(10):
            call()
        st.sync()
        passes = []
        for _ in range(2):
            e0, e1 = ev.new(), ev.new()
            t0 = time.perf_counter()
            ev.record(e0, st)
            for _ in range(100):
                call()
            ev.record(e1, st)
            span = ev.ms(e0, e1) / 100
            passes.append({"wall_ms_per_call": (time.perf_counter() - t0) * 1e3 / 100, "device_span_ms_per_call": span})
        wall = sum(p_["wall_ms_per_call"] for p_ in passes) / 2
        h200 = sum(H200_GDN_WALL_MS[T]) / 2
        res.append({"tokens": T, "passes": passes, "h200_published_wall_ms": H200_GDN_WALL_MS[T],
                    "speedup_vs_h200_wall": h200 / wall,
                    "achieved_TFLOPs_device_span": 180224.0 * T * H / (passes[1]["device_span_ms_per_call"] * 1e-3) / 1e12})
    return res


def O_bf16(x):
    """float32 -> bf16 bits (round to nearest even)."""
    u_ = np.ascontiguousarray(x, np.float32).view(np.uint32)
    return ((u_ + 0x7FFF + ((u_ >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def bench_hbm_ops(api, st, ev, steps, warmup):
    """The HBM-bound operations around the two layers, each against the HBM peak with its
    algorithmic bytes (read once + written once): the GDN gates and gated RMSNorm at config 2
    (T=8192, 32 v heads, D=128) and the attention q/k prep at the config-3 attention shape
    (T=4096, 16 q / 4 kv heads, Dh=256, rotary half 32)."""
    rng = np.random.default_rng(3)
    res = {}

    def entry(name, workload, nbytes, fn):
        wall, per = timed(st, ev, steps, warmup, [(name, fn)])
        gbs = nbytes / (per[name] * 1e-3) / 1e9
        res[name] = {"workload": workload, "kernel_ms": per[name], "bound": "hbm", "achieved": gbs,
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS, "algorithmic_bytes": nbytes}

    T, H, D = 8192, 32, 128
    ab = hip.to_device(bf16(rng, 2 * T * 2 * H), st)  # rows [b (H) | a (H)], ld = 2 H
    alog = hip.to_device(bf16(rng, H, 0.5), st)
    dtb = hip.to_device(bf16(rng, H), st)
    beta, g = hip.DeviceBuffer(T * H * 2), hip.DeviceBuffer(T * H * 4)
    entry("gdn_gates", "cfg2 gates T=8192 H=32", T * H * 10,
          lambda: hip.check(api.cs1_gdn_gates(ab.at(0), ab.at(H * 2), 2 * H, alog.at(0), dtb.at(0), beta.at(0),
                                              g.at(0), T, H, st.handle), "gates"))
    x = hip.to_device(bf16(rng, T * H * D), st)
    z = hip.to_device(bf16(rng, T * H * D), st)
    w = hip.to_device(bf16(rng, D), st)
    out = hip.DeviceBuffer(T * H * D * 2)
    entry("gated_rms_norm", "cfg2 gated RMSNorm T=8192 H=32 D=128", 3 * T * H * D * 2,
          lambda: hip.check(api.cs1_gated_rms_norm(x.at(0), z.at(0), H * D, w.at(0), out.at(0), T, H, D, 1e-6,
                                                   st.handle), "gated norm"))
    T, Hq, Hk, Dh, half = 4096, 16, 4, 256, 32
    ld = Hq * 2 * Dh + 2 * Hk * Dh
    row = hip.to_device(bf16(rng, T * ld), st)
    qw, kw = hip.to_device(bf16(rng, Dh, 0.1), st), hip.to_device(bf16(rng, Dh, 0.1), st)
    cs, sn = hip.to_device(bf16(rng, T * half), st), hip.to_device(bf16(rng, T * half), st)
    q, gate, k = hip.DeviceBuffer(T * Hq * Dh * 2), hip.DeviceBuffer(T * Hq * Dh * 2), hip.DeviceBuffer(T * Hk * Dh * 2)
    nbytes = T * (Hq * 2 * Dh + Hk * Dh) * 2 + 2 * T * half * 2 + T * (2 * Hq + Hk) * Dh * 2
    entry("attn_prep", "cfg3 attention prep T=4096 Hq=16 Hk=4 Dh=256 half=32", nbytes,
          lambda: hip.check(api.cs1_attn_prep(row.at(0), row.at(Hq * 2 * Dh * 2), ld, qw.at(0), kw.at(0), cs.at(0),
                                              sn.at(0), q.at(0), gate.at(0), k.at(0), T, Hq, Hk, Dh, half, 1e-6,
                                              st.handle), "attn prep"))
    # the decoder glue of config 3 (T=4096, hidden 2560, SwiGLU 9728): residual norms, SwiGLU,
    # embedding gather (norm.cu:11-73, elementwise.cu:11-16, 75-87)
    T, Dm, I = 4096, 2560, 9728
    xr = hip.to_device(bf16(rng, T * Dm), st)
    dl = hip.to_device(bf16(rng, T * Dm), st)
    wn = hip.to_device(bf16(rng, Dm, 0.1), st)
    on = hip.DeviceBuffer(T * Dm * 2)
    entry("rms_norm", "cfg3 RMSNorm T=4096 D=2560", 2 * T * Dm * 2,
          lambda: hip.check(api.cs1_rms_norm(xr.at(0), wn.at(0), on.at(0), T, Dm, 1e-6, st.handle), "rms norm"))
    # the residual is updated in place: every launch reads and writes it (values drift, bytes do not)
    entry("add_rms_norm", "cfg3 residual add + RMSNorm T=4096 D=2560", 4 * T * Dm * 2,
          lambda: hip.check(api.cs1_add_rms_norm(xr.at(0), dl.at(0), wn.at(0), on.at(0), T, Dm, 1e-6, st.handle),
                            "add rms norm"))
    gu = hip.to_device(bf16(rng, T * 2 * I), st)
    act = hip.DeviceBuffer(T * I * 2)
    entry("silu_mul", "cfg3 SwiGLU T=4096 I=9728", 3 * T * I * 2,
          lambda: hip.check(api.cs1_silu_mul(gu.at(0), 2 * I, act.at(0), T, I, st.handle), "silu mul"))
    V = 151936
    table = hip.to_device(bf16(rng, V * Dm, 0.02), st)
    ids = hip.to_device(rng.integers(0, V, T).astype(np.int32), st)
    entry("embed", "cfg3 embedding gather T=4096 D=2560 vocab 151936", 2 * T * Dm * 2 + T * 4,
          lambda: hip.check(api.cs1_embed(ids.at(0), table.at(0), on.at(0), T, Dm, st.handle), "embed"))
    return res


def bench_decision_prefill(steps, warmup, T=4096, tune=False, graph=True):
    """Config 3: one 4096-token decision prefill of the random-init 4B-class hybrid
    decoder (32 layers, 3:1 GDN:attention, hidden 2560, SwiGLU 9728, 16/4 x 256 attention,
    GDN 16 qk / 32 v heads) through the native runner, then the 8-label head on the last
    hidden state. A step is one complete q35m_decide call: id upload, embedding, the layer
    stack (a captured hipGraph after the first call at this length), the last-row download
    and the host head; wall-clock ms."""
    from qwen3_5_native import model as QM

    cfg = QM.CFG3_4B
    m = QM.Model(cfg, seed=0, max_tokens=T)
    try:
        m.set_graph(graph)
        m.set_gemm_tuning(tune)
        rng = np.random.default_rng(4)
        ids = rng.integers(0, cfg.vocab, T).astype(np.int32)
        labels = (np.arange(8) * 997 + 151).astype(np.int32)
        for _ in range(max(warmup, 2)):
            logits = m.decide(ids, labels)
        tw = time.perf_counter()
        while time.perf_counter() - tw < SETTLE_S:
            logits = m.decide(ids, labels)
        t0 = time.perf_counter()
        for _ in range(steps):
            logits = m.decide(ids, labels)
        ms = (time.perf_counter() - t0) * 1e3 / steps
    finally:
        m.close()
    kd, vd = cfg.lin_k_heads * cfg.lin_k_dim, cfg.lin_v_heads * cfg.lin_v_dim
    n_attn = sum(cfg.is_full(i) for i in range(cfg.layers))
    n_gdn = cfg.layers - n_attn
    gdn_w = 2 * kd + 2 * vd + 2 * cfg.lin_v_heads
    attn_w = 2 * cfg.heads * cfg.head_dim + 2 * cfg.kv_heads * cfg.head_dim
    per_token_gemm = (n_gdn * (gdn_w * cfg.hidden + cfg.hidden * vd) +
                      n_attn * (attn_w * cfg.hidden + cfg.hidden * cfg.heads * cfg.head_dim) +
                      cfg.layers * 3 * cfg.hidden * cfg.intermediate)
    flop = (2.0 * T * per_token_gemm + n_attn * 2.0 * T * T * cfg.head_dim * cfg.heads +
            n_gdn * 180224.0 * T * cfg.lin_v_heads)
    return ms, {"workload": "cfg3 random-init 4B-class hybrid decoder (32 layers, 24 GDN + 8 gated attention), "
                            "T=4096 decision prefill + 8-label head, hipGraph replay",
                "gemm_plans": gemm_plan_mode(tune),
                "ms_per_decision": ms, "argmax": int(np.argmax(logits)),
                "algorithmic_flop": flop, "achieved_TFLOPs": flop / (ms * 1e-3) / 1e12,
                "frac_of_bf16_peak": flop / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS}


def bench_candidates(steps, warmup, P=2048, n=8, tune=False):
    """Config 4: the random-init 27B-class hybrid decoder (64 layers, 3:1, hidden
    5120, 24/4 x 256 attention, GDN 16 qk / 48 v heads, SwiGLU 17408, vocabulary 248320, untied
    LM head). A step captures a 2048-token prefix, then scores 8 candidate continuations of
    U[64, 256] tokens (seeded) packed into one pass from the shared prefix state, returning
    each candidate's summed token log-probability; wall-clock ms, with the capture and the
    scoring pass also timed apart."""
    from qwen3_5_native import model as QM

    cfg = QM.CFG4_27B
    rng = np.random.default_rng(6)
    prefix = rng.integers(0, cfg.vocab, P).astype(np.int32)
    lens = rng.integers(64, 257, n)
    cands = [rng.integers(0, cfg.vocab, int(k)).astype(np.int32) for k in lens]
    m = QM.Model(cfg, seed=0, max_tokens=P + 256 if sum(lens) <= P + 256 else int(sum(lens)))
    try:
        m.set_gemm_tuning(tune)
        tw = time.perf_counter()
        for _ in range(max(warmup, 1)):
            m.capture(prefix)
            scores = m.score(cands)
        while time.perf_counter() - tw < 2 * SETTLE_S:
            m.capture(prefix)
            scores = m.score(cands)
        cap = sco = 0.0
        for _ in range(steps):
            t0 = time.perf_counter()
            m.capture(prefix)
            t1 = time.perf_counter()
            scores = m.score(cands)
            t2 = time.perf_counter()
            cap += t1 - t0
            sco += t2 - t1
    finally:
        m.close()
    return {"workload": "cfg4 random-init 27B-class hybrid decoder (64 layers), 2048-token prefix captured, "
                        f"{n} candidates of {', '.join(str(int(k)) for k in lens)} tokens scored from it",
            "ms_per_job": (cap + sco) * 1e3 / steps, "capture_ms": cap * 1e3 / steps, "score_ms": sco * 1e3 / steps,
            "candidate_tokens": int(sum(lens)), "best_candidate": int(np.argmax(scores)), "gemm_plans": gemm_plan_mode(tune),
            "scores": [round(float(x), 3) for x in scores]}


def gemm_plan_mode(tune):
    """How cs1_gemm picks its hipBLASLt kernels in the run."""
    if tune:
        return "tuned: fastest of up to 16 heuristic candidates per shape (cs1_gemm_tune on the first eager call)"
    return "deterministic: hipBLASLt's first heuristic choice per shape (cs1_gemm default)"


def cpu_baseline_attention():
    """The oracle's emulation of the reference flash kernel (C, OpenMP) on this host, over
    the full config-1 layer, repeated until about 10 s of work."""
    import oracle as O

    T, Hq, Hk, Dh = 2048, 16, 4, 128
    rng = np.random.default_rng(1)
    q, k, v, gate = (bf16(rng, T * h * Dh) for h in (Hq, Hk, Hk, Hq))
    n, t0 = 0, time.perf_counter()
    while True:
        O.attention_emul(q, k, v, Hk * Dh, gate, T, Hq, Hk, Dh, Dh ** -0.5, want_lse=True)
        n += 1
        if time.perf_counter() - t0 > 10:
            break
    dt = time.perf_counter() - t0
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": T * n / dt, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"full cfg1 layer (T=2048, 16/4 heads, Dh=128, gate, LSE) x{n} through the oracle's C "
                      f"emulation of the reference flash kernel, OpenMP over query rows"}


def cpu_baseline_gdn_cfg0():
    """The oracle's C emulation of the reference's chunked GDN prefill (gdn_prefill.cu, with
    the TF32 pair products and blocked inverse) on this host at config 0, repeated for about
    5 s (OpenMP over the 16 heads)."""
    import oracle as O

    T, H, HK = 512, 16, 16
    rng = np.random.default_rng(0)
    q, k = unit_rows_bf16(rng, T * HK, 128), unit_rows_bf16(rng, T * HK, 128)
    v = bf16(rng, T * H * 128)
    beta = O.f32_to_bf16((1 / (1 + np.exp(-rng.standard_normal(T * H)))).astype(np.float32))
    g = (-np.log1p(np.exp(rng.standard_normal(T * H))) * 0.1).astype(np.float32)
    n, t0 = 0, time.perf_counter()
    while True:
        O.gdn_chunk_emul(q, k, v, g, beta, T, H, HK)
        n += 1
        if time.perf_counter() - t0 > 5:
            break
    dt = time.perf_counter() - t0
    cores = min(H, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)))
    return {"value": T * n / dt, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"config 0 (T=512, H=HK=16) x{n} through the oracle's C emulation of the reference's "
                      f"chunked GDN prefill, OpenMP over heads"}


def calibrate(st, ev):
    """The bf16 MFMA and HBM streaming rates this GPU reaches (libq35_calibrate.so, built with
    the op library), after the same clock settling as every measured region: the published
    peaks the rooflines use, read against what the machine delivers."""
    cal = ctypes.CDLL(os.path.join(ROOT, "system1-omni_amd", "libq35_calibrate.so"))
    cal.q35cal_mfma.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    cal.q35cal_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    blocks, iters = 512, 4000  # two waves per SIMD, four independent accumulator chains each
    out = hip.DeviceBuffer(blocks * 256 * 4)
    mf = lambda: hip.check(cal.q35cal_mfma(out.at(0), blocks, iters, st.handle), "mfma calibration")  # noqa: E731
    _, per = timed(st, ev, 5, 1, [("mfma", mf)])
    flop = 2.0 * 32 * 32 * 16 * 4 * 4 * iters * blocks
    nbytes = 1 << 30
    src, dst = hip.DeviceBuffer(nbytes), hip.DeviceBuffer(nbytes)
    cp = lambda: hip.check(cal.q35cal_copy(src.at(0), dst.at(0), nbytes, st.handle), "copy calibration")  # noqa: E731
    _, per_c = timed(st, ev, 10, 1, [("copy", cp)])
    api = hip.api()
    rt = lambda: hip.check(api.cs1_copy_dd(dst.at(0), src.at(0), nbytes, st.handle), "runtime copy")  # noqa: E731
    _, per_r = timed(st, ev, 10, 1, [("copy", rt)])
    return {"mfma_bf16_TFLOPs": flop / (per["mfma"] * 1e-3) / 1e12,
            "hbm_copy_GBs": 2.0 * nbytes / (per_c["copy"] * 1e-3) / 1e9,
            "hbm_runtime_copy_GBs": 2.0 * nbytes / (per_r["copy"] * 1e-3) / 1e9,
            "note": "32x32x16 bf16 MFMA chains (2 waves per SIMD, 4 chains each) and a 1 GiB 16-byte copy "
                    "(read + write bytes) by this library's kernel and by the runtime's device copy, each after the "
                    "clock settling"}


PROBE_COPY_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_bench_probe.txt")


def probe(api, st):
    """A short fixed sequence for the rocprofv3 counter passes: each workload's kernels a few
    times, then a plain device-to-device copy of PROBE_COPY_BYTES that calibrates the
    FETCH_SIZE / WRITE_SIZE counters (it reads and writes exactly that many bytes)."""
    ev = Events()
    bench_attention(api, st, ev, 3, 0)
    bench_attention(api, st, ev, 3, 0, T=8192)
    bench_attention(api, st, ev, 3, 0, T=4096, Dh=256)
    bench_gdn(api, st, ev, 3, 0, 8192, 32, 16, True, 0.01, 2, "cfg2")
    bench_gdn(api, st, ev, 3, 0, 512, 16, 16, False, 0.0, 0, "cfg0")
    bench_hbm_ops(api, st, ev, 3, 0)
    # the MFMA-bound calibration kernel: the counter pass's reference for a fully busy MFMA
    cal = ctypes.CDLL(os.path.join(ROOT, "system1-omni_amd", "libq35_calibrate.so"))
    cal.q35cal_mfma.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    out = hip.DeviceBuffer(512 * 256 * 4)
    for _ in range(3):
        hip.check(cal.q35cal_mfma(out.at(0), 512, 4000, st.handle), "mfma calibration")
    src, dst = hip.DeviceBuffer(PROBE_COPY_BYTES), hip.DeviceBuffer(PROBE_COPY_BYTES)
    for _ in range(3):
        hip.check(api.cs1_copy_dd(dst.at(0), src.at(0), PROBE_COPY_BYTES, st.handle), "copy")
    st.sync()


def _kernel_base(name):
    """Demangled kernel name without its trailing argument list and leading `void `."""
    name = name.strip()
    if name.endswith(")"):
        depth = 0
        for i in range(len(name) - 1, -1, -1):
            depth += {")": 1, "(": -1}.get(name[i], 0)
            if depth == 0:
                name = name[:i]
                break
    return name[5:] if name.startswith("void ") else name


def summarize_pmc(dirs):
    """Per-kernel averages from rocprofv3 counter CSVs of `bench.py --probe`: FETCH_SIZE /
    WRITE_SIZE (KiB per dispatch) scaled by the calibration copy (bytes = KiB * scale, scale =
    copy bytes / the copy's own counter reading), and, where those counters were collected,
    the MFMA busy fraction and the counted bf16 MFMA flop per dispatch."""
    import csv
    import glob
    from collections import defaultdict

    vals = defaultdict(lambda: defaultdict(list))
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                name = r["Kernel_Name"]
                key = ("copy" if "copyBuffer" in name else _kernel_base(name)) + f" grid={r['Grid_Size']}"
                vals[key][r["Counter_Name"]].append(float(r["Counter_Value"]))
    avg = {k: {c: sum(v) / len(v) for c, v in cs.items()} for k, cs in vals.items()}
    copy = [v for k, v in avg.items() if k.startswith("copy")]
    lines = []
    scale = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        got = [v[c] for v in copy if c in v]
        if got:
            scale[c] = PROBE_COPY_BYTES / max(got)
            lines.append(f"calibration {c}: copy of {PROBE_COPY_BYTES} B reads {max(got):.0f} KiB -> "
                         f"{scale[c]:.2f} B per counted KiB")
    # MFMA busy: busy cycles per GPU-active cycle, relative to the calibration kernel (four
    # independent MFMA chains per wave, which keeps the MFMA units busy)
    ref = [v["SQ_VALU_MFMA_BUSY_CYCLES"] / v["GRBM_GUI_ACTIVE"] for k, v in avg.items()
           if "mfma_rate_kernel" in k and v.get("GRBM_GUI_ACTIVE")]
    if ref:
        lines.append(f"calibration MFMA: the MFMA-bound kernel reads {ref[0]:.2f} busy cycles per GPU-active "
                     f"cycle -> mfma_busy 1.000")
    for k, v in sorted(avg.items()):
        if k.startswith("copy") or "mfma_rate_kernel" in k:
            continue
        if "FETCH_SIZE" in v or "WRITE_SIZE" in v:
            f = v.get("FETCH_SIZE", 0.0) * scale.get("FETCH_SIZE", 1024.0)
            w = v.get("WRITE_SIZE", 0.0) * scale.get("WRITE_SIZE", 1024.0)
            lines.append(f"traffic {k} fetch_kib={v.get('FETCH_SIZE', float('nan')):.0f} "
                         f"write_kib={v.get('WRITE_SIZE', float('nan')):.0f} bytes={f + w:.0f}")
        if "SQ_VALU_MFMA_BUSY_CYCLES" in v and v.get("GRBM_GUI_ACTIVE"):
            # MFMA busy cycles (summed over the SIMDs) per GPU-active cycle of the serialised
            # dispatch, as a fraction of the calibration kernel's; MOPS counts bf16 MFMA work in
            # units of 512 flop
            busy = v["SQ_VALU_MFMA_BUSY_CYCLES"] / v["GRBM_GUI_ACTIVE"] / ref[0] if ref else float("nan")
            flop = v.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", float("nan")) * 512
            lines.append(f"mfma {k} bf16_flop={flop:.4g} busy_cycles={v['SQ_VALU_MFMA_BUSY_CYCLES']:.4g} "
                         f"gpu_active_cycles={v['GRBM_GUI_ACTIVE']:.4g} mfma_busy={busy:.3f}")
    return "\n".join(lines)


def summarize_trace(dirs):
    """Per-kernel dispatch count and average / min / max duration (us) by grid size from
    rocprofv3 --kernel-trace CSVs."""
    import csv
    import glob
    from collections import defaultdict

    dur = defaultdict(list)
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                key = _kernel_base(r["Kernel_Name"]) + f" grid={r['Grid_Size_X']}x{r['Grid_Size_Y']}"
                dur[key].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    return "\n".join(f"kernel {k} n={len(v)} avg_us={sum(v) / len(v):.2f} min_us={min(v):.2f} max_us={max(v):.2f}"
                     for k, v in sorted(dur.items()))


def traffic_bytes(kernel_prefix):
    """HBM bytes per launch of a kernel from the committed counter summary, or None."""
    try:
        for ln in open(TRAFFIC_FILE):
            if ln.startswith("traffic " + kernel_prefix):
                return float(ln.rsplit("bytes=", 1)[1])
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--probe", action="store_true", help="short kernel sequence for rocprofv3 counter passes")
    ap.add_argument("--no-model", action="store_true", help="skip the config-3 and config-4 model runs")
    ap.add_argument("--models-only", action="store_true", help="only the config-3 and config-4 model runs")
    ap.add_argument("--no-graph", action="store_true", help="config 3 without hipGraph replay (eager launches)")
    ap.add_argument("--summarize-pmc", nargs="+", metavar="DIR", help="summarize rocprofv3 --pmc output of --probe")
    ap.add_argument("--summarize-trace", nargs="+", metavar="DIR", help="summarize rocprofv3 --kernel-trace output")
    args = ap.parse_args()
    if args.summarize_pmc:
        print(summarize_pmc(args.summarize_pmc))
        return
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace))
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the prefill is sharded by heads in "
              "design only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    api = hip.load()
    hip.set_device(0)
    st = hip.Stream()
    if args.probe:
        probe(api, st)
        return
    if args.models_only:
        dec_ms, dec = bench_decision_prefill(min(args.steps, 10), args.warmup, graph=not args.no_graph)
        dec["graph"] = not args.no_graph
        dec["tuned_gemm_ms_per_decision"] = bench_decision_prefill(min(args.steps, 10), args.warmup, tune=True,
                                                                   graph=not args.no_graph)[0]
        cand = bench_candidates(min(args.steps, 3), 1)
        cand["tuned_gemm_ms_per_job"] = bench_candidates(min(args.steps, 3), 1, tune=True)["ms_per_job"]
        print(json.dumps({"decision_prefill_ms_4k": dec_ms, "model_cfg3": dec, "model_cfg4": cand}), flush=True)
        return
    ev = Events()
    attn = bench_attention(api, st, ev, args.steps, args.warmup)
    attn8k = bench_attention(api, st, ev, max(2, args.steps // 4), 1, T=8192, label="north-star shape")
    attn256 = bench_attention(api, st, ev, max(2, args.steps // 2), 1, T=4096, Dh=256, label="cfg3 layer")
    g2 = bench_gdn(api, st, ev, args.steps, args.warmup, 8192, 32, 16, True, 0.01, 2,
                   "cfg2 conv1d(k=4)+SiLU then GDN chunked prefill T=8192 HK=16 H=32 D=128, S0~N(0,0.01)")
    g0 = bench_gdn(api, st, ev, args.steps, args.warmup, 512, 16, 16, False, 0.0, 0,
                   "cfg0 GDN chunked prefill T=512 H=HK=16 D=128, S0=0")
    hbm = bench_hbm_ops(api, st, ev, args.steps, args.warmup)
    gref = bench_gdn_reference_shapes(api, st, ev)
    dec_ms, dec = (None, None) if args.no_model else bench_decision_prefill(min(args.steps, 10), args.warmup)
    cand = None if args.no_model else bench_candidates(min(args.steps, 3), 1)
    if not args.no_model:
        dec["tuned_gemm_ms_per_decision"] = bench_decision_prefill(min(args.steps, 10), args.warmup, tune=True)[0]
        cand["tuned_gemm_ms_per_job"] = bench_candidates(min(args.steps, 3), 1, tune=True)["ms_per_job"]
    cpu = None if args.no_cpu else cpu_baseline_attention()
    if not args.no_cpu:
        g0["cpu_baseline"] = cpu_baseline_gdn_cfg0()
    cal = calibrate(st, ev)
    line = {
        "metric": "prefill tokens/s per layer type + ms per 4k-token hybrid decision prefill",
        "value": attn["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": attn["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,1) inputs of the benchmark shapes)",
        "config": {"workload": attn["workload"], "global_batch": 1, "seq_len": 2048, "parallelism": "none"},
        "roofline": {k: attn["roofline"][k] for k in ("bound", "achieved", "peak", "unit", "frac")} |
                    {"traffic": traffic_bytes("q35::(anonymous namespace)::flash32_kernel<true, false> grid=131072 "),
                     # HBM bytes per launch are not counted in this run: they come from the committed
                     # FETCH_SIZE / WRITE_SIZE counter passes over `bench.py --probe`
                     "traffic_source": os.path.relpath(TRAFFIC_FILE, ROOT)},
        "cpu_baseline": cpu,
        "layers": {"attention_cfg1": attn, "attention_t8192": attn8k, "attention_cfg3_dh256": attn256,
                   "gdn_cfg2": g2, "gdn_cfg0": g0},
        "hbm_ops": hbm,
        "calibration": cal,
        "gdn_reference_shapes": gref,
        "decision_prefill_ms_4k": dec_ms,
        "model_cfg3": dec,
        "model_cfg4": cand,
    }
    print(json.dumps(line), flush=True)
    st.destroy()


if __name__ == "__main__":
    main()
