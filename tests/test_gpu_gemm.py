"""GPU parity of cs1_gemm (hipBLASLt, reference interface ops.h:117-124, gemm.cu:123-134):
y [M, N] (rows of ldy) = x [M, K] w [N, K]^T, bf16 in and out, float32 accumulation."""
import numpy as np
import pytest

import oracle as O
from gpu_helpers import dev, empty, get_bf16, say, stream, ulp_diff
from qwen3_5_native import hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gemm():
    api = hip.api()
    stream()
    h = api.cs1_gemm_create(32 << 20)
    assert h
    yield h
    api.cs1_gemm_destroy(h)


def run(h, x, w, M, N, K, ldy=None, y_init=None):
    api, st = hip.api(), stream()
    ldy = ldy or N
    dx, dw = dev(x), dev(w)
    y = dev(y_init) if y_init is not None else empty(M * ldy * 2)
    hip.check(api.cs1_gemm(h, dx.at(0), dw.at(0), y.at(0), M, N, K, ldy, st.handle), "gemm")
    return get_bf16(y, M * ldy).reshape(M, ldy)


def ref(x, w, M, N, K):
    """float64 product of the bf16 values, rounded once to bfloat16."""
    xf = O.bf16_to_f32(x).reshape(M, K).astype(np.float64)
    wf = O.bf16_to_f32(w).reshape(N, K).astype(np.float64)
    return O.f32_to_bf16((xf @ wf.T).astype(np.float32))


@pytest.mark.parametrize("M,N,K", [(1, 256, 2560), (200, 512, 256), (4096, 2560, 9728 // 8), (37, 4168, 2560)])
def test_gemm_matches_float64(gemm, M, N, K):
    say(f"gemm M={M} N={N} K={K}")
    rng = np.random.default_rng(M + N + K)
    x = O.f32_to_bf16(rng.standard_normal(M * K).astype(np.float32))
    w = O.f32_to_bf16((rng.standard_normal(N * K) * 0.02).astype(np.float32))
    got = run(gemm, x, w, M, N, K)
    want = ref(x, w, M, N, K)
    # float32 accumulation in another order than the float64 sum: one bf16 rounding step
    # apart at most, except where the sum cancels to a tiny value
    d = np.abs(O.bf16_to_f32(got).astype(np.float64) - O.bf16_to_f32(want).astype(np.float64))
    scale = np.abs(O.bf16_to_f32(want)).max()
    say(f"  max diff {d.max():.3e} of max |y| {scale:.3e}, ulp {ulp_diff(got[np.abs(O.bf16_to_f32(want)) > 1e-3 * scale], want[np.abs(O.bf16_to_f32(want)) > 1e-3 * scale])}")
    assert d.max() <= 2 ** -7 * scale
    assert ulp_diff(got[np.abs(O.bf16_to_f32(want)) > 1e-2 * scale], want[np.abs(O.bf16_to_f32(want)) > 1e-2 * scale]) <= 1


def test_gemm_strided_output_and_repeatable(gemm):
    """ldy > N fills a column slice of a wider buffer and leaves the rest untouched; a shape
    reuses its plan, so repeated calls are bitwise identical (gemm.cu:1-10). The unstrided
    call is another shape with a plan of its own (possibly another tuned kernel), so it
    agrees to one bf16 step."""
    M, N, K, ldy = 130, 192, 512, 320
    say(f"gemm strided M={M} N={N} K={K} ldy={ldy}")
    rng = np.random.default_rng(5)
    x = O.f32_to_bf16(rng.standard_normal(M * K).astype(np.float32))
    w = O.f32_to_bf16((rng.standard_normal(N * K) * 0.05).astype(np.float32))
    fill = np.full(M * ldy, 0x7F7F, np.uint16)
    a = run(gemm, x, w, M, N, K, ldy, fill)
    b = run(gemm, x, w, M, N, K, ldy, fill)
    np.testing.assert_array_equal(a, b)
    assert (a[:, N:] == 0x7F7F).all()
    assert ulp_diff(a[:, :N], run(gemm, x, w, M, N, K)) <= 1


def test_gemm_edge_arguments(gemm):
    api, st = hip.api(), stream()
    say("gemm argument checks")
    assert api.cs1_gemm(gemm, None, None, None, 0, 16, 16, 16, st.handle) == 0
    assert api.cs1_gemm(gemm, None, None, None, 4, 16, 16, 8, st.handle) == hip.HIP_ERROR_INVALID_VALUE
    assert api.cs1_gemm(None, None, None, None, 4, 16, 16, 16, st.handle) == hip.HIP_ERROR_INVALID_VALUE
    # null operands of a valid shape are an argument error, and the shape's plan is unaffected
    assert api.cs1_gemm(gemm, None, None, None, 4, 16, 16, 16, st.handle) == hip.HIP_ERROR_INVALID_VALUE


def test_gemm_tuned_and_default_plans_agree():
    """cs1_gemm_tune (the fastest of hipBLASLt's heuristic candidates, timed on these
    operands) and the default plan (the first heuristic choice without atomic split-K) both
    stay within one bf16 step of the float64 product, and each is bitwise repeatable once
    built. The shape is one of the 27B-class candidate-scoring projections, where the
    measured choice differs from the first."""
    api, st = hip.api(), stream()
    M, N, K = 1217, 5120, 6144
    say(f"gemm tuned vs default M={M} N={N} K={K}")
    rng = np.random.default_rng(11)
    x = O.f32_to_bf16(rng.standard_normal(M * K).astype(np.float32))
    w = O.f32_to_bf16((rng.standard_normal(N * K) * 0.02).astype(np.float32))
    want = ref(x, w, M, N, K)
    mask = np.abs(O.bf16_to_f32(want)) > 1e-2 * np.abs(O.bf16_to_f32(want)).max()
    outs = []
    for tune in (True, False):
        h = api.cs1_gemm_create(32 << 20)
        assert h
        try:
            if tune:
                dx, dw, y = dev(x), dev(w), empty(M * N * 2)
                hip.check(api.cs1_gemm_tune(h, dx.at(0), dw.at(0), y.at(0), M, N, K, N, st.handle), "gemm tune")
                tuned_out = get_bf16(y, M * N).reshape(M, N)
            a = run(h, x, w, M, N, K)
            np.testing.assert_array_equal(a, run(h, x, w, M, N, K))
            if tune:
                np.testing.assert_array_equal(a, tuned_out)
        finally:
            api.cs1_gemm_destroy(h)
        say(f"  tune={tune}: ulp vs float64 {ulp_diff(a[mask], want[mask])}")
        assert ulp_diff(a[mask], want[mask]) <= 1
        outs.append(a)
    assert ulp_diff(outs[0][mask], outs[1][mask]) <= 1


def test_gemm_default_plan_is_the_same_in_every_handle():
    """Without tuning, a shape's plan does not depend on the handle or on timing: two fresh
    handles give bitwise identical results (what makes model outputs repeatable from one
    process to the next)."""
    api = hip.api()
    M, N, K = 1217, 17408 // 8, 5120
    say(f"gemm default plan in two handles M={M} N={N} K={K}")
    rng = np.random.default_rng(12)
    x = O.f32_to_bf16(rng.standard_normal(M * K).astype(np.float32))
    w = O.f32_to_bf16((rng.standard_normal(N * K) * 0.02).astype(np.float32))
    outs = []
    for _ in range(2):
        h = api.cs1_gemm_create(32 << 20)
        assert h
        try:
            outs.append(run(h, x, w, M, N, K))
        finally:
            api.cs1_gemm_destroy(h)
    np.testing.assert_array_equal(outs[0], outs[1])


def test_gemm_tune_refused_under_capture():
    """cs1_gemm_tune waits on the host, so under stream capture it refuses with
    hipErrorStreamCaptureUnsupported and records nothing; the capture then still ends and
    replays a plain cs1_gemm."""
    api, st = hip.api(), stream()
    M, N, K = 64, 256, 256
    say("gemm tune under capture")
    rng = np.random.default_rng(3)
    x = O.f32_to_bf16(rng.standard_normal(M * K).astype(np.float32))
    w = O.f32_to_bf16((rng.standard_normal(N * K) * 0.05).astype(np.float32))
    dx, dw, y = dev(x), dev(w), empty(M * N * 2)
    h = api.cs1_gemm_create(32 << 20)
    assert h
    codes = []
    graph = None
    try:
        def body():
            codes.append(api.cs1_gemm_tune(h, dx.at(0), dw.at(0), y.at(0), M, N, K, N, st.handle))
            hip.check(api.cs1_gemm(h, dx.at(0), dw.at(0), y.at(0), M, N, K, N, st.handle), "gemm")
        graph = hip.Graph(st, body)
        graph.launch(st)
        got = get_bf16(y, M * N).reshape(M, N)
    finally:
        graph = None
        api.cs1_gemm_destroy(h)
    assert codes == [hip.HIP_ERROR_STREAM_CAPTURE_UNSUPPORTED]
    h0 = api.cs1_gemm_create(32 << 20)
    try:
        np.testing.assert_array_equal(got, run(h0, x, w, M, N, K))
    finally:
        api.cs1_gemm_destroy(h0)


def test_gemm_plan_first_built_under_capture():
    """A shape whose first call is recorded into a HIP graph gets the same deterministic
    plan as an eager call, so every replay equals an eager call of a fresh handle bit for
    bit (with eager work on the stream between the replays)."""
    api, st = hip.api(), stream()
    M, N, K = 96, 384, 640
    say(f"gemm plan built under capture M={M} N={N} K={K}")
    rng = np.random.default_rng(23)
    x = O.f32_to_bf16(rng.standard_normal(M * K).astype(np.float32))
    w = O.f32_to_bf16((rng.standard_normal(N * K) * 0.05).astype(np.float32))
    dx, dw, y = dev(x), dev(w), empty(M * N * 2)
    h = api.cs1_gemm_create(32 << 20)
    assert h
    graph = None
    try:
        graph = hip.Graph(st, lambda: hip.check(api.cs1_gemm(h, dx.at(0), dw.at(0), y.at(0), M, N, K, N, st.handle),
                                                "gemm under capture"))
        replays = []
        for i in range(3):
            hip.upload(y, np.zeros(M * N, np.uint16), st)  # eager work between replays
            graph.launch(st)
            replays.append(get_bf16(y, M * N))
            say(f"  replay {i} done")
    finally:
        graph = None
        api.cs1_gemm_destroy(h)
    h0 = api.cs1_gemm_create(32 << 20)
    assert h0
    try:
        want = run(h0, x, w, M, N, K).reshape(-1)
    finally:
        api.cs1_gemm_destroy(h0)
    for r in replays:
        np.testing.assert_array_equal(r, want)
