"""GPU tests of the runtime entry points' failure recovery (the reference's
tests/qwen3_5/kernels.rs:203-273) and of the model runner's prefix-state rejection rules
(kernels.rs:634-692): every failure returns a code, leaves the stream capturable again, and
a graph captured before the failure keeps replaying with updated inputs."""
import ctypes

import numpy as np
import pytest

from gpu_helpers import dev, empty, get, say, stream
from qwen3_5_native import hip
from qwen3_5_native import model as QM

pytestmark = pytest.mark.gpu


def _capture(st, record):
    """(code, exec handle) of capturing what record() queues; the capture is always ended."""
    api = hip.api()
    rc = api.cs1_graph_begin(st.handle)
    if rc != 0:
        return rc, None
    inner = 0
    try:
        inner = record()
    finally:
        ex = ctypes.c_void_p()
        end = api.cs1_graph_end(st.handle, ctypes.byref(ex))
    if inner:
        if ex.value:
            api.cs1_graph_destroy(ex.value)
        return inner, None
    return end, ex.value


def test_graph_capture_failures_recover():
    api, st = hip.api(), stream()
    say("runtime: graph capture failure recovery")
    # a recording that fails must still end the capture so the stream can be captured again
    rc, ex = _capture(st, lambda: 1)
    assert rc == 1 and ex is None
    table = np.array([np.float32(i) for i in range(24)], np.float32)
    bf = (table.view(np.uint32) >> 16).astype(np.uint16)  # exact: small integers
    weights = dev(bf)
    ids = empty(8)
    out = empty(32)

    def embed():
        return api.cs1_embed(ids.at(0), weights.at(0), out.at(0), 2, 8, st.handle)

    def replay(ex, rows):
        hip.upload(ids, np.array(rows, np.int32), st)
        hip.check(api.cs1_graph_launch(ex, st.handle), "replay")
        got = get(out, np.uint16, 16)
        want = np.concatenate([bf[r * 8:(r + 1) * 8] for r in rows])
        np.testing.assert_array_equal(got, want)

    rc, graph = _capture(st, embed)
    assert rc == 0 and graph
    try:
        for rows in ([0, 1], [2, 0], [1, 2]):
            replay(graph, rows)
        # capturing the null (legacy default) stream is refused without poisoning the thread
        assert api.cs1_graph_begin(None) != 0
        rc, rec = _capture(st, embed)
        assert rc == 0
        replay(rec, [0, 1])
        api.cs1_graph_destroy(rec)
        # launching a null graph is an argument error
        assert api.cs1_graph_launch(None, st.handle) == hip.HIP_ERROR_INVALID_VALUE
        rc, rec = _capture(st, embed)
        assert rc == 0
        replay(rec, [2, 0])
        api.cs1_graph_destroy(rec)
        # a host wait inside capture is refused (900) and spoils the capture: ending it reports
        # 901 and yields no graph, whether or not the recording passes the 900 on
        # (uploads and downloads are host waits too: the caller reuses its host buffer right
        # after the call, so a copy recorded into a graph would replay stale or freed memory)
        host = np.zeros(8, np.int32)
        waits = {
            "sync": lambda: api.cs1_stream_sync(st.handle),
            "upload": lambda: api.cs1_upload(ids.at(0), host.ctypes.data, 32, st.handle),
            "download": lambda: api.cs1_download(host.ctypes.data, ids.at(0), 32, st.handle),
        }
        for kind, propagate in [(k, p) for k in waits for p in (True, False)]:
            seen = []

            def record():
                rc = embed()
                if rc:
                    return rc
                code = waits[kind]()
                seen.append(code)
                return code if propagate else 0

            rc, rec = _capture(st, record)
            say(f"  {kind} inside capture (propagate={propagate}): wait {seen}, capture {rc}")
            assert seen == [hip.HIP_ERROR_STREAM_CAPTURE_UNSUPPORTED]
            assert rec is None
            assert rc == (hip.HIP_ERROR_STREAM_CAPTURE_UNSUPPORTED if propagate
                          else hip.HIP_ERROR_STREAM_CAPTURE_INVALIDATED)
            # the retained graph still replays, and recapture works on this thread
            replay(graph, [2, 1])
            rc, rec = _capture(st, embed)
            assert rc == 0
            replay(rec, [0, 2])
            api.cs1_graph_destroy(rec)
    finally:
        api.cs1_graph_destroy(graph)


def test_empty_copies_and_null_frees_succeed():
    api, st = hip.api(), stream()
    say("runtime: empty copies")
    assert api.cs1_copy_dd(None, None, 0, st.handle) == 0
    assert api.cs1_copy2d(None, 0, None, 0, 0, 5, st.handle) == 0
    assert api.cs1_upload(None, None, 0, st.handle) == 0
    assert api.cs1_download(None, None, 0, st.handle) == 0
    assert api.cs1_free(None) == 0
    assert api.cs1_graph_destroy(None) == 0
    # an error string exists for runtime and hipBLASLt codes
    assert api.cs1_error_string(hip.HIP_ERROR_STREAM_CAPTURE_INVALIDATED)
    assert b"hipBLASLt" in api.cs1_error_string(1007)


def test_null_operands_are_argument_errors():
    """A call that would launch work with a null operand returns hipErrorInvalidValue (1) and
    launches nothing; the same calls with nothing to do still succeed."""
    api, st = hip.api(), stream()
    say("runtime: null operands")
    buf = empty(1 << 20)
    x = buf.at(0)
    cu = np.array([0, 64], np.int32)
    h = st.handle
    calls = {
        "embed": lambda: api.cs1_embed(None, None, None, 4, 64, h),
        "rms_norm": lambda: api.cs1_rms_norm(None, None, None, 4, 64, 1e-6, h),
        "add_rms_norm": lambda: api.cs1_add_rms_norm(None, None, None, None, 4, 64, 1e-6, h),
        "gated_rms_norm": lambda: api.cs1_gated_rms_norm(None, None, 128, None, None, 4, 1, 128, 1e-6, h),
        "gdn_conv": lambda: api.cs1_gdn_conv(None, 24, None, None, None, None, 4, 8, 8, h),
        "gdn_conv_varlen": lambda: api.cs1_gdn_conv_varlen(None, 24, None, None, None, None, cu.ctypes.data, 1, None,
                                                           8, 8, h),
        "gdn_gates": lambda: api.cs1_gdn_gates(None, None, 8, None, None, None, None, 4, 8, h),
        "sigmoid_gate": lambda: api.cs1_sigmoid_gate(None, None, 64, h),
        "silu_mul": lambda: api.cs1_silu_mul(None, 16, None, 4, 8, h),
        "attn_prep": lambda: api.cs1_attn_prep(None, None, 1536, None, None, None, None, None, None, None, 4, 4, 1, 256,
                                               32, 1e-6, h),
        "attention_ex": lambda: api.cs1_attention_ex(None, None, None, 128, None, None, None, 64, 4, 1, 128, 0.1, 0, h),
        "attention_varlen": lambda: api.cs1_attention_varlen(None, None, None, 128, None, None, None, cu.ctypes.data, 1,
                                                             4, 1, 128, 0.1, h),
        "gdn_prefill_x": lambda: api.cs1_gdn_prefill_x(None, None, None, None, None, None, None, 64, 2, 1, 0.1, None,
                                                       None, h),
        # every operand but g set: still an argument error
        "gdn_prefill_x g": lambda: api.cs1_gdn_prefill_x(x, x, x, None, x, x, x, 64, 2, 1, 0.1, None, None, h),
        "gdn_prefill_gated_x": lambda: api.cs1_gdn_prefill_gated_x(x, x, x, x, x, 2, x, x, None, x, 64, 2, 1, 0.1,
                                                                   None, None, h),
    }
    for name, call in calls.items():
        say(f"  {name}")
        assert call() == 1, name
    st.sync()
    # nothing to do: success, whatever the pointers
    assert api.cs1_embed(None, None, None, 0, 64, h) == 0
    assert api.cs1_gdn_gates(None, None, 8, None, None, None, None, 0, 8, h) == 0
    assert api.cs1_attention_ex(None, None, None, 128, None, None, None, 0, 4, 1, 128, 0.1, 0, h) == 0


TINY = QM.Config(layers=4, hidden=256, intermediate=512, vocab=1024, heads=4, kv_heads=1, lin_k_heads=2,
                 lin_v_heads=4, lm_head=1)


def test_prefix_state_rejection_rules():
    """The runner's capture / score guards (the reference rejects oversized prefixes, continuing
    before capture and cached prompts that overflow the maximum, model.rs:955-1062): each is an
    argument error before any work is queued, and a valid capture afterwards still scores. The
    reference's foreign-model rule has no counterpart here: the prefix state lives inside the
    model that captured it."""
    stream()
    say("model prefix rejection rules")
    m = QM.Model(TINY, seed=3, max_tokens=256)
    try:
        rng = np.random.default_rng(0)
        c1 = [rng.integers(0, TINY.vocab, 10)]
        with pytest.raises(hip.HipError):
            m.score(c1)  # no capture yet
        for P in (320, 256 + 64):  # beyond max_tokens
            with pytest.raises(hip.HipError):
                m.capture(rng.integers(0, TINY.vocab, P))
        for P in (0, 63, 100):  # not a positive multiple of 64
            with pytest.raises(hip.HipError):
                m.capture(rng.integers(0, TINY.vocab, P))
        with pytest.raises(hip.HipError):
            m.capture(np.full(64, TINY.vocab, np.int32))  # token id out of range
        prefix = rng.integers(0, TINY.vocab, 192)
        m.capture(prefix)
        with pytest.raises(hip.HipError):
            m.score([rng.integers(0, TINY.vocab, 65)])  # 192 + 65 > 256 rows
        with pytest.raises(hip.HipError):
            m.score([np.zeros(0, np.int32)])  # an empty candidate
        ok = m.score([rng.integers(0, TINY.vocab, 64), rng.integers(0, TINY.vocab, 5)])
        assert np.isfinite(ok).all()
    finally:
        m.close()
