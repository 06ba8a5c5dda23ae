"""cs1_gdn_prefill_x_static (the GDN prefill with the library's own per-GPU workspace, for
callers that cannot allocate) against cs1_gdn_prefill_x with a caller workspace: bitwise equal
outputs and final states on two calls in a row, the second smaller, so stale workspace
contents from the first call cannot leak into the second; shapes beyond the 64 MiB workspace
are refused."""
import numpy as np
import pytest

from gpu_helpers import dev, empty, get, get_bf16, say, stream
from qwen3_5_native import hip

pytestmark = pytest.mark.gpu

D = 128


def inputs(T, H, HK, seed):
    rng = np.random.default_rng(seed)

    def unit(x):
        return x / np.sqrt((x * x).sum(-1, keepdims=True))

    import oracle as O
    q = O.f32_to_bf16(unit(rng.standard_normal((T, HK, D))).astype(np.float32)).reshape(-1)
    k = O.f32_to_bf16(unit(rng.standard_normal((T, HK, D))).astype(np.float32)).reshape(-1)
    v = O.f32_to_bf16(rng.standard_normal((T, H, D)).astype(np.float32)).reshape(-1)
    beta = O.f32_to_bf16((1 / (1 + np.exp(-rng.standard_normal(T * H)))).astype(np.float32))
    g = (-np.log1p(np.exp(rng.standard_normal(T * H))) * 0.1).astype(np.float32)
    s0 = (rng.standard_normal((H, D, D)) * 0.01).astype(np.float32)
    return q, k, v, g, beta, s0


def run_both(T, H, HK, seed):
    api, st = hip.api(), stream()
    q, k, v, g, beta, s0 = inputs(T, H, HK, seed)
    bufs = [dev(x) for x in (q, k, v, g, beta, s0.reshape(-1))]
    o1, o2 = empty(T * H * D * 2), empty(T * H * D * 2)
    so1, so2 = empty(H * D * D * 4), empty(H * D * D * 4)
    ws = empty(api.cs1_gdn_workspace_floats(T, H) * 4)
    say(f"gdn prefill static workspace T={T} H={H} HK={HK}")
    hip.check(api.cs1_gdn_prefill_x(*(b.at(0) for b in bufs[:5]), o1.at(0), ws.at(0), T, H, HK, D ** -0.5,
                                    bufs[5].at(0), so1.at(0), st.handle), "with workspace")
    hip.check(api.cs1_gdn_prefill_x_static(*(b.at(0) for b in bufs[:5]), o2.at(0), T, H, HK, D ** -0.5,
                                           bufs[5].at(0), so2.at(0), st.handle), "static workspace")
    np.testing.assert_array_equal(get_bf16(o2, T * H * D), get_bf16(o1, T * H * D))
    np.testing.assert_array_equal(get(so2, np.float32, H * D * D), get(so1, np.float32, H * D * D))


def test_static_workspace_matches_caller_workspace_twice():
    run_both(4480, 13, 1, seed=1)    # exactly 910 records (70 chunks x 13 heads): the whole array
    run_both(1792, 32, 16, seed=3)   # the largest T at H = 32 (28 x 32 = 896 records)
    run_both(130, 8, 4, seed=2)      # smaller, a partial last chunk, other heads


def test_static_workspace_limits():
    api, st = hip.api(), stream()
    say("gdn prefill static workspace: limits")
    # 1793 tokens at 32 heads need 29 * 32 = 928 records > 910, 4481 at 13 heads 71 * 13 = 923:
    # refused before any launch
    assert api.cs1_gdn_prefill_x_static(None, None, None, None, None, None, 4481, 13, 1, 0.1, None, None,
                                        st.handle) == hip.HIP_ERROR_INVALID_VALUE
    assert api.cs1_gdn_prefill_x_static(None, None, None, None, None, None, 1793, 32, 16, 0.1, None, None,
                                        st.handle) == hip.HIP_ERROR_INVALID_VALUE
    assert api.cs1_gdn_prefill_x_static(None, None, None, None, None, None, -1, 32, 16, 0.1, None, None,
                                        st.handle) == hip.HIP_ERROR_INVALID_VALUE
    # T = 0 passes the state through, as cs1_gdn_prefill_x does
    H = 2
    s = np.arange(H * D * D, dtype=np.float32)
    si, so = dev(s), empty(H * D * D * 4)
    hip.check(api.cs1_gdn_prefill_x_static(None, None, None, None, None, None, 0, H, 1, 0.1, si.at(0), so.at(0),
                                           st.handle), "T = 0")
    np.testing.assert_array_equal(get(so, np.float32, H * D * D), s)
