"""The drop-in boundary, checked without a GPU.

* libqwen3_5_hip.so loads, reports ABI 6 and exports every symbol include/qwen3_5_ops.h
  declares; the reference loader's table (cuda.rs:50-133) is a subset of the header;
  libqwen3_5_model.so exports every symbol include/qwen3_5_model.h declares.
* Argument validation returns hipErrorInvalidValue before any device work, with the
  reference's rules (attention.cu:239-243, 266-268; gdn_prefill.cu:571; elementwise.cu:97,
  106, 117, 134; norm.cu:281), and empty work succeeds without a launch.
"""
import os
import re

import pytest

from qwen3_5_native import hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qwen3_5_ops.h")
INVALID = hip.HIP_ERROR_INVALID_VALUE


@pytest.fixture(scope="module")
def api():
    return hip.load()


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(cs1_\w+)\s*\(", text))


def test_library_exports_every_declared_symbol(api):
    names = declared_symbols()
    assert len(names) >= 45
    for n in names:
        assert hasattr(api._lib, n), n
    # the reference loader resolves these names; all are declared here
    assert set(hip.SYMBOLS) <= names
    assert set(hip.ADDITIONS) <= names
    assert api.cs1_abi_version() == 6


def test_workspace_size_is_pure_and_monotone(api):
    assert api.cs1_gdn_workspace_floats(0, 4) == 0
    a = api.cs1_gdn_workspace_floats(64, 4)
    assert a == api.cs1_gdn_workspace_floats(1, 4) > 0
    assert api.cs1_gdn_workspace_floats(65, 4) > a
    # per (head, chunk): w, u, qd, kd^T (64x128 bf16) + pb (64x64 bf16) + decay, 256-B aligned parts;
    # a sequence long enough to run in segments (records > 200 MiB) adds two float32 states
    rec = 4 * 64 * 128 * 2 + 64 * 64 * 2
    mid = api.cs1_gdn_workspace_floats(4096, 32) * 4
    assert 32 * 64 * rec <= mid < 32 * 64 * (rec + 4) + 4096
    big = api.cs1_gdn_workspace_floats(8192, 32) * 4
    states = 2 * 32 * 128 * 128 * 4
    assert 32 * 128 * rec + states <= big < 32 * 128 * (rec + 4) + 4096 + states


def test_argument_errors_and_empty_work(api):
    n = None
    # GDN: H % HK, negative T
    assert api.cs1_gdn_prefill(n, n, n, n, n, n, n, 4, 6, 4, 1.0, n) == INVALID
    assert api.cs1_gdn_prefill(n, n, n, n, n, n, n, -1, 4, 2, 1.0, n) == INVALID
    assert api.cs1_gdn_prefill_x(n, n, n, n, n, n, n, 0, 4, 2, 1.0, n, n, n) == 0  # nothing to do
    # attention: Dh must be 256 on the reference entry points, 128/256 on the extension
    assert api.cs1_attention(n, n, n, 1024, n, 4, 16, 4, 128, 0.1, n) == INVALID
    assert api.cs1_attention_ex(n, n, n, 512, n, n, n, 4, 16, 4, 64, 0.1, 0, n) == INVALID
    assert api.cs1_attention(n, n, n, 1024, n, 4, 6, 4, 256, 0.1, n) == INVALID  # Hq % Hk
    assert api.cs1_attention(n, n, n, 1020, n, 4, 16, 4, 256, 0.1, n) == INVALID  # ldv % 8, ldv < Hk Dh
    assert api.cs1_attention_gated_prefix(n, n, n, 1024, n, n, 128, 16, 4, 256, 0.1, 32, n) == INVALID
    assert api.cs1_attention_gated_prefix(n, n, n, 1024, n, n, 128, 16, 4, 256, 0.1, 192, n) == INVALID
    # kernels.rs:355-389: empty work is valid without a gate, non-empty work needs one
    assert api.cs1_attention_gated(n, n, n, 256, n, n, 0, 1, 1, 256, 0.0625, n) == 0
    assert api.cs1_attention_gated(n, n, n, 256, n, n, 1, 1, 1, 256, 0.0625, n) != 0
    assert api.cs1_attention_gated_prefix(n, n, n, 1024, n, n, 128, 16, 4, 256, 0.1, 128, n) == 0
    # attn_prep: half % 8, 2 half <= Dh, ld % 8
    assert api.cs1_attn_prep(n, n, 2048, n, n, n, n, n, n, n, 4, 2, 1, 256, 12, 1e-6, n) == INVALID
    assert api.cs1_attn_prep(n, n, 2048, n, n, n, n, n, n, n, 4, 2, 1, 128, 72, 1e-6, n) == INVALID
    assert api.cs1_attn_prep(n, n, 2050, n, n, n, n, n, n, n, 4, 2, 1, 256, 32, 1e-6, n) == INVALID
    assert api.cs1_attn_prep(n, n, 2048, n, n, n, n, n, n, n, 0, 2, 1, 256, 32, 1e-6, n) == 0
    # elementwise and norms
    assert api.cs1_gated_rms_norm(n, n, 4096, n, n, 4, 32, 64, 1e-6, n) == INVALID
    assert api.cs1_gated_rms_norm(n, n, 100, n, n, 4, 32, 128, 1e-6, n) == INVALID
    assert api.cs1_gated_rms_norm(n, n, 4096, n, n, 0, 32, 128, 1e-6, n) == 0
    assert api.cs1_gdn_conv(n, 100, n, n, n, n, 4, 32, 64, n) == INVALID
    assert api.cs1_gdn_conv(n, 128, n, n, n, n, 0, 32, 64, n) == 0
    assert api.cs1_gdn_gates(n, n, 3, n, n, n, n, 4, 4, n) == INVALID
    assert api.cs1_gdn_gates(n, n, 4, n, n, n, n, 0, 4, n) == 0
    assert api.cs1_silu_mul(n, 10, n, 4, 6, n) == INVALID
    assert api.cs1_silu_mul(n, 12, n, 0, 6, n) == 0
    assert api.cs1_embed(n, n, n, 4, 12, n) == INVALID
    assert api.cs1_embed(n, n, n, 0, 16, n) == 0
    assert api.cs1_sigmoid_gate(n, n, 0, n) == 0
    assert api.cs1_rms_norm(n, n, n, 0, 2560, 1e-6, n) == 0
    assert api.cs1_add_rms_norm(n, n, n, n, 0, 2560, 1e-6, n) == 0


def test_vision_symbols_report_not_supported(api):
    n = None
    assert api.cs1_vision_gelu(n, 0, 1, n) == hip.HIP_ERROR_NOT_SUPPORTED
    assert api.cs1_vision_attention(n, n, n, n, 0, n) == hip.HIP_ERROR_NOT_SUPPORTED
    assert api.cs1_gemm_f32(n, n, n, n, 0, 0, 0, n) == hip.HIP_ERROR_NOT_SUPPORTED


def test_error_strings(api):
    assert api.cs1_error_string(0)
    assert b"hipBLASLt" in api.cs1_error_string(1003)
    with pytest.raises(hip.HipError) as e:
        hip.check(INVALID, "attention")
    assert e.value.code == INVALID and "attention" in str(e.value)


def test_model_library_exports_and_validates():
    """libqwen3_5_model.so loads, exports the runner's symbols and rejects a bad config
    before touching the device."""
    import ctypes
    from qwen3_5_native import model as QM

    lib = QM.load()
    text = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "qwen3_5_model.h")).read(), flags=re.S)
    declared = set(re.findall(r"\b(q35m_\w+)\s*\(", text))
    assert declared and set(QM.SYMBOLS) <= declared
    for name in declared:
        assert hasattr(lib, name), name
    bad = QM._cfg(QM.Config(layers=2, hidden=512, intermediate=1024, vocab=100, heads=4, kv_heads=3))
    h = ctypes.c_void_p()
    assert lib.q35m_create(ctypes.byref(bad), 0, 16, ctypes.byref(h)) == hip.HIP_ERROR_INVALID_VALUE
    assert lib.q35m_forward(None, None, 0, None) == hip.HIP_ERROR_INVALID_VALUE
