"""Host side of the MI355X Qwen3.5 prefill path.

``hip`` loads ``libqwen3_5_hip.so`` and exposes its C ABI the way the reference's Rust
loader does (src/models/qwen3_5/native/src/cuda.rs): one symbol table resolved at load
time, an ABI-version check, error-code mapping, RAII device buffers, streams and graphs.
"""
from . import hip  # noqa: F401
