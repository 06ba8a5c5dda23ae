"""Helpers shared by the GPU tests: every device call goes through the C ABI."""
import sys

import numpy as np

import oracle as O
from qwen3_5_native import hip

_STREAM = None


def stream():
    global _STREAM
    if _STREAM is None:
        hip.load()
        hip.set_device(0)
        _STREAM = hip.Stream()
    return _STREAM


def dev(arr):
    return hip.to_device(np.ascontiguousarray(arr), stream())


def empty(nbytes):
    return hip.DeviceBuffer(nbytes)


def get(buf, dtype, count, offset=0):
    return hip.from_device(buf, dtype, count, stream(), offset)


def get_bf16(buf, count, offset=0):
    return get(buf, np.uint16, count, offset)


def say(*a):
    """Name the case before each GPU step (flushed, so a hard failure still shows it)."""
    print(*a, flush=True)
    sys.stdout.flush()


def bf16_errors(got_u16, want):
    """max-abs and mean-abs difference of a bf16 result against float reference values."""
    g = O.bf16_to_f32(got_u16).astype(np.float64).reshape(-1)
    w = np.asarray(want, np.float64).reshape(-1)
    d = np.abs(g - w)
    return float(d.max()) if d.size else 0.0, float(d.mean()) if d.size else 0.0


def ulp_diff(a_u16, b_u16):
    """Largest distance in bf16 units in the last place (same-sign values)."""
    a = np.asarray(a_u16, np.uint16).astype(np.int32)
    b = np.asarray(b_u16, np.uint16).astype(np.int32)
    a = np.where(a & 0x8000, -(a & 0x7FFF), a)
    b = np.where(b & 0x8000, -(b & 0x7FFF), b)
    return int(np.abs(a - b).max()) if a.size else 0
