"""CPU oracle for the Qwen3.5 prefill hot path (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may import
this package, and only as the checker. The product library never calls it.

The arithmetic lives in ``oracle.c`` (built to ``liboracle.so`` by ``oracle/Makefile``);
this module wraps it with numpy. bfloat16 arrays are carried as ``np.uint16`` bit
patterns. Each wrapper names the reference function it restates; the C file cites
file:line for every rounding point.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")


def build() -> str:
    """Compile liboracle.so from oracle.c (gcc, OpenMP)."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB_PATH


def _nullable(tp):
    class _N:
        @classmethod
        def from_param(cls, obj):
            if obj is None:
                return None
            return tp.from_param(obj)

    return _N


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH) or os.path.getmtime(_LIB_PATH) < os.path.getmtime(
        os.path.join(_HERE, "oracle.c")
    ):
        build()
    L = ctypes.CDLL(_LIB_PATH)
    c_int, c_float, c_double, c_size, c_u64 = (
        ctypes.c_int,
        ctypes.c_float,
        ctypes.c_double,
        ctypes.c_size_t,
        ctypes.c_uint64,
    )
    nf32 = _nullable(f32p)
    nf64 = _nullable(f64p)
    nu16 = _nullable(u16p)
    L.orc_xorshift_bf16.argtypes = [u16p, c_size, c_u64, c_float]
    L.orc_f32_to_bf16.argtypes = [f32p, u16p, c_size]
    L.orc_f32_to_tf32.argtypes = [f32p, f32p, c_size]
    L.orc_gdn_recurrent_f64.argtypes = [u16p, u16p, u16p, f32p, u16p, c_int, c_int, c_int, c_int, c_double,
                                        nf32, f64p, nf64]
    L.orc_gdn_chunk_emul.argtypes = [u16p, u16p, u16p, f32p, u16p, c_int, c_int, c_int, c_float, nf32, u16p, nf32]
    L.orc_gdn_chunk_emul.restype = c_int
    L.orc_tri_inverse_blocked.argtypes = [f32p, f32p]
    L.orc_attention_f64.argtypes = [u16p, u16p, u16p, c_int, c_int, c_int, c_int, c_int, c_double, c_int,
                                    _nullable(np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")), c_int, f64p, nf64]
    L.orc_attention_emul.argtypes = [u16p, u16p, u16p, c_int, nu16, c_int, c_int, c_int, c_int, c_float, c_int,
                                     u16p, nf32]
    L.orc_attention_emul_rows.argtypes = [u16p, u16p, u16p, c_int, nu16, c_int, c_int, c_int, c_int, c_float,
                                          np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS"), c_int, u16p, nf32]
    L.orc_gdn_conv.argtypes = [u16p, c_int, u16p, u16p, u16p, u16p, c_int, c_int, c_int]
    L.orc_gdn_gates.argtypes = [u16p, u16p, c_int, u16p, u16p, u16p, f32p, c_int, c_int]
    L.orc_gated_rms_norm.argtypes = [u16p, u16p, c_int, u16p, u16p, c_int, c_int, c_int, c_float]
    L.orc_attn_prep.argtypes = [u16p, u16p, c_int, u16p, u16p, u16p, u16p, u16p, u16p, u16p, c_int, c_int, c_int,
                                c_int, c_int, c_float]
    L.orc_sigmoid_gate.argtypes = [u16p, u16p, c_size]
    L.orc_silu_mul.argtypes = [u16p, c_int, u16p, c_int, c_int]
    L.orc_rms_norm.argtypes = [u16p, u16p, u16p, c_int, c_int, c_float]
    L.orc_add_rms_norm.argtypes = [u16p, u16p, u16p, u16p, c_int, c_int, c_float]
    L.orc_rotary_tables.argtypes = [i64p, c_int, c_int, c_double, u16p, u16p]
    _lib = L
    return L


# ---------------------------------------------------------------- bf16 helpers


def bf16_to_f32(x: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(x, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round to nearest even (the C oracle's conversion)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16(x.reshape(-1), out.reshape(-1), x.size)
    return out


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_to_f32(f32_to_bf16(x))


def tf32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().orc_f32_to_tf32(x.reshape(-1), out.reshape(-1), x.size)
    return out


# ---------------------------------------------------------------- generators


def xorshift_bf16(n: int, seed: int, amp: float) -> np.ndarray:
    """kernels.rs:26-36 ``random(n, seed, amp)``: bf16 bit patterns."""
    out = np.empty(n, dtype=np.uint16)
    lib().orc_xorshift_bf16(out, n, seed, amp)
    return out


def gdn_test_inputs(t: int, h: int, hk: int, decay_scale: float, qk_amp: float, d: int = 128):
    """The inputs of kernels.rs:557-575: k ~ U(-a, a), q = bf16(0.8 k + 0.2 n),
    v ~ U(-1, 1), g = (U(-1,1) - 1) * decay_scale (float32), beta = bf16(U(-.5,.5) + .5)."""
    k = xorshift_bf16(t * hk * d, 12, qk_amp)
    n = xorshift_bf16(t * hk * d, 11, qk_amp)
    q = f32_to_bf16(np.float32(0.8) * bf16_to_f32(k) + np.float32(0.2) * bf16_to_f32(n))
    v = xorshift_bf16(t * h * d, 13, 1.0)
    g = (bf16_to_f32(xorshift_bf16(t * h, 14, 1.0)) - np.float32(1.0)) * np.float32(decay_scale)
    beta = f32_to_bf16(bf16_to_f32(xorshift_bf16(t * h, 15, 0.5)) + np.float32(0.5))
    return q, k, v, g.astype(np.float32), beta


# --------------------------------------------------------- gated delta rule


def gdn_recurrent_f64(q, k, v, g, beta, T, H, HK, d=128, scale=None, s_in=None, want_state=False):
    """kernels.rs:479-525 (float64 token-by-token). Returns out [T,H,d] f64 (and state)."""
    scale = d ** -0.5 if scale is None else scale
    out = np.empty(T * H * d, dtype=np.float64)
    s_out = np.empty(H * d * d, dtype=np.float64) if want_state else None
    lib().orc_gdn_recurrent_f64(q, k, v, np.ascontiguousarray(g, np.float32), beta, T, H, HK, d, scale,
                                None if s_in is None else np.ascontiguousarray(s_in, np.float32), out, s_out)
    out = out.reshape(T, H, d)
    return (out, s_out.reshape(H, d, d)) if want_state else out


def gdn_chunk_emul(q, k, v, g, beta, T, H, HK, scale=128 ** -0.5, s_in=None, want_state=True):
    """Emulation of cs1_gdn_prefill_x (gdn_prefill.cu). Returns (o bf16 [T,H,128], s_out f32 [H,128,128])."""
    o = np.zeros(max(T, 0) * H * 128, dtype=np.uint16)
    s_out = np.empty(H * 128 * 128, dtype=np.float32) if want_state else None
    rc = lib().orc_gdn_chunk_emul(q, k, v, np.ascontiguousarray(g, np.float32), beta, T, H, HK, scale,
                                  None if s_in is None else np.ascontiguousarray(s_in, np.float32), o, s_out)
    if rc != 0:
        raise ValueError("invalid gdn shape")
    return o.reshape(T, H, 128), (s_out.reshape(H, 128, 128) if want_state else None)


def tri_inverse_blocked(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    t = np.empty((64, 64), np.float32)
    lib().orc_tri_inverse_blocked(a.reshape(-1), t.reshape(-1))
    return t


# ---------------------------------------------------------------- attention


def attention_f64(q, k, v, ldv, T, Hq, Hk, Dh, scale, q_base=0, want_lse=False, rows=None):
    """kernels.rs:436-469 brute force in float64; out [T,Hq,Dh], lse [Hq,T].
    ``rows`` restricts the work to those query rows (others stay zero)."""
    out = np.zeros(T * Hq * Dh, np.float64)
    lse = np.zeros(Hq * T, np.float64) if want_lse else None
    r = None if rows is None else np.ascontiguousarray(rows, np.int32)
    lib().orc_attention_f64(q, k, v, ldv, T, Hq, Hk, Dh, scale, q_base, r, 0 if r is None else r.size, out, lse)
    out = out.reshape(T, Hq, Dh)
    return (out, lse.reshape(Hq, T)) if want_lse else out


def attention_emul(q, k, v, ldv, gate, T, Hq, Hk, Dh, scale, q_base=0, want_lse=False, rows=None):
    """Emulation of flash_kernel (attention.cu:84-234); out bf16 [T,Hq,Dh], lse f32 [Hq,T].
    ``rows`` restricts the work to those query rows (others stay zero; q_base is then unused)."""
    out = np.zeros(T * Hq * Dh, np.uint16)
    lse = np.zeros(Hq * T, np.float32) if want_lse else None
    if rows is not None:
        r = np.ascontiguousarray(rows, np.int32)
        assert r.size == 0 or (r.min() >= 0 and r.max() < T)
        lib().orc_attention_emul_rows(q, k, v, ldv, gate, T, Hq, Hk, Dh, scale, r, r.size, out, lse)
    else:
        lib().orc_attention_emul(q, k, v, ldv, gate, T, Hq, Hk, Dh, scale, q_base, out, lse)
    out = out.reshape(T, Hq, Dh)
    return (out, lse.reshape(Hq, T)) if want_lse else out


# --------------------------------------------------------------- elementwise


def gdn_conv(qkv, ld, w, T, key_dim, value_dim):
    q = np.empty(T * key_dim, np.uint16)
    k = np.empty(T * key_dim, np.uint16)
    v = np.empty(T * value_dim, np.uint16)
    lib().orc_gdn_conv(qkv, ld, w, q, k, v, T, key_dim, value_dim)
    return q, k, v


def gdn_gates(b, a, ld, A_log, dt_bias, T, H):
    beta = np.empty(T * H, np.uint16)
    g = np.empty(T * H, np.float32)
    lib().orc_gdn_gates(b, a, ld, A_log, dt_bias, beta, g, T, H)
    return beta, g


def gated_rms_norm(x, z, ldz, w, T, H, D=128, eps=1e-6):
    out = np.empty(T * H * D, np.uint16)
    lib().orc_gated_rms_norm(x, z, ldz, w, out, T, H, D, eps)
    return out


def attn_prep(qg, kr, ld, qw, kw, cos, sin, T, Hq, Hk, Dh, half, eps=1e-6):
    q = np.empty(T * Hq * Dh, np.uint16)
    gate = np.empty(T * Hq * Dh, np.uint16)
    k = np.empty(T * Hk * Dh, np.uint16)
    lib().orc_attn_prep(qg, kr, ld, qw, kw, cos, sin, q, gate, k, T, Hq, Hk, Dh, half, eps)
    return q, gate, k


def sigmoid_gate(x, gate):
    x = np.array(x, dtype=np.uint16, copy=True)
    lib().orc_sigmoid_gate(x, gate, x.size)
    return x


def silu_mul(gate_up, ld, T, I):
    out = np.empty(T * I, np.uint16)
    lib().orc_silu_mul(gate_up, ld, out, T, I)
    return out


def rms_norm(x, w, rows, D, eps=1e-6):
    out = np.empty(rows * D, np.uint16)
    lib().orc_rms_norm(x, w, out, rows, D, eps)
    return out


def add_rms_norm(residual, delta, w, rows, D, eps=1e-6):
    res = np.array(residual, dtype=np.uint16, copy=True)
    out = np.empty(rows * D, np.uint16)
    lib().orc_add_rms_norm(res, delta, w, out, rows, D, eps)
    return res, out


def rotary_tables(positions, half, theta):
    positions = np.ascontiguousarray(positions, np.int64)
    T = positions.size
    cs = np.empty(T * half, np.uint16)
    sn = np.empty(T * half, np.uint16)
    lib().orc_rotary_tables(positions, T, half, theta, cs, sn)
    return cs, sn
