"""ctypes binding of libqwen3_5_model.so (include/qwen3_5_model.h): the native host runner of
the Qwen3.5-style hybrid decoder prefill over the cs1_* operations.

Mirrors the reference executor's text path (src/models/qwen3_5/native/src/model.rs:763-826,
1119-1318) and the cua_s1 decision head (src/models/cua_s1/native/src/executor.rs:61-78).
"""
import ctypes
import os
from dataclasses import dataclass, fields

import numpy as np

from . import hip

_HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT_LIB = os.path.join(os.path.dirname(_HERE), "libqwen3_5_model.so")

EMBED, FINAL_NORM, INPUT_NORM, POST_NORM = 0, 1, 2, 3
GDN_IN, GDN_CONV, GDN_A_LOG, GDN_DT_BIAS, GDN_NORM, GDN_OUT = 4, 5, 6, 7, 8, 9
ATTN_QKV, ATTN_Q_NORM, ATTN_K_NORM, ATTN_O = 10, 11, 12, 13
MLP_GATE_UP, MLP_DOWN, LM_HEAD = 14, 15, 16

SYMBOLS = ["q35m_create", "q35m_destroy", "q35m_set_graph", "q35m_set_gemm_tuning", "q35m_forward", "q35m_decide", "q35m_capture",
           "q35m_score", "q35m_logprobs", "q35m_tensor", "q35m_stream", "q35m_letter_logits"]


class _Config(ctypes.Structure):
    _fields_ = [("layers", ctypes.c_int), ("hidden", ctypes.c_int), ("intermediate", ctypes.c_int),
                ("vocab", ctypes.c_int), ("heads", ctypes.c_int), ("kv_heads", ctypes.c_int),
                ("head_dim", ctypes.c_int), ("rotary_half", ctypes.c_int), ("rope_theta", ctypes.c_double),
                ("lin_k_heads", ctypes.c_int), ("lin_v_heads", ctypes.c_int), ("lin_k_dim", ctypes.c_int),
                ("lin_v_dim", ctypes.c_int), ("full_attention_interval", ctypes.c_int), ("eps", ctypes.c_float),
                ("lm_head", ctypes.c_int)]


@dataclass(frozen=True)
class Config:
    layers: int
    hidden: int
    intermediate: int
    vocab: int
    heads: int
    kv_heads: int
    head_dim: int = 256
    rotary_half: int = 32
    rope_theta: float = 1e7
    lin_k_heads: int = 16
    lin_v_heads: int = 32
    lin_k_dim: int = 128
    lin_v_dim: int = 128
    full_attention_interval: int = 4
    eps: float = 1e-6
    lm_head: int = 0

    def is_full(self, layer: int) -> bool:
        return (layer + 1) % self.full_attention_interval == 0


# Config 3: the 4B-class hybrid decoder (32 layers, 3:1 GDN:attention).
CFG3_4B = Config(layers=32, hidden=2560, intermediate=9728, vocab=151936, heads=16, kv_heads=4)
# Config 4: the 27B-class hybrid decoder (64 layers, 3:1), with the remaining sizes
# (SwiGLU 17408, vocabulary 248320, untied LM head) from the reference's test config
# tests/qwen3_5/data/config.json.
CFG4_27B = Config(layers=64, hidden=5120, intermediate=17408, vocab=248320, heads=24, kv_heads=4, lin_k_heads=16,
                  lin_v_heads=48, lm_head=1)

_LIB = None


def load(path: str = None) -> ctypes.CDLL:
    """Load the runner (after the op library it links against)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    hip.load()
    path = path or os.environ.get("CS1_MODEL_LIB", DEFAULT_LIB)
    if not os.path.exists(path):
        raise hip.HipError(f"{path} is missing: build it with `make -C system1-omni_amd`")
    lib = ctypes.CDLL(path)
    vp, i32p, f32p = ctypes.c_void_p, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_float)
    lib.q35m_create.argtypes = [ctypes.POINTER(_Config), ctypes.c_uint64, ctypes.c_int, ctypes.POINTER(vp)]
    lib.q35m_destroy.argtypes = [vp]
    lib.q35m_destroy.restype = None
    lib.q35m_set_graph.argtypes = [vp, ctypes.c_int]
    lib.q35m_set_gemm_tuning.argtypes = [vp, ctypes.c_int]
    lib.q35m_forward.argtypes = [vp, i32p, ctypes.c_int, f32p]
    lib.q35m_decide.argtypes = [vp, i32p, ctypes.c_int, i32p, ctypes.c_int, f32p]
    lib.q35m_letter_logits.argtypes = [f32p, f32p, ctypes.c_int, ctypes.c_int, f32p]
    lib.q35m_capture.argtypes = [vp, i32p, ctypes.c_int]
    lib.q35m_score.argtypes = [vp, i32p, i32p, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    lib.q35m_logprobs.argtypes = [vp, i32p, ctypes.c_int, f32p]
    lib.q35m_tensor.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.POINTER(vp), ctypes.POINTER(ctypes.c_size_t)]
    lib.q35m_stream.argtypes = [vp]
    lib.q35m_stream.restype = vp
    _LIB = lib
    return lib


def letter_logits(letters: np.ndarray, last: np.ndarray, n: int) -> np.ndarray:
    """The decision head alone (q35m_letter_logits; executor.rs:61-78): float32 logits of the
    first n rows of `letters` [*, H] against `last` [H], float64 accumulation. Raises
    hip.HipError if a logit is not finite."""
    lib = load()
    letters = np.ascontiguousarray(letters, np.float32).reshape(-1)
    last = np.ascontiguousarray(last, np.float32)
    out = np.zeros(n, np.float32)
    f32p = ctypes.POINTER(ctypes.c_float)
    hip.check(lib.q35m_letter_logits(letters.ctypes.data_as(f32p), last.ctypes.data_as(f32p), last.size, n,
                                     out.ctypes.data_as(f32p)), "q35m_letter_logits")
    return out


def _cfg(c: Config) -> _Config:
    return _Config(**{f.name: getattr(c, f.name) for f in fields(Config)})


class Model:
    """A randomly initialised model on the current device."""

    def __init__(self, cfg: Config, seed: int = 0, max_tokens: int = 4096):
        self.lib = load()
        self.cfg = cfg
        h = ctypes.c_void_p()
        hip.check(self.lib.q35m_create(ctypes.byref(_cfg(cfg)), seed, max_tokens, ctypes.byref(h)), "q35m_create")
        self.handle = h.value

    def close(self):
        if getattr(self, "handle", None):
            self.lib.q35m_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def set_graph(self, enabled: bool):
        hip.check(self.lib.q35m_set_graph(self.handle, int(enabled)), "q35m_set_graph")

    def set_gemm_tuning(self, enabled: bool):
        hip.check(self.lib.q35m_set_gemm_tuning(self.handle, int(enabled)), "q35m_set_gemm_tuning")

    def forward(self, ids) -> np.ndarray:
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty(self.cfg.hidden, np.float32)
        hip.check(self.lib.q35m_forward(self.handle, ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), len(ids),
                                        out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))), "q35m_forward")
        return out

    def decide(self, ids, labels) -> np.ndarray:
        ids = np.ascontiguousarray(ids, np.int32)
        labels = np.ascontiguousarray(labels, np.int32)
        out = np.empty(len(labels), np.float32)
        hip.check(self.lib.q35m_decide(self.handle, ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), len(ids),
                                       labels.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), len(labels),
                                       out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))), "q35m_decide")
        return out

    def capture(self, ids):
        """Run a prompt prefix (length a multiple of 64) and keep its per-layer state."""
        ids = np.ascontiguousarray(ids, np.int32)
        hip.check(self.lib.q35m_capture(self.handle, ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), len(ids)),
                  "q35m_capture")

    def score(self, candidates) -> np.ndarray:
        """Summed token log-probabilities of each candidate continuing the captured prefix."""
        ids = np.ascontiguousarray(np.concatenate([np.asarray(c) for c in candidates]), np.int32)
        lens = np.ascontiguousarray([len(c) for c in candidates], np.int32)
        out = np.empty(len(candidates), np.float64)
        hip.check(self.lib.q35m_score(self.handle, ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                      lens.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), len(candidates),
                                      out.ctypes.data_as(ctypes.POINTER(ctypes.c_double))), "q35m_score")
        return out

    def logprobs(self, ids) -> np.ndarray:
        """log p(ids[t + 1] | ids[:t + 1]) for t < len(ids) - 1, from one full forward."""
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty(len(ids) - 1, np.float32)
        hip.check(self.lib.q35m_logprobs(self.handle, ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), len(ids),
                                         out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))), "q35m_logprobs")
        return out

    def tensor(self, which: int, layer: int = 0) -> np.ndarray:
        """A weight tensor downloaded as raw bf16 bits."""
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        hip.check(self.lib.q35m_tensor(self.handle, layer, which, ctypes.byref(p), ctypes.byref(n)), "q35m_tensor")
        out = np.empty(n.value, np.uint16)
        hip.check(hip.api().cs1_download(out.ctypes.data, p.value, out.nbytes, self.stream()), "download")
        return out

    def stream(self):
        return self.lib.q35m_stream(self.handle)
