"""ctypes wrapper of the CPU oracle (liboracle.so). TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, as the
results the GPU path is compared with or as the timed CPU baseline; the product path never does. bf16 tensors are numpy
uint16 arrays of raw bits. ``mode`` is GPU_ORDER (bit-exact mirror of the HIP kernels'
summation order) or EXACT (double accumulation, libm transcendentals).
"""
import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

GPU_ORDER = 0
EXACT = 1
ATTN_BLOCK = 64

_lib = None


def build():
    """Compiles liboracle.so from oracle.c (gcc, OpenMP)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


_u16p = ctypes.POINTER(ctypes.c_uint16)
_i32p = ctypes.POINTER(ctypes.c_int)
_c_int = ctypes.c_int
_c_float = ctypes.c_float
_c_size = ctypes.c_size_t


class OrcConfig(ctypes.Structure):
    _fields_ = [("hidden_size", _c_int), ("intermediate_size", _c_int), ("n_layers", _c_int),
                ("n_heads", _c_int), ("n_kv_heads", _c_int), ("head_dim", _c_int),
                ("vocab_size", _c_int), ("rms_norm_eps", _c_float), ("rope_theta", _c_float)]


class OrcLayer(ctypes.Structure):
    _fields_ = [(n, _u16p) for n in ("attn_norm", "wq", "wk", "wv", "q_norm", "k_norm", "wo",
                                     "mlp_norm", "w_gate", "w_up", "w_down")]


class OrcWeights(ctypes.Structure):
    _fields_ = [("embed", _u16p), ("final_norm", _u16p), ("lm_head", _u16p),
                ("layers", ctypes.POINTER(OrcLayer))]


class OrcState(ctypes.Structure):
    _fields_ = [(n, _u16p) for n in ("x", "xb", "q", "k", "v", "attn_out", "hb", "logits",
                                     "key_cache", "value_cache")] + [("max_seq", _c_int)]


def _declare(L):
    sig = {
        "orc_f32_to_bf16": (ctypes.c_uint16, [_c_float]),
        "orc_bf16_to_f32": (_c_float, [ctypes.c_uint16]),
        "orc_exp_f32": (_c_float, [_c_float]),
        "orc_exp_ref": (_c_float, [_c_float]),
        "orc_sincos_d": (None, [ctypes.c_double, ctypes.POINTER(ctypes.c_double),
                                ctypes.POINTER(ctypes.c_double)]),
        "orc_inv_freq": (_c_float, [_c_float, _c_int, _c_int]),
        "orc_silu": (_c_float, [_c_float, _c_int]),
        "orc_embedding": (None, [_u16p, _u16p, _c_int, _c_int]),
        "orc_rmsnorm": (None, [_u16p, _u16p, _u16p, _c_int, _c_int, _c_float, _c_int]),
        "orc_dot": (_c_float, [_u16p, _u16p, _c_int, _c_int]),
        "orc_gemv": (None, [_u16p, _u16p, _u16p, _c_int, _c_int, _c_int]),
        "orc_gemv_residual": (None, [_u16p, _u16p, _u16p, _c_int, _c_int, _u16p, _c_int]),
        "orc_qkv": (None, [_u16p] * 7 + [_c_int] * 4),
        "orc_gate_up": (None, [_u16p] * 4 + [_c_int, _c_int, _u16p, _u16p, _c_int]),
        "orc_swiglu": (None, [_u16p, _u16p, _u16p, _c_size, _c_int]),
        "orc_qk_norm_rope_rows": (None, [_u16p] * 7 + [_i32p] + [_c_int] * 4 +
                                  [_c_float, _c_float, _u16p, _u16p, _c_int]),
        "orc_attention": (None, [_u16p] * 4 + [_c_int] * 4 + [_c_float, _c_int]),
        "orc_argmax": (_c_int, [_u16p, _c_int]),
        "orc_sample": (_c_int, [_u16p, _c_int, ctypes.c_float, ctypes.c_float]),
        "orc_forward": (_c_int, [ctypes.POINTER(OrcConfig), ctypes.POINTER(OrcWeights),
                                 ctypes.POINTER(OrcState), _c_int, _c_int, _c_int]),
        "orc_weight_bytes_per_step": (_c_size, [ctypes.POINTER(OrcConfig)]),
        "orc_kv_bytes_per_position": (_c_size, [ctypes.POINTER(OrcConfig)]),
        "orc_num_threads": (_c_int, []),
        "orc_selfcheck_exp": (ctypes.c_int64, [_c_float, _c_float, ctypes.POINTER(ctypes.c_int64),
                                               ctypes.POINTER(ctypes.c_int64)]),
        "orc_selfcheck_sincos": (ctypes.c_int64, [_c_float, _c_int, _c_int,
                                                  ctypes.POINTER(ctypes.c_int64)]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def _p(a):
    if a is None:
        return None
    assert a.dtype == np.uint16 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_u16p)


# ---- bf16 helpers (numpy, vectorized; checked against orc_f32_to_bf16 in the tests) ----

def f32_to_bf16(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- op wrappers (all return new arrays; in-place ops take copies) ----

def exp_f32(x):
    return lib().orc_exp_f32(float(x))


def sincos(x):
    s, c = ctypes.c_double(), ctypes.c_double()
    lib().orc_sincos_d(float(x), ctypes.byref(s), ctypes.byref(c))
    return s.value, c.value


def inv_freq(theta, head_dim):
    return np.array([lib().orc_inv_freq(theta, j, head_dim) for j in range(head_dim // 2)],
                    dtype=np.float32)


def embedding(table, token, hidden):
    out = np.empty(hidden, np.uint16)
    lib().orc_embedding(_p(out), _p(table), int(token), int(hidden))
    return out


def rmsnorm(x, w, eps, mode=GPU_ORDER):
    x = np.ascontiguousarray(x, dtype=np.uint16)
    rows, dim = (1, x.shape[0]) if x.ndim == 1 else x.shape
    out = np.empty_like(x)
    lib().orc_rmsnorm(_p(out), _p(x), _p(w), rows, dim, eps, mode)
    return out


def gemv(w, x, mode=GPU_ORDER):
    rows, cols = w.shape
    out = np.empty(rows, np.uint16)
    lib().orc_gemv(_p(out), _p(w), _p(x), rows, cols, mode)
    return out


def gemv_residual(x, w, inp, mode=GPU_ORDER, with_tap=False):
    rows, cols = w.shape
    x = x.copy()
    tap = np.empty(rows, np.uint16) if with_tap else None
    lib().orc_gemv_residual(_p(x), _p(w), _p(inp), rows, cols, _p(tap), mode)
    return (x, tap) if with_tap else x


def qkv(wq, wk, wv, x, mode=GPU_ORDER):
    q = np.empty(wq.shape[0], np.uint16)
    k = np.empty(wk.shape[0], np.uint16)
    v = np.empty(wv.shape[0], np.uint16)
    lib().orc_qkv(_p(q), _p(k), _p(v), _p(wq), _p(wk), _p(wv), _p(x), wq.shape[0], wk.shape[0],
                  wq.shape[1], mode)
    return q, k, v


def gate_up(wg, wu, x, mode=GPU_ORDER, with_taps=False):
    rows, cols = wg.shape
    act = np.empty(rows, np.uint16)
    gt = np.empty(rows, np.uint16) if with_taps else None
    ut = np.empty(rows, np.uint16) if with_taps else None
    lib().orc_gate_up(_p(act), _p(wg), _p(wu), _p(x), rows, cols, _p(gt), _p(ut), mode)
    return (act, gt, ut) if with_taps else act


def swiglu(gate, up, mode=GPU_ORDER):
    gate = np.ascontiguousarray(gate, dtype=np.uint16)
    up = np.ascontiguousarray(up, dtype=np.uint16)
    act = np.empty_like(gate)
    lib().orc_swiglu(_p(act), _p(gate), _p(up), gate.size, mode)
    return act


def qk_norm_rope_rows(q, k, v, qn, kn, key_cache, value_cache, positions, n_heads, n_kv_heads,
                      head_dim, eps, theta, mode=GPU_ORDER, with_taps=False):
    """Returns (q', k', key_cache', value_cache'[, q_tap, k_tap]); inputs are not modified."""
    q = np.ascontiguousarray(q, dtype=np.uint16).copy()
    k = np.ascontiguousarray(k, dtype=np.uint16).copy()
    v = np.ascontiguousarray(v, dtype=np.uint16)
    kc = key_cache.copy()
    vc = value_cache.copy()
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    qt = np.empty_like(q) if with_taps else None
    kt = np.empty_like(k) if with_taps else None
    lib().orc_qk_norm_rope_rows(_p(q), _p(k), _p(v), _p(qn), _p(kn), _p(kc), _p(vc),
                                pos.ctypes.data_as(_i32p), pos.size, n_heads, n_kv_heads,
                                head_dim, eps, theta, _p(qt), _p(kt), mode)
    return (q, k, kc, vc, qt, kt) if with_taps else (q, k, kc, vc)


def attention(q, key_cache, value_cache, n_heads, n_kv_heads, head_dim, pos, scale,
              mode=GPU_ORDER):
    out = np.empty(n_heads * head_dim, np.uint16)
    lib().orc_attention(_p(out), _p(q), _p(key_cache), _p(value_cache), n_heads, n_kv_heads,
                        head_dim, pos, scale, mode)
    return out


def argmax(x):
    return lib().orc_argmax(_p(np.ascontiguousarray(x, dtype=np.uint16)), x.size)


def sample(x, inv_temp, u):
    x = np.ascontiguousarray(x, dtype=np.uint16)
    return lib().orc_sample(_p(x), x.size, inv_temp, u)


def selfcheck_exp(lo, hi):
    """(worst ulp distance, inputs checked, inputs differing) of exp_f32 vs libm over [lo, hi]."""
    n, d = ctypes.c_int64(), ctypes.c_int64()
    worst = lib().orc_selfcheck_exp(lo, hi, ctypes.byref(n), ctypes.byref(d))
    return worst, n.value, d.value


def selfcheck_sincos(theta, head_dim, n_pos):
    """(differing fp32 results, results checked) of the double sincos vs libm at RoPE angles."""
    n = ctypes.c_int64()
    diff = lib().orc_selfcheck_sincos(theta, head_dim, n_pos, ctypes.byref(n))
    return diff, n.value


def num_threads():
    return lib().orc_num_threads()


class Model:
    """Host-memory Qwen3 decode state for orc_forward. `weights` is a dict of uint16 arrays named
    as the safetensors tensors (model.embed_tokens.weight, model.layers.N.*, model.norm.weight,
    optional lm_head.weight)."""

    LAYER_KEYS = {"attn_norm": "input_layernorm.weight", "wq": "self_attn.q_proj.weight",
                  "wk": "self_attn.k_proj.weight", "wv": "self_attn.v_proj.weight",
                  "q_norm": "self_attn.q_norm.weight", "k_norm": "self_attn.k_norm.weight",
                  "wo": "self_attn.o_proj.weight", "mlp_norm": "post_attention_layernorm.weight",
                  "w_gate": "mlp.gate_proj.weight", "w_up": "mlp.up_proj.weight",
                  "w_down": "mlp.down_proj.weight"}

    def __init__(self, cfg, weights, max_seq):
        self.cfg = OrcConfig(cfg["hidden_size"], cfg["intermediate_size"], cfg["n_layers"],
                             cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"],
                             cfg["vocab_size"], cfg["rms_norm_eps"], cfg["rope_theta"])
        self._keep = weights
        nl = cfg["n_layers"]
        self._layers = (OrcLayer * nl)()
        for i in range(nl):
            for field, key in self.LAYER_KEYS.items():
                setattr(self._layers[i], field, _p(weights[f"model.layers.{i}.{key}"]))
        lm = weights.get("lm_head.weight", weights["model.embed_tokens.weight"])
        self.weights = OrcWeights(_p(weights["model.embed_tokens.weight"]),
                                  _p(weights["model.norm.weight"]), _p(lm), self._layers)
        H, D = cfg["hidden_size"], cfg["head_dim"]
        kv_dim = cfg["n_kv_heads"] * D
        self.bufs = {
            "x": np.zeros(H, np.uint16), "xb": np.zeros(H, np.uint16),
            "q": np.zeros(cfg["n_heads"] * D, np.uint16), "k": np.zeros(kv_dim, np.uint16),
            "v": np.zeros(kv_dim, np.uint16), "attn_out": np.zeros(cfg["n_heads"] * D, np.uint16),
            "hb": np.zeros(cfg["intermediate_size"], np.uint16),
            "logits": np.zeros(cfg["vocab_size"], np.uint16),
            "key_cache": np.zeros(nl * max_seq * kv_dim, np.uint16),
            "value_cache": np.zeros(nl * max_seq * kv_dim, np.uint16),
        }
        self.state = OrcState(*[_p(self.bufs[n]) for n in
                                ("x", "xb", "q", "k", "v", "attn_out", "hb", "logits",
                                 "key_cache", "value_cache")], max_seq)

    def forward(self, token, pos, mode=GPU_ORDER):
        """One decode position; returns the greedy next token."""
        return lib().orc_forward(ctypes.byref(self.cfg), ctypes.byref(self.weights),
                                 ctypes.byref(self.state), int(token), int(pos), mode)

    @property
    def logits(self):
        return self.bufs["logits"]

    def weight_bytes_per_step(self):
        return lib().orc_weight_bytes_per_step(ctypes.byref(self.cfg))

    def kv_bytes_per_position(self):
        return lib().orc_kv_bytes_per_position(ctypes.byref(self.cfg))
