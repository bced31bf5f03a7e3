"""Model, run state and decode-step bindings (include/llm_amd/forward.h, which replaces the
reference's src/model.cuh and src/forward.cuh).

``Decoder`` owns a Config, device Weights (seeded synthetic or loaded from safetensors) and a
RunState, and exposes the reference's step API: ``forward(token, pos)``, ``sample_argmax()``,
``capture_graph()``, plus ``generate_greedy`` (the whole greedy loop on the device).
"""
import ctypes

from . import LlmError, check, lib

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t

MAX_SHARDS = 8
MAX_EOS = 8


class Config(ctypes.Structure):
    _fields_ = [("hidden_size", _i), ("intermediate_size", _i), ("n_layers", _i),
                ("n_heads", _i), ("n_kv_heads", _i), ("head_dim", _i), ("vocab_size", _i),
                ("max_seq_len", _i), ("rms_norm_eps", _f), ("rope_theta", _f),
                ("tie_word_embeddings", _i), ("eos_ids", _i * MAX_EOS), ("n_eos", _i)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_ if k != "eos_ids"}


class LayerWeights(ctypes.Structure):
    _fields_ = [(n, _vp) for n in ("attn_norm", "wq", "wk", "wv", "q_norm", "k_norm", "wo",
                                   "mlp_norm", "w_gate", "w_up", "w_down")]


class TensorRef(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 96), ("data", _vp), ("numel", _sz)]


class Weights(ctypes.Structure):
    _fields_ = [("embed", _vp), ("layers", ctypes.POINTER(LayerWeights)), ("final_norm", _vp),
                ("lm_head", _vp), ("tensors", ctypes.POINTER(TensorRef)), ("n_tensors", _i),
                ("gpu_buffers", _vp * MAX_SHARDS), ("n_buffers", _i), ("gpu_bytes", _sz)]


class RunState(ctypes.Structure):
    _fields_ = [("x", _vp), ("xb", _vp), ("q", _vp), ("k", _vp), ("v", _vp), ("attn_out", _vp),
                ("att", _vp), ("key_cache", _vp), ("value_cache", _vp), ("max_seq", _i),
                ("hb", _vp), ("tap1", _vp), ("tap2", _vp), ("logits", _vp),
                ("next_token", _vp), ("pos", _vp), ("stream", _vp), ("graph", _vp),
                ("argmax_partials", _vp), ("token_out", _vp), ("token_capacity", _i),
                ("pos_base", _vp), ("error_flag", _vp), ("loop_graph", _vp), ("step_mode", _i),
                ("persistent", _i), ("step_ws", _vp), ("layers_dev", _vp), ("step_grid", _i),
                ("next_token_valid", _i), ("step_trace", ctypes.POINTER(ctypes.c_longlong)),
                ("attn_mode", _i), ("attn_one_pass_ws", _vp),
                ("rope_table", ctypes.POINTER(ctypes.c_float)), ("step_switch_pos", _i),
                ("step_split_blocks", _i)]


STEP_MODES = {"auto": 0, "graph": 1, "persistent": 2}
ATTN_MODES = {"auto": 0, "separate": 1, "in_scores": 2, "one_pass": 3}


_PC, _PW, _PS = ctypes.POINTER(Config), ctypes.POINTER(Weights), ctypes.POINTER(RunState)

_SIGS = {
    "load_config": (None, [ctypes.c_char_p, _PC]),
    "load_weights": (None, [ctypes.c_char_p, _PC, _PW]),
    "free_weights": (None, [_PW]),
    "print_weight_checksums": (None, [_PW]),
    "alloc_run_state": (None, [_PS, _PC]),
    "alloc_run_state_seq": (None, [_PS, _PC, _i]),
    "free_run_state": (None, [_PS]),
    "capture_graph": (None, [_PC, _PW, _PS]),
    "forward": (None, [_PC, _PW, _PS, _i, _i]),
    "sample_argmax": (_i, [_PC, _PS]),
    "sample_temperature": (_i, [_PC, _PS, _f, _f]),
    "weight_bytes_per_step": (_sz, [_PC]),
    "kv_bytes_per_position": (_sz, [_PC]),
    "synth_weights": (None, [_PC, _PW, ctypes.c_uint64, _f, _f]),
    "synth_fill": (None, [_vp, _sz, ctypes.c_uint64, ctypes.c_uint64, _f, _f, _vp]),
    "generate_greedy": (_i, [_PC, _PW, _PS, _i, _i, _i, ctypes.POINTER(_i)]),
}


def _declare(L):
    for name, (res, args) in _SIGS.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


# Qwen3 shapes of the benchmark configurations (hidden, intermediate, layers, q/kv heads,
# head_dim 128, vocab 151936, rope theta 1e6, eps 1e-6, tied embeddings).
QWEN3 = {
    "0.6B": dict(hidden_size=1024, intermediate_size=3072, n_layers=28, n_heads=16, n_kv_heads=8),
    "1.7B": dict(hidden_size=2048, intermediate_size=6144, n_layers=28, n_heads=16, n_kv_heads=8),
    "4B": dict(hidden_size=2560, intermediate_size=9728, n_layers=36, n_heads=32, n_kv_heads=8),
}


def make_config(hidden_size, intermediate_size, n_layers, n_heads, n_kv_heads, head_dim=128,
                vocab_size=151936, max_seq_len=4096, rms_norm_eps=1e-6, rope_theta=1e6,
                tie_word_embeddings=1, eos_ids=(151645, 151643)):
    cfg = Config()
    cfg.hidden_size = hidden_size
    cfg.intermediate_size = intermediate_size
    cfg.n_layers = n_layers
    cfg.n_heads = n_heads
    cfg.n_kv_heads = n_kv_heads
    cfg.head_dim = head_dim
    cfg.vocab_size = vocab_size
    cfg.max_seq_len = max_seq_len
    cfg.rms_norm_eps = rms_norm_eps
    cfg.rope_theta = rope_theta
    cfg.tie_word_embeddings = tie_word_embeddings
    for i, e in enumerate(eos_ids[:MAX_EOS]):
        cfg.eos_ids[i] = e
    cfg.n_eos = min(len(eos_ids), MAX_EOS)
    return cfg


def qwen3_config(size, **overrides):
    args = dict(QWEN3[size])
    args.update(overrides)
    return make_config(**args)


def load_config(model_dir):
    cfg = Config()
    lib().load_config(str(model_dir).encode(), ctypes.byref(cfg))
    check()
    return cfg


_hip_rt = None


def _hip():
    """The HIP runtime the library is bound to (already loaded by torch; same SONAME)."""
    global _hip_rt
    if _hip_rt is None:
        lib()
        _hip_rt = ctypes.CDLL("libamdhip64.so.7")
        _hip_rt.hipMemcpy.restype = _i
        _hip_rt.hipMemcpy.argtypes = [_vp, _vp, _sz, _i]
        _hip_rt.hipDeviceSynchronize.restype = _i
    return _hip_rt


def copy_to_host(ptr, nbytes, out=None):
    """Synchronous device-to-host copy of nbytes at device address ptr into a numpy uint8 array
    (or into `out`, a writable contiguous numpy array of nbytes)."""
    import numpy as np
    if out is None:
        out = np.empty(nbytes, np.uint8)
    rt = _hip()
    rc = rt.hipMemcpy(out.ctypes.data, ptr, nbytes, 2)  # hipMemcpyDeviceToHost
    if rc != 0:
        raise LlmError(f"hipMemcpy device-to-host failed ({rc})")
    return out


def copy_to_device(ptr, arr, capacity):
    """Synchronous host-to-device copy of a contiguous numpy array to device address ptr, whose
    allocation holds `capacity` bytes (a larger array is refused before anything is copied)."""
    import numpy as np
    arr = np.ascontiguousarray(arr)
    if arr.nbytes > capacity:
        raise LlmError(f"copy_to_device: {arr.nbytes} bytes for a {capacity}-byte destination")
    rt = _hip()
    rc = rt.hipMemcpy(ptr, arr.ctypes.data, arr.nbytes, 1)  # hipMemcpyHostToDevice
    if rc != 0:
        raise LlmError(f"hipMemcpy host-to-device failed ({rc})")


def weight_bytes_per_step(cfg):
    return lib().weight_bytes_per_step(ctypes.byref(cfg))


def kv_bytes_per_position(cfg):
    return lib().kv_bytes_per_position(ctypes.byref(cfg))


class Decoder:
    """Config + device weights + run state, with the reference's step API.

    weights: ("synth", seed, std, gamma_std) for seeded random init, or a model directory.
    """

    def __init__(self, cfg, weights=("synth", 0, 0.02, 0.1), max_seq=None, mode="auto"):
        L = lib()
        self.cfg = cfg
        self.mode = mode
        self.w = Weights()
        self.s = RunState()
        self._w_ok = self._s_ok = False
        if isinstance(weights, tuple) and weights[0] == "synth":
            _, seed, std, gamma_std = weights
            L.synth_weights(ctypes.byref(cfg), ctypes.byref(self.w), seed, std, gamma_std)
        else:
            L.load_weights(str(weights).encode(), ctypes.byref(cfg), ctypes.byref(self.w))
        check()
        self._w_ok = True
        L.alloc_run_state_seq(ctypes.byref(self.s), ctypes.byref(cfg),
                              max_seq if max_seq else cfg.max_seq_len)
        check()
        self._s_ok = True

    def close(self):
        L = lib()
        if self._s_ok:
            L.free_run_state(ctypes.byref(self.s))
            self._s_ok = False
        if self._w_ok:
            L.free_weights(ctypes.byref(self.w))
            self._w_ok = False
        check()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self):
        return self.s.stream

    def capture_graph(self, mode=None):
        """Prepares the replayed step: "auto" (the persistent step kernel below its switch
        position where the shapes have a specialisation, the hipGraph of the per-layer kernels
        from there on), "persistent" (the kernel at every position) or "graph"."""
        self.s.step_mode = STEP_MODES[mode or self.mode]
        lib().capture_graph(ctypes.byref(self.cfg), ctypes.byref(self.w), ctypes.byref(self.s))
        check()

    @property
    def persistent(self):
        """The persistent step kernel is prepared (it runs the positions below
        `s.step_switch_pos`)."""
        return bool(self.s.persistent)

    def kernel_tokens(self, pos, n):
        """How many of n tokens decoded from `pos` run in the persistent step kernel (one
        launch); the others run one hipGraph replay each."""
        if not self.s.persistent:
            return 0
        return max(0, min(n, self.s.step_switch_pos - pos))

    def step_kind(self, pos, n):
        """Which step decodes n tokens from `pos`: the persistent kernel (its attention one
        workgroup per query head, or split over (kv head, block) items from
        `s.step_split_blocks` blocks of history on) and/or the hipGraph."""
        k = self.kernel_tokens(pos, n)
        if k == 0:
            return "hipGraph of per-layer kernels"
        split_from = (self.s.step_split_blocks - 1) * 64
        heads = 0 if pos >= split_from else min(k, split_from - pos)
        form = ("one workgroup per query head" if heads == k else "split attention" if heads == 0
                else f"one workgroup per query head for {heads} tokens, then split attention")
        kind = f"persistent step kernel, {form}"
        return kind if k == n else f"{kind}, for {k} tokens, then hipGraph of per-layer kernels"

    def forward(self, token, pos):
        lib().forward(ctypes.byref(self.cfg), ctypes.byref(self.w), ctypes.byref(self.s), token,
                      pos)
        check()

    def sample_argmax(self):
        t = lib().sample_argmax(ctypes.byref(self.cfg), ctypes.byref(self.s))
        check()
        return t

    def sample_temperature(self, temperature, coin):
        """A token drawn from softmax(logits / temperature) at coin in [0, 1)
        (src/forward.cu:238-251)."""
        t = lib().sample_temperature(ctypes.byref(self.cfg), ctypes.byref(self.s), temperature,
                                     coin)
        check()
        return t

    def generate_greedy(self, token, pos, n_steps):
        out = (_i * n_steps)()
        rc = lib().generate_greedy(ctypes.byref(self.cfg), ctypes.byref(self.w),
                                   ctypes.byref(self.s), token, pos, n_steps, out)
        check()
        if rc != 0:
            raise LlmError("generate_greedy: a token left the vocabulary")
        return list(out)

    def tensors(self):
        """{name: (device pointer, numel)} of every weight tensor."""
        return {self.w.tensors[i].name.decode(): (self.w.tensors[i].data, self.w.tensors[i].numel)
                for i in range(self.w.n_tensors)}

    def host_tensor(self, name):
        """A weight tensor copied to the host as numpy uint16 (raw bf16 bits)."""
        import numpy as np
        ptr, numel = self.tensors()[name]
        out = np.empty(numel, np.uint16)
        copy_to_host(ptr, numel * 2, out)
        return out

    def set_weights(self, weights):
        """Overwrites device weight tensors with host arrays {safetensors name: uint16 bf16 bits}
        (every name must exist, with the tensor's element count)."""
        import numpy as np
        t = self.tensors()
        for name, arr in weights.items():
            if name not in t:
                raise LlmError(f"no weight tensor {name}")
            ptr, numel = t[name]
            a = np.ascontiguousarray(arr, dtype=np.uint16).reshape(-1)
            if a.size != numel:
                raise LlmError(f"{name}: {a.size} elements for a tensor of {numel}")
            copy_to_device(ptr, a, numel * 2)

    def host_weights(self):
        """{safetensors name: uint16 numpy array} of every weight (2-D for matrices)."""
        c = self.cfg
        shapes = {"model.embed_tokens.weight": (c.vocab_size, c.hidden_size)}
        q_dim, kv_dim = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim
        for l in range(c.n_layers):
            p = f"model.layers.{l}."
            shapes[p + "self_attn.q_proj.weight"] = (q_dim, c.hidden_size)
            shapes[p + "self_attn.k_proj.weight"] = (kv_dim, c.hidden_size)
            shapes[p + "self_attn.v_proj.weight"] = (kv_dim, c.hidden_size)
            shapes[p + "self_attn.o_proj.weight"] = (c.hidden_size, q_dim)
            shapes[p + "mlp.gate_proj.weight"] = (c.intermediate_size, c.hidden_size)
            shapes[p + "mlp.up_proj.weight"] = (c.intermediate_size, c.hidden_size)
            shapes[p + "mlp.down_proj.weight"] = (c.hidden_size, c.intermediate_size)
        out = {}
        for name in self.tensors():
            t = self.host_tensor(name)
            out[name] = t.reshape(shapes[name]) if name in shapes else t
        return out

    def logits(self):
        import numpy as np
        out = np.empty(self.cfg.vocab_size, np.uint16)
        copy_to_host(self.s.logits, out.nbytes, out)
        return out

    def kv_cache(self):
        """(key_cache, value_cache) as uint16 [n_layers, max_seq, kv_dim]."""
        import numpy as np
        c = self.cfg
        shape = (c.n_layers, self.s.max_seq, c.n_kv_heads * c.head_dim)
        k = np.empty(shape, np.uint16)
        v = np.empty(shape, np.uint16)
        copy_to_host(self.s.key_cache, k.nbytes, k)
        copy_to_host(self.s.value_cache, v.nbytes, v)
        return k, v

    def set_kv_cache(self, k, v):
        """Overwrites the device KV caches with uint16 arrays [n_layers, max_seq, kv_dim] (the
        run state's max_seq; any other shape or dtype is refused)."""
        import numpy as np
        c = self.cfg
        shape = (c.n_layers, self.s.max_seq, c.n_kv_heads * c.head_dim)
        for name, a in (("k", k), ("v", v)):
            if a.dtype != np.uint16 or tuple(a.shape) != shape:
                raise LlmError(f"set_kv_cache: {name} is {a.dtype}{list(a.shape)}, the cache is "
                               f"uint16{list(shape)}")
        nbytes = int(np.prod(shape)) * 2
        copy_to_device(self.s.key_cache, k, nbytes)
        copy_to_device(self.s.value_cache, v, nbytes)

    def weight_bytes_per_step(self):
        return weight_bytes_per_step(self.cfg)

    def kv_bytes_per_position(self):
        return kv_bytes_per_position(self.cfg)
