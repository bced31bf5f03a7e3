"""Python host side of the MI355X (gfx950) decode kernels.

Thin ctypes bindings of libllm_amd.so, whose C ABI (include/llm_amd/kernels.h, forward.h)
replaces the reference's src/kernels.cuh and src/forward.cuh launchers and step API
(William-Lamer/llm-inference). The wrappers take torch tensors for device memory and a torch
stream (or the current one); torch is only the allocator and stream provider. Every call goes to
the HIP kernels: there is no CPU path, and a missing library raises.

Errors the reference reports with exit(EXIT_FAILURE) raise LlmError here (the library is
switched to recording mode on load).
"""
import ctypes
import os
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libllm_amd.so"

__all__ = [
    "LlmError", "lib", "embedding_forward", "rmsnorm_forward", "gemv_forward",
    "gemv_residual_forward", "qkv_forward", "gate_up_forward", "qk_norm_rope_forward",
    "qk_norm_rope_rows", "attention_forward", "argmax_forward", "swiglu_forward",
    "attention_workspace_floats", "rmsnorm_qkv_forward", "rmsnorm_gemv_forward",
    "rmsnorm_gate_up_forward", "hbm_stream_probe", "hbm_read_peak_probe", "hbm_copy_peak_probe", "sample_forward",
    "qk_norm_rope_attention_forward", "dump_open",
    "dump_close", "dump_enabled", "attention_forward_noalloc", "EXPORTED_SYMBOLS",
    "qk_norm_rope_attention_one_pass", "attention_one_pass_bytes", "attention_one_pass_supported",
]

# Every symbol include/llm_amd/*.h declares.
EXPORTED_SYMBOLS = [
    "embedding_forward", "rmsnorm_forward", "gemv_forward", "gemv_residual_forward",
    "qkv_forward", "gate_up_forward", "qk_norm_rope_forward", "attention_forward",
    "argmax_forward", "qk_norm_rope_rows", "swiglu_forward", "attention_workspace_floats",
    "rmsnorm_qkv_forward", "rmsnorm_gemv_forward", "rmsnorm_gate_up_forward",
    "hbm_stream_probe", "hbm_read_peak_probe", "hbm_copy_peak_probe", "sample_forward", "sample_temperature",
    "dump_open", "dump_close",
    "dump_enabled", "dump_bf16", "dump_f32", "llm_set_exit_on_error", "llm_last_error", "llm_clear_error",
    "load_config", "load_weights", "free_weights", "print_weight_checksums",
    "alloc_run_state", "free_run_state", "capture_graph", "forward", "sample_argmax",
    "weight_bytes_per_step", "kv_bytes_per_position", "alloc_run_state_seq", "synth_weights",
    "synth_fill", "generate_greedy", "attention_forward_noalloc",
    "qk_norm_rope_attention_forward", "qk_norm_rope_attention_one_pass",
    "attention_one_pass_bytes", "attention_one_pass_supported",
]


class LlmError(RuntimeError):
    """A shape, alignment or HIP error reported by libllm_amd."""


_lib = None

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t

_SIGS = {
    "embedding_forward": (None, [_vp, _vp, _vp, _i, _vp]),
    "rmsnorm_forward": (None, [_vp, _vp, _vp, _i, _i, _f, _vp]),
    "gemv_forward": (None, [_vp, _vp, _vp, _i, _i, _vp]),
    "gemv_residual_forward": (None, [_vp, _vp, _vp, _i, _i, _vp, _vp]),
    "qkv_forward": (None, [_vp] * 7 + [_i, _i, _i, _vp]),
    "gate_up_forward": (None, [_vp] * 4 + [_i, _i, _vp, _vp, _vp]),
    "qk_norm_rope_forward": (None, [_vp] * 8 + [_i, _i, _i, _f, _f, _vp, _vp, _vp]),
    "qk_norm_rope_rows": (None, [_vp] * 8 + [_i, _i, _i, _i, _f, _f, _vp, _vp, _vp]),
    "attention_forward": (None, [_vp] * 5 + [_i, _i, _i, _vp, _i, _f, _vp]),
    "attention_forward_noalloc": (None, [_vp] * 4 + [_i, _i, _i, _vp, _i, _f, _vp]),
    "argmax_forward": (None, [_vp, _vp, _i, _vp]),
    "swiglu_forward": (None, [_vp, _vp, _vp, _sz, _vp]),
    "attention_workspace_floats": (_sz, [_i, _i, _i]),
    "rmsnorm_qkv_forward": (None, [_vp] * 8 + [_f, _i, _i, _i, _vp]),
    "rmsnorm_gemv_forward": (None, [_vp] * 4 + [_f, _i, _i, _vp]),
    "rmsnorm_gate_up_forward": (None, [_vp] * 5 + [_f, _i, _i, _vp]),
    "hbm_stream_probe": (None, [_vp, _vp, _vp, _sz, _i, _vp]),
    "hbm_read_peak_probe": (None, [_vp, _vp, _sz, _i, _i, _i, _i, _vp]),
    "hbm_copy_peak_probe": (None, [_vp, _vp, _sz, _i, _i, _i, _vp]),
    "qk_norm_rope_attention_forward": (None, [_vp] * 9 + [_vp, _i, _i, _i, _f, _f, _i, _f, _vp]),
    "qk_norm_rope_attention_one_pass": (None, [_vp] * 11 + [_i, _i, _i, _f, _f, _i, _f, _vp]),
    "attention_one_pass_bytes": (_sz, [_i, _i, _i]),
    "attention_one_pass_supported": (_i, [_i, _i, _i, _i]),
    "sample_forward": (None, [_vp, _vp, _i, _f, _f, _vp]),
    "dump_open": (None, [ctypes.c_char_p]),
    "dump_close": (None, []),
    "dump_enabled": (_i, []),
    "dump_bf16": (None, [ctypes.c_char_p, _vp, _i]),
    "dump_f32": (None, [ctypes.c_char_p, _vp, _i]),
    "llm_set_exit_on_error": (_i, [_i]),
    "llm_last_error": (ctypes.c_char_p, []),
    "llm_clear_error": (None, []),
}


def lib():
    """The loaded libllm_amd.so (raises LlmError if it has not been built)."""
    global _lib
    if _lib is None:
        # torch first: its bundled HIP runtime then satisfies the library's libamdhip64.so.7
        # dependency (same SONAME), so both share one runtime and torch's streams are valid here.
        import torch  # noqa: F401
        if not LIB_PATH.exists():
            raise LlmError(f"{LIB_PATH} is missing: build it with `make -C {HERE}` "
                           "(or __graft_entry__.build())")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        L.llm_set_exit_on_error(0)
        _lib = L
        from . import model  # noqa: F401  (declares the step API signatures)
        model._declare(L)
    return _lib


def check():
    """Raises LlmError with the library's message if the last call recorded an error."""
    L = lib()
    msg = L.llm_last_error()
    if msg is not None:
        L.llm_clear_error()
        raise LlmError(msg.decode())


def _ptr(t):
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if not t.is_cuda:
        raise LlmError("tensors passed to the HIP kernels must live on the GPU")
    if not t.is_contiguous():
        raise LlmError("tensors passed to the HIP kernels must be contiguous")
    return t.data_ptr()


def _bf16(t, name):
    import torch
    if t is not None and not isinstance(t, int) and t.dtype not in (torch.bfloat16, torch.int16,
                                                                     torch.uint16):
        raise LlmError(f"{name} must be bfloat16 (or its raw 16-bit view), got {t.dtype}")
    return _ptr(t)


def _stream(stream):
    import torch
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _call(fn, *args):
    fn(*args)
    check()


# ---- launchers (include/llm_amd/kernels.h) ----

def embedding_forward(out, table, d_token, hidden, stream=None):
    _call(lib().embedding_forward, _bf16(out, "out"), _bf16(table, "table"), _ptr(d_token),
          hidden, _stream(stream))


def rmsnorm_forward(out, inp, weight, rows, dim, eps, stream=None):
    _call(lib().rmsnorm_forward, _bf16(out, "out"), _bf16(inp, "in"), _bf16(weight, "weight"),
          rows, dim, eps, _stream(stream))


def gemv_forward(out, w, x, rows, cols, stream=None):
    _call(lib().gemv_forward, _bf16(out, "out"), _bf16(w, "w"), _bf16(x, "x"), rows, cols,
          _stream(stream))


def gemv_residual_forward(x, w, inp, rows, cols, tap=None, stream=None):
    _call(lib().gemv_residual_forward, _bf16(x, "x"), _bf16(w, "w"), _bf16(inp, "in"), rows,
          cols, _bf16(tap, "tap"), _stream(stream))


def qkv_forward(q, k, v, wq, wk, wv, x, q_rows, kv_rows, cols, stream=None):
    _call(lib().qkv_forward, _bf16(q, "q"), _bf16(k, "k"), _bf16(v, "v"), _bf16(wq, "wq"),
          _bf16(wk, "wk"), _bf16(wv, "wv"), _bf16(x, "x"), q_rows, kv_rows, cols,
          _stream(stream))


def gate_up_forward(act, w_gate, w_up, x, rows, cols, gate_tap=None, up_tap=None, stream=None):
    _call(lib().gate_up_forward, _bf16(act, "act"), _bf16(w_gate, "w_gate"), _bf16(w_up, "w_up"),
          _bf16(x, "x"), rows, cols, _bf16(gate_tap, "gate_tap"), _bf16(up_tap, "up_tap"),
          _stream(stream))


def rmsnorm_qkv_forward(q, k, v, wq, wk, wv, x, norm_w, eps, q_rows, kv_rows, cols,
                        stream=None):
    _call(lib().rmsnorm_qkv_forward, _bf16(q, "q"), _bf16(k, "k"), _bf16(v, "v"),
          _bf16(wq, "wq"), _bf16(wk, "wk"), _bf16(wv, "wv"), _bf16(x, "x"),
          _bf16(norm_w, "norm_w"), eps, q_rows, kv_rows, cols, _stream(stream))


def rmsnorm_gemv_forward(out, w, x, norm_w, eps, rows, cols, stream=None):
    _call(lib().rmsnorm_gemv_forward, _bf16(out, "out"), _bf16(w, "w"), _bf16(x, "x"),
          _bf16(norm_w, "norm_w"), eps, rows, cols, _stream(stream))


def rmsnorm_gate_up_forward(act, w_gate, w_up, x, norm_w, eps, rows, cols, stream=None):
    _call(lib().rmsnorm_gate_up_forward, _bf16(act, "act"), _bf16(w_gate, "w_gate"),
          _bf16(w_up, "w_up"), _bf16(x, "x"), _bf16(norm_w, "norm_w"), eps, rows, cols,
          _stream(stream))


def qk_norm_rope_forward(q, k, v, q_norm_w, k_norm_w, key_cache, value_cache, d_pos, n_heads,
                         n_kv_heads, head_dim, eps, theta, q_tap=None, k_tap=None, stream=None):
    _call(lib().qk_norm_rope_forward, _bf16(q, "q"), _bf16(k, "k"), _bf16(v, "v"),
          _bf16(q_norm_w, "q_norm_w"), _bf16(k_norm_w, "k_norm_w"), _bf16(key_cache, "key_cache"),
          _bf16(value_cache, "value_cache"), _ptr(d_pos), n_heads, n_kv_heads, head_dim, eps,
          theta, _bf16(q_tap, "q_tap"), _bf16(k_tap, "k_tap"), _stream(stream))


def qk_norm_rope_rows(q, k, v, q_norm_w, k_norm_w, key_cache, value_cache, d_positions,
                      n_tokens, n_heads, n_kv_heads, head_dim, eps, theta, q_tap=None,
                      k_tap=None, stream=None):
    _call(lib().qk_norm_rope_rows, _bf16(q, "q"), _bf16(k, "k"), _bf16(v, "v"),
          _bf16(q_norm_w, "q_norm_w"), _bf16(k_norm_w, "k_norm_w"), _bf16(key_cache, "key_cache"),
          _bf16(value_cache, "value_cache"), _ptr(d_positions), n_tokens, n_heads, n_kv_heads,
          head_dim, eps, theta, _bf16(q_tap, "q_tap"), _bf16(k_tap, "k_tap"), _stream(stream))


def attention_workspace_floats(n_heads, head_dim, max_seq):
    return lib().attention_workspace_floats(n_heads, head_dim, max_seq)


def attention_forward(out, q, key_cache, value_cache, att, n_heads, n_kv_heads, head_dim, d_pos,
                      max_seq, scale, stream=None):
    """att: a device pointer (int) to the caller's own allocation of at least [n_heads, max_seq]
    floats (the library checks that allocation's size), or a torch tensor of at least
    attention_workspace_floats(n_heads, head_dim, max_seq) floats: torch's caching allocator
    carves tensors out of larger allocations, whose size says nothing of the tensor's."""
    need = attention_workspace_floats(n_heads, head_dim, max_seq)
    if not isinstance(att, int) and att.numel() < need:
        raise LlmError(f"att holds {att.numel()} floats, attention needs {need}")
    _call(lib().attention_forward, _bf16(out, "out"), _bf16(q, "q"),
          _bf16(key_cache, "key_cache"), _bf16(value_cache, "value_cache"), _ptr(att), n_heads,
          n_kv_heads, head_dim, _ptr(d_pos), max_seq, scale, _stream(stream))


def qk_norm_rope_attention_forward(out, q, k, v, q_norm_w, k_norm_w, key_cache, value_cache, att,
                                   d_pos, n_heads, n_kv_heads, head_dim, eps, theta, max_seq,
                                   scale, stream=None):
    """qk_norm_rope_forward + attention_forward, the QK-norm + RoPE inside the scores pass."""
    need = attention_workspace_floats(n_heads, head_dim, max_seq)
    if not isinstance(att, int) and att.numel() < need:
        raise LlmError(f"att holds {att.numel()} floats, attention needs {need}")
    _call(lib().qk_norm_rope_attention_forward, _bf16(out, "out"), _bf16(q, "q"), _bf16(k, "k"),
          _bf16(v, "v"), _bf16(q_norm_w, "q_norm_w"), _bf16(k_norm_w, "k_norm_w"),
          _bf16(key_cache, "key_cache"), _bf16(value_cache, "value_cache"), _ptr(att), _ptr(d_pos),
          n_heads, n_kv_heads, head_dim, eps, theta, max_seq, scale, _stream(stream))


def attention_one_pass_bytes(n_heads, head_dim, max_seq):
    return lib().attention_one_pass_bytes(n_heads, head_dim, max_seq)


def attention_one_pass_supported(n_heads, n_kv_heads, head_dim, max_seq):
    return bool(lib().attention_one_pass_supported(n_heads, n_kv_heads, head_dim, max_seq))


def qk_norm_rope_attention_one_pass(out, q, k, v, q_norm_w, k_norm_w, key_cache, value_cache, ws,
                                    err, d_pos, n_heads, n_kv_heads, head_dim, eps, theta,
                                    max_seq, scale, stream=None):
    """qk_norm_rope_forward + attention_forward in one launch. ws: a zeroed device buffer of
    attention_one_pass_bytes() bytes kept between calls; err: a device int32 (2 on timeout)."""
    need = attention_one_pass_bytes(n_heads, head_dim, max_seq)
    if not isinstance(ws, int) and ws.numel() * ws.element_size() < need:
        raise LlmError(f"ws holds {ws.numel() * ws.element_size()} bytes, one-pass attention "
                       f"needs {need}")
    _call(lib().qk_norm_rope_attention_one_pass, _bf16(out, "out"), _bf16(q, "q"), _bf16(k, "k"),
          _bf16(v, "v"), _bf16(q_norm_w, "q_norm_w"), _bf16(k_norm_w, "k_norm_w"),
          _bf16(key_cache, "key_cache"), _bf16(value_cache, "value_cache"), _ptr(ws), _ptr(err),
          _ptr(d_pos), n_heads, n_kv_heads, head_dim, eps, theta, max_seq, scale,
          _stream(stream))


def attention_forward_noalloc(out, q, key_cache, value_cache, n_heads, n_kv_heads, head_dim,
                              d_pos, max_seq, scale, stream=None):
    """attention_forward with the library's own workspace (allocates nothing)."""
    _call(lib().attention_forward_noalloc, _bf16(out, "out"), _bf16(q, "q"),
          _bf16(key_cache, "key_cache"), _bf16(value_cache, "value_cache"), n_heads, n_kv_heads,
          head_dim, _ptr(d_pos), max_seq, scale, _stream(stream))


def hbm_stream_probe(dst, a, b, n_bytes, mode, stream=None):
    need = (1 << 20) if mode == 0 else n_bytes
    if not isinstance(dst, int) and dst.numel() * dst.element_size() < need:
        raise LlmError(f"dst holds {dst.numel() * dst.element_size()} bytes, the probe needs {need}")
    _call(lib().hbm_stream_probe, _ptr(dst), _ptr(a), _ptr(b), n_bytes, mode, _stream(stream))


def hbm_read_peak_probe(out, a, n_bytes, blocks, threads, loads_in_flight=4, contiguous=0,
                        stream=None):
    """Reads n_bytes of `a` with `blocks` workgroups of `threads` threads, loads_in_flight
    16-byte loads per thread per round, grid-stride (contiguous=0) or one range per workgroup
    (contiguous=1) (the read-peak probe); `out` is a device word written only if a thread's xor
    equals 0x9e3779b9."""
    _call(lib().hbm_read_peak_probe, _ptr(out), _ptr(a), n_bytes, blocks, threads,
          loads_in_flight, contiguous, _stream(stream))


def hbm_copy_peak_probe(dst, a, n_bytes, blocks, threads, chunks_in_flight=4, stream=None):
    """Copies n_bytes of `a` to `dst` grid-stride with `blocks` workgroups of `threads` threads,
    each thread requesting chunks_in_flight 16-byte loads before it stores them (the copy-peak
    probe)."""
    for name, t in (("dst", dst), ("a", a)):
        if not isinstance(t, int) and t.numel() * t.element_size() < n_bytes:
            raise LlmError(f"{name} holds {t.numel() * t.element_size()} bytes, the probe copies "
                           f"{n_bytes}")
    _call(lib().hbm_copy_peak_probe, _ptr(dst), _ptr(a), n_bytes, blocks, threads,
          chunks_in_flight, _stream(stream))


def sample_forward(out, x, n, inv_temp, u, stream=None):
    _call(lib().sample_forward, _ptr(out), _bf16(x, "x"), n, inv_temp, u, _stream(stream))


def dump_open(directory):
    """Activation dumps of the eager step into `directory` (include/llm_amd/dump.h)."""
    _call(lib().dump_open, str(directory).encode())


def dump_close():
    lib().dump_close()


def argmax_forward(out, x, n, stream=None):
    _call(lib().argmax_forward, _ptr(out), _bf16(x, "x"), n, _stream(stream))


def swiglu_forward(act, gate, up, n, stream=None):
    _call(lib().swiglu_forward, _bf16(act, "act"), _bf16(gate, "gate"), _bf16(up, "up"), n,
          _stream(stream))
