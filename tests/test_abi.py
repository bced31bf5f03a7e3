"""C-ABI library checks that need no GPU: every symbol include/llm_amd/*.h declares is exported,
shape/argument validation reports the reference's messages (recorded, or exit(EXIT_FAILURE) in
the default mode, as src/kernels.cu:147-152 and :392-396 do), and the config/safetensors parsing
errors of src/loader.cu:29-139 and :143-180."""
import json
import re
import struct
import subprocess
import sys
from pathlib import Path

import pytest

from conftest import PKG_DIR, ROOT, load_package

HEADERS = sorted((ROOT / "include" / "llm_amd").glob("*.h"))


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"\b([A-Za-z_]\w*)\s*\(([^;{}]*)\)\s*;", text):
            if m.group(1) not in ("if", "while", "for", "sizeof"):
                names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def L():
    pkg = load_package()
    return pkg.lib()


def test_library_exports_every_declared_symbol(L):
    declared = declared_functions()
    assert len(declared) >= 30
    out = subprocess.run(["nm", "-D", "--defined-only", str(PKG_DIR / "libllm_amd.so")],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = declared - exported
    assert not missing, missing
    for name in declared:
        getattr(L, name)
    pkg = load_package()
    assert set(pkg.EXPORTED_SYMBOLS) == declared


def test_library_does_not_link_the_oracle():
    out = subprocess.run(["ldd", str(PKG_DIR / "libllm_amd.so")], capture_output=True, text=True,
                         check=True).stdout
    assert "oracle" not in out
    nm = subprocess.run(["nm", "-D", str(PKG_DIR / "libllm_amd.so")], capture_output=True,
                        text=True, check=True).stdout
    assert "orc_" not in nm


def _err(L, fn, *args):
    L.llm_clear_error()
    fn(*args)
    msg = L.llm_last_error()
    L.llm_clear_error()
    return msg.decode() if msg else None


def test_shape_errors_are_recorded(L):
    # fake but 16-byte-aligned pointers: validation happens before anything touches the GPU
    p = 0x1000
    assert "cols 7 is not a multiple of 8" in _err(L, L.gemv_forward, p, p, p, 4, 7, None)
    assert "cols 12 is not a multiple of 8" in _err(L, L.gemv_residual_forward, p, p, p, 4, 12, None, None)
    assert "in must not alias x" in _err(L, L.gemv_residual_forward, p, p, p, 4, 8, None, None)
    assert "multiple of 8" in _err(L, L.gate_up_forward, p, p, p, p, 4, 10, None, None, None)
    assert "multiple of 8" in _err(L, L.qkv_forward, p, p, p, p, p, p, p, 4, 4, 6, None)
    assert "16-byte aligned" in _err(L, L.gemv_forward, p, p + 2, p, 4, 8, None)
    assert "head_dim 96" in _err(L, L.qk_norm_rope_forward, p, p, p, p, p, p, p, p, 2, 1, 96,
                                 1e-6, 1e6, None, None, None)
    assert "not a multiple of n_kv_heads" in _err(L, L.attention_forward, p, p, p, p, p, 6, 4, 128,
                                                  p, 16, 0.1, None)
    assert "is not 1, 2, 4 or 8" in _err(L, L.attention_forward, p, p, p, p, p, 12, 4, 128, p, 16,
                                         0.1, None)
    assert "n 0 must be positive" in _err(L, L.argmax_forward, p, p, 0, None)
    assert _err(L, L.swiglu_forward, p, p, p, 0, None) is None  # nothing to do


def test_workspace_size(L):
    # [n_heads, max_seq] scores + [n_heads, ceil(max_seq/64)] x (2 stats + D partial)
    assert L.attention_workspace_floats(16, 128, 4096) == 16 * 4096 + 16 * 64 * 130
    assert L.attention_workspace_floats(32, 128, 8448) == 32 * 8448 + 32 * 132 * 130


def test_exit_on_error_mode_exits_like_the_reference():
    code = (
        "import sys; sys.path.insert(0, 'tests'); from conftest import load_package;"
        "L = load_package().lib(); L.llm_set_exit_on_error(1);"
        "L.gemv_forward(0x1000, 0x1000, 0x1000, 4, 7, None); print('not reached')")
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True)
    assert r.returncode == 1
    assert "gemv: cols 7 is not a multiple of 8" in r.stderr
    assert "not reached" not in r.stdout


# ---------------------------------------------------------------- loader (host-only paths)

CFG = {"hidden_size": 256, "intermediate_size": 512, "num_hidden_layers": 2,
       "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 128,
       "vocab_size": 1000, "max_position_embeddings": 4096, "rms_norm_eps": 1e-6,
       "rope_theta": 1000000.0, "tie_word_embeddings": True}


def _model_dir(tmp_path, cfg=CFG, gen={"eos_token_id": [151645, 151643]}):
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    if gen is not None:
        (tmp_path / "generation_config.json").write_text(json.dumps(gen))
    return tmp_path


def test_load_config_parses_fields(tmp_path):
    pkg = load_package()
    from llm_inference_amd import model
    cfg = model.load_config(_model_dir(tmp_path))
    assert (cfg.hidden_size, cfg.intermediate_size, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads,
            cfg.head_dim, cfg.vocab_size, cfg.max_seq_len) == (256, 512, 2, 4, 2, 128, 1000, 4096)
    assert cfg.rms_norm_eps == pytest.approx(1e-6) and cfg.rope_theta == 1e6
    assert cfg.tie_word_embeddings == 1 and list(cfg.eos_ids[:cfg.n_eos]) == [151645, 151643]
    _model_dir(tmp_path, gen={"eos_token_id": 7})
    assert list(model.load_config(tmp_path).eos_ids[:1]) == [7]


@pytest.mark.parametrize("mutate,message", [
    (lambda c: c.pop("head_dim"), 'no number "head_dim"'),
    (lambda c: c.update(tie_word_embeddings=1), 'no bool "tie_word_embeddings"'),
    (lambda c: c.update(num_key_value_heads=3), "multiple of num_key_value_heads"),
    (lambda c: c.update(rope_theta="big"), 'no number "rope_theta"'),
])
def test_load_config_errors(tmp_path, mutate, message):
    pkg = load_package()
    from llm_inference_amd import model
    cfg = dict(CFG)
    mutate(cfg)
    with pytest.raises(pkg.LlmError, match=re.escape(message)):
        model.load_config(_model_dir(tmp_path, cfg))


def test_load_config_eos_errors(tmp_path):
    pkg = load_package()
    from llm_inference_amd import model
    with pytest.raises(pkg.LlmError, match="has no \"eos_token_id\""):
        model.load_config(_model_dir(tmp_path, gen={"bos_token_id": 1}))
    with pytest.raises(pkg.LlmError, match="bad \"eos_token_id\""):
        model.load_config(_model_dir(tmp_path, gen={"eos_token_id": [1, "x"]}))
    (tmp_path / "config.json").write_text("{not json")
    with pytest.raises(pkg.LlmError, match="cannot parse"):
        model.load_config(tmp_path)


def _write_raw(path, header_bytes, data=b"", header_len=None):
    n = len(header_bytes) if header_len is None else header_len
    path.write_bytes(struct.pack("<Q", n) + header_bytes + data)


def test_load_weights_header_errors(tmp_path):
    """Shard errors caught before any device allocation (src/loader.cu:159-173)."""
    pkg = load_package()
    from llm_inference_amd import model
    d = _model_dir(tmp_path)
    cfg = model.load_config(d)
    L = pkg.lib()
    w = model.Weights()
    import ctypes
    (d / "model.safetensors").write_bytes(b"1234")
    L.load_weights(str(d).encode(), ctypes.byref(cfg), ctypes.byref(w))
    assert "too small to be a safetensors file" in L.llm_last_error().decode()
    L.llm_clear_error()
    _write_raw(d / "model.safetensors", b"{}", header_len=1000)
    L.load_weights(str(d).encode(), ctypes.byref(cfg), ctypes.byref(w))
    assert "bad header length" in L.llm_last_error().decode()
    L.llm_clear_error()
    _write_raw(d / "model.safetensors", b"{\"a\": [1,")
    L.load_weights(str(d).encode(), ctypes.byref(cfg), ctypes.byref(w))
    assert "cannot parse header" in L.llm_last_error().decode()
    L.llm_clear_error()
    (d / "model.safetensors").unlink()
    L.load_weights(str(d).encode(), ctypes.byref(cfg), ctypes.byref(w))
    assert "no .safetensors files" in L.llm_last_error().decode()
    L.llm_clear_error()


# ---------------------------------------------------------------- loader: manifest and schema

def _small_tensors():
    """{name: (dtype, shape, bytes)} of a complete checkpoint for CFG (zero-filled BF16)."""
    H, I, D, V = 256, 512, 128, 1000
    qd, kvd = 4 * D, 2 * D
    shapes = {"model.embed_tokens.weight": (V, H), "model.norm.weight": (H,)}
    for l in range(2):
        p = f"model.layers.{l}."
        shapes.update({p + "input_layernorm.weight": (H,), p + "self_attn.q_proj.weight": (qd, H),
                       p + "self_attn.k_proj.weight": (kvd, H),
                       p + "self_attn.v_proj.weight": (kvd, H),
                       p + "self_attn.q_norm.weight": (D,), p + "self_attn.k_norm.weight": (D,),
                       p + "self_attn.o_proj.weight": (H, qd),
                       p + "post_attention_layernorm.weight": (H,),
                       p + "mlp.gate_proj.weight": (I, H), p + "mlp.up_proj.weight": (I, H),
                       p + "mlp.down_proj.weight": (H, I)})
    out = {}
    for name, shape in shapes.items():
        n = 1
        for s in shape:
            n *= s
        out[name] = ("BF16", list(shape), n * 2)
    return out


def _write_checkpoint(path, tensors, patch=None):
    """One safetensors file; `patch(header)` may edit the header dict before it is written."""
    header, off = {}, 0
    for name, (dtype, shape, nbytes) in tensors.items():
        header[name] = {"dtype": dtype, "shape": shape, "data_offsets": [off, off + nbytes]}
        off += nbytes + (-nbytes) % 16
    if patch:
        patch(header)
    h = json.dumps(header).encode()
    h += b" " * ((-len(h)) % 16)
    path.write_bytes(struct.pack("<Q", len(h)) + h + b"\0" * off)


def _load_error(tmp_path, tensors, patch=None, cfg=CFG):
    pkg = load_package()
    from llm_inference_amd import model
    import ctypes
    d = _model_dir(tmp_path, cfg)
    for f in d.glob("*.safetensors"):
        f.unlink()
    _write_checkpoint(d / "model.safetensors", tensors, patch)
    c = model.load_config(d)
    L = pkg.lib()
    w = model.Weights()
    L.llm_clear_error()
    L.load_weights(str(d).encode(), ctypes.byref(c), ctypes.byref(w))
    msg = L.llm_last_error()
    L.llm_clear_error()
    assert w.n_tensors == 0 and w.n_buffers == 0  # nothing kept on failure
    return msg.decode() if msg else ""


def _set(name, key, value):
    def patch(h):
        h[name][key] = value
    return patch


@pytest.mark.parametrize("case,message", [
    ("missing", "tensor model.layers.1.mlp.up_proj.weight not found"),
    ("dtype", "is F16, only BF16 is supported"),
    ("shape", "has shape [512, 255], config.json implies [512, 256]"),
    ("unaligned", "offset 8 is not 16-byte aligned"),
    ("negative", "data_offsets must be non-negative integers"),
    ("fraction", "data_offsets must be non-negative integers"),
    ("string_dim", "dims must be non-negative integers"),
    ("negative_dim", "dims must be non-negative integers"),
    ("outside", "outside the"),
    ("size", "bytes for 131072 bf16 elements"),
    ("unused", "1 tensor(s) in the checkpoint are not read by the engine (first: extra.weight)"),
    ("untied_head", "tensor lm_head.weight not found"),
])
def test_load_weights_validation_errors(tmp_path, case, message):
    """Every format and shape rule is checked before any device memory is touched (so these run
    without a GPU): missing tensors, dtypes other than BF16, shapes config.json does not imply,
    misaligned, negative, fractional or out-of-range data offsets, malformed dims, byte counts
    that disagree with the shape, and tensors the engine would not read."""
    t = _small_tensors()
    patch, cfg = None, CFG
    up = "model.layers.1.mlp.up_proj.weight"
    if case == "missing":
        del t[up]
    elif case == "dtype":
        t[up] = ("F16",) + t[up][1:]
    elif case == "shape":
        t[up] = ("BF16", [512, 255], 512 * 255 * 2)
    elif case == "unaligned":
        patch = _set("model.norm.weight", "data_offsets", [8, 8 + 512])
    elif case == "negative":
        patch = _set("model.norm.weight", "data_offsets", [-16, 496])
    elif case == "fraction":
        patch = _set("model.norm.weight", "data_offsets", [0.5, 512])
    elif case == "string_dim":
        patch = _set("model.norm.weight", "shape", ["256"])
    elif case == "negative_dim":
        patch = _set("model.norm.weight", "shape", [-256])
    elif case == "outside":
        patch = _set("model.norm.weight", "data_offsets", [1 << 40, (1 << 40) + 512])
    elif case == "size":
        patch = _set(up, "data_offsets", [0, 1000])
    elif case == "unused":
        t["extra.weight"] = ("BF16", [8], 16)
    elif case == "untied_head":
        cfg = dict(CFG, tie_word_embeddings=False)
    msg = _load_error(tmp_path, t, patch, cfg)
    assert message in msg, msg


def test_load_weights_duplicate_across_shards(tmp_path):
    """A tensor name in two shards is an error, whichever shard would be read."""
    pkg = load_package()
    from llm_inference_amd import model
    import ctypes
    d = _model_dir(tmp_path)
    t = _small_tensors()
    _write_checkpoint(d / "a.safetensors", t)
    _write_checkpoint(d / "b.safetensors", {"model.norm.weight": t["model.norm.weight"]})
    c = model.load_config(d)
    L = pkg.lib()
    w = model.Weights()
    L.llm_clear_error()
    L.load_weights(str(d).encode(), ctypes.byref(c), ctypes.byref(w))
    msg = L.llm_last_error().decode()
    L.llm_clear_error()
    assert "tensor model.norm.weight appears in more than one place" in msg


def test_load_weights_tied_head_may_be_present(tmp_path):
    """With tie_word_embeddings an lm_head.weight in the files is allowed (not read): a complete
    checkpoint passes every check and only then reaches the device (without a GPU the first HIP
    call reports the error; on a machine with a GPU the load succeeds)."""
    t = _small_tensors()
    t["lm_head.weight"] = ("BF16", [1000, 256], 1000 * 256 * 2)
    msg = _load_error_or_none(tmp_path, t)
    assert msg is None or msg.startswith("HIP error"), msg


def _load_error_or_none(tmp_path, tensors):
    pkg = load_package()
    from llm_inference_amd import model
    import ctypes
    d = _model_dir(tmp_path)
    _write_checkpoint(d / "model.safetensors", tensors)
    c = model.load_config(d)
    L = pkg.lib()
    w = model.Weights()
    L.llm_clear_error()
    L.load_weights(str(d).encode(), ctypes.byref(c), ctypes.byref(w))
    msg = L.llm_last_error()
    L.llm_clear_error()
    if msg is None:
        L.free_weights(ctypes.byref(w))
    return msg.decode() if msg else None


def test_load_config_rejects_fractional_sizes(tmp_path):
    pkg = load_package()
    from llm_inference_amd import model
    with pytest.raises(pkg.LlmError, match='"hidden_size" must be a non-negative integer'):
        model.load_config(_model_dir(tmp_path, dict(CFG, hidden_size=256.5)))
    with pytest.raises(pkg.LlmError, match='bad "eos_token_id"'):
        model.load_config(_model_dir(tmp_path, gen={"eos_token_id": [-1]}))


# ---------------------------------------------------------------- byte counts

def test_byte_counts_match_the_published_figures():
    """weight_bytes_per_step and kv_bytes_per_position through the C ABI: the bytes per token
    at the mean position of a 5-token prompt + 256 tokens (133.5) equal the reference's published
    counts for Qwen3-0.6B / 1.7B / 4B (bench/results.csv:289, :317, :345), and the 4B line of the
    8192-position config (mean position 8320.5) equals 9,271,848,960 B."""
    load_package()
    from llm_inference_amd import model
    published = {"0.6B": 1207412736, "1.7B": 3456464896, "4B": 8064626688}
    for size, want in published.items():
        c = model.qwen3_config(size)
        w, kv = model.weight_bytes_per_step(c), model.kv_bytes_per_position(c)
        assert kv == 2 * c.n_layers * c.n_kv_heads * c.head_dim * 2
        assert w + kv * 133.5 == want, size
    c = model.qwen3_config("4B")
    assert model.weight_bytes_per_step(c) + model.kv_bytes_per_position(c) * 8320.5 == 9271848960
    # a model with untied-size terms: every weight once, plus one embedding row
    c = model.make_config(hidden_size=64, intermediate_size=96, n_layers=3, n_heads=4,
                          n_kv_heads=2, head_dim=16, vocab_size=50)
    H, I, D, qd, kvd = 64, 96, 16, 64, 32
    layer = H + qd * H + 2 * kvd * H + 2 * D + H * qd + H + 2 * I * H + H * I
    assert model.weight_bytes_per_step(c) == 2 * (3 * layer + H + 50 * H + H)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 exits with status 2 and says why, before any GPU
    or library work (the argument check comes first)."""
    r = subprocess.run([sys.executable, str(Path(ROOT) / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "--gpus 2 is not supported" in r.stderr
    assert r.stdout == ""
