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
