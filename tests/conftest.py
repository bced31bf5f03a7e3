import importlib.util
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "llm-inference_amd"
sys.path.insert(0, str(ROOT / "oracle"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def load_package():
    """Imports llm-inference_amd/ (a directory name that is not an identifier) as
    llm_inference_amd."""
    if "llm_inference_amd" in sys.modules:
        return sys.modules["llm_inference_amd"]
    spec = importlib.util.spec_from_file_location(
        "llm_inference_amd", PKG_DIR / "__init__.py", submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["llm_inference_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.lib()
    return o


@pytest.fixture(scope="session")
def pkg():
    return load_package()


@pytest.fixture(scope="session")
def gpu(pkg):
    """The HIP library on cuda:0. Fails (does not skip) without a GPU: a gpu-marked test that
    cannot reach the GPU is a broken run, not a pass."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("no GPU visible: gpu tests must run on the MI355X")
    pkg.lib()
    return pkg


def bf16_bits(a):
    """float32 array -> bf16 bits, round to nearest even."""
    import oracle as o
    return o.f32_to_bf16(np.asarray(a, dtype=np.float32))


def bf16_vals(b):
    import oracle as o
    return o.bf16_to_f32(b)


def rand_bf16(rng, shape, std=1.0, mean=0.0):
    return bf16_bits(rng.standard_normal(shape, dtype=np.float32) * np.float32(std) + np.float32(mean))


def ulp_bf16(v):
    """Spacing of bf16 numbers at |v| (fp32 array)."""
    v = np.abs(np.asarray(v, dtype=np.float32))
    e = np.floor(np.log2(np.maximum(v, np.float32(2.0 ** -126))))
    return np.float32(2.0) ** (e - 7)


def bf16_ulp_diff(a, b):
    """Distance in bf16 ulps between two bf16 bit arrays (ordered encoding)."""
    def ordered(x):
        x = np.asarray(x, dtype=np.uint16).astype(np.int32)
        mag = x & 0x7FFF
        return np.where(x & 0x8000, 0x8000 - mag, 0x8000 + mag)

    return np.abs(ordered(a) - ordered(b))


def bf16_step(b, k):
    """The bf16 value k representable steps away from b (bits), through zero if needed."""
    if k == 0:
        return np.asarray(b, dtype=np.uint16)  # keeps the sign of zero
    x = np.asarray(b, dtype=np.uint16).astype(np.int32)
    mag = x & 0x7FFF
    o = np.where(x & 0x8000, -mag, mag) + k
    return np.where(o < 0, 0x8000 | (-o), o).astype(np.uint16)


def within_one_ulp_then_scale(y, n_exact, scale):
    """True where y = bf16(m * scale) for some m within one bf16 ulp of n_exact: the parity
    1-ulp tolerance applied at HF's first rounding point (bf16(x * inv_rms) for RMSNorm,
    bf16(silu(g)) for SwiGLU), followed by the same bf16 multiply by gamma (or up)."""
    y = np.asarray(y, dtype=np.uint16)
    s = bf16_vals(scale)
    ok = np.zeros(y.shape, bool)
    # products past the float range are inf, as the bf16 arithmetic gives (exhaustive sweeps)
    with np.errstate(over="ignore"):
        for k in (-1, 0, 1):
            ok |= y == bf16_bits(bf16_vals(bf16_step(n_exact, k)) * s)
    return ok


# Seeded Qwen3 weights as bf16 bits in the checkpoint's names: N(0, 0.02) matrices and
# 1 + N(0, 0.1) norm weights, drawn in this fixed order from numpy's default_rng(seed), so the HF
# golden fixtures (tests/golden) and the GPU tests build the same model.
SMALL = dict(hidden_size=256, intermediate_size=512, n_layers=2, n_heads=4, n_kv_heads=2,
             head_dim=128, vocab_size=1000)
QWEN3_06B = dict(hidden_size=1024, intermediate_size=3072, n_layers=28, n_heads=16, n_kv_heads=8,
                 head_dim=128, vocab_size=151936)


def qwen3_np_weights(c, seed=0):
    rng = np.random.default_rng(seed)
    H, I, D = c["hidden_size"], c["intermediate_size"], c["head_dim"]
    qd, kvd = c["n_heads"] * D, c["n_kv_heads"] * D
    w = {"model.embed_tokens.weight": rand_bf16(rng, (c["vocab_size"], H), 0.02)}
    for l in range(c["n_layers"]):
        p = f"model.layers.{l}."
        w[p + "input_layernorm.weight"] = rand_bf16(rng, H, 0.1, 1.0)
        w[p + "self_attn.q_proj.weight"] = rand_bf16(rng, (qd, H), 0.02)
        w[p + "self_attn.k_proj.weight"] = rand_bf16(rng, (kvd, H), 0.02)
        w[p + "self_attn.v_proj.weight"] = rand_bf16(rng, (kvd, H), 0.02)
        w[p + "self_attn.q_norm.weight"] = rand_bf16(rng, D, 0.1, 1.0)
        w[p + "self_attn.k_norm.weight"] = rand_bf16(rng, D, 0.1, 1.0)
        w[p + "self_attn.o_proj.weight"] = rand_bf16(rng, (H, qd), 0.02)
        w[p + "post_attention_layernorm.weight"] = rand_bf16(rng, H, 0.1, 1.0)
        w[p + "mlp.gate_proj.weight"] = rand_bf16(rng, (I, H), 0.02)
        w[p + "mlp.up_proj.weight"] = rand_bf16(rng, (I, H), 0.02)
        w[p + "mlp.down_proj.weight"] = rand_bf16(rng, (H, I), 0.02)
    w["model.norm.weight"] = rand_bf16(rng, H, 0.1, 1.0)
    return w


def small_weights(seed=0):
    return qwen3_np_weights(SMALL, seed)
