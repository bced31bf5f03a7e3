"""Writes the HF golden fixtures: the HF-transformers Qwen3 path (the reference's parity path,
ref/dump.py:124: bf16 weights, eager attention), run on the CPU in this container, on models whose
weights come from tests/conftest.py's seeded generator.

tests/golden/hf_small_qwen3.npz, the small model (SMALL, small_weights(0)), token sequence TOKENS:
  logits      [len(TOKENS), vocab] fp32: teacher-forced logits at every position (one forward)
  greedy      [GREEDY_STEPS] int32: greedy tokens after PROMPT (model.generate, no sampling)
  greedy_gap  [GREEDY_STEPS] fp32: top-1 minus top-2 logit at each greedy step
tests/golden/hf_small_qwen3_dumps.npz, the small model's activation dumps (the reference's
  dump taxonomy, ref/dump.py:39-86) at the positions of TOKENS, as bf16 bits
tests/golden/hf_qwen3_06b_greedy.npz, the Qwen3-0.6B shapes (QWEN3_06B, qwen3_np_weights(., 0)),
the bench's 5 seeded prompt ids:
  greedy, greedy_gap  [256]; top_values, top_indices [256, 8]: the 8 largest logits per step
  full_steps [9]; full_logits [9, vocab] bf16 bits: every logit at steps 0, 32, ..., 224, 255

These pin what no closed form does: the HF fp32/bf16 CPU arithmetic end to end (the e2e logits
within 2e-2 and the greedy sequence up to near ties). The fixtures are data; this script is the
only place transformers is imported, and only here (never by the GPU tests or the bench).

Run from the repository root:  python tests/golden/make_hf_fixtures.py [small] [dumps] [0.6B]
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))  # tests/ (conftest helpers)

TOKENS = [17, 999, 0, 512, 3, 77, 640, 1, 2, 900, 45, 300]
PROMPT = [5, 60, 700, 8, 91]
GREEDY_STEPS = 40
# The Qwen3-0.6B-shaped model (28 layers) of the bench's decode: 5 seeded prompt ids, 256 greedy
# tokens; per step the top-2 gap and the 8 largest logits (values, indices).
GREEDY_06B_STEPS = 256
TOPK = 8
FULL_06B_STEPS = list(range(0, GREEDY_06B_STEPS, 32)) + [GREEDY_06B_STEPS - 1]


def hf_model(c, w, max_pos=64):
    """transformers' Qwen3ForCausalLM (bf16, eager attention) with the given bf16-bit weights."""
    import torch
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(
        vocab_size=c["vocab_size"], hidden_size=c["hidden_size"],
        intermediate_size=c["intermediate_size"], num_hidden_layers=c["n_layers"],
        num_attention_heads=c["n_heads"], num_key_value_heads=c["n_kv_heads"],
        head_dim=c["head_dim"], max_position_embeddings=max_pos, rms_norm_eps=1e-6,
        rope_parameters={"rope_type": "default", "rope_theta": 1e6}, tie_word_embeddings=True,
        attention_bias=False, hidden_act="silu", attn_implementation="eager")
    torch.manual_seed(0)
    model = Qwen3ForCausalLM(cfg).to(torch.bfloat16).eval()
    state = {}
    for name, bits in w.items():
        t = torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16))
        state[name] = t.view(torch.bfloat16).clone()
    state["lm_head.weight"] = state["model.embed_tokens.weight"]
    missing, unexpected = model.load_state_dict(state, strict=False)
    assert not unexpected, unexpected
    assert all(m == "lm_head.weight" for m in missing) or not missing, missing
    assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr() or \
        torch.equal(model.lm_head.weight, model.model.embed_tokens.weight)
    assert model.config._attn_implementation == "eager"
    return model


def small_fixture():
    import torch
    import transformers

    from conftest import SMALL, small_weights

    c = SMALL
    model = hf_model(c, small_weights(0))
    with torch.no_grad():
        ids = torch.tensor([TOKENS])
        logits = model(ids).logits[0].float().numpy()
        out = model.generate(torch.tensor([PROMPT]), max_new_tokens=GREEDY_STEPS, do_sample=False,
                             output_logits=True, return_dict_in_generate=True,
                             pad_token_id=0, eos_token_id=None)
    greedy = out.sequences[0, len(PROMPT):].numpy().astype(np.int32)
    gaps = []
    for step_logits in out.logits:
        top = torch.topk(step_logits[0].float(), 2).values
        gaps.append(float(top[0] - top[1]))
    meta = {"transformers": transformers.__version__, "torch": torch.__version__,
            "dtype": "bfloat16", "attn_implementation": "eager", "device": "cpu",
            "model": {k: v for k, v in c.items()}, "weights": "tests/conftest.py small_weights(0)",
            "tokens": TOKENS, "prompt": PROMPT}
    np.savez_compressed(os.path.join(HERE, "hf_small_qwen3.npz"), logits=logits,
                        greedy=greedy, greedy_gap=np.array(gaps, np.float32),
                        meta=np.array(json.dumps(meta)))
    print("wrote hf_small_qwen3.npz:", logits.shape, greedy[:8], "min gap", min(gaps))


# The tensors of one decoder layer in dump order, with the module whose output (or, marked "in",
# whose input) holds it; q_rope/k_rope come from the RoPE function (ref/dump.py:39-86 taxonomy).
LAYER_TAPS = [("attn_norm", "input_layernorm", "out"), ("q_proj", "self_attn.q_proj", "out"),
              ("k_proj", "self_attn.k_proj", "out"), ("v_proj", "self_attn.v_proj", "out"),
              ("q_norm", "self_attn.q_norm", "out"), ("k_norm", "self_attn.k_norm", "out"),
              ("attn_out", "self_attn.o_proj", "in"), ("o_proj", "self_attn.o_proj", "out"),
              ("attn_resid", "post_attention_layernorm", "in"),
              ("mlp_norm", "post_attention_layernorm", "out"), ("gate", "mlp.gate_proj", "out"),
              ("up", "mlp.up_proj", "out"), ("mlp_act", "mlp.down_proj", "in"),
              ("down", "mlp.down_proj", "out"), ("out", "", "out")]


def small_dumps_fixture():
    """tests/golden/hf_small_qwen3_dumps.npz: every dumped tensor of the small model at the
    positions of TOKENS (one teacher-forced forward; causal, so row t is position t's decode),
    as bf16 bits [len(TOKENS), width] (HF computes them all in bf16)."""
    import torch
    from transformers.models.qwen3 import modeling_qwen3

    from conftest import SMALL, small_weights

    model = hf_model(SMALL, small_weights(0))
    acts, hooks = {}, []

    def rows(t):
        return t[0].detach().to(torch.bfloat16).reshape(t.shape[1], -1).contiguous()

    def tap(name, where):
        if where == "in":
            return lambda mod, args: acts.__setitem__(name, rows(args[0]))
        return lambda mod, args, out: acts.__setitem__(name, rows(out[0] if isinstance(out, tuple) else out))

    inner = model.model
    hooks.append(inner.embed_tokens.register_forward_hook(tap("embed", "out")))
    layer_of = {}
    for i, layer in enumerate(inner.layers):
        for name, path, where in LAYER_TAPS:
            mod = layer
            for part in filter(None, path.split(".")):
                mod = getattr(mod, part)
            fn = tap(f"L{i:02d}.{name}", where)
            hooks.append(mod.register_forward_pre_hook(fn) if where == "in"
                         else mod.register_forward_hook(fn))
        layer_of[id(layer.self_attn)] = i
        hooks.append(layer.self_attn.register_forward_pre_hook(
            lambda mod, args, kwargs: acts.__setitem__("_layer", layer_of[id(mod)]),
            with_kwargs=True))
    hooks.append(inner.norm.register_forward_hook(tap("final_norm", "out")))
    hooks.append(model.lm_head.register_forward_hook(tap("logits", "out")))
    rope = modeling_qwen3.apply_rotary_pos_emb

    def rope_tap(q, k, cos, sin, *a, **kw):
        qe, ke = rope(q, k, cos, sin, *a, **kw)
        p = f"L{acts['_layer']:02d}"
        acts[p + ".q_rope"] = rows(qe.transpose(1, 2))  # [batch, seq, heads, dim]
        acts[p + ".k_rope"] = rows(ke.transpose(1, 2))
        return qe, ke

    modeling_qwen3.apply_rotary_pos_emb = rope_tap
    try:
        with torch.no_grad():
            model(torch.tensor([TOKENS]))
    finally:
        modeling_qwen3.apply_rotary_pos_emb = rope
        for h in hooks:
            h.remove()
    acts.pop("_layer")
    n_expected = 1 + SMALL["n_layers"] * (len(LAYER_TAPS) + 2) + 2
    assert len(acts) == n_expected, (len(acts), n_expected)
    out = {name: t.view(torch.int16).numpy().view(np.uint16) for name, t in acts.items()}
    np.savez_compressed(os.path.join(HERE, "hf_small_qwen3_dumps.npz"), **out)
    print("wrote hf_small_qwen3_dumps.npz:", len(out), "tensors")


def qwen06b_fixture():
    import torch
    import transformers

    from conftest import QWEN3_06B, qwen3_np_weights

    c = QWEN3_06B
    model = hf_model(c, qwen3_np_weights(c, 0), max_pos=4096)
    prompt = [int(t) for t in np.random.default_rng(0).integers(0, c["vocab_size"], 5)]
    with torch.no_grad():
        out = model.generate(torch.tensor([prompt]), max_new_tokens=GREEDY_06B_STEPS,
                             do_sample=False, output_logits=True, return_dict_in_generate=True,
                             pad_token_id=0, eos_token_id=None)
    greedy = out.sequences[0, len(prompt):].numpy().astype(np.int32)
    gaps, top_v, top_i = [], [], []
    for step_logits in out.logits:
        top = torch.topk(step_logits[0].float(), TOPK)
        gaps.append(float(top.values[0] - top.values[1]))
        top_v.append(top.values.numpy())
        top_i.append(top.indices.numpy().astype(np.int32))
    # HF's logits are the bf16 lm_head output (generate hands them out widened to fp32, which is
    # exact): kept as their bf16 bits, all 151936 of them
    full = []
    for i in FULL_06B_STEPS:
        row = out.logits[i][0]
        b = row.to(torch.bfloat16)
        assert torch.equal(b.float(), row.float()), "logits are not bf16 values"
        full.append(b.contiguous().view(torch.int16).numpy().view(np.uint16))
    full = np.stack(full)
    meta = {"transformers": transformers.__version__, "torch": torch.__version__,
            "dtype": "bfloat16", "attn_implementation": "eager", "device": "cpu",
            "model": dict(c), "weights": "tests/conftest.py qwen3_np_weights(QWEN3_06B, 0)",
            "prompt": prompt}
    np.savez_compressed(os.path.join(HERE, "hf_qwen3_06b_greedy.npz"), greedy=greedy,
                        greedy_gap=np.array(gaps, np.float32), top_values=np.array(top_v),
                        top_indices=np.array(top_i), full_steps=np.array(FULL_06B_STEPS, np.int32),
                        full_logits=full, meta=np.array(json.dumps(meta)))
    print("wrote hf_qwen3_06b_greedy.npz:", greedy[:8], "min gap", min(gaps))


if __name__ == "__main__":
    which = sys.argv[1:] or ["small", "dumps", "0.6B"]
    if "small" in which:
        small_fixture()
    if "dumps" in which:
        small_dumps_fixture()
    if "0.6B" in which:
        qwen06b_fixture()
