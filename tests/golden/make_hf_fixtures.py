"""Writes tests/golden/hf_small_qwen3.npz: the HF-transformers Qwen3 path (the reference's parity
path, ref/dump.py:124: bf16 weights, eager attention, on the CPU) run on the small seeded model of
tests/conftest.py (SMALL, small_weights(0)).

Recorded, for the token sequence TOKENS:
  logits      [len(TOKENS), vocab] fp32: teacher-forced logits at every position (one forward)
  greedy      [GREEDY_STEPS] int32: greedy tokens after PROMPT (model.generate, no sampling)
  greedy_gap  [GREEDY_STEPS] fp32: top-1 minus top-2 logit at each greedy step

These pin what no closed form does: the HF fp32/bf16 CPU arithmetic end to end (the e2e logits
within 2e-2 and the greedy sequence up to near ties). The fixture is data; this script is the
only place transformers is imported, and only here (never on the GPU box).

Run from the repository root:  python tests/golden/make_hf_fixtures.py
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


def main():
    import torch
    import transformers
    from transformers import Qwen3Config, Qwen3ForCausalLM

    from conftest import SMALL, small_weights

    c = SMALL
    cfg = Qwen3Config(
        vocab_size=c["vocab_size"], hidden_size=c["hidden_size"],
        intermediate_size=c["intermediate_size"], num_hidden_layers=c["n_layers"],
        num_attention_heads=c["n_heads"], num_key_value_heads=c["n_kv_heads"],
        head_dim=c["head_dim"], max_position_embeddings=64, rms_norm_eps=1e-6,
        rope_parameters={"rope_type": "default", "rope_theta": 1e6}, tie_word_embeddings=True,
        attention_bias=False, hidden_act="silu", attn_implementation="eager")
    torch.manual_seed(0)
    model = Qwen3ForCausalLM(cfg).to(torch.bfloat16).eval()
    w = small_weights(0)
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


if __name__ == "__main__":
    main()
