"""How far exact arithmetic is from HF transformers' CPU path over the whole vocabulary, at the
Qwen3-0.6B fixture's full-logit steps (tests/golden/hf_qwen3_06b_greedy.npz): the oracle's EXACT
mode (double accumulation, libm transcendentals, bf16 at HF's rounding points) and its GPU_ORDER
mode (the HIP kernels' fp32 order, which the GPU step equals bit for bit) are teacher-forced on
HF's tokens, and each step's 151936 logits are compared with HF's. This separates what any
summation order loses to 28 layers of bf16 rounding from what the kernels' order adds.

Writes tests/golden/exact_oracle_vs_hf.json: per full-logit step, each mode's max-abs difference
from HF and the bf16 ulp of HF's largest |logit| in that row. The GPU step test holds the GPU's
per-step max-abs to the EXACT mode's plus one such ulp.

CPU only, about 5 minutes on 8 cores. Run from the repository root:
    python tests/golden/exact_oracle_vs_hf.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(HERE)), "oracle"))

import oracle  # noqa: E402
from conftest import QWEN3_06B, bf16_vals, qwen3_np_weights, ulp_bf16  # noqa: E402


def main():
    f = np.load(os.path.join(HERE, "hf_qwen3_06b_greedy.npz"))
    meta = json.loads(str(f["meta"]))
    c = QWEN3_06B
    cfg = dict(hidden_size=c["hidden_size"], intermediate_size=c["intermediate_size"],
               n_layers=c["n_layers"], n_heads=c["n_heads"], n_kv_heads=c["n_kv_heads"],
               head_dim=c["head_dim"], vocab_size=c["vocab_size"], rms_norm_eps=1e-6,
               rope_theta=1e6)
    w = qwen3_np_weights(c, 0)
    prompt, ref = meta["prompt"], [int(x) for x in f["greedy"]]
    full_steps = [int(x) for x in f["full_steps"]]
    last = max(full_steps)
    record = {"full_steps": full_steps, "source": "oracle teacher-forced on HF's tokens vs "
              "tests/golden/hf_qwen3_06b_greedy.npz full_logits"}
    for mode, name in [(oracle.EXACT, "EXACT"), (oracle.GPU_ORDER, "GPU_ORDER")]:
        orc = oracle.Model(cfg, w, max_seq=len(prompt) + last + 8)
        for pos, tok in enumerate(prompt[:-1]):
            orc.forward(tok, pos, mode)
        tok, worst, over, ulps = prompt[-1], 0.0, 0, 0.0
        per_step, units = [], []
        for i in range(last + 1):
            orc.forward(tok, len(prompt) - 1 + i, mode)
            if i in full_steps:
                lg = bf16_vals(orc.logits).astype(np.float64)
                hf = bf16_vals(f["full_logits"][full_steps.index(i)]).astype(np.float64)
                d = np.abs(lg - hf)
                worst = max(worst, float(d.max()))
                over += int(np.sum(d > 2e-2))
                unit = float(ulp_bf16(np.abs(hf).max()))
                ulps = max(ulps, float(d.max()) / unit)
                per_step.append(float(d.max()))
                units.append(unit)
            tok = ref[i]
        n = len(full_steps) * f["full_logits"].shape[1]
        print(f"{name}: max-abs {worst:.4f} over {n} logits at steps {full_steps}; {over} above "
              f"2e-2; at most {ulps:.2f} bf16 ulps of the row's largest logit", flush=True)
        record[name] = {"max_abs_per_step": per_step, "max_abs": worst, "above_2e-2": over}
        record["row_ulp_per_step"] = units
    with open(os.path.join(HERE, "exact_oracle_vs_hf.json"), "w") as fh:
        json.dump(record, fh, indent=1)


if __name__ == "__main__":
    main()
