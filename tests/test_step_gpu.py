"""End-to-end decode on the GPU against the CPU oracle's whole-step restatement.

The step (src/forward.cu:118-193 order, the gfx950 kernels) must give logits bit-identical to
the oracle's GPU-order step at every position, eager and graph-replayed alike, and greedy
sequences bit-identical over 32 (Qwen3-0.6B shapes) and 256 tokens. A small model goes through
the safetensors loader so the loader's tensors, checksums and tied LM head are checked on the
same path."""
import json
import struct

import numpy as np
import pytest

from conftest import SMALL, bf16_bits, bf16_vals, rand_bf16, small_weights, ulp_bf16

pytestmark = pytest.mark.gpu

TIE_GAP = 0.25  # ref/compare.py:18: a greedy flip is accepted only below this top-2 gap


def ident(name):
    print(f"[case] {name}", flush=True)


def write_safetensors(path, tensors):
    """safetensors: u64 header length, JSON header, data; 16-byte-aligned offsets."""
    header, blobs, off = {}, [], 0
    for name, arr in tensors.items():
        b = np.ascontiguousarray(arr, dtype=np.uint16).tobytes()
        header[name] = {"dtype": "BF16", "shape": list(arr.shape), "data_offsets": [off, off + len(b)]}
        pad = (-len(b)) % 16
        blobs.append(b + b"\0" * pad)
        off += len(b) + pad
    h = json.dumps(header).encode()
    h += b" " * ((-len(h)) % 16)
    path.write_bytes(struct.pack("<Q", len(h)) + h + b"".join(blobs))


def oracle_cfg(c):
    return dict(hidden_size=c.hidden_size, intermediate_size=c.intermediate_size,
                n_layers=c.n_layers, n_heads=c.n_heads, n_kv_heads=c.n_kv_heads,
                head_dim=c.head_dim, vocab_size=c.vocab_size, rms_norm_eps=c.rms_norm_eps,
                rope_theta=c.rope_theta)


@pytest.fixture(scope="module")
def small_model(gpu, tmp_path_factory):
    from llm_inference_amd import model
    d = tmp_path_factory.mktemp("small_qwen3")
    w = small_weights()
    cfg = {"hidden_size": 256, "intermediate_size": 512, "num_hidden_layers": 2,
           "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 128,
           "vocab_size": 1000, "max_position_embeddings": 64, "rms_norm_eps": 1e-6,
           "rope_theta": 1000000.0, "tie_word_embeddings": True}
    (d / "config.json").write_text(json.dumps(cfg))
    (d / "generation_config.json").write_text(json.dumps({"eos_token_id": 3}))
    # split over two shards, in reverse name order, to exercise the multi-shard lookup
    names = list(w)
    write_safetensors(d / "model-00002.safetensors", {n: w[n] for n in names[::2]})
    write_safetensors(d / "model-00001.safetensors", {n: w[n] for n in names[1::2]})
    c = model.load_config(d)
    dec = model.Decoder(c, d)
    yield dec, w
    dec.close()


def test_loader_tensors_and_checksums(small_model, capfd):
    """Every tensor round-trips bit-exactly; print_weight_checksums matches the numpy
    computation of ref/weight_checksums.py (sum and index-weighted sum of the raw bits, mod 2^64)."""
    ident("loader checksums")
    dec, w = small_model
    assert dec.w.n_tensors == len(w) and dec.w.lm_head == dec.w.embed
    for name, arr in w.items():
        assert np.array_equal(dec.host_tensor(name), arr.reshape(-1)), name
    import ctypes
    from llm_inference_amd import lib
    capfd.readouterr()
    lib().print_weight_checksums(ctypes.byref(dec.w))
    lines = capfd.readouterr().out.strip().splitlines()
    got = {l.split()[0]: l.split()[1:] for l in lines}
    for name, arr in w.items():
        bits = arr.reshape(-1).astype(np.uint64)
        with np.errstate(over="ignore"):
            total = int(bits.sum(dtype=np.uint64))
            weighted = int((bits * np.arange(1, bits.size + 1, dtype=np.uint64)).sum(dtype=np.uint64))
        first = float(bf16_vals(arr.reshape(-1)[:1])[0])
        assert got[name][:3] == [str(bits.size), str(total), str(weighted)], name
        assert float(got[name][3]) == pytest.approx(first, rel=1e-5)


def test_small_model_logits_bit_exact(small_model, oracle):
    """Eager step vs the oracle step: logits and KV caches bit-identical at every position;
    then the captured graph replays the same positions with identical logits."""
    ident("small model eager + graph vs oracle")
    dec, w = small_model
    orc = oracle.Model(oracle_cfg(dec.cfg), w, max_seq=dec.s.max_seq)
    tokens = [17, 999, 0, 512, 3, 77, 640, 1, 2, 900, 45, 300]
    eager = []
    for pos, tok in enumerate(tokens):
        dec.forward(tok, pos)
        nxt = dec.sample_argmax()
        lg = dec.logits()
        eo = orc.forward(tok, pos, oracle.GPU_ORDER)
        assert np.array_equal(lg, orc.logits), pos
        assert nxt == eo
        eager.append(lg)
    k, v = dec.kv_cache()
    n = len(tokens)
    assert np.array_equal(k[:, :n].reshape(-1), orc.bufs["key_cache"].reshape(k.shape)[:, :n].reshape(-1))
    assert np.array_equal(v[:, :n].reshape(-1), orc.bufs["value_cache"].reshape(v.shape)[:, :n].reshape(-1))
    dec.capture_graph()
    for pos, tok in enumerate(tokens):
        dec.forward(tok, pos)
        dec.sample_argmax()
        assert np.array_equal(dec.logits(), eager[pos]), pos


def test_generate_greedy_matches_step_loop(small_model, oracle):
    """The on-device loop (argmax fed back, position advanced by a kernel) gives the same tokens
    as forward + sample_argmax per step and as the oracle."""
    ident("generate_greedy vs step loop")
    dec, w = small_model
    prompt = [5, 60, 700, 8, 91]
    for pos, tok in enumerate(prompt):
        dec.forward(tok, pos)
    first = dec.sample_argmax()
    loop = dec.generate_greedy(first, len(prompt), 40)
    for pos, tok in enumerate(prompt):
        dec.forward(tok, pos)
    t = dec.sample_argmax()
    step = []
    for i in range(40):
        dec.forward(t, len(prompt) + i)
        t = dec.sample_argmax()
        step.append(t)
    assert loop == step
    orc = oracle.Model(oracle_cfg(dec.cfg), w, max_seq=dec.s.max_seq)
    for pos, tok in enumerate(prompt):
        t = orc.forward(tok, pos)
    ref = []
    for i in range(40):
        t = orc.forward(t, len(prompt) + i)
        ref.append(t)
    assert loop == ref


def test_sample_temperature_step(small_model, oracle):
    """sample_temperature after a step draws from the step's logits as the oracle does
    (src/forward.cu:238-251), with the same coin; coin 0 gives the first token with weight."""
    ident("sample_temperature")
    dec, _ = small_model
    dec.capture_graph()
    for pos, tok in enumerate([4, 8, 15, 16]):
        dec.forward(tok, pos)
    lg = dec.logits()
    for temp, coin in [(1.0, 0.3), (0.5, 0.77), (2.0, 0.05), (1.0, 0.0)]:
        assert dec.sample_temperature(temp, coin) == oracle.sample(lg, np.float32(1.0 / temp), coin)


# ref/compare.py:13-18: worst-row relative L2 error per dumped tensor (embed and layer 0 held
# tighter), and the near-tie rule for the logits' argmax
DUMP_TOL_FIRST, DUMP_TOL = 0.02, 0.15


def test_small_model_dumps_match_hf(small_model, tmp_path):
    """Activation dumps (include/llm_amd/dump.h) of the eager step over the fixture's tokens
    against HF transformers' own tensors at the same points (tests/golden/hf_small_qwen3_dumps.npz,
    the reference's dump taxonomy): every tensor present with one row per position, worst-row
    relative L2 within ref/compare.py's tolerances, embedding rows bit-exact, the residual adds
    exactly bf16(x + y) (ref/dump.py:101-108), and the logits' argmax equal up to a near tie."""
    import json
    import os
    import llm_inference_amd as lia
    ident("dumps vs HF")
    dec, _ = small_model
    here = os.path.dirname(os.path.abspath(__file__))
    ref = np.load(os.path.join(here, "golden", "hf_small_qwen3_dumps.npz"))
    tokens = json.loads(str(np.load(os.path.join(here, "golden", "hf_small_qwen3.npz"))["meta"]))["tokens"]
    d = tmp_path / "dumps"
    lia.dump_open(d)
    try:
        for pos, tok in enumerate(tokens):
            dec.forward(tok, pos)
            dec.sample_argmax()
    finally:
        lia.dump_close()
    mine = {}
    for name in ref.files:
        raw = np.fromfile(d / f"{name}.bin", dtype=np.float32)
        width = ref[name].shape[1]
        assert raw.size == len(tokens) * width, (name, raw.size)
        mine[name] = raw.reshape(len(tokens), width).astype(np.float64)
    assert sorted(mine) == sorted(ref.files)
    assert len([f for f in os.listdir(d) if f.endswith(".bin")]) == len(ref.files)
    worst = {}
    for name in ref.files:
        r = bf16_vals(ref[name]).astype(np.float64)
        err = (np.linalg.norm(mine[name] - r, axis=1) / np.linalg.norm(r, axis=1)).max()
        tol = DUMP_TOL_FIRST if name == "embed" or name.startswith("L00.") else DUMP_TOL
        assert err <= tol, (name, float(err))
        worst[name] = float(err)
    assert np.array_equal(mine["embed"], bf16_vals(ref["embed"]).astype(np.float64))

    def bf16_add(a, b):
        return bf16_vals(bf16_bits((a + b).astype(np.float32))).astype(np.float64)
    x = mine["embed"]
    for l in range(SMALL["n_layers"]):
        p = f"L{l:02d}."
        assert np.array_equal(mine[p + "attn_resid"], bf16_add(x, mine[p + "o_proj"]))
        x = mine[p + "out"]
        assert np.array_equal(x, bf16_add(mine[p + "attn_resid"], mine[p + "down"]))
    lg, rl = mine["logits"], bf16_vals(ref["logits"]).astype(np.float64)
    for t in range(len(tokens)):
        a, b = int(lg[t].argmax()), int(rl[t].argmax())
        assert a == b or rl[t, b] - rl[t, a] <= TIE_GAP, (t, a, b)
    top = sorted(worst.items(), key=lambda kv: -kv[1])[:3]
    print("[case] worst tensors: " + ", ".join(f"{n} {e:.4f}" for n, e in top), flush=True)


def test_small_model_matches_hf_fixture(small_model):
    """The GPU step (loaded through the safetensors loader) against HF transformers' Qwen3 on the
    same weights (tests/golden/hf_small_qwen3.npz: bf16, eager attention, CPU): teacher-forced
    logits within 2e-2 at every position, and the greedy tokens after the fixture's prompt equal
    to HF's up to a near tie (top-2 gap <= TIE_GAP where they part)."""
    import json
    import os
    ident("small model vs HF fixture")
    dec, _ = small_model
    f = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                             "hf_small_qwen3.npz"))
    meta = json.loads(str(f["meta"]))
    dec.capture_graph()
    for pos, tok in enumerate(meta["tokens"]):
        dec.forward(tok, pos)
        dec.sample_argmax()
        diff = np.abs(bf16_vals(dec.logits()).astype(np.float64) - f["logits"][pos])
        assert diff.max() <= 2e-2, (pos, float(diff.max()))
    prompt = meta["prompt"]
    for pos, tok in enumerate(prompt):
        dec.forward(tok, pos)
    first = dec.sample_argmax()
    got = [first] + dec.generate_greedy(first, len(prompt), len(f["greedy"]) - 1)
    for i, (a, b) in enumerate(zip(got, [int(x) for x in f["greedy"]])):
        if a != b:
            assert f["greedy_gap"][i] <= TIE_GAP, (i, a, b, float(f["greedy_gap"][i]))
            break


def test_qwen3_06b_greedy_256_vs_hf_fixture(gpu):
    """Qwen3-0.6B shapes with the seeded numpy weights of the HF fixture
    (tests/golden/hf_qwen3_06b_greedy.npz: transformers' Qwen3, bf16, eager attention, CPU; 256
    greedy tokens after the bench's prompt), persistent step, teacher-forced on HF's tokens so
    every step sees HF's context: at all 256 steps the GPU's logits at HF's 8 largest indices are
    within 2 bf16 ulps of HF's, and wherever HF's top-2 gap exceeds 0.07 (more than the two
    sides' combined error) the GPU's argmax is HF's token. Two ulps, not the 2e-2 logit bound:
    after 28 layers of bf16 rounding, the oracle's exact-arithmetic mode (double accumulation,
    libm transcendentals) is itself 2 ulps (0.031 at |logit| ~2.7) from HF's CPU path at some of
    these steps, so no summation order meets 2e-2 everywhere. At the fixture's 9 full-vocabulary
    steps (0, 32, ..., 224, 255) every one of the 151936 logits is compared: the max-abs
    difference is printed against the 2e-2 logit bound (with the count of logits above it), and
    at every such step the GPU's max-abs difference from HF may exceed the exact mode's (the
    oracle teacher-forced the same way, tests/golden/exact_oracle_vs_hf.json, written by
    exact_oracle_vs_hf.py) by at most one bf16 ulp of the row's largest logit: the GPU is as
    close to HF as exact arithmetic is, step by step. (With N(0, 0.02) weights the logits are
    flat: most steps are near ties, where either token is a correct greedy choice,
    ref/greedy.py:14-31.)"""
    import json
    import os
    from llm_inference_amd import model
    from conftest import QWEN3_06B, qwen3_np_weights
    ident("0.6B 256 steps vs HF fixture (teacher-forced)")
    f = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                             "hf_qwen3_06b_greedy.npz"))
    meta = json.loads(str(f["meta"]))
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                           "exact_oracle_vs_hf.json")) as fh:
        rel = json.load(fh)
    ref = [int(x) for x in f["greedy"]]
    cfg = model.qwen3_config("0.6B", max_seq_len=len(meta["prompt"]) + len(ref) + 8)
    dec = model.Decoder(cfg, ("synth", 0, 0.02, 0.1))
    try:
        dec.set_weights(qwen3_np_weights(QWEN3_06B, 0))
        dec.capture_graph("persistent")
        prompt = meta["prompt"]
        for pos, tok in enumerate(prompt):
            dec.forward(tok, pos)
        decided = agree = 0
        worst = 0.0
        full_steps = [int(x) for x in f["full_steps"]]
        assert rel["full_steps"] == full_steps
        full_worst, full_ulps, full_over = 0.0, 0, 0
        beyond_exact = []  # per full step: GPU max-abs - exact mode's, in row ulps
        for i in range(len(ref)):
            got = dec.sample_argmax()
            lg = bf16_vals(dec.logits()).astype(np.float64)
            hf = f["top_values"][i].astype(np.float64)
            diff = np.abs(lg[f["top_indices"][i]] - hf)
            worst = max(worst, float(diff.max()))
            assert np.all(diff <= 2 * ulp_bf16(hf)), (i, float(diff.max()))
            if i in full_steps:
                # every logit of the step against HF's (bf16 bits)
                hf_all = bf16_vals(f["full_logits"][full_steps.index(i)]).astype(np.float64)
                d_all = np.abs(lg - hf_all)
                full_worst = max(full_worst, float(d_all.max()))
                full_over += int(np.sum(d_all > 2e-2))
                # in ulps of the row's largest logit: the error of a logit comes from the error
                # of the final hidden vector, on the scale of the row, not of its own value
                unit = float(ulp_bf16(np.abs(hf_all).max()))
                full_ulps = max(full_ulps, float(d_all.max()) / unit)
                j = full_steps.index(i)
                assert unit == rel["row_ulp_per_step"][j], i
                beyond_exact.append((float(d_all.max()) - rel["EXACT"]["max_abs_per_step"][j])
                                    / unit)
                assert float(d_all.max()) <= rel["EXACT"]["max_abs_per_step"][j] + unit, \
                    (i, float(d_all.max()), rel["EXACT"]["max_abs_per_step"][j], unit)
            if f["greedy_gap"][i] > 0.07:
                decided += 1
                agree += got == ref[i]
                assert got == ref[i], (i, got, ref[i], float(f["greedy_gap"][i]))
            if i + 1 < len(ref):
                dec.forward(ref[i], len(prompt) + i)  # HF's token: the same context as HF's
        print(f"[case] max logit diff {worst:.4f}; argmax equal at {agree}/{decided} decided steps",
              flush=True)
        print(f"[case] all {f['full_logits'].shape[1]} logits at steps {full_steps}: max-abs "
              f"{full_worst:.4f} (logit bound 2e-2), {full_over} of "
              f"{len(full_steps) * f['full_logits'].shape[1]} logits above 2e-2, at most "
              f"{full_ulps:.2f} bf16 ulps of the row's largest logit; beyond the exact "
              f"mode's max-abs by at most {max(beyond_exact):.2f} such ulps (bound 1)", flush=True)
    finally:
        dec.close()


@pytest.fixture(scope="module")
def qwen06b(gpu):
    from llm_inference_amd import model
    cfg = model.qwen3_config("0.6B", max_seq_len=512)
    dec = model.Decoder(cfg, ("synth", 0, 0.02, 0.1))
    w = dec.host_weights()
    yield dec, w
    dec.close()


def _prompt(seed=0):
    return [int(t) for t in np.random.default_rng(seed).integers(0, 151936, 5)]


@pytest.mark.parametrize("mode", ["graph", "persistent"])
def test_qwen3_06b_greedy_32_bit_exact(qwen06b, oracle, mode):
    """Qwen3-0.6B shapes, seeded N(0, 0.02) weights: 5-token prompt + 32 greedy tokens, GPU
    (hipGraph of the per-layer kernels, or the persistent step kernel; both replayed on the
    device) == oracle GPU-order, token for token."""
    ident(f"0.6B greedy 32 {mode}")
    dec, w = qwen06b
    prompt = _prompt()
    dec.capture_graph(mode)
    assert dec.persistent == (mode == "persistent")
    for pos, tok in enumerate(prompt):
        dec.forward(tok, pos)
    first = dec.sample_argmax()
    got = [first] + dec.generate_greedy(first, len(prompt), 31)
    orc = oracle.Model(oracle_cfg(dec.cfg), w, max_seq=dec.s.max_seq)
    for pos, tok in enumerate(prompt):
        t = orc.forward(tok, pos, oracle.GPU_ORDER)
    ref = [t]
    for i in range(31):
        t = orc.forward(t, len(prompt) + i, oracle.GPU_ORDER)
        ref.append(t)
    assert got == ref


def test_qwen3_06b_greedy_256_vs_exact_oracle(qwen06b, oracle):
    """256 greedy tokens: identical to the GPU-order oracle; against the exact-arithmetic oracle
    (double accumulation) the sequences may part only at a near tie (top-2 gap <= TIE_GAP,
    ref/greedy.py:14-31)."""
    ident("0.6B greedy 256")
    dec, w = qwen06b
    dec.capture_graph("persistent")
    prompt = _prompt(1)
    for pos, tok in enumerate(prompt):
        dec.forward(tok, pos)
    first = dec.sample_argmax()
    got = [first] + dec.generate_greedy(first, len(prompt), 255)
    orc = oracle.Model(oracle_cfg(dec.cfg), w, max_seq=dec.s.max_seq)
    for pos, tok in enumerate(prompt):
        t = orc.forward(tok, pos, oracle.GPU_ORDER)
    ref = [t]
    for i in range(255):
        t = orc.forward(t, len(prompt) + i, oracle.GPU_ORDER)
        ref.append(t)
    assert got == ref
    ex = oracle.Model(oracle_cfg(dec.cfg), w, max_seq=dec.s.max_seq)
    for pos, tok in enumerate(prompt):
        t = ex.forward(tok, pos, oracle.EXACT)
    exact, gaps = [t], [float(np.diff(np.sort(bf16_vals(ex.logits))[-2:])[0])]
    for i in range(255):
        t = ex.forward(got[i], len(prompt) + i, oracle.EXACT)  # teacher-forced on our tokens
        exact.append(t)
        gaps.append(float(np.diff(np.sort(bf16_vals(ex.logits))[-2:])[0]))
    flips = [(i, gaps[i]) for i in range(256) if exact[i] != got[i]]
    print(f"teacher-forced agreement with exact arithmetic: {256 - len(flips)}/256, flips {flips}")
    assert all(g <= TIE_GAP for _, g in flips), flips


def test_persistent_step_logits_per_position(gpu, oracle):
    """The persistent step on the smallest specialised shapes (hidden 512, 8/4 heads,
    intermediate 1024): logits and the fused argmax bit-identical to the oracle at every
    position, and identical to the hipGraph step."""
    ident("persistent step small shapes")
    from llm_inference_amd import model
    cfg = model.make_config(hidden_size=512, intermediate_size=1024, n_layers=3, n_heads=8,
                            n_kv_heads=4, vocab_size=5000, max_seq_len=200)
    dec = model.Decoder(cfg, ("synth", 3, 0.02, 0.1))
    try:
        w = dec.host_weights()
        orc = oracle.Model(oracle_cfg(cfg), w, max_seq=200)
        tokens = [int(t) for t in np.random.default_rng(5).integers(0, 5000, 150)]
        dec.capture_graph("persistent")
        per = []
        for pos, tok in enumerate(tokens):
            dec.forward(tok, pos)
            nxt = dec.sample_argmax()
            ref = orc.forward(tok, pos, oracle.GPU_ORDER)
            assert np.array_equal(dec.logits(), orc.logits), pos
            assert nxt == ref, pos
            per.append(dec.logits())
        dec.capture_graph("graph")
        for pos, tok in enumerate(tokens[:70]):
            dec.forward(tok, pos)
            dec.sample_argmax()
            assert np.array_equal(dec.logits(), per[pos]), pos
    finally:
        dec.close()


def test_persistent_generate_one_launch_small(gpu, oracle):
    """generate_greedy in persistent mode decodes every token in ONE launch (each token's argmax
    feeds the next inside the kernel; KV rows written earlier in the launch are read back by the
    other heads of the group). 150 tokens on the smallest specialised shapes cross the 64- and
    128-position block edges: tokens equal the oracle's and per-token persistent launches'."""
    ident("persistent one-launch generate small shapes")
    from llm_inference_amd import model
    cfg = model.make_config(hidden_size=512, intermediate_size=1024, n_layers=3, n_heads=8,
                            n_kv_heads=4, vocab_size=5000, max_seq_len=200)
    dec = model.Decoder(cfg, ("synth", 4, 0.02, 0.1))
    try:
        w = dec.host_weights()
        prompt = [17, 4000, 250, 3]
        dec.capture_graph("persistent")
        for pos, tok in enumerate(prompt):
            dec.forward(tok, pos)
        first = dec.sample_argmax()
        got = dec.generate_greedy(first, len(prompt), 150)
        t, per = first, []
        for i in range(150):
            dec.forward(t, len(prompt) + i)
            t = dec.sample_argmax()
            per.append(t)
        assert got == per
        orc = oracle.Model(oracle_cfg(cfg), w, max_seq=200)
        for pos, tok in enumerate(prompt):
            t = orc.forward(tok, pos, oracle.GPU_ORDER)
        ref = []
        for i in range(150):
            t = orc.forward(t, len(prompt) + i, oracle.GPU_ORDER)
            ref.append(t)
        assert got == ref
        # a second call continues from the state the first left
        more = dec.generate_greedy(got[-1], len(prompt) + 150, 20)
        for i in range(20):
            t = orc.forward(t, len(prompt) + 150 + i, oracle.GPU_ORDER)
            assert more[i] == t, i
    finally:
        dec.close()


@pytest.mark.parametrize("head_dim,attn", [(64, "in_scores"), (64, "separate"),
                                           (256, "in_scores"), (256, "separate")])
def test_graph_step_other_head_dims(gpu, oracle, head_dim, attn):
    """The hipGraph step at head_dim 64 and 256 (shapes with no persistent kernel: STEP_AUTO
    captures the graph), in both attention forms: QK-norm + RoPE inside the scores pass reading
    the step's RoPE table (rope_table_kernel), and qk_norm_rope_forward + attention_forward; at
    these head dims the PV and combine passes are two launches. Logits bit-identical to the
    oracle at positions 0-69 (crossing the first 64-position block) of a prompt fed one token at
    a time, then a 24-token generate_greedy equal to the oracle's."""
    ident(f"graph step head_dim {head_dim} {attn}")
    from llm_inference_amd import model
    cfg = model.make_config(hidden_size=512, intermediate_size=1024, n_layers=2, n_heads=8,
                            n_kv_heads=4, head_dim=head_dim, vocab_size=3000, max_seq_len=128)
    dec = model.Decoder(cfg, ("synth", head_dim, 0.02, 0.1))
    try:
        w = dec.host_weights()
        orc = oracle.Model(oracle_cfg(cfg), w, max_seq=128)
        dec.s.attn_mode = model.ATTN_MODES[attn]
        dec.capture_graph("auto")
        assert not dec.persistent
        rng = np.random.default_rng(head_dim)
        tok = 0
        for pos in range(70):
            tok = int(rng.integers(0, cfg.vocab_size))
            dec.forward(tok, pos)
            nxt = dec.sample_argmax()
            ref = orc.forward(tok, pos, oracle.GPU_ORDER)
            assert np.array_equal(dec.logits(), orc.logits), pos
            assert nxt == ref, pos
        got = dec.generate_greedy(nxt, 70, 24)
        want, t = [], nxt
        for i in range(24):
            t = orc.forward(t, 70 + i, oracle.GPU_ORDER)
            want.append(t)
        assert got == want
    finally:
        dec.close()


@pytest.mark.parametrize("n_heads", [4, 8, 16, 32])
def test_graph_step_pv_combine_one_launch(gpu, oracle, n_heads):
    """At head_dim 128 the graph step runs attention's PV and combine passes as one launch
    (attn_pv_combine_kernel): every item publishes its block partials as tagged words and the
    items of the T last blocks of each kv head add them in block order, T the largest power of
    two <= min(blocks, REP * 128 / 16). 4 kv heads with n_heads / 4 = 1, 2, 4 or 8 query heads
    each, a 16580-position N(0, 1) cache: logits bit-identical to the oracle at positions holding
    1 to 260 blocks (T = 1 to 32; two staged chunks of partials past 256 blocks), in both
    attention forms, then a short generate_greedy equal to the oracle's."""
    ident(f"graph step one-launch PV + combine, {n_heads}/4 heads")
    from llm_inference_amd import model
    max_seq = 16640
    cfg = model.make_config(hidden_size=512, intermediate_size=1024, n_layers=1,
                            n_heads=n_heads, n_kv_heads=4, vocab_size=3000, max_seq_len=max_seq)
    dec = model.Decoder(cfg, ("synth", 40 + n_heads, 0.02, 0.1))
    try:
        rng = np.random.default_rng(n_heads)
        kvd = cfg.n_kv_heads * cfg.head_dim
        k = np.zeros((1, max_seq, kvd), np.uint16)
        v = np.zeros_like(k)
        k[:, :16580] = rand_bf16(rng, (1, 16580, kvd))
        v[:, :16580] = rand_bf16(rng, (1, 16580, kvd))
        dec.set_kv_cache(k, v)
        w = dec.host_weights()
        orc = oracle.Model(oracle_cfg(cfg), w, max_seq=max_seq)
        orc.bufs["key_cache"][:] = k.reshape(-1)
        orc.bufs["value_cache"][:] = v.reshape(-1)
        for attn in ("in_scores", "separate"):
            dec.s.attn_mode = model.ATTN_MODES[attn]
            dec.capture_graph("graph")
            assert not dec.persistent
            for pos in (0, 63, 64, 191, 500, 1023, 1100, 2100, 16383, 16384, 16579):
                tok = int(rng.integers(0, cfg.vocab_size))
                dec.forward(tok, pos)
                nxt = dec.sample_argmax()
                ref = orc.forward(tok, pos, oracle.GPU_ORDER)
                assert np.array_equal(dec.logits(), orc.logits), (attn, pos)
                assert nxt == ref, (attn, pos)
            got = dec.generate_greedy(nxt, 16580, 6)
            t, want = nxt, []
            for i in range(6):
                t = orc.forward(t, 16580 + i, oracle.GPU_ORDER)
                want.append(t)
            assert got == want, attn
    finally:
        dec.close()


@pytest.mark.parametrize("n_heads,n_kv_heads,max_seq", [(8, 1, 100), (8, 8, 130), (2, 2, 64)])
def test_graph_step_pv_combine_small_grids(gpu, oracle, n_heads, n_kv_heads, max_seq):
    """The one-launch PV + combine on small grids: one kv head with 8 query heads (1024 columns,
    4 per thread when one item combines them all), 8 kv heads of one query head, and a cache of
    a single 64-position block (one item per kv head, which both computes and combines). Every
    position of the cache stepped through in both attention forms: logits bit-identical to the
    oracle."""
    ident(f"graph step one-launch PV + combine, {n_heads}/{n_kv_heads} heads, {max_seq} slots")
    from llm_inference_amd import model
    cfg = model.make_config(hidden_size=512, intermediate_size=1024, n_layers=1,
                            n_heads=n_heads, n_kv_heads=n_kv_heads, vocab_size=2000,
                            max_seq_len=max_seq)
    dec = model.Decoder(cfg, ("synth", 60 + n_heads + n_kv_heads, 0.02, 0.1))
    try:
        w = dec.host_weights()
        orc = oracle.Model(oracle_cfg(cfg), w, max_seq=max_seq)
        rng = np.random.default_rng(max_seq)
        for attn in ("in_scores", "separate"):
            dec.s.attn_mode = model.ATTN_MODES[attn]
            dec.capture_graph("graph")
            assert not dec.persistent
            for pos in range(max_seq):
                tok = int(rng.integers(0, cfg.vocab_size))
                dec.forward(tok, pos)
                nxt = dec.sample_argmax()
                ref = orc.forward(tok, pos, oracle.GPU_ORDER)
                assert np.array_equal(dec.logits(), orc.logits), (attn, pos)
                assert nxt == ref, (attn, pos)
    finally:
        dec.close()


def test_auto_step_switches_to_graph_at_switch_pos(gpu, oracle):
    """STEP_AUTO prepares the persistent kernel for the positions below its switch position
    (736 at hidden <= 1024) and the hipGraph from there on: single steps on either side of the
    switch and one generate_greedy call that crosses it (36 tokens in the kernel's launch, 28
    graph replays continuing from the token and position it left) equal the oracle, on the
    smallest specialised shapes after a 700-position N(0, 1) cache."""
    ident("auto step switch small shapes")
    from llm_inference_amd import model
    cfg = model.make_config(hidden_size=512, intermediate_size=1024, n_layers=3, n_heads=8,
                            n_kv_heads=4, vocab_size=5000, max_seq_len=800)
    dec = model.Decoder(cfg, ("synth", 6, 0.02, 0.1))
    try:
        rng = np.random.default_rng(736)
        kvd = cfg.n_kv_heads * cfg.head_dim
        k = np.zeros((cfg.n_layers, 800, kvd), np.uint16)
        v = np.zeros_like(k)
        k[:, :700] = rand_bf16(rng, (cfg.n_layers, 700, kvd))
        v[:, :700] = rand_bf16(rng, (cfg.n_layers, 700, kvd))
        dec.set_kv_cache(k, v)
        w = dec.host_weights()
        orc = oracle.Model(oracle_cfg(cfg), w, max_seq=800)
        orc.bufs["key_cache"][:] = k.reshape(-1)
        orc.bufs["value_cache"][:] = v.reshape(-1)
        dec.capture_graph("auto")
        assert dec.persistent and dec.s.step_switch_pos == 736
        assert dec.kernel_tokens(700, 64) == 36
        got = dec.generate_greedy(1234, 700, 64)
        t, ref = 1234, []
        for i in range(64):
            t = orc.forward(t, 700 + i, oracle.GPU_ORDER)
            ref.append(t)
        assert got == ref
        # single steps (rewriting a row as the oracle does): 735 in the kernel, 736 and 764 in
        # the graph
        for pos in (735, 736, 764):
            dec.forward(77 + pos, pos)
            nxt = dec.sample_argmax()
            want = orc.forward(77 + pos, pos, oracle.GPU_ORDER)
            assert np.array_equal(dec.logits(), orc.logits), pos
            assert nxt == want, pos
    finally:
        dec.close()


@pytest.mark.parametrize("split_blocks", [1, 3])
def test_persistent_split_attention_small(gpu, oracle, split_blocks):
    """The persistent step's split attention ((kv head, 64-position block) items over every
    workgroup, block statistics and partials exchanged as tagged words, the partials of half a
    head's columns added in block order by each of the last workgroups) on the smallest
    specialised shapes (8/4 heads): with the split from the first block (split_blocks 1) and
    from 128 positions (3), single steps at positions 0-69 and 1000-1003 after an N(0, 1) cache,
    and a generate_greedy call of 100 tokens from 100 (which crosses the 64-position block
    edges and, when split_blocks is 3, runs 100-127 in one launch of the per-head instance and
    128-199 in one of the split instance): logits, argmax and tokens bit-identical to the
    oracle."""
    ident(f"persistent split attention small shapes, split from {split_blocks} blocks")
    from llm_inference_amd import model
    S = 1100
    cfg = model.make_config(hidden_size=512, intermediate_size=1024, n_layers=3, n_heads=8,
                            n_kv_heads=4, vocab_size=5000, max_seq_len=S)
    dec = model.Decoder(cfg, ("synth", 8, 0.02, 0.1))
    try:
        rng = np.random.default_rng(split_blocks)
        kvd = cfg.n_kv_heads * cfg.head_dim
        k = np.zeros((cfg.n_layers, S, kvd), np.uint16)
        v = np.zeros_like(k)
        k[:, 200:1000] = rand_bf16(rng, (cfg.n_layers, 800, kvd))
        v[:, 200:1000] = rand_bf16(rng, (cfg.n_layers, 800, kvd))
        dec.set_kv_cache(k, v)
        w = dec.host_weights()
        orc = oracle.Model(oracle_cfg(cfg), w, max_seq=S)
        orc.bufs["key_cache"][:] = k.reshape(-1)
        orc.bufs["value_cache"][:] = v.reshape(-1)
        dec.capture_graph("persistent")
        assert dec.persistent
        dec.s.step_split_blocks = split_blocks
        tokens = [int(t) for t in rng.integers(0, cfg.vocab_size, 70)]
        for pos, tok in enumerate(tokens):
            dec.forward(tok, pos)
            nxt = dec.sample_argmax()
            ref = orc.forward(tok, pos, oracle.GPU_ORDER)
            assert np.array_equal(dec.logits(), orc.logits), pos
            assert nxt == ref, pos
        got = dec.generate_greedy(nxt, 70, 30)
        got += dec.generate_greedy(got[-1], 100, 100)
        t, want = nxt, []
        for pos in range(70, 200):
            t = orc.forward(t, pos, oracle.GPU_ORDER)
            want.append(t)
        assert got == want
        for pos in range(1000, 1004):
            tok = int(rng.integers(0, cfg.vocab_size))
            dec.forward(tok, pos)
            nxt = dec.sample_argmax()
            ref = orc.forward(tok, pos, oracle.GPU_ORDER)
            assert np.array_equal(dec.logits(), orc.logits), pos
            assert nxt == ref, pos
    finally:
        dec.close()


@pytest.mark.parametrize("size", ["1.7B", "4B"])
def test_persistent_step_wide_shapes(gpu, oracle, size):
    """The Qwen3-1.7B and -4B specialisations of the persistent step (their widths and heads,
    3 layers to keep the oracle quick): logits and argmax bit-identical to the oracle at 70
    positions (two 64-position attention blocks), then a one-launch generate of 20 tokens equal
    to the oracle's greedy tokens."""
    ident(f"persistent step {size} widths")
    from llm_inference_amd import model
    cfg = model.qwen3_config(size, n_layers=3, max_seq_len=128)
    dec = model.Decoder(cfg, ("synth", 11, 0.02, 0.1))
    try:
        dec.capture_graph("persistent")
        assert dec.persistent
        w = dec.host_weights()
        orc = oracle.Model(oracle_cfg(cfg), w, max_seq=128)
        tokens = [int(t) for t in np.random.default_rng(12).integers(0, cfg.vocab_size, 70)]
        for pos, tok in enumerate(tokens):
            dec.forward(tok, pos)
            nxt = dec.sample_argmax()
            ref = orc.forward(tok, pos, oracle.GPU_ORDER)
            assert np.array_equal(dec.logits(), orc.logits), pos
            assert nxt == ref, pos
        got = dec.generate_greedy(nxt, len(tokens), 20)
        t, want = nxt, []
        for i in range(20):
            t = orc.forward(t, len(tokens) + i, oracle.GPU_ORDER)
            want.append(t)
        assert got == want
    finally:
        dec.close()


def test_persistent_step_long_context(qwen06b, oracle):
    """One decode position at 5000 with the KV cache below it filled with N(0, 1): the
    persistent step's attention over 79 blocks of 64 positions is bit-identical to the
    oracle's."""
    ident("persistent step pos 5000")
    from llm_inference_amd import model
    dec0, w = qwen06b
    cfg = model.qwen3_config("0.6B", max_seq_len=5008)
    dec = model.Decoder(cfg, ("synth", 0, 0.02, 0.1))
    try:
        rng = np.random.default_rng(7)
        kvd = cfg.n_kv_heads * cfg.head_dim
        k = rand_bf16(rng, (cfg.n_layers, 5008, kvd))
        v = rand_bf16(rng, (cfg.n_layers, 5008, kvd))
        dec.set_kv_cache(k, v)
        orc = oracle.Model(oracle_cfg(cfg), w, max_seq=5008)
        orc.bufs["key_cache"][:] = k.reshape(-1)
        orc.bufs["value_cache"][:] = v.reshape(-1)
        dec.capture_graph("persistent")
        dec.forward(1234, 5000)
        nxt = dec.sample_argmax()
        ref = orc.forward(1234, 5000, oracle.GPU_ORDER)
        assert np.array_equal(dec.logits(), orc.logits)
        assert nxt == ref
        kk, vv = dec.kv_cache()
        assert np.array_equal(kk[:, 5000].reshape(-1),
                              orc.bufs["key_cache"].reshape(k.shape)[:, 5000].reshape(-1))
        assert np.array_equal(vv[:, 5000].reshape(-1),
                              orc.bufs["value_cache"].reshape(v.shape)[:, 5000].reshape(-1))
    finally:
        dec.close()


def test_persistent_step_4b_longest_history(gpu, oracle):
    """The 4B specialisation of the persistent step (four query heads per kv head) up to the end
    of an 8192-position cache (split attention over 128 blocks, two items per half-slot): one
    position at 8183, then an 8-token generate in one launch ending at 8191, after a KV cache
    filled with N(0, 1) below, full widths with 2 layers. Logits, argmax, the KV rows written and
    the generated tokens bit-identical to the oracle; position 8192 is refused."""
    ident("persistent step 4B widths at positions 8183..8191")
    from llm_inference_amd import LlmError, model
    S = 8192
    cfg = model.qwen3_config("4B", n_layers=2, max_seq_len=S)
    dec = model.Decoder(cfg, ("synth", 37, 0.02, 0.1))
    try:
        rng = np.random.default_rng(8183)
        kvd = cfg.n_kv_heads * cfg.head_dim
        k = rand_bf16(rng, (cfg.n_layers, S, kvd))
        v = rand_bf16(rng, (cfg.n_layers, S, kvd))
        dec.set_kv_cache(k, v)
        w = dec.host_weights()
        orc = oracle.Model(oracle_cfg(cfg), w, max_seq=S)
        del w
        orc.bufs["key_cache"][:] = k.reshape(-1)
        orc.bufs["value_cache"][:] = v.reshape(-1)
        dec.capture_graph("persistent")
        assert dec.persistent
        tok = int(rng.integers(0, cfg.vocab_size))
        dec.forward(tok, 8183)
        nxt = dec.sample_argmax()
        ref = orc.forward(tok, 8183, oracle.GPU_ORDER)
        assert np.array_equal(dec.logits(), orc.logits)
        assert nxt == ref
        kk, vv = dec.kv_cache()
        assert np.array_equal(kk[:, 8183], orc.bufs["key_cache"].reshape(k.shape)[:, 8183])
        assert np.array_equal(vv[:, 8183], orc.bufs["value_cache"].reshape(v.shape)[:, 8183])
        got = dec.generate_greedy(nxt, 8184, 8)
        t, want = nxt, []
        for i in range(8):
            t = orc.forward(t, 8184 + i, oracle.GPU_ORDER)
            want.append(t)
        assert got == want
        kk, vv = dec.kv_cache()
        assert np.array_equal(kk[:, 8184:], orc.bufs["key_cache"].reshape(k.shape)[:, 8184:])
        assert np.array_equal(vv[:, 8184:], orc.bufs["value_cache"].reshape(v.shape)[:, 8184:])
        with pytest.raises(LlmError, match="past the kv cache size 8192"):
            dec.forward(t, 8192)
        with pytest.raises(LlmError, match="pass the kv cache size 8192"):
            dec.generate_greedy(t, 8185, 8)
    finally:
        dec.close()


def test_persistent_step_4b_after_8192_positions(gpu, oracle):
    """The Qwen3-4B 8192-position config on the persistent step (split attention: 129-132 blocks,
    so some half-slots hold three (kv head, block) items): full 4B widths, 2 layers, the KV
    cache's first 8192 positions filled with N(0, 1), max_seq 8448. Logits and argmax
    bit-identical to the oracle at 8192 and 8193, one generate_greedy launch of 8 tokens from
    8194, and the last position 8447."""
    ident("persistent step 4B from 8192 positions")
    from llm_inference_amd import model
    S = 8448
    cfg = model.qwen3_config("4B", n_layers=2, max_seq_len=S)
    dec = model.Decoder(cfg, ("synth", 41, 0.02, 0.1))
    try:
        rng = np.random.default_rng(8448)
        kvd = cfg.n_kv_heads * cfg.head_dim
        k = np.zeros((cfg.n_layers, S, kvd), np.uint16)
        v = np.zeros_like(k)
        k[:, :8192] = rand_bf16(rng, (cfg.n_layers, 8192, kvd))
        v[:, :8192] = rand_bf16(rng, (cfg.n_layers, 8192, kvd))
        k[:, 8202:] = rand_bf16(rng, (cfg.n_layers, S - 8202, kvd))
        v[:, 8202:] = rand_bf16(rng, (cfg.n_layers, S - 8202, kvd))
        dec.set_kv_cache(k, v)
        w = dec.host_weights()
        orc = oracle.Model(oracle_cfg(cfg), w, max_seq=S)
        del w
        orc.bufs["key_cache"][:] = k.reshape(-1)
        orc.bufs["value_cache"][:] = v.reshape(-1)
        dec.capture_graph("persistent")
        assert dec.persistent
        tok = int(rng.integers(0, cfg.vocab_size))
        for pos in (8192, 8193):
            dec.forward(tok, pos)
            nxt = dec.sample_argmax()
            ref = orc.forward(tok, pos, oracle.GPU_ORDER)
            assert np.array_equal(dec.logits(), orc.logits), pos
            assert nxt == ref, pos
            tok = nxt
        got = dec.generate_greedy(tok, 8194, 8)
        want = []
        for i in range(8):
            tok = orc.forward(tok, 8194 + i, oracle.GPU_ORDER)
            want.append(tok)
        assert got == want
        kk, vv = dec.kv_cache()
        ok = orc.bufs["key_cache"].reshape(k.shape)
        ov = orc.bufs["value_cache"].reshape(v.shape)
        assert np.array_equal(kk[:, 8192:8202], ok[:, 8192:8202])
        assert np.array_equal(vv[:, 8192:8202], ov[:, 8192:8202])
        dec.forward(99, 8447)
        nxt = dec.sample_argmax()
        ref = orc.forward(99, 8447, oracle.GPU_ORDER)
        assert np.array_equal(dec.logits(), orc.logits)
        assert nxt == ref
    finally:
        dec.close()


def test_persistent_split_attention_longest_history(gpu, oracle):
    """The split attention at the longest history the persistent kernel holds: 192 blocks of 64
    positions (three items on half of the half-slots at Qwen3-0.6B's 8 kv heads on 256 CUs, the
    combine over every block the workspace holds), full 0.6B widths with 2 layers after an
    N(0, 1) cache. Position 12286 alone, then a generate of the last position, bit-identical to
    the oracle; a run state one position longer has no persistent step."""
    ident("persistent split attention at the longest history")
    from llm_inference_amd import LlmError, model
    probe = model.Decoder(model.qwen3_config("0.6B", n_layers=1, max_seq_len=64),
                          ("synth", 1, 0.02, 0.1))
    try:
        probe.capture_graph("persistent")
        grid = probe.s.step_grid
    finally:
        probe.close()
    S = min(192, 3 * (2 * grid // 8)) * 64
    cfg = model.qwen3_config("0.6B", n_layers=2, max_seq_len=S)
    dec = model.Decoder(cfg, ("synth", 43, 0.02, 0.1))
    try:
        rng = np.random.default_rng(S)
        kvd = cfg.n_kv_heads * cfg.head_dim
        k = rand_bf16(rng, (cfg.n_layers, S, kvd))
        v = rand_bf16(rng, (cfg.n_layers, S, kvd))
        dec.set_kv_cache(k, v)
        w = dec.host_weights()
        orc = oracle.Model(oracle_cfg(cfg), w, max_seq=S)
        del w
        orc.bufs["key_cache"][:] = k.reshape(-1)
        orc.bufs["value_cache"][:] = v.reshape(-1)
        dec.capture_graph("auto")
        assert dec.persistent and dec.s.step_switch_pos == S  # 0.6B: the kernel throughout
        tok = int(rng.integers(0, cfg.vocab_size))
        dec.forward(tok, S - 2)
        nxt = dec.sample_argmax()
        ref = orc.forward(tok, S - 2, oracle.GPU_ORDER)
        assert np.array_equal(dec.logits(), orc.logits)
        assert nxt == ref
        got = dec.generate_greedy(nxt, S - 1, 1)
        assert got == [orc.forward(nxt, S - 1, oracle.GPU_ORDER)]
        assert np.array_equal(dec.logits(), orc.logits)
        kk, vv = dec.kv_cache()
        assert np.array_equal(kk[:, S - 2:], orc.bufs["key_cache"].reshape(k.shape)[:, S - 2:])
        assert np.array_equal(vv[:, S - 2:], orc.bufs["value_cache"].reshape(v.shape)[:, S - 2:])
    finally:
        dec.close()
    longer = model.Decoder(model.qwen3_config("0.6B", n_layers=1, max_seq_len=S + 1),
                           ("synth", 1, 0.02, 0.1))
    try:
        with pytest.raises(LlmError, match="no persistent step kernel"):
            longer.capture_graph("persistent")
    finally:
        longer.close()


@pytest.mark.parametrize("size", ["1.7B", "4B"])
def test_persistent_step_wide_shapes_long_history(gpu, oracle, size):
    """The 1.7B and 4B specialisations of the persistent step (2 and 4 query heads per kv head)
    around their switch from one workgroup per query head to the split attention (from 384 / 512
    positions): single positions 260 and sp - 1 (per head) and sp (split) after a KV cache filled
    with N(0, 1) below them, at full widths with 2 layers; logits, argmax and the KV rows
    written bit-identical to the oracle. Then one generate_greedy call of 16 tokens from sp - 7,
    which runs its first 7 tokens in one launch of the per-head instance and the rest in one of
    the split instance, continuing from the token and position the first left."""
    sp = {"1.7B": 384, "4B": 512}[size]
    ident(f"persistent step {size} widths at positions 260, {sp - 1}, {sp}")
    from llm_inference_amd import model
    S = 528
    cfg = model.qwen3_config(size, n_layers=2, max_seq_len=S)
    dec = model.Decoder(cfg, ("synth", 31, 0.02, 0.1))
    try:
        rng = np.random.default_rng(447)
        kvd = cfg.n_kv_heads * cfg.head_dim
        k = rand_bf16(rng, (cfg.n_layers, S, kvd))
        v = rand_bf16(rng, (cfg.n_layers, S, kvd))
        dec.set_kv_cache(k, v)
        w = dec.host_weights()
        orc = oracle.Model(oracle_cfg(cfg), w, max_seq=S)
        del w
        orc.bufs["key_cache"][:] = k.reshape(-1)
        orc.bufs["value_cache"][:] = v.reshape(-1)
        dec.capture_graph("auto")
        assert dec.s.step_split_blocks == sp // 64 + 1 and dec.s.step_switch_pos == S
        dec.capture_graph("persistent")
        assert dec.persistent
        for pos in (260, sp - 1, sp):
            tok = int(rng.integers(0, cfg.vocab_size))
            dec.forward(tok, pos)
            nxt = dec.sample_argmax()
            ref = orc.forward(tok, pos, oracle.GPU_ORDER)
            assert np.array_equal(dec.logits(), orc.logits), pos
            assert nxt == ref, pos
            kk, vv = dec.kv_cache()
            ok = orc.bufs["key_cache"].reshape(k.shape)
            ov = orc.bufs["value_cache"].reshape(v.shape)
            assert np.array_equal(kk[:, pos], ok[:, pos]), pos
            assert np.array_equal(vv[:, pos], ov[:, pos]), pos
        got = dec.generate_greedy(nxt, sp - 7, 16)
        t, want = nxt, []
        for i in range(16):
            t = orc.forward(t, sp - 7 + i, oracle.GPU_ORDER)
            want.append(t)
        assert got == want
    finally:
        dec.close()


@pytest.mark.parametrize("mode", ["graph", "persistent"])
def test_step_keeps_an_earlier_error_code(gpu, mode):
    """A wait between workgroups that finds the error flag already set stops at once and leaves
    the code alone: with the flag set to 1 (token or position out of range) from the host before
    a step whose attention waits on other workgroups (graph step: the PV + combine launch at
    position 200, four blocks; persistent step: every tagged-vector poll), the error reported
    afterwards is the out-of-range one, not a timed-out wait. Every wait ends at once, so the
    kernels exit normally."""
    ident(f"earlier error code kept ({mode} step)")
    from llm_inference_amd import LlmError, model
    cfg = model.make_config(hidden_size=512, intermediate_size=1024, n_layers=2, n_heads=8,
                            n_kv_heads=4, vocab_size=3000, max_seq_len=256)
    dec = model.Decoder(cfg, ("synth", 9, 0.02, 0.1))
    try:
        dec.capture_graph(mode)
        assert dec.persistent == (mode == "persistent")
        model.copy_to_device(dec.s.error_flag, np.array([1], np.int32), 4)
        dec.forward(17, 200)
        with pytest.raises(LlmError, match="out of range"):
            dec.sample_argmax()
        # the flag was reported and cleared: the next step runs normally
        dec.forward(17, 200)
        assert 0 <= dec.sample_argmax() < cfg.vocab_size
    finally:
        dec.close()


@pytest.mark.parametrize("attn", ["one_pass", "fused", "unfused"])
def test_graph_step_4b_after_8192_positions(gpu, oracle, attn):
    """The Qwen3-4B 8192-position config on the step it runs on (the hipGraph of per-layer
    kernels): full 4B widths (hidden 2560, 32/8 heads, intermediate 9728, vocab 151936), 2 layers
    to keep the oracle quick, the KV cache's first 8192 positions filled with N(0, 1). Logits and
    argmax bit-identical to the oracle's GPU order at positions 8192-8199 (each step's KV rows
    written past the reference's 4096-slot cap and read back by the next), then a one-call
    generate_greedy of 8 tokens from 8200 equal to the oracle's. Every attention form of the
    step: QK-norm + RoPE + attention in one launch (ATTN_ONE_PASS, opt-in), QK-norm + RoPE inside
    the attention's scores pass (what ATTN_AUTO takes at these shapes), and qk_norm_rope_forward
    + attention_forward."""
    ident(f"4B graph step from 8192 positions, {attn} attention")
    from llm_inference_amd import model
    cfg = model.qwen3_config("4B", n_layers=2, max_seq_len=8448)
    dec = model.Decoder(cfg, ("synth", 21, 0.02, 0.1))
    try:
        rng = np.random.default_rng(8192)
        kvd = cfg.n_kv_heads * cfg.head_dim
        k = np.zeros((cfg.n_layers, 8448, kvd), np.uint16)
        v = np.zeros_like(k)
        k[:, :8192] = rand_bf16(rng, (cfg.n_layers, 8192, kvd))
        v[:, :8192] = rand_bf16(rng, (cfg.n_layers, 8192, kvd))
        dec.set_kv_cache(k, v)
        w = dec.host_weights()
        orc = oracle.Model(oracle_cfg(cfg), w, max_seq=8448)
        del w
        orc.bufs["key_cache"][:] = k.reshape(-1)
        orc.bufs["value_cache"][:] = v.reshape(-1)
        dec.s.attn_mode = model.ATTN_MODES[{"one_pass": "one_pass", "fused": "in_scores",
                                            "unfused": "separate"}[attn]]
        dec.capture_graph("graph")
        assert not dec.persistent
        tok = int(rng.integers(0, cfg.vocab_size))
        for pos in range(8192, 8200):
            dec.forward(tok, pos)
            nxt = dec.sample_argmax()
            ref = orc.forward(tok, pos, oracle.GPU_ORDER)
            assert np.array_equal(dec.logits(), orc.logits), pos
            assert nxt == ref, pos
            tok = nxt
        kk, vv = dec.kv_cache()
        ok = orc.bufs["key_cache"].reshape(k.shape)
        ov = orc.bufs["value_cache"].reshape(v.shape)
        assert np.array_equal(kk[:, 8192:8200], ok[:, 8192:8200])
        assert np.array_equal(vv[:, 8192:8200], ov[:, 8192:8200])
        assert np.array_equal(kk[:, 8200:], k[:, 8200:])  # rows past the position untouched
        got = dec.generate_greedy(tok, 8200, 8)
        want = []
        for i in range(8):
            tok = orc.forward(tok, 8200 + i, oracle.GPU_ORDER)
            want.append(tok)
        assert got == want
    finally:
        dec.close()


def test_recapture_after_new_weights_drops_old_graphs(gpu, oracle):
    """capture_graph after the caller swaps in new Weights (a separate allocation): the hipGraph
    step's generate_greedy must read the new weights, not replay a loop graph captured over the
    old pointers. The old allocation stays alive until the end, so a stale graph would show up
    as the old model's tokens, not as a memory fault."""
    ident("recapture with new weights")
    import ctypes
    from llm_inference_amd import lib, model
    cfg = model.make_config(hidden_size=512, intermediate_size=1024, n_layers=2, n_heads=8,
                            n_kv_heads=4, vocab_size=3000, max_seq_len=64)
    dec = model.Decoder(cfg, ("synth", 5, 0.02, 0.1))
    old = dec.w
    try:
        dec.capture_graph("graph")
        first = dec.generate_greedy(7, 0, 12)
        new = model.Weights()
        lib().synth_weights(ctypes.byref(cfg), ctypes.byref(new), 99, 0.02, 0.1)
        dec.w = new
        dec.capture_graph("graph")
        got = dec.generate_greedy(7, 0, 12)
        orc = oracle.Model(oracle_cfg(cfg), dec.host_weights(), max_seq=64)
        t, want = 7, []
        for pos in range(12):
            t = orc.forward(t, pos, oracle.GPU_ORDER)
            want.append(t)
        assert got == want
        assert got != first
    finally:
        dec.close()
        lib().free_weights(ctypes.byref(old))


def test_generate_greedy_while_dumping(gpu, tmp_path):
    """With dumps open, generate_greedy runs each step eagerly and writes one row per tensor and
    position, with the same tokens as the captured loop."""
    ident("generate_greedy with dumps")
    import ctypes
    from llm_inference_amd import lib, model
    cfg = model.make_config(hidden_size=512, intermediate_size=1024, n_layers=2, n_heads=8,
                            n_kv_heads=4, vocab_size=3000, max_seq_len=64)
    dec = model.Decoder(cfg, ("synth", 6, 0.02, 0.1))
    try:
        dec.capture_graph("graph")
        want = dec.generate_greedy(11, 0, 6)
        lib().dump_open(str(tmp_path).encode())
        try:
            got = dec.generate_greedy(11, 0, 6)
        finally:
            lib().dump_close()
        assert got == want
        rows = np.fromfile(tmp_path / "logits.bin", dtype=np.float32)
        assert rows.size == 6 * cfg.vocab_size
        assert np.fromfile(tmp_path / "L01.out.bin", dtype=np.float32).size == 6 * cfg.hidden_size
    finally:
        dec.close()
