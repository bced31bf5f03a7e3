"""Parity of every HIP launcher with the CPU oracle on the same seeded inputs.

GPU results must be bit-identical to the oracle's GPU-order mode (same fp32 operations in the
same order) and within the parity tolerance of its exact mode: 1 bf16 ulp for RMSNorm,
RoPE and SwiGLU, bit-exact for the embedding rows, KV-cache slots and argmax. Shapes are the
Qwen3-0.6B decode layer (hidden 1024, 16q/8kv heads of 128, intermediate 3072, vocab 151936),
the Qwen3-4B widths (2560, 32/8, 9728) and the many-row roofline sweep sizes, plus ragged and
tiny edge cases."""
import math

import numpy as np
import pytest

from conftest import (bf16_bits, bf16_ulp_diff, bf16_vals, rand_bf16, ulp_bf16,
                      within_one_ulp_then_scale)

pytestmark = pytest.mark.gpu


def dev(bits):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint16)


def dev_i32(a):
    import torch
    return torch.tensor(np.asarray(a, dtype=np.int32)).cuda()


def ident(name):
    print(f"[case] {name}", flush=True)


# ---------------------------------------------------------------- embedding

def test_embedding_rows_bit_exact(gpu, oracle):
    import torch
    ident("embedding 151936x1024 and 1000x2560")
    rng = np.random.default_rng(20)
    for vocab, hidden in [(151936, 1024), (1000, 2560), (50, 20)]:
        table = torch.randn(vocab, hidden, device="cuda").to(torch.bfloat16).view(torch.int16)
        for tok in [0, 1, vocab // 2, vocab - 1, int(rng.integers(0, vocab))]:
            out = torch.zeros(hidden, dtype=torch.int16, device="cuda")
            gpu.embedding_forward(out, table, dev_i32([tok]), hidden)
            assert np.array_equal(host(out), host(table[tok]))


# ---------------------------------------------------------------- RMSNorm

@pytest.mark.parametrize("rows,dim", [(1, 1024), (1, 2560), (4096, 2560), (3, 100), (2, 9000),
                                      (5, 8200), (7, 8192), (1, 8)])
def test_rmsnorm(gpu, oracle, rows, dim):
    ident(f"rmsnorm {rows}x{dim}")
    rng = np.random.default_rng(rows * 7 + dim)
    x = rand_bf16(rng, (rows, dim))
    w = rand_bf16(rng, dim, 0.1, 1.0)
    out = dev(np.zeros((rows, dim), np.uint16))
    gpu.rmsnorm_forward(out, dev(x), dev(w), rows, dim, 1e-6)
    y = host(out).reshape(rows, dim)
    assert np.array_equal(y, oracle.rmsnorm(x, w, 1e-6, oracle.GPU_ORDER))
    n_exact = oracle.rmsnorm(x, bf16_bits(np.ones(dim)), 1e-6, oracle.EXACT)
    assert within_one_ulp_then_scale(y, n_exact, w).all()


# ---------------------------------------------------------------- GEMV family

GEMV_SHAPES = [(4096, 1024), (1024, 2048), (1024, 3072), (2560, 9728), (2560, 4096),
               (151936, 1024), (37, 520), (5, 8), (3, 16400)]


@pytest.mark.parametrize("rows,cols", GEMV_SHAPES)
def test_gemv(gpu, oracle, rows, cols):
    ident(f"gemv {rows}x{cols}")
    rng = np.random.default_rng(rows + cols)
    w = rand_bf16(rng, (rows, cols), 0.02)
    x = rand_bf16(rng, cols)
    out = dev(np.zeros(rows, np.uint16))
    gpu.gemv_forward(out, dev(w), dev(x), rows, cols)
    y = host(out)
    assert np.array_equal(y, oracle.gemv(w, x, oracle.GPU_ORDER))
    # against exact arithmetic: one bf16 ulp after the single rounding, plus the fp32
    # accumulation bound 2 * cols * 2^-24 * sum|w x|
    wv, xv = bf16_vals(w).astype(np.float64), bf16_vals(x).astype(np.float64)
    exact = wv @ xv
    bound = ulp_bf16(exact) + 2 * cols * 2.0 ** -24 * (np.abs(wv) @ np.abs(xv))
    assert np.all(np.abs(bf16_vals(y) - exact) <= bound)


@pytest.mark.parametrize("rows,cols", [(1024, 2048), (1024, 3072), (2560, 4096), (2560, 9728),
                                       (33, 64)])
def test_gemv_residual(gpu, oracle, rows, cols):
    ident(f"gemv_residual {rows}x{cols}")
    rng = np.random.default_rng(rows * 3 + cols)
    w = rand_bf16(rng, (rows, cols), 0.02)
    inp = rand_bf16(rng, cols)
    x = rand_bf16(rng, rows)
    xd, tap = dev(x), dev(np.zeros(rows, np.uint16))
    gpu.gemv_residual_forward(xd, dev(w), dev(inp), rows, cols, tap)
    ex, et = oracle.gemv_residual(x, w, inp, oracle.GPU_ORDER, with_tap=True)
    assert np.array_equal(host(tap), et)
    assert np.array_equal(host(xd), ex)
    xd = dev(x)
    gpu.gemv_residual_forward(xd, dev(w), dev(inp), rows, cols, None)
    assert np.array_equal(host(xd), ex)


@pytest.mark.parametrize("hq,hkv,H", [(16, 8, 1024), (32, 8, 2560), (3, 1, 64)])
def test_qkv(gpu, oracle, hq, hkv, H):
    ident(f"qkv {hq}/{hkv} x {H}")
    rng = np.random.default_rng(hq + H)
    wq = rand_bf16(rng, (hq * 128, H), 0.02)
    wk = rand_bf16(rng, (hkv * 128, H), 0.02)
    wv = rand_bf16(rng, (hkv * 128, H), 0.02)
    x = rand_bf16(rng, H)
    q, k, v = (dev(np.zeros(n, np.uint16)) for n in (hq * 128, hkv * 128, hkv * 128))
    gpu.qkv_forward(q, k, v, dev(wq), dev(wk), dev(wv), dev(x), hq * 128, hkv * 128, H)
    eq, ek, ev = oracle.qkv(wq, wk, wv, x, oracle.GPU_ORDER)
    assert np.array_equal(host(q), eq)
    assert np.array_equal(host(k), ek)
    assert np.array_equal(host(v), ev)


@pytest.mark.parametrize("rows,cols", [(3072, 1024), (6144, 2048), (9728, 2560), (77, 136)])
def test_gate_up(gpu, oracle, rows, cols):
    ident(f"gate_up {rows}x{cols}")
    rng = np.random.default_rng(rows + 5 * cols)
    wg = rand_bf16(rng, (rows, cols), 0.02)
    wu = rand_bf16(rng, (rows, cols), 0.02)
    x = rand_bf16(rng, cols)
    act, gt, ut = (dev(np.zeros(rows, np.uint16)) for _ in range(3))
    gpu.gate_up_forward(act, dev(wg), dev(wu), dev(x), rows, cols, gt, ut)
    ea, eg, eu = oracle.gate_up(wg, wu, x, oracle.GPU_ORDER, with_taps=True)
    assert np.array_equal(host(gt), eg) and np.array_equal(host(ut), eu)
    assert np.array_equal(host(act), ea)
    s_exact = oracle.swiglu(eg, bf16_bits(np.ones(rows)), oracle.EXACT)
    assert within_one_ulp_then_scale(host(act), s_exact, eu).all()
    act2 = dev(np.zeros(rows, np.uint16))
    gpu.gate_up_forward(act2, dev(wg), dev(wu), dev(x), rows, cols, None, None)
    assert np.array_equal(host(act2), ea)


# ---------------------------------------------------------------- RMSNorm fused into the GEMV

FUSED_NORM_SHAPES = [(1024, 16, 8), (2560, 32, 8), (2048, 16, 8), (136, 3, 1),
                     (8192, 2, 1)]


@pytest.mark.parametrize("H,hq,hkv", FUSED_NORM_SHAPES)
def test_rmsnorm_fused_gemvs(gpu, oracle, H, hq, hkv):
    """The fused forms equal rmsnorm_forward followed by the plain launcher, bit for bit."""
    ident(f"rmsnorm fused qkv/gemv/gate_up H={H} {hq}/{hkv}")
    rng = np.random.default_rng(H + hq)
    x = rand_bf16(rng, H, 1.0, 4.0)
    g = rand_bf16(rng, H, 0.1, 1.0)
    xn = oracle.rmsnorm(x[None], g, 1e-6, oracle.GPU_ORDER)[0]
    wq = rand_bf16(rng, (hq * 128, H), 0.02)
    wk = rand_bf16(rng, (hkv * 128, H), 0.02)
    wv = rand_bf16(rng, (hkv * 128, H), 0.02)
    q, k, v = (dev(np.zeros(n, np.uint16)) for n in (hq * 128, hkv * 128, hkv * 128))
    gpu.rmsnorm_qkv_forward(q, k, v, dev(wq), dev(wk), dev(wv), dev(x), dev(g), 1e-6, hq * 128,
                            hkv * 128, H)
    eq, ek, ev = oracle.qkv(wq, wk, wv, xn, oracle.GPU_ORDER)
    assert np.array_equal(host(q), eq)
    assert np.array_equal(host(k), ek)
    assert np.array_equal(host(v), ev)
    rows = 3 * H + 5 if H <= 2560 else 1029
    w = rand_bf16(rng, (rows, H), 0.02)
    out = dev(np.zeros(rows, np.uint16))
    gpu.rmsnorm_gemv_forward(out, dev(w), dev(x), dev(g), 1e-6, rows, H)
    assert np.array_equal(host(out), oracle.gemv(w, xn, oracle.GPU_ORDER))
    wg = rand_bf16(rng, (rows, H), 0.02)
    act = dev(np.zeros(rows, np.uint16))
    gpu.rmsnorm_gate_up_forward(act, dev(wg), dev(w), dev(x), dev(g), 1e-6, rows, H)
    assert np.array_equal(host(act), oracle.gate_up(wg, w, xn, oracle.GPU_ORDER))


def test_rmsnorm_fused_gemv_rejects_wide_rows(gpu):
    """A row wider than 8192 columns is refused before any launch."""
    H = 8200
    x, g = dev(np.zeros(H, np.uint16)), dev(np.zeros(H, np.uint16))
    w = dev(np.zeros((4, H), np.uint16))
    out = dev(np.zeros(4, np.uint16))
    with pytest.raises(gpu.LlmError, match="do not fit one panel"):
        gpu.rmsnorm_gemv_forward(out, w, x, g, 1e-6, 4, H)


# ---------------------------------------------------------------- SwiGLU

@pytest.mark.parametrize("n", [65280, 4096 * 9728, 1001, 7])
def test_swiglu(gpu, oracle, n):
    ident(f"swiglu n={n}")
    rng = np.random.default_rng(n)
    if n == 65280:  # every finite bf16 gate value
        g = np.arange(65536, dtype=np.uint32).astype(np.uint16)
        g = g[np.isfinite(bf16_vals(g))]
    else:
        g = rand_bf16(rng, n, 2.0)
    u = rand_bf16(rng, g.size)
    act = dev(np.zeros(g.size, np.uint16))
    gpu.swiglu_forward(act, dev(g), dev(u), g.size)
    y = host(act)
    assert np.array_equal(y, oracle.swiglu(g, u, oracle.GPU_ORDER))
    s_exact = oracle.swiglu(g, bf16_bits(np.ones(g.size)), oracle.EXACT)
    assert within_one_ulp_then_scale(y, s_exact, u).all()
    if n == 65280:
        # u = 1: the rounded SiLU itself, for every finite bf16 gate value (the kernel's fast
        # estimate must round like the precise formula everywhere)
        ones = bf16_bits(np.ones(g.size))
        act1 = dev(np.zeros(g.size, np.uint16))
        gpu.swiglu_forward(act1, dev(g), dev(ones), g.size)
        assert np.array_equal(host(act1), oracle.swiglu(g, ones, oracle.GPU_ORDER))


# ---------------------------------------------------------------- QK-norm + RoPE + KV write

def rope_rotate(tap, positions, D, theta, oracle):
    """HF's apply_rotary_pos_emb on bf16 heads, computed independently: angles fp32(pos *
    inv_freq_j) (inv_freq pinned to decimal arithmetic), cos/sin from libm rounded through fp32
    to bf16, each product and the sum rounded to bf16 (modeling_qwen3.py:126-170)."""
    inv = oracle.inv_freq(theta, D)
    T = len(positions)
    y = bf16_vals(np.asarray(tap, dtype=np.uint16).reshape(T, -1, D))
    out = np.empty(y.shape, np.uint16)
    r = lambda z: bf16_vals(bf16_bits(z))
    for t, p in enumerate(positions):
        ang = (np.float32(p) * inv).astype(np.float32)
        c = bf16_vals(bf16_bits(np.array([math.cos(float(a)) for a in ang], np.float32)))
        s = bf16_vals(bf16_bits(np.array([math.sin(float(a)) for a in ang], np.float32)))
        a, b = y[t, :, :D // 2], y[t, :, D // 2:]
        out[t, :, :D // 2] = bf16_bits(r(a * c) - r(b * s))
        out[t, :, D // 2:] = bf16_bits(r(b * c) + r(a * s))
    return out


def _rope_case(rng, n_tokens, hq, hkv, D, max_seq):
    q = rand_bf16(rng, (n_tokens, hq * D))
    k = rand_bf16(rng, (n_tokens, hkv * D))
    v = rand_bf16(rng, (n_tokens, hkv * D))
    qn = rand_bf16(rng, D, 0.1, 1.0)
    kn = rand_bf16(rng, D, 0.1, 1.0)
    kc = np.full((max_seq, hkv * D), 0x7FC1, np.uint16)
    vc = np.full((max_seq, hkv * D), 0x7FC3, np.uint16)
    return q, k, v, qn, kn, kc, vc


@pytest.mark.parametrize("hq,hkv,D,pos", [(16, 8, 128, 0), (16, 8, 128, 1), (16, 8, 128, 3071),
                                          (32, 8, 128, 4095), (4, 2, 64, 77), (4, 2, 256, 500),
                                          (3, 1, 128, 9), (32, 8, 128, 4096), (32, 8, 128, 8191),
                                          (32, 8, 128, 8447)])
def test_qk_norm_rope_decode(gpu, oracle, hq, hkv, D, pos):
    """Config-1 decode: q/k rotated in place bit-exactly, k'/v written to cache row pos only.
    Positions past the reference's 4096-slot cap (src/forward.cu:7-8) use an 8448-slot cache, the
    size of the Qwen3-4B 8192-position config: the rows at 4096, 8191 and 8447 are written and
    every other row keeps its sentinel."""
    ident(f"qk_norm_rope decode {hq}/{hkv} D{D} pos{pos}")
    rng = np.random.default_rng(hq * 1000 + pos)
    max_seq = 4096 if pos < 4096 else 8448
    q, k, v, qn, kn, kc, vc = _rope_case(rng, 1, hq, hkv, D, max_seq)
    qd, kd, kcd, vcd = dev(q), dev(k), dev(kc), dev(vc)
    qt, kt = dev(np.zeros_like(q)), dev(np.zeros_like(k))
    gpu.qk_norm_rope_forward(qd, kd, dev(v), dev(qn), dev(kn), kcd, vcd, dev_i32([pos]), hq, hkv,
                             D, 1e-6, 1e6, qt, kt)
    eq, ek, ekc, evc, eqt, ekt = oracle.qk_norm_rope_rows(q, k, v, qn, kn, kc, vc, [pos], hq, hkv,
                                                          D, 1e-6, 1e6, oracle.GPU_ORDER,
                                                          with_taps=True)
    assert np.array_equal(host(qt).reshape(eqt.shape), eqt)
    assert np.array_equal(host(kt).reshape(ekt.shape), ekt)
    assert np.array_equal(host(qd).reshape(eq.shape), eq)
    assert np.array_equal(host(kd).reshape(ek.shape), ek)
    gkc, gvc = host(kcd).reshape(kc.shape), host(vcd).reshape(vc.shape)
    assert np.array_equal(gkc, ekc) and np.array_equal(gvc, evc)
    assert np.array_equal(gkc[pos], host(kd).reshape(-1)) and np.array_equal(gvc[pos], v[0])
    # tolerance against exact arithmetic: the normed heads within 1 ulp at HF's rounding point,
    # and the rotation of the GPU's own normed heads bit-exact against libm cos/sin
    ones = bf16_bits(np.ones(D))
    nq = oracle.qk_norm_rope_rows(q, k, v, ones, ones, kc, vc, [pos], hq, hkv, D, 1e-6, 1e6,
                                  oracle.EXACT, with_taps=True)
    assert within_one_ulp_then_scale(host(qt).reshape(-1), nq[4].reshape(-1), np.tile(qn, hq)).all()
    assert within_one_ulp_then_scale(host(kt).reshape(-1), nq[5].reshape(-1), np.tile(kn, hkv)).all()
    assert np.array_equal(host(qd).reshape(-1), rope_rotate(host(qt), [pos], D, 1e6, oracle).reshape(-1))
    assert np.array_equal(host(kd).reshape(-1), rope_rotate(host(kt), [pos], D, 1e6, oracle).reshape(-1))


def test_qk_norm_rope_rows_sweep(gpu, oracle):
    """Config-5 sweep: 4096 tokens x (32 q + 8 kv) heads of 128 at positions 0..4095."""
    ident("qk_norm_rope rows 4096 tokens 32/8")
    rng = np.random.default_rng(30)
    T, hq, hkv, D = 4096, 32, 8, 128
    q, k, v, qn, kn, kc, vc = _rope_case(rng, T, hq, hkv, D, T)
    pos = np.arange(T, dtype=np.int32)
    qd, kd, kcd, vcd = dev(q), dev(k), dev(kc), dev(vc)
    gpu.qk_norm_rope_rows(qd, kd, dev(v), dev(qn), dev(kn), kcd, vcd, dev_i32(pos), T, hq, hkv, D,
                          1e-6, 1e6)
    eq, ek, ekc, evc = oracle.qk_norm_rope_rows(q, k, v, qn, kn, kc, vc, pos, hq, hkv, D, 1e-6,
                                                1e6, oracle.GPU_ORDER)
    assert np.array_equal(host(qd).reshape(eq.shape), eq)
    assert np.array_equal(host(kd).reshape(ek.shape), ek)
    assert np.array_equal(host(kcd).reshape(kc.shape), ekc)
    assert np.array_equal(host(vcd).reshape(vc.shape), evc)


# ---------------------------------------------------------------- attention

@pytest.mark.parametrize("hq,hkv,pos", [(16, 8, 0), (16, 8, 4), (16, 8, 63), (16, 8, 64),
                                        (16, 8, 260), (32, 8, 4095), (32, 8, 8447), (8, 8, 100),
                                        (8, 1, 130), (3, 3, 4100)])
def test_attention(gpu, oracle, hq, hkv, pos):
    ident(f"attention {hq}/{hkv} pos{pos}")
    rng = np.random.default_rng(hq * 10000 + pos)
    D = 128
    max_seq = max(pos + 1, 4096) if pos < 8000 else 8448
    q = rand_bf16(rng, hq * D)
    kc = rand_bf16(rng, (max_seq, hkv * D))
    vc = rand_bf16(rng, (max_seq, hkv * D))
    import torch
    att = torch.zeros(gpu.attention_workspace_floats(hq, D, max_seq), dtype=torch.float32,
                      device="cuda")
    out = dev(np.zeros(hq * D, np.uint16))
    scale = float(np.float32(1.0 / np.sqrt(D)))
    gpu.attention_forward(out, dev(q), dev(kc), dev(vc), att, hq, hkv, D, dev_i32([pos]), max_seq,
                          scale)
    y = host(out)
    assert np.array_equal(y, oracle.attention(q, kc, vc, hq, hkv, D, pos, scale, oracle.GPU_ORDER))
    assert bf16_ulp_diff(y, oracle.attention(q, kc, vc, hq, hkv, D, pos, scale,
                                             oracle.EXACT)).max() <= 2


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("rep", [1, 2, 4, 8])
def test_attention_head_dims(gpu, oracle, D, rep):
    """The head_dim 64 and 256 instantiations of the split-softmax kernels, for every GQA ratio
    they are built for, at a position that spans several 64-position blocks and ends inside one:
    bit-identical to the oracle's GPU order, within 2 bf16 ulps of exact arithmetic."""
    import torch
    hkv = 2
    hq, pos = hkv * rep, 200 + 37 * rep
    ident(f"attention D{D} rep{rep} pos{pos}")
    rng = np.random.default_rng(D * 100 + rep)
    max_seq = 512
    q = rand_bf16(rng, hq * D)
    kc = rand_bf16(rng, (max_seq, hkv * D))
    vc = rand_bf16(rng, (max_seq, hkv * D))
    att = torch.zeros(gpu.attention_workspace_floats(hq, D, max_seq), dtype=torch.float32,
                      device="cuda")
    out = dev(np.zeros(hq * D, np.uint16))
    scale = float(np.float32(1.0 / np.sqrt(D)))
    gpu.attention_forward(out, dev(q), dev(kc), dev(vc), att, hq, hkv, D, dev_i32([pos]), max_seq,
                          scale)
    y = host(out)
    assert np.array_equal(y, oracle.attention(q, kc, vc, hq, hkv, D, pos, scale, oracle.GPU_ORDER))
    assert bf16_ulp_diff(y, oracle.attention(q, kc, vc, hq, hkv, D, pos, scale,
                                             oracle.EXACT)).max() <= 2


FUSED_ATTN_CASES = [(16, 8, 128, 0, 4096), (16, 8, 128, 63, 4096), (16, 8, 128, 64, 4096),
                    (16, 8, 128, 260, 4096), (32, 8, 128, 8192, 8448), (32, 8, 128, 8447, 8448),
                    (8, 8, 128, 100, 512), (8, 1, 128, 130, 512), (2, 2, 64, 301, 512),
                    (16, 2, 64, 200, 512), (4, 2, 256, 777, 1024), (16, 2, 256, 150, 512),
                    (3, 3, 128, 4100, 4200)]


@pytest.mark.parametrize("hq,hkv,D,pos,max_seq", FUSED_ATTN_CASES)
def test_qk_norm_rope_attention_fused(gpu, oracle, hq, hkv, D, pos, max_seq):
    """qk_norm_rope_attention_forward (QK-norm + RoPE inside the attention's scores pass): the
    output is bit-identical to the oracle's GPU order of the two steps (QK-norm + RoPE of q and
    k, k'/v written to row pos, then attention over rows 0..pos), the caches equal the oracle's
    (row pos written, every other row keeps its value), q and k are not rewritten. Three calls
    on one workspace: the case, an earlier position with new inputs, then the first position
    again with new inputs."""
    import torch
    ident(f"qk_norm_rope_attention {hq}/{hkv} D{D} pos{pos} max_seq{max_seq}")
    rng = np.random.default_rng(hq * 7919 + hkv * 31 + D + pos)
    kc = rand_bf16(rng, (max_seq, hkv * D))
    vc = rand_bf16(rng, (max_seq, hkv * D))
    kcd, vcd = dev(kc), dev(vc)
    att = torch.zeros(gpu.attention_workspace_floats(hq, D, max_seq), dtype=torch.float32,
                      device="cuda")
    scale = float(np.float32(1.0 / np.sqrt(D)))
    qn = rand_bf16(rng, D, 0.1, 1.0)
    kn = rand_bf16(rng, D, 0.1, 1.0)
    for p in [pos, pos // 2, pos]:
        q = rand_bf16(rng, hq * D)
        k = rand_bf16(rng, hkv * D)
        v = rand_bf16(rng, hkv * D)
        qd, kd = dev(q), dev(k)
        out = dev(np.zeros(hq * D, np.uint16))
        gpu.qk_norm_rope_attention_forward(out, qd, kd, dev(v), dev(qn), dev(kn), kcd, vcd, att,
                                           dev_i32([p]), hq, hkv, D, 1e-6, 1e6, max_seq, scale)
        eq, ek, ekc, evc = oracle.qk_norm_rope_rows(q[None], k[None], v[None], qn, kn, kc, vc, [p],
                                                    hq, hkv, D, 1e-6, 1e6, oracle.GPU_ORDER)
        want = oracle.attention(eq.reshape(-1), ekc, evc, hq, hkv, D, p, scale, oracle.GPU_ORDER)
        got = host(out)
        assert np.array_equal(got, want), p
        assert np.array_equal(host(kcd).reshape(kc.shape), ekc), p
        assert np.array_equal(host(vcd).reshape(vc.shape), evc), p
        assert np.array_equal(host(qd), q) and np.array_equal(host(kd), k)
        kc, vc = ekc, evc


ONE_PASS_CASES = [(16, 8, 128, 0, 4096), (16, 8, 128, 63, 4096), (16, 8, 128, 64, 4096),
                  (16, 8, 128, 260, 4096), (16, 8, 128, 4095, 4096), (32, 8, 128, 8192, 8448),
                  (32, 8, 128, 8447, 8448), (32, 8, 128, 30001, 32768), (8, 8, 128, 100, 512),
                  (8, 1, 128, 130, 512), (8, 1, 128, 9000, 9100), (2, 2, 128, 301, 512),
                  (16, 2, 128, 2000, 2048), (3, 3, 128, 4100, 4200)]


@pytest.mark.parametrize("hq,hkv,D,pos,max_seq", ONE_PASS_CASES)
def test_qk_norm_rope_attention_one_pass(gpu, oracle, hq, hkv, D, pos, max_seq):
    """qk_norm_rope_attention_one_pass (QK-norm + RoPE + attention in one launch, the
    workgroups of a kv head handing block statistics and partial outputs to each other): the
    output is bit-identical to the oracle's GPU order of the two steps, the caches equal the
    oracle's (row pos written, every other row unchanged), q and k are not rewritten and the
    error flag stays 0. Five calls on one workspace (its launch counter tags the handoffs): the
    case, an earlier position, the case again, the first position and the case once more, each
    with new inputs, so a stale word of an earlier call would be read as current."""
    import torch
    if not gpu.attention_one_pass_supported(hq, hkv, D, max_seq):
        pytest.skip("no one-pass attention for this shape on this device")
    ident(f"one-pass attention {hq}/{hkv} D{D} pos{pos} max_seq{max_seq}")
    rng = np.random.default_rng(hq * 7919 + hkv * 31 + D + pos + 17)
    kc = rand_bf16(rng, (max_seq, hkv * D))
    vc = rand_bf16(rng, (max_seq, hkv * D))
    kcd, vcd = dev(kc), dev(vc)
    ws = torch.zeros(gpu.attention_one_pass_bytes(hq, D, max_seq), dtype=torch.uint8,
                     device="cuda")
    err = dev_i32([0])
    scale = float(np.float32(1.0 / np.sqrt(D)))
    qn = rand_bf16(rng, D, 0.1, 1.0)
    kn = rand_bf16(rng, D, 0.1, 1.0)
    for p in [pos, pos // 2, pos, 0, pos]:
        q = rand_bf16(rng, hq * D)
        k = rand_bf16(rng, hkv * D)
        v = rand_bf16(rng, hkv * D)
        qd, kd = dev(q), dev(k)
        out = dev(np.zeros(hq * D, np.uint16))
        gpu.qk_norm_rope_attention_one_pass(out, qd, kd, dev(v), dev(qn), dev(kn), kcd, vcd, ws,
                                            err, dev_i32([p]), hq, hkv, D, 1e-6, 1e6, max_seq,
                                            scale)
        eq, ek, ekc, evc = oracle.qk_norm_rope_rows(q[None], k[None], v[None], qn, kn, kc, vc, [p],
                                                    hq, hkv, D, 1e-6, 1e6, oracle.GPU_ORDER)
        want = oracle.attention(eq.reshape(-1), ekc, evc, hq, hkv, D, p, scale, oracle.GPU_ORDER)
        got = host(out)
        assert int(err.cpu()[0]) == 0, p
        assert np.array_equal(got, want), p
        assert np.array_equal(host(kcd).reshape(kc.shape), ekc), p
        assert np.array_equal(host(vcd).reshape(vc.shape), evc), p
        assert np.array_equal(host(qd), q) and np.array_equal(host(kd), k)
        kc, vc = ekc, evc


def test_qk_norm_rope_attention_one_pass_rejects(gpu):
    """Shapes the one-pass attention is not built for are refused with a message, and report
    themselves as unsupported."""
    import torch
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    x = dev(np.zeros(4096, np.uint16))
    err = dev_i32([0])
    for hq, hkv, D, max_seq in [(4, 2, 64, 16), (6, 2, 128, 16), (16, 8, 128, 40000)]:
        assert not gpu.attention_one_pass_supported(hq, hkv, D, max_seq)
        with pytest.raises(gpu.LlmError):
            gpu.qk_norm_rope_attention_one_pass(x, x, x, x, x, x, x, x, ws, err, dev_i32([0]), hq,
                                                hkv, D, 1e-6, 1e6, max_seq, 0.1)
    with pytest.raises(gpu.LlmError):  # no norm weights
        gpu.qk_norm_rope_attention_one_pass(x, x, x, x, None, None, x, x, ws, err, dev_i32([0]),
                                            4, 2, 128, 1e-6, 1e6, 16, 0.1)


def test_attention_rejects_a_workspace_too_small(gpu):
    """The C-ABI guard on `att`: a workspace sized for fewer positions than max_seq (here a
    RunState's own att, allocated for 64 positions, passed with max_seq 4096, as a caller sizing
    it [n_heads, max_seq] the reference's way would under-size it) is an error, not an overrun;
    the same buffer at its own size runs."""
    from llm_inference_amd import model
    cfg = model.make_config(hidden_size=512, intermediate_size=1024, n_layers=1, n_heads=8,
                            n_kv_heads=4, vocab_size=256, max_seq_len=64)
    dec = model.Decoder(cfg, ("synth", 1, 0.02, 0.1))
    try:
        D, hq, hkv = 128, 8, 4
        q = dev(np.zeros(hq * D, np.uint16))
        kc = dev(np.zeros((4096, hkv * D), np.uint16))
        out = dev(np.zeros(hq * D, np.uint16))
        att = int(dec.s.att)
        with pytest.raises(gpu.LlmError, match="att has room"):
            gpu.attention_forward(out, q, kc, kc, att, hq, hkv, D, dev_i32([10]), 4096, 0.1)
        gpu.attention_forward(out, q, kc, kc, att, hq, hkv, D, dev_i32([10]), 64, 0.1)
        host(out)
    finally:
        dec.close()


@pytest.mark.parametrize("hq,hkv,pos,max_seq", [(32, 8, 8447, 8448), (16, 8, 4095, 4096),
                                                 (16, 8, 300, 4096)])
def test_attention_reference_sized_att(gpu, oracle, hq, hkv, pos, max_seq):
    """attention_forward with `att` allocated the reference's way (src/forward.cu:10-51: its own
    hipMalloc of [n_heads, max_seq] floats, src/forward.cuh:13): the scores go there and the
    block statistics and partial outputs to the library's own array. Bit-identical to the
    oracle's GPU order; a call with the full workspace in between leaves the next reference-sized
    call unaffected (every value it reads it wrote)."""
    import ctypes
    import torch
    from llm_inference_amd import model
    ident(f"attention reference-sized att {hq}/{hkv} pos{pos}")
    rt = model._hip()
    D = 128
    nbytes = hq * max_seq * 4
    ptr = ctypes.c_void_p()
    assert rt.hipMalloc(ctypes.byref(ptr), ctypes.c_size_t(nbytes)) == 0
    try:
        base, size = ctypes.c_void_p(), ctypes.c_size_t()
        assert rt.hipMemGetAddressRange(ctypes.byref(base), ctypes.byref(size), ptr) == 0
        full = gpu.attention_workspace_floats(hq, D, max_seq) * 4
        print(f"[case] att allocation {size.value} bytes; the full workspace needs {full}",
              flush=True)
        if (hq, max_seq) == (32, 8448):
            assert size.value < full  # this case runs on the library's array
        rng = np.random.default_rng(hq * 1000 + pos)
        scale = float(np.float32(1.0 / np.sqrt(D)))
        for rnd in range(2):
            q = rand_bf16(rng, hq * D)
            kc = rand_bf16(rng, (max_seq, hkv * D))
            vc = rand_bf16(rng, (max_seq, hkv * D))
            qd, kd, vd = dev(q), dev(kc), dev(vc)
            out = dev(np.full(hq * D, 0x7FC1, np.uint16))
            gpu.attention_forward(out, qd, kd, vd, ptr.value, hq, hkv, D, dev_i32([pos]),
                                  max_seq, scale)
            assert np.array_equal(host(out), oracle.attention(q, kc, vc, hq, hkv, D, pos, scale,
                                                              oracle.GPU_ORDER)), rnd
            if rnd == 0:  # the full-workspace form in between, on other data
                att = torch.zeros(full // 4, dtype=torch.float32, device="cuda")
                gpu.attention_forward(out, dev(rand_bf16(rng, hq * D)), kd, vd, att, hq, hkv, D,
                                      dev_i32([pos // 2]), max_seq, scale)
                host(out)
    finally:
        torch.cuda.synchronize()
        rt.hipFree(ptr)


def test_qk_norm_rope_attention_fused_rejects(gpu):
    """Shapes the kernels are not built for are refused with a message."""
    import torch
    att = torch.zeros(1 << 16, dtype=torch.float32, device="cuda")
    x = dev(np.zeros(4096, np.uint16))
    with pytest.raises(gpu.LlmError):  # head_dim 96
        gpu.qk_norm_rope_attention_forward(x, x, x, x, x, x, x, x, att, dev_i32([0]), 4, 2, 96,
                                           1e-6, 1e6, 16, 0.1)
    with pytest.raises(gpu.LlmError):  # 3 query heads per kv head
        gpu.qk_norm_rope_attention_forward(x, x, x, x, x, x, x, x, att, dev_i32([0]), 6, 2, 128,
                                           1e-6, 1e6, 16, 0.1)
    with pytest.raises(gpu.LlmError):  # no norm weights
        gpu.qk_norm_rope_attention_forward(x, x, x, x, None, None, x, x, att, dev_i32([0]), 4, 2,
                                           128, 1e-6, 1e6, 16, 0.1)


def test_hbm_stream_probe(gpu):
    """The ceiling probe's three modes compute what they claim (copy, xor of two streams, and a
    per-thread xor of the read chunks), including a length that is not a multiple of the grid."""
    import torch
    ident("hbm_stream_probe")
    n16 = 1024 * 256 * 4 * 3 + 5  # grid-stride remainder for the read mode
    a = torch.randint(0, 1 << 30, (n16 * 4,), dtype=torch.int32, device="cuda")
    b = torch.randint(0, 1 << 30, (n16 * 4,), dtype=torch.int32, device="cuda")
    dst = torch.zeros(n16 * 4, dtype=torch.int32, device="cuda")
    gpu.hbm_stream_probe(dst, a, None, n16 * 16, 1)
    assert torch.equal(dst, a)
    gpu.hbm_stream_probe(dst, a, b, n16 * 16, 2)
    assert torch.equal(dst, a ^ b)
    out = torch.zeros(1 << 18, dtype=torch.int32, device="cuda")
    gpu.hbm_stream_probe(out, a, None, n16 * 16, 0)
    # thread b * 256 + i xors chunks b * 1024 + i + 256 u + (1024 * 1024) j (all four words)
    chunks = a.view(n16, 4).cpu().numpy().astype(np.uint32)
    words = np.bitwise_xor.reduce(chunks, axis=1)
    c = np.arange(n16) % (1024 * 1024)
    thread = (c // 1024) * 256 + c % 256
    expect = np.zeros(1 << 18, np.uint32)
    np.bitwise_xor.at(expect, thread, words)
    assert np.array_equal(out.cpu().numpy().astype(np.uint32), expect)


def test_hbm_read_peak_probe(gpu):
    """The read-peak probe reads every chunk of its walk: a buffer of zeros with the magic word in
    one chunk of a late round (grid-stride: thread 5, third pass, last load; one range per
    workgroup: workgroup 1's thread 5, third pass, last load) makes exactly that thread store
    it; without it nothing is stored. Every loads-in-flight count and both layouts, with a
    length that is not a multiple of the grid; bad launch shapes are refused."""
    import torch
    ident("hbm_read_peak_probe")
    magic = 0x9e3779b9 - (1 << 32)  # as int32
    for contiguous in (0, 1):
        for U in (4, 8, 16):
            for blocks, threads in [(3, 256), (2, 1024), (7, 64)]:
                T = blocks * threads
                if contiguous:
                    span = U * threads * 3
                    n16 = blocks * span - 5  # the last workgroup's range is short
                    hit = span + U * threads * 2 + (U - 1) * threads + 5
                else:
                    n16 = U * T * 3 + 7
                    hit = U * T * 2 + (U - 1) * T + 5
                a = torch.zeros(n16 * 4, dtype=torch.int32, device="cuda")
                out = torch.zeros(1, dtype=torch.int32, device="cuda")
                gpu.hbm_read_peak_probe(out, a, n16 * 16, blocks, threads, U, contiguous)
                torch.cuda.synchronize()
                assert int(out.item()) == 0, (contiguous, U, blocks, threads)
                a[4 * hit] = magic
                gpu.hbm_read_peak_probe(out, a, n16 * 16, blocks, threads, U, contiguous)
                torch.cuda.synchronize()
                assert int(out.item()) == magic, (contiguous, U, blocks, threads)
    with pytest.raises(gpu.LlmError):
        gpu.hbm_read_peak_probe(out, a, 64, 4, 100)
    with pytest.raises(gpu.LlmError):
        gpu.hbm_read_peak_probe(out, a, 24, 4, 256)
    with pytest.raises(gpu.LlmError):
        gpu.hbm_read_peak_probe(out, a, 64, 4, 256, 6)
    with pytest.raises(gpu.LlmError):
        gpu.hbm_read_peak_probe(out, a, 64, 4, 256, 4, 2)


def test_hbm_copy_peak_probe(gpu):
    """The copy-peak probe copies every chunk exactly once and nothing past n_bytes: random words
    into a destination filled with a sentinel one chunk longer, for every chunks-in-flight count,
    with lengths that are not multiples of the grid's tile; bad launch shapes are refused."""
    import torch
    ident("hbm_copy_peak_probe")
    g = torch.Generator(device="cpu").manual_seed(11)
    for U in (1, 2, 4, 8):
        for blocks, threads in [(3, 256), (2, 1024), (7, 64)]:
            n16 = U * blocks * threads * 3 + 5
            a = torch.randint(-2**31, 2**31 - 1, (n16 * 4,), generator=g, dtype=torch.int32).cuda()
            d = torch.full((n16 * 4 + 4,), 0x5a5a5a5a, dtype=torch.int32, device="cuda")
            gpu.hbm_copy_peak_probe(d, a, n16 * 16, blocks, threads, U)
            torch.cuda.synchronize()
            assert torch.equal(d[:n16 * 4], a), (U, blocks, threads)
            assert torch.all(d[n16 * 4:] == 0x5a5a5a5a), (U, blocks, threads)
    with pytest.raises(gpu.LlmError):
        gpu.hbm_copy_peak_probe(d, a, 64, 4, 100)
    with pytest.raises(gpu.LlmError):
        gpu.hbm_copy_peak_probe(d, a, 24, 4, 256)
    with pytest.raises(gpu.LlmError):
        gpu.hbm_copy_peak_probe(d, a, 64, 4, 256, 3)


# ---------------------------------------------------------------- temperature sampling

def test_sample_forward(gpu, oracle):
    """sample_forward equals the oracle's inverse-CDF draw (same weights, same order of additions)
    on random rows, one-hot rows and uniform rows, for several temperatures and coins."""
    import torch
    ident("sample_forward")
    rng = np.random.default_rng(11)
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    n = 151936
    rows = [rand_bf16(rng, n, s) for s in (0.5, 2.0, 4.0)]
    hot = bf16_bits(np.full(n, -50.0, np.float32))
    hot[123456] = bf16_bits(np.array([50.0], np.float32))[0]
    rows += [hot, bf16_bits(np.zeros(n, np.float32)), rand_bf16(rng, 1000, 1.0),
             rand_bf16(rng, 1023, 1.0)]
    for row in rows:
        xd = dev(row)
        for inv_temp in (1.0, 0.7, 1.5):
            for u in (0.0, 0.25, 0.5, 0.9, 0.999):
                gpu.sample_forward(out, xd, row.size, inv_temp, u)
                assert int(out.item()) == oracle.sample(row, inv_temp, u), (row.size, inv_temp, u)


# ---------------------------------------------------------------- argmax

def test_argmax(gpu, oracle):
    import torch
    ident("argmax")
    rng = np.random.default_rng(40)
    cases = [rand_bf16(rng, 151936) for _ in range(5)]
    cases.append(bf16_bits(np.full(151936, 2.5)))                     # all equal -> 0
    x = rand_bf16(rng, 151936); x[[7, 90000, 151935]] = bf16_bits(np.full(3, 50.0)); cases.append(x)
    x = rand_bf16(rng, 151936); x[151935] = bf16_bits(np.float32(60.0)).item(); cases.append(x)
    cases.append(bf16_bits(np.full(1000, -np.inf)))                   # all -inf -> 0
    x = rand_bf16(rng, 5000); x[::3] = 0x7FC0; cases.append(x)        # NaNs never taken
    cases.append(np.full(17, 0x7FC0, np.uint16))                      # all NaN -> INT_MAX
    cases.append(rand_bf16(rng, 1))
    cases.append(rand_bf16(rng, 13))
    out = dev_i32([-5])
    for x in cases:
        gpu.argmax_forward(out, dev(x), x.size)
        torch.cuda.synchronize()
        assert int(out.cpu()[0]) == oracle.argmax(x)
    # an unaligned view (falls back to 2-byte loads)
    x = rand_bf16(rng, 1001)
    xd = dev(x)
    gpu.argmax_forward(out, xd[1:], 1000)
    torch.cuda.synchronize()
    assert int(out.cpu()[0]) == oracle.argmax(x[1:])
