"""Pins the CPU oracle (oracle/oracle.c) with checks that do not restate its formulas: libm,
exact decimal arithmetic, closed forms, invariants, brute force, and the reference's published
byte counts. Each test names the oracle function and the plausible mistake it would catch."""
import json
import math
import os
from decimal import Decimal, getcontext

import numpy as np
import pytest

from conftest import (bf16_bits, bf16_ulp_diff, bf16_vals, rand_bf16, ulp_bf16,
                      within_one_ulp_then_scale)


# ---------------------------------------------------------------- numerics

def test_bf16_rounding_round_half_even(oracle):
    """orc_f32_to_bf16 against an independent round-half-even on exact rationals."""
    rng = np.random.default_rng(1)
    u = rng.integers(0, 2**32, size=200000, dtype=np.uint64).astype(np.uint32)
    # include exact ties and their neighbours
    ties = (rng.integers(0, 2**16, size=5000, dtype=np.uint32) << 16) | 0x8000
    u = np.concatenate([u, ties, ties + 1, ties - 1]).astype(np.uint32)
    f = u.view(np.float32)
    finite = np.isfinite(f)
    got = np.array([oracle.lib().orc_f32_to_bf16(float(x)) for x in f[:3000]], dtype=np.uint16)
    assert np.array_equal(got, oracle.f32_to_bf16(f[:3000]))
    b = oracle.f32_to_bf16(f[finite])
    # independent: nearest of the two bf16 candidates by exact difference, ties to even
    x = f[finite].astype(np.float64)
    lo = (u[finite] & 0xFFFF0000).view(np.float32).astype(np.float64)
    hi_bits = ((u[finite] >> 16) + 1).astype(np.uint32) << 16
    hi = hi_bits.view(np.float32).astype(np.float64)
    # past the largest bf16 the next candidate is +-2^128 (IEEE rounds as if unbounded, then
    # overflows to inf)
    hi = np.where(np.isinf(hi), np.sign(hi) * 2.0 ** 128, hi)
    dlo, dhi = np.abs(x - lo), np.abs(hi - x)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (((u[finite] >> 16) & 1) == 1))
    expect = np.where(pick_hi, (u[finite] >> 16) + 1, u[finite] >> 16).astype(np.uint16)
    assert np.array_equal(b, expect)
    nan = oracle.f32_to_bf16(np.array([np.nan, -np.nan], dtype=np.float32))
    assert np.all(np.isnan(bf16_vals(nan)))


def test_exp_f32_exhaustive_within_one_ulp(oracle):
    """orc_exp_f32 (the kernels' exp) on every fp32 input in [-104, 89] against libm exp in
    double rounded to fp32: a wrong coefficient, reduction constant or scaling shows up as
    a multi-ulp error somewhere in 2.2e9 inputs."""
    worst, n, ndiff = oracle.selfcheck_exp(-104.0, 89.0)
    assert n > 2_000_000_000
    assert worst <= 1
    assert ndiff / n < 0.02
    assert oracle.exp_f32(0.0) == 1.0
    assert oracle.exp_f32(-200.0) == 0.0 and math.isinf(oracle.exp_f32(90.0))
    assert math.isnan(oracle.exp_f32(float("nan")))


def test_sincos_matches_libm_at_rope_angles(oracle):
    """orc_sincos_d rounded to fp32 against libm at every RoPE angle of the benchmark shapes
    (theta 1e6, D 128, positions < 8448) and of a theta 1e4 / D 64 / 40960-position table."""
    diff, n = oracle.selfcheck_sincos(1e6, 128, 8448)
    assert n == 2 * 8448 * 64 and diff == 0
    diff, n = oracle.selfcheck_sincos(1e4, 64, 40960)
    assert diff == 0
    s, c = oracle.sincos(0.0)
    assert (s, c) == (0.0, 1.0)
    s, c = oracle.sincos(math.pi / 2)
    assert abs(s - 1) < 1e-15 and abs(c - math.cos(math.pi / 2)) < 1e-15


def _cr_pow_f32(theta, e):
    getcontext().prec = 60
    v = Decimal(float(np.float32(theta))) ** Decimal(float(np.float32(e)))
    return np.float32(float(v))  # float(Decimal) rounds correctly to double, then fp32


def test_inv_freq_correctly_rounded(oracle):
    """orc_inv_freq = 1 / fp32(theta^(2j/D)): the power against 60-digit decimal arithmetic."""
    for theta, D in [(1e6, 128), (1e4, 128), (1e6, 64)]:
        got = oracle.inv_freq(theta, D)
        for j in range(D // 2):
            e = np.float32(2 * j) / np.float32(D)
            expect = np.float32(1.0) / _cr_pow_f32(theta, e)
            assert got[j] == expect, (theta, D, j)
    assert oracle.inv_freq(1e6, 128)[0] == 1.0


# ---------------------------------------------------------------- RMSNorm

@pytest.mark.parametrize("mode", [0, 1])
def test_rmsnorm_closed_forms(oracle, mode):
    """orc_rmsnorm: zero row -> 0; constant row c -> sign(c) * gamma (eps negligible);
    power-of-two scaling of x leaves y unchanged when eps = 0."""
    rng = np.random.default_rng(2)
    for dim in (1024, 2560, 8200, 100):
        w = rand_bf16(rng, dim, 0.1, 1.0)
        y = oracle.rmsnorm(np.zeros(dim, np.uint16), w, 1e-6, mode)
        assert np.all(bf16_vals(y) == 0)
        for c in (0.75, -3.0):
            x = bf16_bits(np.full(dim, c))
            y = oracle.rmsnorm(x, w, 1e-6, mode)
            assert np.array_equal(y, bf16_bits(np.sign(c) * bf16_vals(w))), (dim, c)
        x = rand_bf16(rng, dim)
        y0 = oracle.rmsnorm(x, w, 0.0, mode)
        y1 = oracle.rmsnorm(bf16_bits(bf16_vals(x) * np.float32(8.0)), w, 0.0, mode)
        assert np.array_equal(y0, y1)


@pytest.mark.parametrize("dim", [1024, 2560, 100, 9000])
def test_rmsnorm_against_double(oracle, dim):
    """Both modes within 1 bf16 ulp of x / sqrt(mean(x^2) + eps) in double, rounded at HF's two
    points; a wrong divisor (dim) or a dropped gamma fails by far more."""
    rng = np.random.default_rng(dim)
    x = rand_bf16(rng, (6, dim))
    w = rand_bf16(rng, dim, 0.1, 1.0)
    xv = bf16_vals(x).astype(np.float64)
    inv = 1.0 / np.sqrt((xv * xv).mean(axis=1, keepdims=True) + 1e-6)
    n = bf16_bits((xv * inv).astype(np.float32))
    ref = bf16_bits(bf16_vals(n) * bf16_vals(w))
    for mode in (0, 1):
        y = oracle.rmsnorm(x, w, 1e-6, mode)
        assert within_one_ulp_then_scale(y, n, w).all()
        assert (y != ref).mean() < 0.01


# ---------------------------------------------------------------- dot / GEMV

def test_dot_against_double_brute_force(oracle):
    """orc_gemv (both modes) against a float64 brute-force dot rounded once: within one bf16 ulp
    plus the fp32 reduction bound. A transposed matrix or dropped chunk fails by far more."""
    rng = np.random.default_rng(3)
    for rows, cols in [(64, 1024), (32, 2560), (16, 9728), (8, 8), (8, 520)]:
        w = rand_bf16(rng, (rows, cols), 0.02)
        x = rand_bf16(rng, cols)
        exact = bf16_vals(w).astype(np.float64) @ bf16_vals(x).astype(np.float64)
        absum = np.abs(bf16_vals(w).astype(np.float64)) @ np.abs(bf16_vals(x).astype(np.float64))
        bound = ulp_bf16(exact) + 2 * cols * 2.0 ** -24 * absum
        for mode in (0, 1):
            y = bf16_vals(oracle.gemv(w, x, mode)).astype(np.float64)
            assert np.all(np.abs(y - exact) <= bound), (rows, cols, mode)
        y0, y1 = oracle.gemv(w, x, 0), oracle.gemv(w, x, 1)
        assert bf16_ulp_diff(y0, y1).max() <= 1


def test_gemv_residual_and_taps(oracle):
    """orc_gemv_residual: tap = bf16(W in); x' = bf16(x + tap) exactly (ref/dump.py:104-108)."""
    rng = np.random.default_rng(4)
    w = rand_bf16(rng, (256, 1024), 0.02)
    inp = rand_bf16(rng, 1024)
    x = rand_bf16(rng, 256)
    x2, tap = oracle.gemv_residual(x, w, inp, 0, with_tap=True)
    assert np.array_equal(tap, oracle.gemv(w, inp, 0))
    assert np.array_equal(x2, bf16_bits(bf16_vals(x) + bf16_vals(tap)))


# ---------------------------------------------------------------- SwiGLU

def test_swiglu_closed_forms(oracle):
    """orc_swiglu: g = 0 -> 0; large +g -> bf16(g * u); large -g -> 0 (signed); and the silu
    value against libm in double for every finite bf16 gate with u = 1."""
    up = bf16_bits(np.array([1.5, -2.0, 3.0], np.float32))
    zero = bf16_bits(np.zeros(3))
    assert np.all(bf16_vals(oracle.swiglu(zero, up)) == 0)
    big = bf16_bits(np.full(3, 100.0))
    assert np.array_equal(oracle.swiglu(big, up), bf16_bits(100.0 * bf16_vals(up)))
    neg = bf16_bits(np.full(3, -200.0))
    assert np.all(bf16_vals(oracle.swiglu(neg, up)) == 0)
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    g = g[np.isfinite(bf16_vals(g))]
    one = bf16_bits(np.ones(g.size))
    gv = bf16_vals(g).astype(np.float64)
    # where exp(-g) fits fp32 the silu is compared with double precision; below that (g < -88.7)
    # fp32 evaluation (HF's and the reference's) overflows exp and gives exactly -0
    fits = gv > -88.0
    with np.errstate(over="ignore"):
        s = gv / (1.0 + np.exp(-gv))
    ref = bf16_bits(s.astype(np.float32))
    for mode in (0, 1):
        got = oracle.swiglu(g, one, mode)
        d = bf16_ulp_diff(got[fits], ref[fits])
        assert d.max() <= 1, mode
        assert (d > 0).sum() < 20
        assert np.all(bf16_vals(got[gv < -89.0]) == 0)


def test_gate_up_composes_gemv_and_swiglu(oracle):
    """orc_gate_up == swiglu(gemv(Wg), gemv(Wu)) with the taps equal to the two GEMVs."""
    rng = np.random.default_rng(5)
    wg = rand_bf16(rng, (300, 1024), 0.02)
    wu = rand_bf16(rng, (300, 1024), 0.02)
    x = rand_bf16(rng, 1024)
    for mode in (0, 1):
        act, gt, ut = oracle.gate_up(wg, wu, x, mode, with_taps=True)
        assert np.array_equal(gt, oracle.gemv(wg, x, mode))
        assert np.array_equal(ut, oracle.gemv(wu, x, mode))
        assert np.array_equal(act, oracle.swiglu(gt, ut, mode))


# ---------------------------------------------------------------- QK-norm + RoPE

def _rope_inputs(rng, n_tokens, hq, hkv, D=128, max_seq=64):
    q = rand_bf16(rng, (n_tokens, hq * D))
    k = rand_bf16(rng, (n_tokens, hkv * D))
    v = rand_bf16(rng, (n_tokens, hkv * D))
    qn = rand_bf16(rng, D, 0.1, 1.0)
    kn = rand_bf16(rng, D, 0.1, 1.0)
    kc = np.full((max_seq, hkv * D), 0x7FC1, np.uint16)  # sentinel NaN pattern
    vc = kc.copy()
    return q, k, v, qn, kn, kc, vc


@pytest.mark.parametrize("mode", [0, 1])
def test_rope_position_zero_is_identity(oracle, mode):
    """At pos 0 cos = 1 and sin = 0, so the output equals the normed head (the tap)."""
    rng = np.random.default_rng(6)
    q, k, v, qn, kn, kc, vc = _rope_inputs(rng, 1, 4, 2)
    q2, k2, kc2, vc2, qt, kt = oracle.qk_norm_rope_rows(q, k, v, qn, kn, kc, vc, [0], 4, 2, 128,
                                                        1e-6, 1e6, mode, with_taps=True)
    assert np.array_equal(q2, qt) and np.array_equal(k2, kt)
    # the tap is the per-head RMSNorm: same as orc_rmsnorm on each head
    assert np.array_equal(qt.reshape(4, 128), oracle.rmsnorm(q.reshape(4, 128), qn, 1e-6, mode))


@pytest.mark.parametrize("mode", [0, 1])
def test_rope_frequency_one_pair(oracle, mode):
    """Pair j = 0 has inv_freq 1, so its rotation angle is pos: checked against libm cos/sin of
    pos rounded through fp32 to bf16, and the 2x2 rotation with bf16 products."""
    rng = np.random.default_rng(7)
    q, k, v, qn, kn, kc, vc = _rope_inputs(rng, 3, 2, 1, max_seq=5000)
    pos = [5, 1000, 4095]
    q2, _, _, _, qt, _ = oracle.qk_norm_rope_rows(q, k, v, qn, kn, kc, vc, pos, 2, 1, 128, 1e-6,
                                                  1e6, mode, with_taps=True)
    for t, p in enumerate(pos):
        c = bf16_vals(bf16_bits(np.float32(math.cos(p))))
        s = bf16_vals(bf16_bits(np.float32(math.sin(p))))
        for h in range(2):
            a = bf16_vals(qt[t, h * 128 + 0])
            b = bf16_vals(qt[t, h * 128 + 64])
            r = lambda z: bf16_vals(bf16_bits(np.float32(z)))
            ea = bf16_bits(r(a * c) - r(b * s))
            eb = bf16_bits(r(b * c) + r(a * s))
            assert q2[t, h * 128] == ea and q2[t, h * 128 + 64] == eb, (t, h)


def test_rope_preserves_norm_and_cache_slots(oracle):
    """Rotation keeps each head's norm (to bf16 rounding); k' and v land in cache row pos
    bit-exactly and every other row keeps its sentinel."""
    rng = np.random.default_rng(8)
    q, k, v, qn, kn, kc, vc = _rope_inputs(rng, 2, 4, 2, max_seq=64)
    pos = [17, 40]
    q2, k2, kc2, vc2, qt, kt = oracle.qk_norm_rope_rows(q, k, v, qn, kn, kc, vc, pos, 4, 2, 128,
                                                        1e-6, 1e6, 0, with_taps=True)
    n_in = np.linalg.norm(bf16_vals(qt).reshape(-1, 128), axis=1)
    n_out = np.linalg.norm(bf16_vals(q2).reshape(-1, 128), axis=1)
    assert np.allclose(n_in, n_out, rtol=1e-2)
    for t, p in enumerate(pos):
        assert np.array_equal(kc2[p], k2[t]) and np.array_equal(vc2[p], v[t])
    untouched = [r for r in range(64) if r not in pos]
    assert np.all(kc2[untouched] == 0x7FC1) and np.all(vc2[untouched] == 0x7FC1)


def test_rope_modes_agree(oracle):
    rng = np.random.default_rng(9)
    q, k, v, qn, kn, kc, vc = _rope_inputs(rng, 16, 16, 8, max_seq=4096)
    pos = rng.integers(0, 4096, 16)
    a = oracle.qk_norm_rope_rows(q, k, v, qn, kn, kc, vc, pos, 16, 8, 128, 1e-6, 1e6, 0)
    b = oracle.qk_norm_rope_rows(q, k, v, qn, kn, kc, vc, pos, 16, 8, 128, 1e-6, 1e6, 1)
    d = bf16_ulp_diff(a[0], b[0])
    assert d.max() <= 2 and (d > 0).mean() < 0.01


# ---------------------------------------------------------------- attention

def _attn_inputs(rng, hq, hkv, n, D=128, max_seq=None):
    max_seq = max_seq or n
    q = rand_bf16(rng, hq * D)
    kc = rand_bf16(rng, (max_seq, hkv * D))
    vc = rand_bf16(rng, (max_seq, hkv * D))
    return q, kc, vc


@pytest.mark.parametrize("mode", [0, 1])
def test_attention_single_position_returns_v(oracle, mode):
    """pos = 0: softmax over one score is 1, so out = v of the GQA-mapped kv head."""
    rng = np.random.default_rng(10)
    q, kc, vc = _attn_inputs(rng, 4, 2, 8)
    out = oracle.attention(q, kc, vc, 4, 2, 128, 0, 128 ** -0.5, mode)
    for h in range(4):
        assert np.array_equal(out[h * 128:(h + 1) * 128], vc[0, (h // 2) * 128:(h // 2 + 1) * 128])


@pytest.mark.parametrize("mode", [0, 1])
def test_attention_equal_keys_average_values(oracle, mode):
    """Identical keys give p_t = bf16(1/n) for every t; out = bf16(sum p v) (fp32 bound)."""
    rng = np.random.default_rng(11)
    n = 150
    q, kc, vc = _attn_inputs(rng, 2, 1, n)
    kc[:] = kc[0]
    out = bf16_vals(oracle.attention(q, kc, vc, 2, 1, 128, n - 1, 128 ** -0.5, mode))
    p = bf16_vals(bf16_bits(np.float32(1.0) / np.float32(n)))
    ref = p * bf16_vals(vc).astype(np.float64).sum(axis=0)
    bound = ulp_bf16(ref) + 1e-5
    assert np.all(np.abs(np.tile(out.reshape(2, 128), 1)[0] - ref) <= bound)


def test_attention_modes_agree_against_double(oracle):
    """GPU-order (split softmax, 64-position blocks) and exact mode both within 2 bf16 ulps of
    a double-precision softmax(q k^T * scale) v with HF's bf16 rounding of scores and p."""
    rng = np.random.default_rng(12)
    hq, hkv, D = 8, 2, 128
    for n in (1, 63, 64, 65, 300):
        q, kc, vc = _attn_inputs(rng, hq, hkv, n)
        scale = np.float32(D ** -0.5)
        ref = np.zeros(hq * D)
        for h in range(hq):
            g = h // (hq // hkv)
            kh = bf16_vals(kc[:, g * D:(g + 1) * D]).astype(np.float64)
            vh = bf16_vals(vc[:, g * D:(g + 1) * D]).astype(np.float64)
            s = kh @ bf16_vals(q[h * D:(h + 1) * D]).astype(np.float64)
            s = bf16_vals(bf16_bits(bf16_vals(bf16_bits(s.astype(np.float32))) * scale))
            e = np.exp(s.astype(np.float64) - s.max())
            p = bf16_vals(bf16_bits((e / e.sum()).astype(np.float32))).astype(np.float64)
            ref[h * D:(h + 1) * D] = p @ vh
        for mode in (0, 1):
            out = oracle.attention(q, kc, vc, hq, hkv, D, n - 1, float(scale), mode)
            d = bf16_ulp_diff(out, bf16_bits(ref.astype(np.float32)))
            assert d.max() <= 2, (n, mode)


# ---------------------------------------------------------------- argmax

def test_argmax_rules(oracle):
    """orc_argmax: brute force on random rows; all-equal -> 0; duplicated maxima -> lowest
    index; -inf entries; max at the last index; NaN is never taken; all-NaN -> INT_MAX."""
    rng = np.random.default_rng(13)
    for _ in range(20):
        x = rand_bf16(rng, 151936)
        assert oracle.argmax(x) == int(np.argmax(bf16_vals(x)))
    assert oracle.argmax(bf16_bits(np.full(100, 2.5))) == 0
    x = bf16_bits(np.array([1, 5, 3, 5, 5], np.float32))
    assert oracle.argmax(x) == 1
    x = bf16_bits(np.array([-np.inf, -np.inf, -np.inf], np.float32))
    assert oracle.argmax(x) == 0
    x = bf16_bits(np.array([-np.inf, -1e30, -np.inf], np.float32))
    assert oracle.argmax(x) == 1
    x = bf16_bits(np.arange(1000, dtype=np.float32))  # 998 and 999 share a bf16: tie -> 998
    assert oracle.argmax(x) == 998
    x[-1] = bf16_bits(np.float32(5000.0)).item()
    assert oracle.argmax(x) == 999
    x = bf16_bits(np.array([1.0, np.nan, 2.0, np.nan], np.float32))
    assert oracle.argmax(x) == 2
    x = bf16_bits(np.full(5, np.nan, np.float32))
    assert oracle.argmax(x) == 2**31 - 1


# ---------------------------------------------------------------- byte counts

def test_byte_counts_match_published(oracle):
    """orc_weight_bytes_per_step / orc_kv_bytes_per_position reproduce the reference's published
    bytes per step (bench/results.csv:289, :317, :345) with its mean-position rule
    bytes = weights + kv * (n_prompt + (steps + 1) / 2), 5-token prompt, 256 steps."""
    published = {"0.6B": ((1024, 3072, 28, 16, 8), 1207412736),
                 "1.7B": ((2048, 6144, 28, 16, 8), 3456464896),
                 "4B": ((2560, 9728, 36, 32, 8), 8064626688)}
    for name, ((H, I, L, hq, hkv), total) in published.items():
        m = oracle.OrcConfig(H, I, L, hq, hkv, 128, 151936, 1e-6, 1e6)
        import ctypes
        wb = oracle.lib().orc_weight_bytes_per_step(ctypes.byref(m))
        kb = oracle.lib().orc_kv_bytes_per_position(ctypes.byref(m))
        assert wb + kb * (5 + 257 / 2) == total, name


# ---------------------------------------------------------------- HF golden fixture

HF_FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "hf_small_qwen3.npz")
LOGIT_TOL = 2e-2  # the final-logits bound against the HF path
TIE_GAP = 0.25    # ref/compare.py:18: a greedy flip is accepted only below this top-2 gap


def hf_fixture():
    f = np.load(HF_FIXTURE)  # allow_pickle=False (default): plain arrays and a JSON string
    return f, json.loads(str(f["meta"]))


def small_oracle(oracle):
    from conftest import SMALL, small_weights
    cfg = dict(SMALL, rms_norm_eps=1e-6, rope_theta=1e6)
    return oracle.Model(cfg, small_weights(0), max_seq=64)


@pytest.mark.parametrize("mode", ["GPU_ORDER", "EXACT"])
def test_oracle_logits_match_hf_fixture(oracle, mode):
    """The oracle's whole step against HF transformers' Qwen3 (bf16, eager attention, CPU) on
    the small seeded model: teacher-forced logits at every position within 2e-2."""
    f, meta = hf_fixture()
    m = small_oracle(oracle)
    worst = 0.0
    for pos, tok in enumerate(meta["tokens"]):
        m.forward(tok, pos, getattr(oracle, mode))
        diff = np.abs(bf16_vals(m.logits).astype(np.float64) - f["logits"][pos])
        worst = max(worst, float(diff.max()))
    assert worst <= LOGIT_TOL, worst
    # and not trivially: the logits are not all near zero
    assert np.abs(f["logits"]).max() > 10 * LOGIT_TOL


def test_oracle_greedy_matches_hf_fixture(oracle):
    """Greedy tokens after the fixture's prompt equal HF's, or part from them only at a near tie
    (HF's top-2 gap at that step <= TIE_GAP, the reference's greedy rule, ref/greedy.py:14-31)."""
    f, meta = hf_fixture()
    m = small_oracle(oracle)
    prompt = meta["prompt"]
    for pos, tok in enumerate(prompt):
        t = m.forward(tok, pos, oracle.GPU_ORDER)
    got = [t]
    for i in range(len(f["greedy"]) - 1):
        t = m.forward(t, len(prompt) + i, oracle.GPU_ORDER)
        got.append(t)
    ref = [int(x) for x in f["greedy"]]
    for i, (a, b) in enumerate(zip(got, ref)):
        if a != b:
            assert f["greedy_gap"][i] <= TIE_GAP, (i, a, b, float(f["greedy_gap"][i]))
            break


# ---------------------------------------------------------------- temperature sampling

def test_sample_closed_forms(oracle):
    """orc_sample (src/kernels.cu:546-597): a uniform row gives floor(u n); a one-hot row gives
    its token for every u; u = 0 gives the first token with weight. Catches an off-by-one in the
    chunk walk or an inverted comparison."""
    n = 151936
    flat = bf16_bits(np.zeros(n, np.float32))
    for u in [0.0, 0.1, 0.37, 0.5, 0.999]:
        assert oracle.sample(flat, 1.0, u) == int(u * n), u
    hot = bf16_bits(np.full(n, -100.0, np.float32))
    for k in [0, 7, 77777, n - 1]:
        h = hot.copy()
        h[k] = bf16_bits(np.array([100.0], np.float32))[0]
        for u in [0.0, 0.5, 0.999999]:
            assert oracle.sample(h, 1.0, u) == k, (k, u)
    row = rand_bf16(np.random.default_rng(3), n, 2.0)
    assert oracle.sample(row, 1.0, 0.0) == 0


def test_sample_against_double_cdf(oracle):
    """Random rows: the chosen index brackets u in the float64 CDF of the same weights (up to the
    fp32 accumulation error), and a higher temperature spreads the draws."""
    rng = np.random.default_rng(5)
    n = 20000
    for trial in range(6):
        row = rand_bf16(rng, n, 3.0)
        inv_temp = [1.0, 0.5, 2.0][trial % 3]
        x = bf16_vals(row).astype(np.float64)
        w = np.exp((x - x.max()) * inv_temp)
        cdf = np.cumsum(w) / w.sum()
        for u in rng.random(8):
            i = oracle.sample(row, inv_temp, float(u))
            lo = cdf[i - 1] if i > 0 else 0.0
            assert lo - 1e-5 <= u <= cdf[i] + 1e-5, (trial, u, i, lo, cdf[i])


def test_hf_dump_fixture_wiring(oracle):
    """The HF dump fixture holds what its names say (ref/dump.py:101-108): the embedding rows of
    the tokens, and each residual add exactly bf16(x + y)."""
    from conftest import SMALL, small_weights
    here = os.path.dirname(os.path.abspath(__file__))
    ref = np.load(os.path.join(here, "golden", "hf_small_qwen3_dumps.npz"))
    tokens = hf_fixture()[1]["tokens"]
    emb = small_weights(0)["model.embed_tokens.weight"]
    assert np.array_equal(ref["embed"], emb[tokens])
    v = {n: bf16_vals(ref[n]).astype(np.float32) for n in ref.files}
    x = v["embed"]
    for l in range(SMALL["n_layers"]):
        p = f"L{l:02d}."
        assert np.array_equal(ref[p + "attn_resid"], bf16_bits(x + v[p + "o_proj"]))
        x = v[p + "out"]
        assert np.array_equal(ref[p + "out"], bf16_bits(v[p + "attn_resid"] + v[p + "down"]))
