/*
 * CPU oracle for the fused Qwen3 decode-layer path. TEST INFRASTRUCTURE ONLY: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it, as the results the GPU path
 * is compared with or as the timed CPU baseline. Nothing in the product path links or calls it.
 *
 * What each function restates (reference = William-Lamer/llm-inference):
 *   orc_embedding      src/kernels.cu:7-15
 *   orc_rmsnorm        src/kernels.cu:25-64, HF modeling_qwen3.py:59-64 (Qwen3RMSNorm)
 *   orc_dot/orc_gemv   src/kernels.cu:79-106, :159-173
 *   orc_gemv_residual  src/kernels.cu:185-203, HF modeling_qwen3.py:316,:322 (residual adds)
 *   orc_qkv            src/kernels.cu:215-247
 *   orc_gate_up        src/kernels.cu:109-144, :260-288, HF modeling_qwen3.py:81-83 (Qwen3MLP)
 *   orc_swiglu         src/kernels.cu:283-286 applied elementwise
 *   orc_qk_norm_rope   src/kernels.cu:301-384, HF modeling_qwen3.py:121,:126-170,:252-253
 *   orc_attention      src/kernels.cu:439-486, HF modeling_qwen3.py:185-207 (eager attention)
 *   orc_argmax         src/kernels.cu:499-538
 *   orc_sample         src/kernels.cu:546-597 (inverse-CDF temperature sampling)
 *   orc_forward        src/forward.cu:118-193 (layer order), :229-236 (greedy sample)
 *   orc_*_bytes        src/forward.cu:83-114
 *
 * Parity pinning (tests/test_oracle.py; no check restates the formula it pins):
 *   bf16 rounding      an independent nearest/ties-to-even selection over 215k patterns
 *                      (exact ties, overflow, denormals, NaN).
 *   orc_exp_f32        every fp32 input in [-104, 89] against (float)exp((double)x): <= 1 ulp.
 *   orc_sincos_d       libm cos/sin at every RoPE angle of two (theta, D) tables: identical
 *                      after fp32 rounding.
 *   orc_inv_freq       60-digit decimal pow: correctly rounded.
 *   orc_rmsnorm        closed forms (zero row, constant row, power-of-two scale invariance) and
 *                      a double-precision reference (<= 1 bf16 ulp at HF's rounding point).
 *   orc_dot/gemv       double brute force (<= 1 bf16 ulp + the fp32 accumulation bound).
 *   orc_gemv_residual  the tap equals the GEMV, the add equals bf16(x + tap) (ref/dump.py:104-108).
 *   orc_swiglu/gate_up closed forms (g = 0, large +-g), every finite bf16 gate against libm
 *                      double silu (1 ulp), gate_up = gemv + swiglu.
 *   orc_qk_norm_rope   pos 0 is the identity, the frequency-1 pair rotates by pos exactly,
 *                      norm preservation, KV slot invariants against a sentinel fill.
 *   orc_attention      single position (output = v), equal keys (mean of v), a double softmax
 *                      reference within 2 ulps.
 *   orc_argmax         brute force, ties, -inf, last index, NaN policy.
 *   orc_sample         u -> 0 and u -> 1 pick the first and last tokens with weight, a one-hot
 *                      row picks its token for every u, uniform rows pick floor(u n).
 *   orc_forward        HF transformers' Qwen3ForCausalLM on the small seeded model
 *                      (tests/golden/hf_small_qwen3.npz): logits within 2e-2, greedy tokens.
 *   byte formulas      the reference's published bytes/step (bench/results.csv:289,:317,:345).
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------ */
/* bf16                                                                                        */
/* ------------------------------------------------------------------------------------------ */

/* Round-to-nearest-even fp32 -> bf16; NaN stays NaN with the quiet bit set. */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float orc_round_bf16(float f) { return orc_bf16_to_f32(orc_f32_to_bf16(f)); }

/* The same conversion as orc_bf16_to_f32, inlined where the hot loops use it (the exported
 * function is called through the PLT in a shared library and would not be inlined). */
static inline float bf(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline uint16_t tobf(float f) { return orc_f32_to_bf16(f); }

/* ------------------------------------------------------------------------------------------ */
/* transcendental functions                                                                   */
/* ------------------------------------------------------------------------------------------ */

static inline float pow2i(int n) { /* 2^n for n in [-126, 127] */
    uint32_t u = (uint32_t)(n + 127) << 23;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/*
 * exp in fp32: k = rint(x*log2(e)); r = x - k*ln2 with ln2 split in a 16-bit head (so k*hi is
 * exact and x - k*hi is exact by Sterbenz) and a tail; e^r by the degree-7 Taylor series
 * (truncation < 0.1 ulp on |r| <= ln2/2) evaluated as 1 + (r + r^2*q(r)); the result scaled by
 * 2^k in two exact-or-single-rounding steps so gradual underflow rounds once.
 */
float orc_exp_f32(float x) {
    if (x != x) return x;
    if (x > 89.0f) return INFINITY;
    if (x < -104.0f) return 0.0f;
    float k = rintf(x * 0x1.715476p+0f);
    float r = fmaf(k, -0x1.62e400p-1f, x);
    r = fmaf(k, -0x1.7f7d1cp-20f, r);
    float q = 0x1.a01a02p-13f;
    q = fmaf(q, r, 0x1.6c16c2p-10f);
    q = fmaf(q, r, 0x1.111112p-7f);
    q = fmaf(q, r, 0x1.555556p-5f);
    q = fmaf(q, r, 0x1.555556p-3f);
    q = fmaf(q, r, 0x1.000000p-1f);
    float r2 = r * r;
    float t = fmaf(r2, q, r);
    float p = 1.0f + t;
    int ki = (int)k;
    int k1 = ki / 2;
    int k2 = ki - k1;
    return p * pow2i(k1) * pow2i(k2);
}

float orc_exp_ref(float x) { return (float)exp((double)x); }

/*
 * sin and cos in double: k = rint(x*2/pi); r = x - k*pi/2 with pi/2 split into two 33-bit
 * heads and a tail (k*head exact for |k| < 2^20); Taylor series to x^17 (sin) and x^18 (cos)
 * on |r| <= pi/4, Horner with fma; quadrant from k mod 4.
 */
void orc_sincos_d(double x, double *s_out, double *c_out) {
    double k = rint(x * 0x1.45f306dc9c883p-1);
    double r = fma(-k, 0x1.921fb54400000p+0, x);
    r = fma(-k, 0x1.0b4611a600000p-34, r);
    r = fma(-k, 0x1.3198a2e037073p-69, r);
    double z = r * r;
    double ps = 0x1.952c77030ad4ap-49;
    ps = fma(ps, z, -0x1.ae7f3e733b81fp-41);
    ps = fma(ps, z, 0x1.6124613a86d09p-33);
    ps = fma(ps, z, -0x1.ae64567f544e4p-26);
    ps = fma(ps, z, 0x1.71de3a556c734p-19);
    ps = fma(ps, z, -0x1.a01a01a01a01ap-13);
    ps = fma(ps, z, 0x1.1111111111111p-7);
    ps = fma(ps, z, -0x1.5555555555555p-3);
    double sr = fma(r * z, ps, r);
    double pc = -0x1.6827863b97d97p-53;
    pc = fma(pc, z, 0x1.ae7f3e733b81fp-45);
    pc = fma(pc, z, -0x1.93974a8c07c9dp-37);
    pc = fma(pc, z, 0x1.1eed8eff8d898p-29);
    pc = fma(pc, z, -0x1.27e4fb7789f5cp-22);
    pc = fma(pc, z, 0x1.a01a01a01a01ap-16);
    pc = fma(pc, z, -0x1.6c16c16c16c17p-10);
    pc = fma(pc, z, 0x1.5555555555555p-5);
    pc = fma(pc, z, -0x1.0000000000000p-1);
    double cr = fma(z, pc, 1.0);
    int quadrant = (int)((long long)k & 3);
    double s, c;
    switch (quadrant) {
    case 0: s = sr; c = cr; break;
    case 1: s = cr; c = -sr; break;
    case 2: s = -sr; c = -cr; break;
    default: s = -cr; c = sr; break;
    }
    *s_out = s;
    *c_out = c;
}

/* 1/theta^(2j/D) in fp32 as HF computes it (modeling_qwen3.py:121): the exponent is an fp32
 * quotient, the power is rounded once from libm's double pow, the reciprocal is fp32. */
float orc_inv_freq(float theta, int j, int head_dim) {
    float e = (float)(2 * j) / (float)head_dim;
    return 1.0f / (float)pow((double)theta, (double)e);
}

float orc_silu(float g, int mode) {
    float e = (mode == ORC_EXACT) ? orc_exp_ref(-g) : orc_exp_f32(-g);
    return g / (1.0f + e);
}

/* ------------------------------------------------------------------------------------------ */
/* reduction trees of the kernels                                                              */
/* ------------------------------------------------------------------------------------------ */

/* xor-butterfly over n lanes (n a power of two): the balanced pairwise tree in lane order. */
static float tree_sum(float *a, int n) {
    for (int s = 1; s < n; s <<= 1)
        for (int l = 0; l < n; l += 2 * s) a[l] = a[l] + a[l + s];
    return a[0];
}

/* A 64-lane wave: lane l takes 8-element chunks l, l+64, ...; each lane fma-accumulates its
 * elements in order; the lanes then meet in the xor tree. cols % 8 == 0. The loops run the 64
 * lanes' chains side by side (the same operations in each lane's order), so the CPU overlaps
 * 64 independent fma chains instead of waiting out one at a time. */
static float dot_gpu(const uint16_t *w, const uint16_t *x, int cols) {
    float acc[64];
    for (int l = 0; l < 64; l++) acc[l] = 0.0f;
    int n_chunks = cols / 8;
    for (int c0 = 0; c0 < n_chunks; c0 += 64) {
        int lanes = n_chunks - c0 < 64 ? n_chunks - c0 : 64;
        const uint16_t *wc = w + 8 * c0, *xc = x + 8 * c0;
        for (int e = 0; e < 8; e++)
            for (int l = 0; l < lanes; l++) acc[l] = fmaf(bf(wc[8 * l + e]), bf(xc[8 * l + e]), acc[l]);
    }
    return tree_sum(acc, 64);
}

static double dot_exact(const uint16_t *w, const uint16_t *x, int cols) {
    double a = 0.0;
    for (int i = 0; i < cols; i++) a += (double)bf(w[i]) * (double)bf(x[i]);
    return a;
}

float orc_dot(const uint16_t *w_row, const uint16_t *x, int cols, int mode) {
    if (mode == ORC_EXACT) return (float)dot_exact(w_row, x, cols);
    return dot_gpu(w_row, x, cols);
}

/* bf16 of a dot product. GPU order rounds its fp32 sum; exact mode rounds the double sum to
 * fp32 then bf16, the same two steps as an fp32-accumulating GEMM with a bf16 output. */
static uint16_t dot_bf16(const uint16_t *w, const uint16_t *x, int cols, int mode) {
    if (mode == ORC_EXACT) return tobf((float)dot_exact(w, x, cols));
    return tobf(dot_gpu(w, x, cols));
}

/* ------------------------------------------------------------------------------------------ */
/* ops                                                                                         */
/* ------------------------------------------------------------------------------------------ */

void orc_embedding(uint16_t *out, const uint16_t *table, int token, int hidden) {
    memcpy(out, table + (size_t)token * hidden, (size_t)hidden * 2);
}

/* Threads per RMSNorm row in the kernel: one wave while every lane holds at most 16 chunks,
 * else enough waves (up to 16) for 16 chunks per lane. */
static int rms_waves(int dim) {
    int n_chunks = (dim + 7) / 8;
    int w = (n_chunks + 64 * 16 - 1) / (64 * 16);
    if (w < 1) w = 1;
    if (w > 16) w = 16;
    return w;
}

static float sumsq_gpu(const uint16_t *x, int dim) {
    int waves = rms_waves(dim);
    int threads = 64 * waves;
    int n_chunks = (dim + 7) / 8;
    float total = 0.0f;
    for (int w = 0; w < waves; w++) {
        float acc[64];
        for (int l = 0; l < 64; l++) {
            int t = w * 64 + l;
            float a = 0.0f;
            for (int c = t; c < n_chunks; c += threads)
                for (int e = 0; e < 8; e++) {
                    int i = 8 * c + e;
                    if (i < dim) a = fmaf(bf(x[i]), bf(x[i]), a);
                }
            acc[l] = a;
        }
        float ws = tree_sum(acc, 64);
        total = (w == 0) ? ws : total + ws;
    }
    return total;
}

void orc_rmsnorm(uint16_t *out, const uint16_t *in, const uint16_t *weight, int rows, int dim,
                 float eps, int mode) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const uint16_t *x = in + (size_t)r * dim;
        uint16_t *y = out + (size_t)r * dim;
        float var;
        if (mode == ORC_EXACT) {
            double s = 0.0;
            for (int i = 0; i < dim; i++) s += (double)bf(x[i]) * (double)bf(x[i]);
            var = (float)(s / dim);
        } else {
            var = sumsq_gpu(x, dim) / (float)dim;
        }
        float inv = 1.0f / sqrtf(var + eps);
        for (int i = 0; i < dim; i++) {
            float n = orc_round_bf16(bf(x[i]) * inv);
            y[i] = tobf(n * bf(weight[i]));
        }
    }
}

void orc_gemv(uint16_t *out, const uint16_t *w, const uint16_t *x, int rows, int cols, int mode) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) out[r] = dot_bf16(w + (size_t)r * cols, x, cols, mode);
}

void orc_gemv_residual(uint16_t *x, const uint16_t *w, const uint16_t *in, int rows, int cols,
                       uint16_t *tap, int mode) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        uint16_t y = dot_bf16(w + (size_t)r * cols, in, cols, mode);
        if (tap) tap[r] = y;
        x[r] = tobf(bf(x[r]) + bf(y));
    }
}

void orc_qkv(uint16_t *q, uint16_t *k, uint16_t *v, const uint16_t *wq, const uint16_t *wk,
             const uint16_t *wv, const uint16_t *x, int q_rows, int kv_rows, int cols, int mode) {
    orc_gemv(q, wq, x, q_rows, cols, mode);
    orc_gemv(k, wk, x, kv_rows, cols, mode);
    orc_gemv(v, wv, x, kv_rows, cols, mode);
}

static uint16_t swiglu1(uint16_t g, uint16_t u, int mode) {
    float s = orc_round_bf16(orc_silu(bf(g), mode));
    return tobf(s * bf(u));
}

void orc_gate_up(uint16_t *act, const uint16_t *w_gate, const uint16_t *w_up, const uint16_t *x,
                 int rows, int cols, uint16_t *gate_tap, uint16_t *up_tap, int mode) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        uint16_t g = dot_bf16(w_gate + (size_t)r * cols, x, cols, mode);
        uint16_t u = dot_bf16(w_up + (size_t)r * cols, x, cols, mode);
        if (gate_tap) {
            gate_tap[r] = g;
            up_tap[r] = u;
        }
        act[r] = swiglu1(g, u, mode);
    }
}

void orc_swiglu(uint16_t *act, const uint16_t *gate, const uint16_t *up, size_t n, int mode) {
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; i++) act[i] = swiglu1(gate[i], up[i], mode);
}

static int next_pow2(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

/* Sum of squares of one head as the kernel forms it: lanes_per_head = next_pow2(D/16) lanes;
 * lane L holds the chunks [8L, 8L+8) and [D/2+8L, D/2+8L+8) (lanes >= D/16 hold nothing),
 * fma-accumulated in that order, then the xor tree over the lanes. */
static float head_sumsq_gpu(const uint16_t *x, int D) {
    int used = D / 16;
    int lanes = next_pow2(used);
    float acc[64];
    for (int L = 0; L < lanes; L++) {
        float a = 0.0f;
        if (L < used) {
            for (int e = 0; e < 8; e++) a = fmaf(bf(x[8 * L + e]), bf(x[8 * L + e]), a);
            for (int e = 0; e < 8; e++)
                a = fmaf(bf(x[D / 2 + 8 * L + e]), bf(x[D / 2 + 8 * L + e]), a);
        }
        acc[L] = a;
    }
    return tree_sum(acc, lanes);
}

/* RMSNorm of one head then RoPE at `pos`, in place; the normed head goes to tap. */
static void norm_rope_head(uint16_t *x, const uint16_t *w, int D, float eps, int pos,
                           const float *cosv, const float *sinv, uint16_t *tap, int mode) {
    float var;
    if (mode == ORC_EXACT) {
        double s = 0.0;
        for (int i = 0; i < D; i++) s += (double)bf(x[i]) * (double)bf(x[i]);
        var = (float)(s / D);
    } else {
        var = head_sumsq_gpu(x, D) / (float)D;
    }
    float inv = 1.0f / sqrtf(var + eps);
    uint16_t y[1024];
    for (int i = 0; i < D; i++) {
        float n = orc_round_bf16(bf(x[i]) * inv);
        y[i] = tobf(n * bf(w[i]));
    }
    if (tap) memcpy(tap, y, (size_t)D * 2);
    int half = D / 2;
    (void)pos;
    for (int j = 0; j < half; j++) {
        float c = cosv[j], s = sinv[j];
        float a = bf(y[j]), b = bf(y[j + half]);
        float a_cos = orc_round_bf16(a * c);
        float b_sin = orc_round_bf16(b * s);
        float b_cos = orc_round_bf16(b * c);
        float a_sin = orc_round_bf16(a * s);
        x[j] = tobf(a_cos - b_sin);
        x[j + half] = tobf(b_cos + a_sin);
    }
}

/* bf16 cos/sin of the RoPE angles at one position: angle = fp32(pos * inv_freq_j), cos/sin
 * to fp32 then bf16 (HF computes emb.cos() in fp32 then casts to the model dtype). */
static void rope_table(int pos, float theta, int D, float *cosv, float *sinv, int mode) {
    for (int j = 0; j < D / 2; j++) {
        float angle = (float)pos * orc_inv_freq(theta, j, D);
        double s, c;
        if (mode == ORC_EXACT) {
            s = sin((double)angle);
            c = cos((double)angle);
        } else {
            orc_sincos_d((double)angle, &s, &c);
        }
        cosv[j] = orc_round_bf16((float)c);
        sinv[j] = orc_round_bf16((float)s);
    }
}

void orc_qk_norm_rope_rows(uint16_t *q, uint16_t *k, const uint16_t *v, const uint16_t *q_norm_w,
                           const uint16_t *k_norm_w, uint16_t *key_cache, uint16_t *value_cache,
                           const int *positions, int n_tokens, int n_heads, int n_kv_heads,
                           int head_dim, float eps, float theta, uint16_t *q_tap, uint16_t *k_tap,
                           int mode) {
    int D = head_dim;
    int q_dim = n_heads * D, kv_dim = n_kv_heads * D;
#pragma omp parallel for schedule(static)
    for (int t = 0; t < n_tokens; t++) {
        int pos = positions[t];
        float cosv[512], sinv[512];
        rope_table(pos, theta, D, cosv, sinv, mode);
        for (int h = 0; h < n_heads; h++) {
            uint16_t *x = q + (size_t)t * q_dim + (size_t)h * D;
            uint16_t *tap = q_tap ? q_tap + (size_t)t * q_dim + (size_t)h * D : NULL;
            norm_rope_head(x, q_norm_w, D, eps, pos, cosv, sinv, tap, mode);
        }
        for (int h = 0; h < n_kv_heads; h++) {
            uint16_t *x = k + (size_t)t * kv_dim + (size_t)h * D;
            uint16_t *tap = k_tap ? k_tap + (size_t)t * kv_dim + (size_t)h * D : NULL;
            norm_rope_head(x, k_norm_w, D, eps, pos, cosv, sinv, tap, mode);
            size_t slot = (size_t)pos * kv_dim + (size_t)h * D;
            memcpy(key_cache + slot, x, (size_t)D * 2);
            memcpy(value_cache + slot, v + (size_t)t * kv_dim + (size_t)h * D, (size_t)D * 2);
        }
    }
}

/* q.k over one head in the kernel's order: D/8 lanes, lane L fma-accumulates elements
 * [8L, 8L+8), then the xor tree over the D/8 lanes. */
static float qk_dot_gpu(const uint16_t *q, const uint16_t *k, int D) {
    float acc[64];
    int lanes = D / 8;
    for (int L = 0; L < lanes; L++) acc[L] = 0.0f;
    /* each lane's chain over its 8 elements in order, the lanes side by side */
    for (int e = 0; e < 8; e++)
        for (int L = 0; L < lanes; L++) acc[L] = fmaf(bf(q[8 * L + e]), bf(k[8 * L + e]), acc[L]);
    return tree_sum(acc, lanes);
}

static void attention_head_exact(uint16_t *out, const uint16_t *qh, const uint16_t *key_cache,
                                 const uint16_t *value_cache, int kv_dim, int kv_off, int D,
                                 int n, float scale, float *sc) {
    float m = -INFINITY;
    for (int t = 0; t < n; t++) {
        const uint16_t *kt = key_cache + (size_t)t * kv_dim + kv_off;
        float d = bf(dot_bf16(qh, kt, D, ORC_EXACT));
        sc[t] = orc_round_bf16(d * scale);
        if (sc[t] > m) m = sc[t];
    }
    double sum = 0.0;
    for (int t = 0; t < n; t++) sum += exp((double)sc[t] - (double)m);
    float sumf = (float)sum;
    for (int t = 0; t < n; t++) sc[t] = orc_round_bf16(orc_exp_ref(sc[t] - m) / sumf);
    for (int d = 0; d < D; d++) {
        double acc = 0.0;
        for (int t = 0; t < n; t++)
            acc += (double)sc[t] * (double)bf(value_cache[(size_t)t * kv_dim + kv_off + d]);
        out[d] = tobf((float)acc);
    }
}

/*
 * The split-softmax kernels' order, blocks of B = ORC_ATTN_BLOCK positions:
 *   scores   s_t = bf16(bf16(q.k_t) * scale), q.k in qk_dot_gpu order
 *   block    m_b = max s_t;  S_b = tree64 over slots i of exp(s_{bB+i} - m_b) (0 past n)
 *   global   M = max m_b;  sum = sequential over chunks of 64 blocks of
 *            tree64 over slots i of S_b * exp(m_b - M) (0 past the last block)
 *   probs    p_t = bf16(exp(s_t - M) / sum)
 *   PV       4 waves; wave w, group G (of 64/(D/8) position groups), iteration it handles
 *            slot w*(B/4) + it*groups + G; each lane fma-accumulates p*v over its iterations,
 *            the groups meet in an xor tree, the waves are added in order 0..3
 *   combine  out = bf16(sequential sum over blocks of the block partials)
 */
static void attention_head_gpu(uint16_t *out, const uint16_t *qh, const uint16_t *key_cache,
                               const uint16_t *value_cache, int kv_dim, int kv_off, int D, int n,
                               float scale, float *sc, float *stats, float *partial) {
    const int B = ORC_ATTN_BLOCK;
    int nb = (n + B - 1) / B;
    for (int t = 0; t < n; t++) {
        const uint16_t *kt = key_cache + (size_t)t * kv_dim + kv_off;
        float d = orc_round_bf16(qk_dot_gpu(qh, kt, D));
        sc[t] = orc_round_bf16(d * scale);
    }
    for (int b = 0; b < nb; b++) {
        float m = -INFINITY;
        for (int i = 0; i < B && b * B + i < n; i++)
            if (sc[b * B + i] > m) m = sc[b * B + i];
        float e[64];
        for (int i = 0; i < 64; i++) e[i] = (b * B + i < n) ? orc_exp_f32(sc[b * B + i] - m) : 0.0f;
        stats[2 * b] = m;
        stats[2 * b + 1] = tree_sum(e, 64);
    }
    float M = -INFINITY;
    for (int b = 0; b < nb; b++)
        if (stats[2 * b] > M) M = stats[2 * b];
    float sum = 0.0f;
    for (int c0 = 0; c0 < nb; c0 += 64) {
        float e[64];
        for (int i = 0; i < 64; i++) {
            int b = c0 + i;
            e[i] = (b < nb) ? stats[2 * b + 1] * orc_exp_f32(stats[2 * b] - M) : 0.0f;
        }
        float cs = tree_sum(e, 64);
        sum = (c0 == 0) ? cs : sum + cs;
    }
    for (int t = 0; t < n; t++) sc[t] = orc_round_bf16(orc_exp_f32(sc[t] - M) / sum);
    int lanes = D / 8;
    int groups = 64 / lanes;
    int per_wave = B / 4;
    int iters = per_wave / groups;
    /* per block: wave w, position group G accumulates its positions (it = 0, 1, ...) in order
     * for every output element d (the loop over d innermost: the same operations per element,
     * a value row read once); then per d the groups' tree and the waves added in order */
    float *acc = (float *)malloc((size_t)4 * groups * D * sizeof(float));
    for (int b = 0; b < nb; b++) {
        for (int w = 0; w < 4; w++)
            for (int G = 0; G < groups; G++) {
                float *a = acc + ((size_t)w * groups + G) * D;
                for (int d = 0; d < D; d++) a[d] = 0.0f;
                for (int it = 0; it < iters; it++) {
                    int t = b * B + w * per_wave + it * groups + G;
                    if (t >= n) continue;
                    const uint16_t *vt = value_cache + (size_t)t * kv_dim + kv_off;
                    for (int d = 0; d < D; d++) a[d] = fmaf(sc[t], bf(vt[d]), a[d]);
                }
            }
        for (int d = 0; d < D; d++) {
            float wave_sum[4];
            for (int w = 0; w < 4; w++) {
                float g[64];
                for (int G = 0; G < groups; G++) g[G] = acc[((size_t)w * groups + G) * D + d];
                wave_sum[w] = tree_sum(g, groups);
            }
            partial[(size_t)b * D + d] = ((wave_sum[0] + wave_sum[1]) + wave_sum[2]) + wave_sum[3];
        }
    }
    free(acc);
    for (int d = 0; d < D; d++) {
        float a = partial[d];
        for (int b = 1; b < nb; b++) a = a + partial[(size_t)b * D + d];
        out[d] = tobf(a);
    }
}

void orc_attention(uint16_t *out, const uint16_t *q, const uint16_t *key_cache,
                   const uint16_t *value_cache, int n_heads, int n_kv_heads, int head_dim, int pos,
                   float scale, int mode) {
    int D = head_dim;
    int kv_dim = n_kv_heads * D;
    int rep = n_heads / n_kv_heads;
    int n = pos + 1;
    int nb = (n + ORC_ATTN_BLOCK - 1) / ORC_ATTN_BLOCK;
#pragma omp parallel for schedule(static)
    for (int h = 0; h < n_heads; h++) {
        float *sc = (float *)malloc((size_t)n * sizeof(float));
        float *stats = (float *)malloc((size_t)nb * 2 * sizeof(float));
        float *partial = (float *)malloc((size_t)nb * D * sizeof(float));
        int kv_off = (h / rep) * D;
        if (mode == ORC_EXACT)
            attention_head_exact(out + (size_t)h * D, q + (size_t)h * D, key_cache, value_cache,
                                 kv_dim, kv_off, D, n, scale, sc);
        else
            attention_head_gpu(out + (size_t)h * D, q + (size_t)h * D, key_cache, value_cache,
                               kv_dim, kv_off, D, n, scale, sc, stats, partial);
        free(sc);
        free(stats);
        free(partial);
    }
}

/* Larger value wins, ties keep the lowest index; starting from (-inf, INT_MAX) no NaN is ever
 * taken (src/kernels.cu:499-505, :509-510). */
int orc_argmax(const uint16_t *x, int n) {
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = 0; i < n; i++) {
        float v = bf(x[i]);
        if (v > best || (v == best && i < idx)) {
            best = v;
            idx = i;
        }
    }
    return idx;
}

/* Inverse-CDF sampling from softmax(x * inv_temp) (src/kernels.cu:546-597): the row's max; the
 * row cut into 1024 contiguous chunks of ceil(n / 1024) elements, each chunk's weights
 * exp_f32((x - max) * inv_temp) added in order; the total as the chunk sums added in order;
 * target = u * total; the first chunk whose running sum would pass the target (never past the
 * last), then the first element of it whose running sum passes. -1 if none does. */
int orc_sample(const uint16_t *x, int n, float inv_temp, float u) {
    enum { T = 1024 };
    float mx = -INFINITY;
    for (int i = 0; i < n; i++) mx = fmaxf(mx, bf(x[i]));
    const int chunk = (n + T - 1) / T;
    float sums[T];
    for (int t = 0; t < T; t++) {
        const int start = t * chunk, end = start + chunk < n ? start + chunk : n;
        float acc = 0.0f;
        for (int i = start; i < end; i++) acc += orc_exp_f32((bf(x[i]) - mx) * inv_temp);
        sums[t] = acc;
    }
    float total = 0.0f;
    for (int t = 0; t < T; t++) total += sums[t];
    const float target = u * total;
    float cdf = 0.0f;
    int t = 0;
    while (t < T - 1 && cdf + sums[t] <= target) cdf += sums[t++];
    const int start = t * chunk, end = start + chunk < n ? start + chunk : n;
    float acc = 0.0f;
    for (int i = start; i < end; i++) {
        acc += orc_exp_f32((bf(x[i]) - mx) * inv_temp);
        if (cdf + acc > target) return i;
    }
    return -1;
}

/* ------------------------------------------------------------------------------------------ */
/* decode step                                                                                 */
/* ------------------------------------------------------------------------------------------ */

int orc_forward(const OrcConfig *cfg, const OrcWeights *w, OrcState *s, int token, int pos,
                int mode) {
    int H = cfg->hidden_size, D = cfg->head_dim;
    int q_dim = cfg->n_heads * D, kv_dim = cfg->n_kv_heads * D, I = cfg->intermediate_size;
    float scale = (float)(1.0 / sqrt((double)D));
    orc_embedding(s->x, w->embed, token, H);
    for (int l = 0; l < cfg->n_layers; l++) {
        const OrcLayer *L = &w->layers[l];
        uint16_t *kc = s->key_cache + (size_t)l * s->max_seq * kv_dim;
        uint16_t *vc = s->value_cache + (size_t)l * s->max_seq * kv_dim;
        orc_rmsnorm(s->xb, s->x, L->attn_norm, 1, H, cfg->rms_norm_eps, mode);
        orc_qkv(s->q, s->k, s->v, L->wq, L->wk, L->wv, s->xb, q_dim, kv_dim, H, mode);
        orc_qk_norm_rope_rows(s->q, s->k, s->v, L->q_norm, L->k_norm, kc, vc, &pos, 1,
                              cfg->n_heads, cfg->n_kv_heads, D, cfg->rms_norm_eps,
                              cfg->rope_theta, NULL, NULL, mode);
        orc_attention(s->attn_out, s->q, kc, vc, cfg->n_heads, cfg->n_kv_heads, D, pos, scale,
                      mode);
        orc_gemv_residual(s->x, L->wo, s->attn_out, H, q_dim, NULL, mode);
        orc_rmsnorm(s->xb, s->x, L->mlp_norm, 1, H, cfg->rms_norm_eps, mode);
        orc_gate_up(s->hb, L->w_gate, L->w_up, s->xb, I, H, NULL, NULL, mode);
        orc_gemv_residual(s->x, L->w_down, s->hb, H, I, NULL, mode);
    }
    orc_rmsnorm(s->xb, s->x, w->final_norm, 1, H, cfg->rms_norm_eps, mode);
    orc_gemv(s->logits, w->lm_head, s->xb, cfg->vocab_size, H, mode);
    return orc_argmax(s->logits, cfg->vocab_size);
}

size_t orc_weight_bytes_per_step(const OrcConfig *c) {
    size_t H = c->hidden_size, D = c->head_dim, qd = (size_t)c->n_heads * D;
    size_t kvd = (size_t)c->n_kv_heads * D, I = c->intermediate_size;
    size_t layer = H + qd * H + 2 * kvd * H + 2 * D + H * qd + H + 2 * I * H + H * I;
    return (layer * c->n_layers + H + (size_t)c->vocab_size * H + H) * 2;
}

size_t orc_kv_bytes_per_position(const OrcConfig *c) {
    return 2 * (size_t)c->n_layers * c->n_kv_heads * c->head_dim * 2;
}

/* ------------------------------------------------------------------------------------------ */
/* self-checks that pin the transcendental algorithms against libm                            */
/* ------------------------------------------------------------------------------------------ */

static int64_t ulp_diff(float a, float b) {
    int32_t ia, ib;
    memcpy(&ia, &a, 4);
    memcpy(&ib, &b, 4);
    if (ia < 0) ia = (int32_t)0x80000000 - ia;
    if (ib < 0) ib = (int32_t)0x80000000 - ib;
    int64_t d = (int64_t)ia - (int64_t)ib;
    return d < 0 ? -d : d;
}

/* Every fp32 x in [lo, hi]: orc_exp_f32(x) against (float)exp((double)x). Returns the largest
 * ulp distance; *n_checked and *n_diff count inputs and inputs whose results differ. */
int64_t orc_selfcheck_exp(float lo, float hi, int64_t *n_checked, int64_t *n_diff) {
    int64_t worst = 0, checked = 0, diff = 0;
    uint32_t ulo, uhi;
    /* walk the positive and negative halves separately by bit pattern */
    for (int sign = 0; sign < 2; sign++) {
        float a = sign ? 0.0f : 0.0f, b = sign ? -lo : hi;
        if (b <= 0.0f) continue;
        memcpy(&ulo, &a, 4);
        memcpy(&uhi, &b, 4);
#pragma omp parallel for reduction(max : worst) reduction(+ : checked, diff) schedule(static)
        for (int64_t u = ulo; u <= (int64_t)uhi; u++) {
            uint32_t bits = (uint32_t)u | (sign ? 0x80000000u : 0u);
            float x;
            memcpy(&x, &bits, 4);
            float g = orc_exp_f32(x), r = orc_exp_ref(x);
            int64_t d = ulp_diff(g, r);
            if (d > worst) worst = d;
            checked++;
            if (d) diff++;
        }
    }
    *n_checked = checked;
    *n_diff = diff;
    return worst;
}

/* RoPE angles fp32(pos * inv_freq_j) for pos < n_pos, j < D/2: orc_sincos_d rounded to fp32
 * against libm sin/cos rounded to fp32. Returns the number of differing fp32 results. */
int64_t orc_selfcheck_sincos(float theta, int head_dim, int n_pos, int64_t *n_checked) {
    int64_t diff = 0;
#pragma omp parallel for reduction(+ : diff) schedule(static)
    for (int pos = 0; pos < n_pos; pos++) {
        for (int j = 0; j < head_dim / 2; j++) {
            float angle = (float)pos * orc_inv_freq(theta, j, head_dim);
            double s, c;
            orc_sincos_d((double)angle, &s, &c);
            if ((float)s != (float)sin((double)angle)) diff++;
            if ((float)c != (float)cos((double)angle)) diff++;
        }
    }
    *n_checked = 2 * (int64_t)n_pos * (head_dim / 2);
    return diff;
}

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
