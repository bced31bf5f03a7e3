/*
 * CPU oracle for the fused Qwen3 decode-layer path. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the results the GPU path is compared with (or the timed CPU baseline). The product path
 * (llm-inference_amd/) never links, loads or calls it.
 *
 * It restates, in plain C on the CPU, the arithmetic of William-Lamer/llm-inference's
 * decode kernels (src/kernels.cu) at their bf16 rounding points, which follow the
 * Hugging Face Qwen3 modules (transformers models/qwen3/modeling_qwen3.py). Each op has
 * two modes:
 *
 *   ORC_GPU_ORDER  fp32 arithmetic in exactly the summation order of the HIP kernels
 *                  (lane decomposition and reduction trees written out below), with the
 *                  same transcendental algorithms, so HIP results must be bit-identical.
 *   ORC_EXACT      reductions accumulated in double and rounded once, transcendentals from
 *                  libm in double rounded once to fp32: the ideal result the HF fp32 path
 *                  approximates. Used for the 1-bf16-ulp tolerance tests.
 *
 * bf16 values are passed as their raw uint16_t bits.
 *
 * Parity pinning (which check fixes each function) is listed in the header of oracle.c.
 */
#ifndef LLM_AMD_ORACLE_H
#define LLM_AMD_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_GPU_ORDER = 0, ORC_EXACT = 1 };

/* Attention split: positions per block in the GPU's split-softmax kernels. */
#define ORC_ATTN_BLOCK 64

/* ---- numerics ---- */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t b);
float orc_round_bf16(float f);
float orc_exp_f32(float x);     /* the kernels' fp32 exp (Cody-Waite + Taylor, fma) */
float orc_exp_ref(float x);     /* (float)exp((double)x) from libm */
void orc_sincos_d(double x, double *s, double *c); /* the kernels' double sincos */
float orc_inv_freq(float theta, int j, int head_dim); /* 1/(float)pow(theta, (2j)/D) */
float orc_silu(float g, int mode);                    /* fp32 g/(1+exp(-g)) */

/* ---- ops (src/kernels.cuh:7-26 counterparts) ---- */
void orc_embedding(uint16_t *out, const uint16_t *table, int token, int hidden);
void orc_rmsnorm(uint16_t *out, const uint16_t *in, const uint16_t *weight, int rows, int dim,
                 float eps, int mode);
float orc_dot(const uint16_t *w_row, const uint16_t *x, int cols, int mode);
void orc_gemv(uint16_t *out, const uint16_t *w, const uint16_t *x, int rows, int cols, int mode);
void orc_gemv_residual(uint16_t *x, const uint16_t *w, const uint16_t *in, int rows, int cols,
                       uint16_t *tap, int mode);
void orc_qkv(uint16_t *q, uint16_t *k, uint16_t *v, const uint16_t *wq, const uint16_t *wk,
             const uint16_t *wv, const uint16_t *x, int q_rows, int kv_rows, int cols, int mode);
void orc_gate_up(uint16_t *act, const uint16_t *w_gate, const uint16_t *w_up, const uint16_t *x,
                 int rows, int cols, uint16_t *gate_tap, uint16_t *up_tap, int mode);
void orc_swiglu(uint16_t *act, const uint16_t *gate, const uint16_t *up, size_t n, int mode);
/* q [n_tokens, n_heads*D], k and v [n_tokens, n_kv_heads*D]; caches [*, n_kv_heads*D] */
void orc_qk_norm_rope_rows(uint16_t *q, uint16_t *k, const uint16_t *v, const uint16_t *q_norm_w,
                           const uint16_t *k_norm_w, uint16_t *key_cache, uint16_t *value_cache,
                           const int *positions, int n_tokens, int n_heads, int n_kv_heads,
                           int head_dim, float eps, float theta, uint16_t *q_tap, uint16_t *k_tap,
                           int mode);
/* one decode position `pos`; caches hold positions 0..pos */
void orc_attention(uint16_t *out, const uint16_t *q, const uint16_t *key_cache,
                   const uint16_t *value_cache, int n_heads, int n_kv_heads, int head_dim, int pos,
                   float scale, int mode);
int orc_argmax(const uint16_t *x, int n);
int orc_sample(const uint16_t *x, int n, float inv_temp, float u);

/* ---- whole decode step (src/forward.cu:118-193, :229-236) ---- */
typedef struct {
    int hidden_size, intermediate_size, n_layers, n_heads, n_kv_heads, head_dim, vocab_size;
    float rms_norm_eps, rope_theta;
} OrcConfig;

typedef struct {
    const uint16_t *attn_norm, *wq, *wk, *wv, *q_norm, *k_norm, *wo, *mlp_norm, *w_gate, *w_up,
        *w_down;
} OrcLayer;

typedef struct {
    const uint16_t *embed, *final_norm, *lm_head;
    const OrcLayer *layers;
} OrcWeights;

typedef struct {
    uint16_t *x, *xb, *q, *k, *v, *attn_out, *hb, *logits;
    uint16_t *key_cache, *value_cache; /* [n_layers, max_seq, kv_dim] */
    int max_seq;
} OrcState;

/* Runs one position and returns the greedy token (argmax of the logits). */
int orc_forward(const OrcConfig *cfg, const OrcWeights *w, OrcState *s, int token, int pos,
                int mode);
size_t orc_weight_bytes_per_step(const OrcConfig *cfg);
size_t orc_kv_bytes_per_position(const OrcConfig *cfg);
int orc_num_threads(void);

/* ---- self-checks pinning the transcendental algorithms against libm ---- */
int64_t orc_selfcheck_exp(float lo, float hi, int64_t *n_checked, int64_t *n_diff);
int64_t orc_selfcheck_sincos(float theta, int head_dim, int n_pos, int64_t *n_checked);

#ifdef __cplusplus
}
#endif
#endif
