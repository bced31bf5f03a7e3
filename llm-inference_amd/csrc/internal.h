// Functions shared between the kernel and step translation units (not part of the C ABI).
#pragma once

#include "llm_amd/kernels.h"

// embedding_forward that checks the token against the vocabulary on the device: a token
// outside [0, vocab) sets *err and leaves `out` unchanged.
void embedding_checked(bf16 *out, const bf16 *table, const int *d_token, int hidden, int vocab,
                       int *err, hipStream_t stream);

// Two-stage argmax into *out using caller-owned partials of argmax_partial_count() entries.
void argmax_launch(int *out, const bf16 *x, int n, float *pv, int *pi, hipStream_t stream);
int argmax_partial_count();

// inv_freq_j = 1 / fp32(pow(theta, fp32(2j / D))) for j < D/2 (D <= 256), cached per (theta, D).
void rope_inv_freq_table(float theta, int D, float *out);

// qk_norm_rope_attention_one_pass, reporting whether it launched.
bool attention_one_pass_launch(bf16 *out, const bf16 *q, const bf16 *k, const bf16 *v,
                               const bf16 *q_norm_w, const bf16 *k_norm_w, bf16 *key_cache,
                               bf16 *value_cache, void *ws, int *err, const int *d_pos,
                               int n_heads, int n_kv_heads, int head_dim, float eps, float theta,
                               int max_seq, float scale, hipStream_t stream);

// Bytes of the workspace of the one-launch PV and combine (attn_pv_combine_kernel: launch
// counters and tagged partials), or 0 for shapes it does not take (head_dim other than 128, more
// than 8192 blocks x kv heads). Zeroed once at allocation; its launch counters then keep it valid
// from call to call (nothing needs clearing between calls or after a timeout).
size_t attention_pv_combine_bytes(int n_heads, int n_kv_heads, int head_dim, int max_seq);

// attention_forward, reporting whether it launched; with pvc (a workspace of
// attention_pv_combine_bytes() bytes, used by one RunState only) and err (the device error flag,
// set to 2 if a wait times out), the PV and combine passes run as one launch (the same bits).
bool attention_launch(bf16 *out, const bf16 *q, const bf16 *key_cache, const bf16 *value_cache,
                      float *att, int n_heads, int n_kv_heads, int head_dim, const int *d_pos,
                      int max_seq, float scale, hipStream_t stream, void *pvc = nullptr,
                      int *err = nullptr);

// qk_norm_rope_attention_forward, reporting whether it launched; with rope_table (the
// rope_table_launch output at *d_pos), the kernel reads the RoPE table instead of computing it;
// pvc and err as for attention_launch.
bool qk_norm_rope_attention_launch(bf16 *out, const bf16 *q, const bf16 *k, const bf16 *v,
                                   const bf16 *q_norm_w, const bf16 *k_norm_w, bf16 *key_cache,
                                   bf16 *value_cache, float *att, const int *d_pos, int n_heads,
                                   int n_kv_heads, int head_dim, float eps, float theta,
                                   int max_seq, float scale, hipStream_t stream,
                                   const float *rope_table = nullptr, void *pvc = nullptr,
                                   int *err = nullptr);

// The RoPE table at *d_pos into table[0, head_dim): cos then sin of the head_dim / 2 rotation
// pairs, the values rope_table computes in the kernels (one launch serves every layer).
bool rope_table_launch(float *table, const int *d_pos, int head_dim, float theta,
                       hipStream_t stream);
