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
