/*
 * Activation dumps of the decode step (replacing src/dump.cuh:5-9 of
 * William-Lamer/llm-inference). While a dump directory is open, the eager step (`forward` with
 * no captured graph or persistent step) writes every intermediate tensor of every position as
 * fp32 rows to <dir>/<name>.bin, in the tensor taxonomy of the reference's HF dumps: "embed",
 * "Lnn.attn_norm", "Lnn.q_proj", "Lnn.k_proj", "Lnn.v_proj", "Lnn.q_norm", "Lnn.k_norm",
 * "Lnn.q_rope", "Lnn.k_rope", "Lnn.attn_out", "Lnn.o_proj", "Lnn.attn_resid", "Lnn.mlp_norm",
 * "Lnn.gate", "Lnn.up", "Lnn.mlp_act", "Lnn.down", "Lnn.out", "final_norm", "logits". The first
 * write of a name after dump_open truncates its file, later writes append a row.
 */
#ifndef LLM_AMD_DUMP_H
#define LLM_AMD_DUMP_H

#include "llm_amd/kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

/* src/dump.cuh:5. Creates the directory if needed; errors as the launchers'. */
void dump_open(const char *dir);
/* src/dump.cuh:6 */
void dump_close(void);
/* src/dump.cuh:7. 1 while a directory is open. */
int dump_enabled(void);
/* src/dump.cuh:8-9. Appends one row: n bf16 (or fp32) device values as fp32, after waiting for
 * all work on the device (the row is the finished tensor). No-op while no directory is open. */
void dump_bf16(const char *name, const bf16 *d_data, int n);
void dump_f32(const char *name, const float *d_data, int n);

#ifdef __cplusplus
}
#endif
#endif
