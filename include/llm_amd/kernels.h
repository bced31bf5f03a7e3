/*
 * Decode-kernel launchers of the MI355X (gfx950) build. C ABI: plain device pointers, sizes and
 * a hipStream_t; bf16 tensors are raw 16-bit patterns (uint16_t). Every pointer is caller-owned
 * device memory and no launcher allocates. Launchers check shapes on the host; on a violation
 * they print to stderr and exit(EXIT_FAILURE) like the reference, unless the error mode was
 * switched with llm_set_exit_on_error(0), in which case they return without launching and
 * llm_last_error() holds the message.
 *
 * Each entry point replaces the reference launcher of the same name in
 * William-Lamer/llm-inference src/kernels.cuh (line numbers cited per function), with the same
 * argument order and meaning.
 */
#ifndef LLM_AMD_KERNELS_H
#define LLM_AMD_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t bf16;

/* src/kernels.cuh:7-8. out[i] = table[*d_token * hidden + i]; the token is read on the device. */
void embedding_forward(bf16 *out, const bf16 *table, const int *d_token, int hidden,
                       hipStream_t stream);

/* src/kernels.cuh:9-10. Per row: y = bf16(bf16(x * 1/sqrt(mean(x^2) + eps)) * weight). */
void rmsnorm_forward(bf16 *out, const bf16 *in, const bf16 *weight, int rows, int dim, float eps,
                     hipStream_t stream);

/* src/kernels.cuh:11. out[r] = bf16(sum_c w[r, c] * x[c]), fp32 accumulation; cols % 8 == 0. */
void gemv_forward(bf16 *out, const bf16 *w, const bf16 *x, int rows, int cols,
                  hipStream_t stream);

/* src/kernels.cuh:12-13. y = bf16(w[r] . in); tap[r] = y if tap != NULL; x[r] = bf16(x[r] + y).
 * `in` must not alias `x`. cols % 8 == 0. */
void gemv_residual_forward(bf16 *x, const bf16 *w, const bf16 *in, int rows, int cols, bf16 *tap,
                           hipStream_t stream);

/* src/kernels.cuh:14-15. q = wq.x, k = wk.x, v = wv.x in one launch. cols % 8 == 0. */
void qkv_forward(bf16 *q, bf16 *k, bf16 *v, const bf16 *wq, const bf16 *wk, const bf16 *wv,
                 const bf16 *x, int q_rows, int kv_rows, int cols, hipStream_t stream);

/* src/kernels.cuh:16-17. g = bf16(w_gate[r].x), u = bf16(w_up[r].x) (taps when non-NULL),
 * act[r] = bf16(bf16(g / (1 + exp(-g))) * u). cols % 8 == 0. */
void gate_up_forward(bf16 *act, const bf16 *w_gate, const bf16 *w_up, const bf16 *x, int rows,
                     int cols, bf16 *gate_tap, bf16 *up_tap, hipStream_t stream);

/* src/kernels.cuh:18-21. Per head: RMSNorm over head_dim with q_norm_w/k_norm_w (normed heads to
 * q_tap/k_tap when non-NULL), then RoPE at position *d_pos with inv_freq_j = 1/theta^(2j/D), in
 * place on q [n_heads*D] and k [n_kv_heads*D]; k' and v are written to key_cache/value_cache
 * (one layer's caches, [max_seq, n_kv_heads*D]) at row *d_pos. head_dim in {64, 128, 256}. */
void qk_norm_rope_forward(bf16 *q, bf16 *k, const bf16 *v, const bf16 *q_norm_w,
                          const bf16 *k_norm_w, bf16 *key_cache, bf16 *value_cache,
                          const int *d_pos, int n_heads, int n_kv_heads, int head_dim, float eps,
                          float theta, bf16 *q_tap, bf16 *k_tap, hipStream_t stream);

/* src/kernels.cuh:22-24. Decode attention of the query at position *d_pos over cache rows
 * 0..*d_pos, GQA kv_head = h / (n_heads / n_kv_heads). scores bf16(bf16(q.k) * scale), softmax
 * probabilities rounded to bf16, out = bf16(sum p v). `att` is 16-byte aligned fp32 scratch
 * holding either the reference's [n_heads, max_seq] score rows (src/forward.cuh:13) or
 * attention_workspace_floats(n_heads, head_dim, max_seq) floats: the score rows followed by the
 * split softmax's block statistics and partial outputs. With the reference's size, those live
 * in a library-owned device array of 2^22 floats per device (n_heads * ceil(max_seq / 64) *
 * (head_dim + 2) floats must fit; larger sizes are an error), and calls on one device that use
 * it must not overlap. A smaller `att` is an error. The size is what the runtime reports for the
 * allocation holding `att`, counted from `att` to its end. head_dim in {64, 128, 256};
 * n_heads / n_kv_heads in {1, 2, 4, 8}. */
void attention_forward(bf16 *out, const bf16 *q, const bf16 *key_cache, const bf16 *value_cache,
                       float *att, int n_heads, int n_kv_heads, int head_dim, const int *d_pos,
                       int max_seq, float scale, hipStream_t stream);

/* src/kernels.cuh:25. *out = index of the largest x; ties keep the lowest index; NaN is never
 * taken (all-NaN input gives INT_MAX). Calls on one device must not overlap: the partial
 * results live in one library-owned device buffer. */
void argmax_forward(int *out, const bf16 *x, int n, hipStream_t stream);

/* src/kernels.cuh:26. *out = a token drawn from softmax(x * inv_temp) by inverse CDF at the
 * coin u in [0, 1): the row's max, 1024 contiguous chunks whose weights exp((x - max) * inv_temp)
 * are added in order, the chunk sums added in order, then the first chunk and element whose
 * running sum passes u * total (-1 if none). */
void sample_forward(int *out, const bf16 *x, int n, float inv_temp, float u, hipStream_t stream);

/* ---- entry points with no counterpart in kernels.cuh (needed by the multi-row workloads) ---- */

/* qk_norm_rope_forward over n_tokens rows: q [n_tokens, n_heads*D], k and v
 * [n_tokens, n_kv_heads*D]; token t uses position d_positions[t] for RoPE and its cache row.
 * Taps, when non-NULL, have the shapes of q and k. */
void qk_norm_rope_rows(bf16 *q, bf16 *k, const bf16 *v, const bf16 *q_norm_w,
                       const bf16 *k_norm_w, bf16 *key_cache, bf16 *value_cache,
                       const int *d_positions, int n_tokens, int n_heads, int n_kv_heads,
                       int head_dim, float eps, float theta, bf16 *q_tap, bf16 *k_tap,
                       hipStream_t stream);

/* act[i] = bf16(bf16(g / (1 + exp(-g))) * up[i]) with g = gate[i], the elementwise tail of
 * gate_up_forward (src/kernels.cu:283-286). */
void swiglu_forward(bf16 *act, const bf16 *gate, const bf16 *up, size_t n, hipStream_t stream);

/* RMSNorm of the single row x (as rmsnorm_forward, eps, weight norm_w) fused into the prologue
 * of the GEMV that reads it: bit-identical to rmsnorm_forward into a temporary followed by
 * qkv_forward / gemv_forward / gate_up_forward on it, without the temporary's store and reload
 * or the extra launch. No counterpart in the reference: each replaces one rmsnorm_forward
 * (src/kernels.cu:25-71) plus the launcher that consumes its output (qkv: src/kernels.cu:215-257,
 * gemv: :79-212, gate_up: :260-298) in a decode step. cols % 8 == 0 and cols <= 8192 (the
 * normed row stays in registers). */
void rmsnorm_qkv_forward(bf16 *q, bf16 *k, bf16 *v, const bf16 *wq, const bf16 *wk,
                         const bf16 *wv, const bf16 *x, const bf16 *norm_w, float eps, int q_rows,
                         int kv_rows, int cols, hipStream_t stream);
void rmsnorm_gemv_forward(bf16 *out, const bf16 *w, const bf16 *x, const bf16 *norm_w, float eps,
                          int rows, int cols, hipStream_t stream);
void rmsnorm_gate_up_forward(bf16 *act, const bf16 *w_gate, const bf16 *w_up, const bf16 *x,
                             const bf16 *norm_w, float eps, int rows, int cols,
                             hipStream_t stream);

/* No counterpart in the reference: qk_norm_rope_forward followed by attention_forward
 * (src/kernels.cuh:18-24) for one decode position, with the same bits, in three launches
 * instead of four: the per-head QK-norm + RoPE is computed inside the attention's scores pass,
 * per block of positions, while the block's keys stream. q and k are read, not rewritten; k'
 * and v are written to the caches' row *d_pos as qk_norm_rope_forward writes them. `att`, the
 * shapes and alignment are attention_forward's. */
void qk_norm_rope_attention_forward(bf16 *out, const bf16 *q, const bf16 *k, const bf16 *v,
                                    const bf16 *q_norm_w, const bf16 *k_norm_w, bf16 *key_cache,
                                    bf16 *value_cache, float *att, const int *d_pos, int n_heads,
                                    int n_kv_heads, int head_dim, float eps, float theta,
                                    int max_seq, float scale, hipStream_t stream);

/* No counterpart in the reference: qk_norm_rope_forward followed by attention_forward
 * (src/kernels.cuh:18-24) for one decode position, with the same bits, in ONE launch: a
 * workgroup per (kv head, 1/ipk of the 64-position blocks), ipk = CUs / n_kv_heads (at most
 * 64), that hand the split softmax's block statistics and partial outputs to each other as
 * tagged words in `ws` instead of through kernel boundaries. The workgroups wait for each
 * other: the grid never exceeds the CU count, no other work may occupy the device's CUs
 * meanwhile, and every wait is bounded (on timeout *err = 2 and the output is not valid).
 * ws: attention_one_pass_bytes(n_heads, head_dim, max_seq) bytes, 256-byte aligned, zeroed
 * once before the first call and then left to these calls (it holds their launch counter);
 * calls sharing a ws must not overlap. q, k and v are read, k' and v are written to the
 * caches' row *d_pos. Supported shapes: attention_one_pass_supported(). */
void qk_norm_rope_attention_one_pass(bf16 *out, const bf16 *q, const bf16 *k, const bf16 *v,
                                     const bf16 *q_norm_w, const bf16 *k_norm_w,
                                     bf16 *key_cache, bf16 *value_cache, void *ws, int *err,
                                     const int *d_pos, int n_heads, int n_kv_heads,
                                     int head_dim, float eps, float theta, int max_seq,
                                     float scale, hipStream_t stream);
/* Bytes of the one-pass attention's workspace for these sizes. */
size_t attention_one_pass_bytes(int n_heads, int head_dim, int max_seq);
/* 1 if qk_norm_rope_attention_one_pass supports these sizes on the current device (head_dim
 * 128, n_heads / n_kv_heads in {1, 2, 4, 8}, at most 32768 positions), else 0. */
int attention_one_pass_supported(int n_heads, int n_kv_heads, int head_dim, int max_seq);

/* Measurement helper, no counterpart in the reference: the streaming ceiling that the
 * bandwidth-bound kernels are compared with. mode 0: read n_bytes of a (dst receives one 32-bit
 * word per thread: at least 1 MiB); mode 1: copy n_bytes from a to dst; mode 2: dst = a ^ b over
 * n_bytes each (two streams in, one out, as SwiGLU). n_bytes % 16 == 0, 16-byte aligned. */
void hbm_stream_probe(void *dst, const void *a, const void *b, size_t n_bytes, int mode,
                      hipStream_t stream);

/* Measurement helper: the device read peak, as the reference measures it beside every bench run
 * (bench/bandwidth.cu:25-116 read_kernel: a grid-stride read, the best of several launch
 * shapes). Reads n_bytes of a (n_bytes % 16 == 0, 16-byte aligned) with `blocks` workgroups of
 * `threads` threads (64..1024, a power of two), each thread keeping loads_in_flight (4, 8 or 16)
 * non-temporal 16-byte loads in flight per round; contiguous 0 walks the buffer grid-stride (the
 * reference's pattern), 1 gives each workgroup one contiguous range (as a GEMV's workgroups read
 * their rows). *out is written only in the unlikely case the xor of a thread's data equals
 * 0x9e3779b9. */
void hbm_read_peak_probe(unsigned *out, const void *a, size_t n_bytes, int blocks, int threads,
                         int loads_in_flight, int contiguous, hipStream_t stream);

/* Measurement helper: the device copy peak (the reference's bench/bandwidth.cu:25-116 measures a
 * device-to-device copy beside its read kernel). Copies n_bytes of a to dst (n_bytes % 16 == 0,
 * both 16-byte aligned, not overlapping) grid-stride with `blocks` workgroups of `threads`
 * threads (64..1024, a power of two), each thread requesting chunks_in_flight (1, 2, 4 or 8)
 * non-temporal 16-byte loads before it stores them. */
void hbm_copy_peak_probe(void *dst, const void *a, size_t n_bytes, int blocks, int threads,
                         int chunks_in_flight, hipStream_t stream);

/* No counterpart in the reference. Decode attention as attention_forward computes it, without
 * the `att` argument, for callers that cannot allocate device memory (code under stream
 * capture, tight serving loops, harnesses that forbid hipMalloc). It allocates nothing: its
 * workspace is a library-owned device array of 2^20 floats (4 MiB) per device, so
 * attention_workspace_floats(n_heads, head_dim, max_seq) must not exceed 1048576 (Qwen3-4B's 32
 * heads of 128 fit up to 10798 positions); larger sizes are an error and nothing is launched.
 * Every call on a device shares that device's array: calls that overlap on one device race. */
void attention_forward_noalloc(bf16 *out, const bf16 *q, const bf16 *key_cache,
                               const bf16 *value_cache, int n_heads, int n_kv_heads, int head_dim,
                               const int *d_pos, int max_seq, float scale, hipStream_t stream);

/* Floats attention_forward needs in `att` for these sizes. */
size_t attention_workspace_floats(int n_heads, int head_dim, int max_seq);

/* Error mode: 1 (default) = print and exit(EXIT_FAILURE) like the reference; 0 = record the
 * message, skip the launch and return. Returns the previous mode. */
int llm_set_exit_on_error(int enable);
/* Message of the last recorded error of this thread, or NULL. */
const char *llm_last_error(void);
void llm_clear_error(void);

#ifdef __cplusplus
}
#endif
#endif
