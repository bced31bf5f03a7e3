/*
 * Model, run state and decode-step API of the MI355X build. C ABI.
 *
 * The types and functions replace William-Lamer/llm-inference src/model.cuh:10-64 and
 * src/forward.cuh:6-34 with the same field names, argument order and fail-fast error
 * behaviour (print to stderr, exit(EXIT_FAILURE); see llm_set_exit_on_error in kernels.h).
 * The reference's 4096-position cap on the KV cache (src/forward.cu:7-8) is lifted: the cache
 * holds max_seq_len positions, or the count given to alloc_run_state_seq.
 */
#ifndef LLM_AMD_FORWARD_H
#define LLM_AMD_FORWARD_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#include "kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

#define MAX_SHARDS 8
#define MAX_EOS 8

/* src/model.cuh:10-24 */
typedef struct {
    int hidden_size;
    int intermediate_size;
    int n_layers;
    int n_heads;
    int n_kv_heads;
    int head_dim;
    int vocab_size;
    int max_seq_len;
    float rms_norm_eps;
    float rope_theta;
    int tie_word_embeddings;
    int eos_ids[MAX_EOS];
    int n_eos;
} Config;

/* src/model.cuh:27-39. Matrices are PyTorch linear weights: [out, in], row-major. */
typedef struct {
    const bf16 *attn_norm;
    const bf16 *wq;
    const bf16 *wk;
    const bf16 *wv;
    const bf16 *q_norm;
    const bf16 *k_norm;
    const bf16 *wo;
    const bf16 *mlp_norm;
    const bf16 *w_gate;
    const bf16 *w_up;
    const bf16 *w_down;
} LayerWeights;

/* src/model.cuh:41-45 */
typedef struct {
    char name[96];
    const bf16 *data;
    size_t numel;
} TensorRef;

/* src/model.cuh:48-59. Host structs; the bf16 pointers point to device memory. */
typedef struct {
    const bf16 *embed;
    LayerWeights *layers;
    const bf16 *final_norm;
    const bf16 *lm_head;

    TensorRef *tensors;
    int n_tensors;
    void *gpu_buffers[MAX_SHARDS];
    int n_buffers;
    size_t gpu_bytes;
} Weights;

/* src/forward.cuh:6-25, plus the device state the gfx950 step keeps after the reference's
 * fields (attention workspace, argmax partials, the on-device token stream). */
typedef struct {
    bf16 *x;
    bf16 *xb;
    bf16 *q;
    bf16 *k;
    bf16 *v;
    bf16 *attn_out;
    float *att;            /* attention_workspace_floats(n_heads, head_dim, max_seq), then
                              (from a 256-byte boundary) the launch counters and tagged block
                              partials of the step's one-launch PV and combine (head_dim 128) */
    bf16 *key_cache;       /* [n_layers, max_seq, n_kv_heads * head_dim] */
    bf16 *value_cache;     /* [n_layers, max_seq, n_kv_heads * head_dim] */
    int max_seq;
    bf16 *hb;
    bf16 *tap1;
    bf16 *tap2;
    bf16 *logits;
    int *next_token;
    int *pos;
    hipStream_t stream;
    hipGraphExec_t graph;
    /* additions */
    void *argmax_partials;  /* per-workgroup (value, index) pairs of the two-stage argmax */
    int *token_out;         /* [token_capacity] tokens written by the on-device decode loop */
    int token_capacity;
    int *pos_base;          /* position of token_out[0] */
    int *error_flag;        /* set on the device when a fed-back token is outside the vocab or a
                               step-kernel wait timed out */
    hipGraphExec_t loop_graph; /* step + argmax + token feedback + pos advance */
    int step_mode;          /* STEP_AUTO, STEP_GRAPH or STEP_PERSISTENT (see capture_graph) */
    int persistent;         /* 1 once capture_graph chose the persistent step kernel */
    void *step_ws;          /* the persistent step's sequence counter, argmax partials and
                               tagged activation vectors */
    void *layers_dev;       /* per-layer weight pointers on the device */
    int step_grid;          /* workgroups of the persistent step (one per CU) */
    int next_token_valid;   /* the last forward() already computed the argmax */
    long long *step_trace;  /* optional [4 * n_layers + 3 + 8 * step_grid] wall-clock stamps
                               (device memory, set by the caller; NULL = off): [0] start, then
                               per layer the moments the first matrix workgroup has its inputs
                               for the q/k/v, o, gate/up and down rows, then for the LM head,
                               and the end; then, for layer 1 and every workgroup, 8 stamps:
                               input staged / results stored for each of its 4 phases */
    int attn_mode;          /* how the graph and eager steps run QK-norm + RoPE + attention (set
                               before capture_graph): ATTN_AUTO, ATTN_SEPARATE
                               (qk_norm_rope_forward + attention_forward), ATTN_IN_SCORES
                               (qk_norm_rope_attention_forward) or ATTN_ONE_PASS
                               (qk_norm_rope_attention_one_pass) */
    void *attn_one_pass_ws; /* the one-pass attention's workspace (zeroed at allocation; NULL
                               where the shapes have no one-pass attention) */
    float *rope_table;      /* [head_dim] cos then sin of the RoPE rotation at *pos, computed
                               once per step for the in-scores attention of every layer */
    int step_switch_pos;    /* with the persistent kernel prepared: positions below this run it,
                               positions from it on the hipGraph step (set by capture_graph) */
    int step_split_blocks;  /* the persistent kernel's attention runs one workgroup per query
                               head below this many blocks of 64 positions of history, and split
                               over (kv head, block) items from it on (1..128; set by
                               capture_graph to the shapes' measured crossover) */
} RunState;

/* RunState::attn_mode. ATTN_AUTO takes ATTN_IN_SCORES when the longest history (max_seq) has at
 * most 256 (64-position block, kv head) items, or when head_dim <= 128 and at most 4 query heads
 * share a kv head: every item then applies the query heads' QK-norm + RoPE with the step's RoPE
 * table (RunState::rope_table, one launch per step) and the scores kernel keeps five workgroups
 * per CU (Qwen3-0.6B graph step, 269 positions: +3% tokens/s; Qwen3-4B at 8192-8448 positions:
 * 433.3-433.8 tokens/s against 431.7 for ATTN_SEPARATE and 412.5 for ATTN_ONE_PASS). Otherwise
 * ATTN_SEPARATE. ATTN_ONE_PASS is taken only when asked for. At head_dim 128 (and at most 8192
 * items) the graph step's ATTN_IN_SCORES and ATTN_SEPARATE run attention's PV and combine passes
 * as one launch, with the same bits. */
enum { ATTN_AUTO = 0, ATTN_SEPARATE = 1, ATTN_IN_SCORES = 2, ATTN_ONE_PASS = 3 };

/* How capture_graph prepares the step. STEP_AUTO: where the shapes have a specialisation
 * (Qwen3-0.6B, 1.7B, 4B), the persistent step kernel (one launch per forward;
 * generate_greedy runs its tokens in one launch, or two where they cross
 * RunState::step_split_blocks) for the positions below RunState::step_switch_pos, and a
 * hipGraph of the per-layer kernels from there on. The kernel's attention runs one workgroup
 * per query head up to 448 / 384 / 512 positions at 0.6B / 1.7B / 4B, and split over
 * (kv head, 64-position block) items on every workgroup from there on, up to the kernel's
 * longest history (12288 positions on 256 CUs: the switch; the graph leads by at most 4%,
 * between ~5000 and ~7500 positions at 1.7B and 4B). 5-token prompt: 2476 / 1145 / 615 tokens/s against
 * 1278 / 893 / 492 for the graph; 0.6B after 4096 / 8192 positions 1450 / 1274 against 1138 /
 * 1035. Other shapes: the hipGraph. STEP_GRAPH: always the hipGraph. STEP_PERSISTENT: the
 * persistent kernel at every position (max_seq at most the kernel's longest history) or an
 * error. */
enum { STEP_AUTO = 0, STEP_GRAPH = 1, STEP_PERSISTENT = 2 };

/* src/loader.cu:105-139 (config.json, generation_config.json) */
void load_config(const char *model_dir, Config *cfg);
/* src/loader.cu:313-380 (safetensors shards; BF16 only; 16-byte-aligned offsets) */
void load_weights(const char *model_dir, const Config *cfg, Weights *w);
void free_weights(Weights *w);
/* src/loader.cu:395-419: "<name> <numel> <sum of bits> <index-weighted sum> <first value>" */
void print_weight_checksums(const Weights *w);

/* src/forward.cuh:27-34. capture_graph prepares the step per RunState::step_mode (set it
 * before the call; the default is STEP_AUTO). */
void alloc_run_state(RunState *s, const Config *cfg);
void free_run_state(RunState *s);
void capture_graph(const Config *cfg, const Weights *w, RunState *s);
void forward(const Config *cfg, const Weights *w, RunState *s, int token, int pos);
int sample_argmax(const Config *cfg, RunState *s);
/* src/forward.cuh:32. A token drawn from softmax(logits / temperature) at the coin in [0, 1)
 * (sample_forward); an error if the draw finds none. */
int sample_temperature(const Config *cfg, RunState *s, float temperature, float coin);
size_t weight_bytes_per_step(const Config *cfg);
size_t kv_bytes_per_position(const Config *cfg);

/* ---- additions ---- */

/* alloc_run_state with a KV cache of max_seq positions (no cap). */
void alloc_run_state_seq(RunState *s, const Config *cfg, int max_seq);

/* Seeded random weights in the layout load_weights produces: every matrix and the embedding
 * N(0, std), norm gammas 1 + N(0, gamma_std), lm_head tied to the embedding. One device buffer.
 * Deterministic in (cfg shapes, seed). */
void synth_weights(const Config *cfg, Weights *w, uint64_t seed, float std, float gamma_std);

/* Fills n bf16 values at dev with mean + std * N(0,1) from the counter-based generator used by
 * synth_weights (stream selects an independent sequence). */
void synth_fill(bf16 *dev, size_t n, uint64_t seed, uint64_t stream_id, float mean, float std,
                hipStream_t stream);

/* Greedy decode entirely on the device: starting from `token` at position `pos`, replays the
 * captured step n_steps times, feeding each argmax back as the next token. The n_steps greedy
 * tokens are copied to out_tokens (host). One host synchronisation at the end. Returns 0, or
 * -1 (error recorded) if a token left the vocabulary or a device-side wait timed out. */
int generate_greedy(const Config *cfg, const Weights *w, RunState *s, int token, int pos,
                    int n_steps, int *out_tokens);

#ifdef __cplusplus
}
#endif
#endif
