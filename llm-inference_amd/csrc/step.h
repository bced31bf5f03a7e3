// Arguments and host entry points of the persistent decode-step kernel (step_kernel.hip).
#pragma once

#include "llm_amd/forward.h"

// Per-layer weight pointers, copied to the device once per RunState.
struct LayerDev {
    const bf16 *attn_norm, *wq, *wk, *wv, *q_norm, *k_norm, *wo, *mlp_norm, *w_gate, *w_up,
        *w_down;
};

// Tagged vectors: element i of a bf16 activation vector travels between workgroups as the
// 32-bit word (bf16 bits << 16) | tag, where tag (1..65535) names the phase that wrote it.
// A consumer polls the words it needs until every tag is the expected one; there is no grid
// barrier. tx: residual stream [H], tqkv: q|k|v [QD + 2 KVD], tattn: attention output [QD],
// thb: SwiGLU output [I]. The vectors read by many workgroups (tx, tattn, thb) have room for
// STEP_REPLICAS copies, step_replica_stride(n) words apart; a model shape writes the first
// R <= STEP_REPLICAS of them and workgroup b reads copy b % R: fewer pollers per cache line make
// a written value visible sooner, more copies cost the writers more stores. The copies sit 1 KB
// off a 4 KB grid (copy q at q (4 KB multiple + 1 KB)): on MI355X the 0.6B decode measured 2328
// tokens/s against 2300 for copies on the 4 KB grid (offsets of 512 B: 2302, 1.5-2 KB: 2319-2321,
// 3 KB: 2309).
constexpr int STEP_REPLICAS = 8;
constexpr size_t step_replica_stride(size_t n) { return (n + 1023) / 1024 * 1024 + 256; }

struct StepArgs {
    const bf16 *embed, *final_norm, *lm_head;
    const LayerDev *layers;
    bf16 *logits, *key_cache, *value_cache;
    uint32_t *tx, *tqkv, *tattn, *thb;
    int *next_token, *pos, *token_out, *pos_base, *error_flag;
    unsigned *epoch;      // tagged phases written over all launches (the tag base)
    unsigned long long *token_word;  // the next token, tagged: (token << 32) | tag
    // per-workgroup argmax partials, tagged 64-bit words AMAX_STRIDE words apart
    unsigned long long *amax;
    long long *trace;     // optional wall-clock stamps of one workgroup's phases
    float eps, scale;
    int n_layers, vocab, max_seq, token_capacity, advance;
    int n_tokens;  // decode steps this launch runs (each feeds its argmax to the next)
    // The split instance's tagged block statistics [n_heads, max_blocks, 2] (max, sum) and
    // block partials [n_heads, max_blocks, head_dim], 64-bit words (float bits << 32) | tag.
    unsigned long long *tstat, *tpart;
    int max_blocks;
    float inv_freq[64];
};

// Each workgroup's argmax partial (one 64-bit word) sits on a 128-byte line of its own, so the
// workgroups' stores at the end of a token do not meet on shared lines.
constexpr int AMAX_STRIDE = 16;

// Workspace the step kernel keeps in RunState::step_ws (zeroed at allocation and after an
// error; a zero tag never matches), followed by the tagged vectors. Its size is 256 bytes past a
// multiple of 4 KB, which places the tagged vectors' copies 1 KB off the 4 KB grid.
struct StepWorkspace {
    unsigned epoch;
    unsigned pad[63];
    // the next token's word at token_word[0], alone on its cache line (every workgroup polls
    // it; sharing the line of a word every workgroup writes once per token cost the 0.6B decode
    // up to 2.8%); the rest of the 4 KB block is padding
    unsigned long long token_word[512];
    unsigned long long amax[1024 * AMAX_STRIDE];      // workgroup b's partial at amax[b * stride]
};
static_assert(sizeof(StepWorkspace) % 4096 == 256, "tagged vectors 256 bytes past the 4 KB grid");

// The workspace for a run state of max_seq positions: the words above, the tagged vectors, then
// the split attention's statistics and partials.
size_t step_workspace_bytes(const Config *cfg, int max_seq);
// Blocks of 64 positions the split attention's workspace holds for max_seq positions, and where
// its statistics and partials sit in the workspace `ws`.
int step_split_max_blocks(const Config *cfg, int max_seq);
void step_split_buffers(const Config *cfg, int max_seq, void *ws, unsigned long long **tstat,
                        unsigned long long **tpart);
// STEP_PERSISTENT: the shapes have a specialisation and every position fits its attention.
bool step_kernel_supported(const Config *cfg, int max_seq);
// The positions the step kernel's attention can hold at most (one workgroup per query head
// below the split, split items above it).
int step_kernel_max_seq(const Config *cfg);
// The history (blocks of 64 positions) from which the shapes' step kernel splits attention over
// (kv head, block) items: the measured crossover of the two attention forms.
int step_kernel_split_blocks(const Config *cfg);
// The shapes have a specialisation (STEP_AUTO then runs it below step_kernel_switch_pos).
bool step_kernel_available(const Config *cfg);
// The first position at which STEP_AUTO runs the hipGraph step instead of the step kernel (the
// measured crossover, at most the kernel's longest history).
int step_kernel_switch_pos(const Config *cfg);
int step_kernel_grid();
// Launches the step kernel; with `split` the instance whose attention runs split over (kv head,
// block) items (long histories), else one workgroup per query head.
bool step_kernel_launch(const Config *cfg, const StepArgs &args, bool split, int grid,
                        hipStream_t stream);
