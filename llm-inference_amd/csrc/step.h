// Arguments and host entry points of the persistent decode-step kernel (step_kernel.hip).
#pragma once

#include "llm_amd/forward.h"

// Per-layer weight pointers, copied to the device once per RunState.
struct LayerDev {
    const bf16 *attn_norm, *wq, *wk, *wv, *q_norm, *k_norm, *wo, *mlp_norm, *w_gate, *w_up,
        *w_down;
};

struct StepArgs {
    const bf16 *embed, *final_norm, *lm_head;
    const LayerDev *layers;
    bf16 *x, *q, *k, *v, *attn_out, *hb, *logits, *key_cache, *value_cache;
    int *next_token, *pos, *token_out, *pos_base, *error_flag;
    unsigned *bar;        // grid-barrier counters, 16 lines of 128 bytes
    unsigned *epoch;      // barriers completed so far (the counters' expected base)
    unsigned *final_ctr;  // workgroups done with the LM head
    float *amax_val;      // per-workgroup argmax partials
    int *amax_idx;
    long long *trace;     // optional: wall-clock stamp after every barrier (workgroup 0)
    float eps, scale;
    int n_layers, vocab, max_seq, token_capacity, advance;
    float inv_freq[64];
};

// Workspace the step kernel keeps in RunState::step_ws (zeroed at allocation).
struct StepWorkspace {
    unsigned bar[16 * 32];
    unsigned epoch;
    unsigned final_ctr;
    unsigned pad[30];
    float amax_val[1024];
    int amax_idx[1024];
};

bool step_kernel_supported(const Config *cfg, int max_seq);
int step_kernel_grid();
bool step_kernel_launch(const Config *cfg, const StepArgs &args, int grid, hipStream_t stream);
