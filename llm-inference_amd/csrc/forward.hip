// Decode step of the gfx950 build: run state, the per-layer launch order of the reference's
// forward_kernels (src/forward.cu:118-193) on the gfx950 kernels, hipGraph capture and replay,
// greedy sampling, and a decode loop that stays on the device (argmax feeds the next step's
// embedding, the position advances in a kernel, tokens are copied out once at the end).
#include <math.h>
#include <string.h>

#include "common.h"
#include "internal.h"
#include "llm_amd/dump.h"
#include "llm_amd/forward.h"
#include "step.h"

using namespace llm;

// ------------------------------------------------------------------------------------------
// run state (src/forward.cu:10-73)
// ------------------------------------------------------------------------------------------

static bool dmalloc(void **p, size_t bytes) {
    *p = nullptr;
    if (!HIP_OK(hipMalloc(p, bytes))) return false;
    return HIP_OK(hipMemset(*p, 0, bytes));
}

// The attention workspace's bytes, rounded up to 256.
static size_t att_bytes(const Config *cfg, int max_seq) {
    return (attention_workspace_floats(cfg->n_heads, cfg->head_dim, max_seq) * 4 + 255) / 256 * 256;
}

// The workspace of the one-launch PV and combine inside RunState::att, or NULL where the shapes
// do not take it.
static void *pvc_workspace(const Config *cfg, const RunState *s) {
    if (!attention_pv_combine_bytes(cfg->n_heads, cfg->n_kv_heads, cfg->head_dim, s->max_seq))
        return nullptr;
    return (char *)s->att + att_bytes(cfg, s->max_seq);
}

extern "C" void alloc_run_state_seq(RunState *s, const Config *cfg, int max_seq) {
    memset(s, 0, sizeof *s);
    if (max_seq <= 0) {
        llm_fail("alloc_run_state: max_seq %d must be positive", max_seq);
        return;
    }
    const size_t q_dim = (size_t)cfg->n_heads * cfg->head_dim;
    const size_t kv_dim = (size_t)cfg->n_kv_heads * cfg->head_dim;
    const size_t H = cfg->hidden_size, I = cfg->intermediate_size;
    s->max_seq = max_seq;
    const size_t cache_len = (size_t)cfg->n_layers * max_seq * kv_dim;
    size_t tap_len = q_dim;
    if (I > tap_len) tap_len = I;
    if (H > tap_len) tap_len = H;
    // `att` holds the attention workspace, then (from a 256-byte boundary) the workspace of the
    // one-launch PV and combine where the shapes take it
    const size_t att = att_bytes(cfg, max_seq) +
                       attention_pv_combine_bytes(cfg->n_heads, cfg->n_kv_heads, cfg->head_dim,
                                                  max_seq);
    bool ok = dmalloc((void **)&s->x, H * 2) && dmalloc((void **)&s->xb, H * 2) &&
              dmalloc((void **)&s->q, q_dim * 2) && dmalloc((void **)&s->k, kv_dim * 2) &&
              dmalloc((void **)&s->v, kv_dim * 2) && dmalloc((void **)&s->attn_out, q_dim * 2) &&
              dmalloc((void **)&s->att, att) && dmalloc((void **)&s->key_cache, cache_len * 2) &&
              dmalloc((void **)&s->value_cache, cache_len * 2) && dmalloc((void **)&s->hb, I * 2) &&
              dmalloc((void **)&s->tap1, tap_len * 2) && dmalloc((void **)&s->tap2, tap_len * 2) &&
              dmalloc((void **)&s->logits, (size_t)cfg->vocab_size * 2) &&
              dmalloc((void **)&s->next_token, 4) && dmalloc((void **)&s->pos, 4) &&
              dmalloc(&s->argmax_partials, (size_t)argmax_partial_count() * 8) &&
              dmalloc((void **)&s->pos_base, 4) && dmalloc((void **)&s->error_flag, 4) &&
              dmalloc(&s->step_ws, step_workspace_bytes(cfg, max_seq)) &&
              dmalloc((void **)&s->rope_table, (size_t)cfg->head_dim * 4);
    if (ok && attention_one_pass_supported(cfg->n_heads, cfg->n_kv_heads, cfg->head_dim, max_seq))
        ok = dmalloc(&s->attn_one_pass_ws,
                     attention_one_pass_bytes(cfg->n_heads, cfg->head_dim, max_seq));
    if (!ok) return;
    HIP_OK(hipStreamCreate(&s->stream));
}

extern "C" void alloc_run_state(RunState *s, const Config *cfg) {
    alloc_run_state_seq(s, cfg, cfg->max_seq_len);
}

extern "C" void free_run_state(RunState *s) {
    void *bufs[] = {s->x,  s->xb,     s->q,      s->k,      s->v,          s->attn_out,
                    s->att, s->key_cache, s->value_cache, s->hb, s->tap1, s->tap2,
                    s->logits, s->next_token, s->pos, s->argmax_partials, s->token_out,
                    s->pos_base, s->error_flag, s->step_ws, s->layers_dev,
                    s->attn_one_pass_ws, s->rope_table};
    for (void *b : bufs)
        if (b) HIP_OK(hipFree(b));
    if (s->graph) HIP_OK(hipGraphExecDestroy(s->graph));
    if (s->loop_graph) HIP_OK(hipGraphExecDestroy(s->loop_graph));
    if (s->stream) HIP_OK(hipStreamDestroy(s->stream));
    memset(s, 0, sizeof *s);
}

// ------------------------------------------------------------------------------------------
// byte counts (src/forward.cu:83-114)
// ------------------------------------------------------------------------------------------

extern "C" size_t weight_bytes_per_step(const Config *cfg) {
    const size_t H = cfg->hidden_size, D = cfg->head_dim;
    const size_t q_dim = (size_t)cfg->n_heads * D, kv_dim = (size_t)cfg->n_kv_heads * D;
    const size_t I = cfg->intermediate_size;
    // norms, q/k/v, q/k norms, o, mlp norm, gate/up/down
    const size_t layer = H + q_dim * H + 2 * kv_dim * H + 2 * D + H * q_dim + H + 2 * I * H + H * I;
    // layers, final norm, LM head, one embedding row
    const size_t elements = layer * cfg->n_layers + H + (size_t)cfg->vocab_size * H + H;
    return elements * 2;
}

extern "C" size_t kv_bytes_per_position(const Config *cfg) {
    return 2 * (size_t)cfg->n_layers * cfg->n_kv_heads * cfg->head_dim * 2;
}

// ------------------------------------------------------------------------------------------
// the step
// ------------------------------------------------------------------------------------------

// One layer tensor of the dumps: "Lnn.<name>" (src/forward.cu:75-79).
static void dump_layer(int l, const char *name, const bf16 *d, int n) {
    char full[64];
    snprintf(full, sizeof full, "L%02d.%s", l, name);
    dump_bf16(full, d, n);
}

static bool forward_kernels(const Config *cfg, const Weights *w, RunState *s) {
    const int H = cfg->hidden_size, D = cfg->head_dim;
    const int q_dim = cfg->n_heads * D, kv_dim = cfg->n_kv_heads * D;
    const int I = cfg->intermediate_size;
    const float scale = (float)(1.0 / sqrt((double)D));
    hipStream_t st = s->stream;
    // While dumping, every intermediate is kept: the RMSNorms run on their own and the fused
    // launchers write their taps (src/forward.cu:127-133). Otherwise RMSNorm runs as the prologue
    // of the GEMV that reads it (same bits, one launch and one store/reload of the normed row
    // fewer) for hidden sizes of up to 8192.
    const bool dumping = dump_enabled() != 0;
    const bool fuse_norm = H <= 8192 && !dumping;
    const long attn_items = (long)((s->max_seq + 63) / 64) * cfg->n_kv_heads;
    const bool one_pass = !dumping && s->attn_mode == ATTN_ONE_PASS;
    if (one_pass && !s->attn_one_pass_ws)
        return llm_fail("forward: no one-pass attention for these shapes");
    const int rep = cfg->n_heads / cfg->n_kv_heads;
    const bool fuse_attn =
        !dumping && !one_pass &&
        (s->attn_mode == ATTN_IN_SCORES ||
         (s->attn_mode == ATTN_AUTO && (attn_items <= 256 || (D <= 128 && rep <= 4))));
    bf16 *tap1 = dumping ? s->tap1 : nullptr, *tap2 = dumping ? s->tap2 : nullptr;
    // PV and combine as one launch (attn_pv_combine_kernel, the same bits) where the shapes
    // take it
    void *pvc = pvc_workspace(cfg, s);
    embedding_checked(s->x, w->embed, s->next_token, H, cfg->vocab_size, s->error_flag, st);
    dump_bf16("embed", s->x, H);
    // The in-scores attention of every layer reads the RoPE table of this position from one
    // launch instead of recomputing it in each of its items.
    if (fuse_attn && !rope_table_launch(s->rope_table, s->pos, D, cfg->rope_theta, st)) return false;
    for (int l = 0; l < cfg->n_layers && !llm_has_error(); l++) {
        const LayerWeights *L = &w->layers[l];
        bf16 *kc = s->key_cache + (size_t)l * s->max_seq * kv_dim;
        bf16 *vc = s->value_cache + (size_t)l * s->max_seq * kv_dim;
        if (fuse_norm) {
            rmsnorm_qkv_forward(s->q, s->k, s->v, L->wq, L->wk, L->wv, s->x, L->attn_norm,
                                cfg->rms_norm_eps, q_dim, kv_dim, H, st);
        } else {
            rmsnorm_forward(s->xb, s->x, L->attn_norm, 1, H, cfg->rms_norm_eps, st);
            dump_layer(l, "attn_norm", s->xb, H);
            qkv_forward(s->q, s->k, s->v, L->wq, L->wk, L->wv, s->xb, q_dim, kv_dim, H, st);
        }
        dump_layer(l, "q_proj", s->q, q_dim);
        dump_layer(l, "k_proj", s->k, kv_dim);
        dump_layer(l, "v_proj", s->v, kv_dim);
        if (one_pass) {
            // QK-norm + RoPE + attention in one launch (same bits)
            attention_one_pass_launch(s->attn_out, s->q, s->k, s->v, L->q_norm, L->k_norm, kc, vc,
                                      s->attn_one_pass_ws, s->error_flag, s->pos, cfg->n_heads,
                                      cfg->n_kv_heads, D, cfg->rms_norm_eps, cfg->rope_theta,
                                      s->max_seq, scale, st);
        } else if (fuse_attn) {
            // QK-norm + RoPE inside the attention's scores pass (same bits, one launch fewer)
            qk_norm_rope_attention_launch(s->attn_out, s->q, s->k, s->v, L->q_norm, L->k_norm, kc,
                                          vc, s->att, s->pos, cfg->n_heads, cfg->n_kv_heads, D,
                                          cfg->rms_norm_eps, cfg->rope_theta, s->max_seq, scale,
                                          st, s->rope_table, pvc, s->error_flag);
        } else {
            qk_norm_rope_forward(s->q, s->k, s->v, L->q_norm, L->k_norm, kc, vc, s->pos,
                                 cfg->n_heads, cfg->n_kv_heads, D, cfg->rms_norm_eps,
                                 cfg->rope_theta, tap1, tap2, st);
            dump_layer(l, "q_norm", tap1, q_dim);
            dump_layer(l, "k_norm", tap2, kv_dim);
            dump_layer(l, "q_rope", s->q, q_dim);
            dump_layer(l, "k_rope", s->k, kv_dim);
            attention_launch(s->attn_out, s->q, kc, vc, s->att, cfg->n_heads, cfg->n_kv_heads, D,
                             s->pos, s->max_seq, scale, st, pvc, s->error_flag);
        }
        dump_layer(l, "attn_out", s->attn_out, q_dim);
        gemv_residual_forward(s->x, L->wo, s->attn_out, H, q_dim, tap1, st);
        dump_layer(l, "o_proj", tap1, H);
        dump_layer(l, "attn_resid", s->x, H);
        if (fuse_norm) {
            rmsnorm_gate_up_forward(s->hb, L->w_gate, L->w_up, s->x, L->mlp_norm,
                                    cfg->rms_norm_eps, I, H, st);
        } else {
            rmsnorm_forward(s->xb, s->x, L->mlp_norm, 1, H, cfg->rms_norm_eps, st);
            dump_layer(l, "mlp_norm", s->xb, H);
            gate_up_forward(s->hb, L->w_gate, L->w_up, s->xb, I, H, tap1, tap2, st);
        }
        dump_layer(l, "gate", tap1, I);
        dump_layer(l, "up", tap2, I);
        dump_layer(l, "mlp_act", s->hb, I);
        gemv_residual_forward(s->x, L->w_down, s->hb, H, I, tap1, st);
        dump_layer(l, "down", tap1, H);
        dump_layer(l, "out", s->x, H);
    }
    if (fuse_norm) {
        rmsnorm_gemv_forward(s->logits, w->lm_head, s->x, w->final_norm, cfg->rms_norm_eps,
                             cfg->vocab_size, H, st);
    } else {
        rmsnorm_forward(s->xb, s->x, w->final_norm, 1, H, cfg->rms_norm_eps, st);
        dump_bf16("final_norm", s->xb, H);
        gemv_forward(s->logits, w->lm_head, s->xb, cfg->vocab_size, H, st);
    }
    dump_bf16("logits", s->logits, cfg->vocab_size);
    return !llm_has_error();
}

static void argmax_into_next(const Config *cfg, RunState *s) {
    float *pv = (float *)s->argmax_partials;
    int *pi = (int *)(pv + argmax_partial_count());
    argmax_launch(s->next_token, s->logits, cfg->vocab_size, pv, pi, s->stream);
}

// Token and position travel as kernel arguments, so no host buffer has to outlive the call.
__global__ void set_token_pos_kernel(int *d_token, int *d_pos, int token, int pos) {
    if (threadIdx.x == 0) {
        *d_token = token;
        *d_pos = pos;
    }
}

// Records the next token and advances the position (the on-device decode loop).
__global__ void advance_kernel(int *d_pos, const int *d_token, int *token_out,
                               const int *pos_base, int capacity) {
    if (threadIdx.x == 0) {
        const int i = *d_pos - *pos_base;
        if (i >= 0 && i < capacity) token_out[i] = *d_token;
        *d_pos = *d_pos + 1;
    }
}

static bool capture(hipStream_t st, hipGraphExec_t *exec, bool (*body)(void *), void *ctx) {
    hipGraph_t graph;
    if (!HIP_OK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal))) return false;
    const bool ok = body(ctx);
    hipError_t end = hipStreamEndCapture(st, &graph);
    if (!ok) {
        if (end == hipSuccess) (void)hipGraphDestroy(graph);
        return false;
    }
    if (!HIP_OK(end)) return false;
    const bool inst = HIP_OK(hipGraphInstantiate(exec, graph, nullptr, nullptr, 0));
    HIP_OK(hipGraphDestroy(graph));
    return inst;
}

struct StepCtx {
    const Config *cfg;
    const Weights *w;
    RunState *s;
};

static bool step_body(void *p) {
    StepCtx *c = (StepCtx *)p;
    return forward_kernels(c->cfg, c->w, c->s);
}

static bool loop_body(void *p) {
    StepCtx *c = (StepCtx *)p;
    if (!forward_kernels(c->cfg, c->w, c->s)) return false;
    argmax_into_next(c->cfg, c->s);
    advance_kernel<<<1, 64, 0, c->s->stream>>>(c->s->pos, c->s->next_token, c->s->token_out,
                                                c->s->pos_base, c->s->token_capacity);
    return LAUNCH_OK();
}

// The persistent step: per-layer pointers on the device, a zeroed workspace, one workgroup per
// CU (at most the workspace's 1024 argmax slots).
static bool prepare_persistent(const Config *cfg, const Weights *w, RunState *s) {
    if (!s->layers_dev) {
        if (!HIP_OK(hipMalloc(&s->layers_dev, sizeof(LayerDev) * cfg->n_layers))) return false;
    }
    LayerDev *host = (LayerDev *)calloc(cfg->n_layers, sizeof(LayerDev));
    if (!host) return llm_fail("capture_graph: out of memory");
    for (int l = 0; l < cfg->n_layers; l++) {
        const LayerWeights *L = &w->layers[l];
        host[l] = LayerDev{L->attn_norm, L->wq, L->wk, L->wv, L->q_norm, L->k_norm,
                           L->wo, L->mlp_norm, L->w_gate, L->w_up, L->w_down};
    }
    const bool ok = HIP_OK(hipMemcpy(s->layers_dev, host, sizeof(LayerDev) * cfg->n_layers,
                                     hipMemcpyHostToDevice)) &&
                    HIP_OK(hipMemset(s->step_ws, 0, step_workspace_bytes(cfg, s->max_seq)));
    free(host);
    if (!ok) return false;
    int grid = step_kernel_grid();
    if (grid <= 0) return llm_fail("capture_graph: cannot read the CU count");
    s->step_grid = grid > 1024 ? 1024 : grid;
    s->step_split_blocks = step_kernel_split_blocks(cfg);
    s->persistent = 1;
    return true;
}

static StepArgs step_args(const Config *cfg, const Weights *w, RunState *s, int advance) {
    StepArgs a;
    memset(&a, 0, sizeof a);
    StepWorkspace *ws = (StepWorkspace *)s->step_ws;
    a.embed = w->embed;
    a.final_norm = w->final_norm;
    a.lm_head = w->lm_head;
    a.layers = (const LayerDev *)s->layers_dev;
    a.logits = s->logits;
    a.key_cache = s->key_cache;
    a.value_cache = s->value_cache;
    a.next_token = s->next_token;
    a.pos = s->pos;
    a.token_out = s->token_out;
    a.pos_base = s->pos_base;
    a.error_flag = s->error_flag;
    uint32_t *tagged = (uint32_t *)(ws + 1);
    const int qd = cfg->n_heads * cfg->head_dim, kvd = cfg->n_kv_heads * cfg->head_dim;
    a.tx = tagged;
    a.tqkv = a.tx + STEP_REPLICAS * step_replica_stride(cfg->hidden_size);
    a.tattn = a.tqkv + step_replica_stride(qd + 2 * kvd);
    a.thb = a.tattn + STEP_REPLICAS * step_replica_stride(qd);
    a.epoch = &ws->epoch;
    a.token_word = &ws->token_word[0];
    a.n_tokens = 1;
    step_split_buffers(cfg, s->max_seq, s->step_ws, &a.tstat, &a.tpart);
    a.max_blocks = step_split_max_blocks(cfg, s->max_seq);
    a.amax = ws->amax;
    a.eps = cfg->rms_norm_eps;
    a.scale = (float)(1.0 / sqrt((double)cfg->head_dim));
    a.n_layers = cfg->n_layers;
    a.vocab = cfg->vocab_size;
    a.max_seq = s->max_seq;
    a.token_capacity = s->token_capacity;
    a.advance = advance;
    a.trace = s->step_trace;
    rope_inv_freq_table(cfg->rope_theta, cfg->head_dim, a.inv_freq);
    return a;
}

// After a synchronisation: a device-side error of the persistent step (bad token or position,
// or a wait that timed out) is reported, and the workspace (sequence counter and tagged
// vectors) is zeroed for the next use.
static bool check_step_error(const Config *cfg, RunState *s) {
    int err = 0;
    if (!HIP_OK(hipMemcpy(&err, s->error_flag, 4, hipMemcpyDeviceToHost))) return false;
    if (err == 0) return true;
    HIP_OK(hipMemset(s->error_flag, 0, 4));
    HIP_OK(hipMemset(s->step_ws, 0, step_workspace_bytes(cfg, s->max_seq)));
    return llm_fail(err == 2 ? "step: a wait for another workgroup's data timed out"
                             : "step: token or position out of range on the device");
}

// src/forward.cu:196-204
extern "C" void capture_graph(const Config *cfg, const Weights *w, RunState *s) {
    StepCtx c{cfg, w, s};
    // Both captured graphs hold the weight pointers of the call that captured them: a new
    // capture (new weights, or a new step mode) drops them, and generate_greedy captures its
    // loop graph again from the current weights when it next needs it.
    if (s->graph) {
        HIP_OK(hipGraphExecDestroy(s->graph));
        s->graph = nullptr;
    }
    if (s->loop_graph) {
        HIP_OK(hipGraphExecDestroy(s->loop_graph));
        s->loop_graph = nullptr;
    }
    s->persistent = 0;
    s->step_switch_pos = 0;
    // while dumping, the step runs eagerly (the reference captures only without --dump,
    // src/main.cu:253): nothing is captured, and forward() dumps as it goes
    if (dump_enabled()) return;
    if (s->step_mode == STEP_PERSISTENT) {
        if (!step_kernel_supported(cfg, s->max_seq)) {
            llm_fail("capture_graph: no persistent step kernel for these shapes");
            return;
        }
        if (prepare_persistent(cfg, w, s)) s->step_switch_pos = s->max_seq;
        return;
    }
    // STEP_AUTO: the step kernel for the positions below its switch position, the hipGraph
    // from there on (captured only when the cache reaches that far)
    if (s->step_mode == STEP_AUTO && step_kernel_available(cfg)) {
        if (!prepare_persistent(cfg, w, s)) return;
        const int sw = step_kernel_switch_pos(cfg);
        s->step_switch_pos = sw < s->max_seq ? sw : s->max_seq;
        if (s->step_switch_pos >= s->max_seq) return;
    }
    capture(s->stream, &s->graph, step_body, &c);
}

// Whether the step at `pos` runs the persistent kernel (else the hipGraph or the eager step).
static bool persistent_at(const RunState *s, int pos) {
    return s->persistent && pos < s->step_switch_pos;
}

// The first position whose step the persistent kernel runs with its split attention, or -1
// (with an error) when RunState::step_split_blocks is outside 1..128.
static int split_from(const RunState *s) {
    if (s->step_split_blocks < 1 || s->step_split_blocks > 128) {
        llm_fail("step: step_split_blocks %d outside 1..128", s->step_split_blocks);
        return -1;
    }
    return (s->step_split_blocks - 1) * 64;
}

static bool check_token_pos(const Config *cfg, const RunState *s, int token, int pos) {
    if (token < 0 || token >= cfg->vocab_size)
        return llm_fail("forward: token %d outside vocab of %d", token, cfg->vocab_size);
    if (pos < 0 || pos >= s->max_seq)
        return llm_fail("forward: position %d past the kv cache size %d", pos, s->max_seq);
    return true;
}

// src/forward.cu:206-227
extern "C" void forward(const Config *cfg, const Weights *w, RunState *s, int token, int pos) {
    if (!check_token_pos(cfg, s, token, pos)) return;
    set_token_pos_kernel<<<1, 64, 0, s->stream>>>(s->next_token, s->pos, token, pos);
    if (!LAUNCH_OK()) return;
    s->next_token_valid = 0;
    if (dump_enabled()) {
        forward_kernels(cfg, w, s);  // the dumps come from the eager step (src/main.cu:253)
    } else if (persistent_at(s, pos)) {
        const int sp = split_from(s);
        if (sp >= 0 &&
            step_kernel_launch(cfg, step_args(cfg, w, s, 0), pos >= sp, s->step_grid, s->stream))
            s->next_token_valid = 1;
    } else if (s->graph) {
        HIP_OK(hipGraphLaunch(s->graph, s->stream));
    } else {
        forward_kernels(cfg, w, s);
    }
}

// src/forward.cu:229-236
// src/forward.cu:238-251: a token drawn from softmax(logits / temperature) at the coin; the
// argmax a persistent step left in next_token is overwritten.
extern "C" int sample_temperature(const Config *cfg, RunState *s, float temperature, float coin) {
    const float inv_temp = 1.0f / temperature;
    sample_forward(s->next_token, s->logits, cfg->vocab_size, inv_temp, coin, s->stream);
    s->next_token_valid = 0;
    int token = -1;
    if (!HIP_OK(hipMemcpyAsync(&token, s->next_token, 4, hipMemcpyDeviceToHost, s->stream)))
        return -1;
    if (!HIP_OK(hipStreamSynchronize(s->stream))) return -1;
    if (!check_step_error(cfg, s)) return -1;
    if (token < 0) {
        llm_fail("sampling found no token (coin %g)", (double)coin);
        return -1;
    }
    return token;
}

extern "C" int sample_argmax(const Config *cfg, RunState *s) {
    if (!s->next_token_valid) argmax_into_next(cfg, s);  // the persistent step already did it
    int token = -1;
    if (!HIP_OK(hipMemcpyAsync(&token, s->next_token, 4, hipMemcpyDeviceToHost, s->stream)))
        return -1;
    if (!HIP_OK(hipStreamSynchronize(s->stream))) return -1;
    if (!check_step_error(cfg, s)) return -1;
    return token;
}

// token_out holds at least n tokens (a larger buffer drops the loop graph, which captured the
// old buffer's address).
static bool ensure_token_capacity(RunState *s, int n) {
    if (s->token_capacity >= n) return true;
    if (s->token_out) HIP_OK(hipFree(s->token_out));
    s->token_out = nullptr;
    s->token_capacity = 0;
    if (s->loop_graph) {
        HIP_OK(hipGraphExecDestroy(s->loop_graph));
        s->loop_graph = nullptr;
    }
    const int cap = n < 256 ? 256 : n;
    if (!dmalloc((void **)&s->token_out, (size_t)cap * 4)) return false;
    s->token_capacity = cap;
    return true;
}

// The n tokens of a device loop to the host, and the loop's error flag (reported and cleared):
// 0, or -1.
static int copy_tokens_out(const Config *cfg, RunState *s, int n, int *out_tokens) {
    if (!HIP_OK(hipMemcpyAsync(out_tokens, s->token_out, (size_t)n * 4, hipMemcpyDeviceToHost,
                               s->stream)) ||
        !HIP_OK(hipStreamSynchronize(s->stream)))
        return -1;
    return check_step_error(cfg, s) ? 0 : -1;
}

extern "C" int generate_greedy(const Config *cfg, const Weights *w, RunState *s, int token,
                               int pos, int n_steps, int *out_tokens) {
    if (n_steps <= 0) return 0;
    if (!check_token_pos(cfg, s, token, pos)) return -1;
    if (pos + n_steps > s->max_seq) {
        llm_fail("generate_greedy: %d steps from position %d pass the kv cache size %d", n_steps,
                 pos, s->max_seq);
        return -1;
    }
    if (dump_enabled()) {
        // While dumping, every step runs eagerly (dumps synchronise and copy to the host, which
        // a captured graph or the persistent kernel cannot do): one forward + argmax + advance
        // per token, writing one row per tensor and position.
        if (!ensure_token_capacity(s, n_steps)) return -1;
        set_token_pos_kernel<<<1, 64, 0, s->stream>>>(s->next_token, s->pos, token, pos);
        set_token_pos_kernel<<<1, 64, 0, s->stream>>>(s->error_flag, s->pos_base, 0, pos);
        if (!LAUNCH_OK()) return -1;
        for (int i = 0; i < n_steps; i++) {
            if (!forward_kernels(cfg, w, s)) return -1;
            argmax_into_next(cfg, s);
            advance_kernel<<<1, 64, 0, s->stream>>>(s->pos, s->next_token, s->token_out,
                                                     s->pos_base, s->token_capacity);
            if (!LAUNCH_OK()) return -1;
        }
        s->next_token_valid = 1;
        return copy_tokens_out(cfg, s, n_steps, out_tokens);
    }
    if (!ensure_token_capacity(s, n_steps)) return -1;
    // the tokens at positions below the switch in one launch of the persistent kernel, the
    // rest by the loop graph, which continues from the token and position that launch left
    // on the device (both steps compute the same bits)
    const int n_kernel = !persistent_at(s, pos) ? 0
                         : pos + n_steps <= s->step_switch_pos ? n_steps
                                                               : s->step_switch_pos - pos;
    if (n_kernel < n_steps && !s->loop_graph) {
        StepCtx c{cfg, w, s};
        if (!capture(s->stream, &s->loop_graph, loop_body, &c)) return -1;
    }
    set_token_pos_kernel<<<1, 64, 0, s->stream>>>(s->next_token, s->pos, token, pos);
    set_token_pos_kernel<<<1, 64, 0, s->stream>>>(s->error_flag, s->pos_base, 0, pos);
    if (!LAUNCH_OK()) return -1;
    if (n_kernel > 0) {
        // one launch decodes every token below the split attention's first position, one more
        // every token from there to the switch (it continues from the token and position the
        // first left on the device)
        const int sp = split_from(s);
        if (sp < 0) return -1;
        const int n_heads = pos >= sp ? 0 : pos + n_kernel <= sp ? n_kernel : sp - pos;
        StepArgs a = step_args(cfg, w, s, 1);
        if (n_heads > 0) {
            a.n_tokens = n_heads;
            if (!step_kernel_launch(cfg, a, false, s->step_grid, s->stream)) return -1;
        }
        if (n_heads < n_kernel) {
            a.n_tokens = n_kernel - n_heads;
            if (!step_kernel_launch(cfg, a, true, s->step_grid, s->stream)) return -1;
        }
    }
    for (int i = n_kernel; i < n_steps; i++)
        if (!HIP_OK(hipGraphLaunch(s->loop_graph, s->stream))) return -1;
    s->next_token_valid = 1;
    return copy_tokens_out(cfg, s, n_steps, out_tokens);
}

// ------------------------------------------------------------------------------------------
// seeded synthetic weights
// ------------------------------------------------------------------------------------------

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Element pair (2i, 2i+1) of stream `sid` comes from two 53-bit uniforms of a counter-based
// SplitMix64 sequence through the Box-Muller transform in double.
__global__ __launch_bounds__(256) void synth_kernel(bf16 *out, size_t n, uint64_t seed,
                                                    uint64_t sid, float mean, float std) {
    const uint64_t key = splitmix64(seed ^ splitmix64(sid + 0x632BE59BD9B4E019ull));
    const size_t pairs = (n + 1) / 2;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < pairs;
         i += (size_t)gridDim.x * blockDim.x) {
        const uint64_t a = splitmix64(key + 2 * i), b = splitmix64(key + 2 * i + 1);
        const double u1 = (double)((a >> 11) + 1) * 0x1.0p-53;  // (0, 1]
        const double u2 = (double)(b >> 11) * 0x1.0p-53;        // [0, 1)
        const double r = sqrt(-2.0 * log(u1));
        double sv, cv;
        sincospi(2.0 * u2, &sv, &cv);
        out[2 * i] = (bf16)f2bf((float)(mean + std * r * cv));
        if (2 * i + 1 < n) out[2 * i + 1] = (bf16)f2bf((float)(mean + std * r * sv));
    }
}

extern "C" void synth_fill(bf16 *dev, size_t n, uint64_t seed, uint64_t stream_id, float mean,
                           float std, hipStream_t stream) {
    if (n == 0) return;
    size_t blocks = ((n + 1) / 2 + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    synth_kernel<<<(unsigned)blocks, 256, 0, stream>>>(dev, n, seed, stream_id, mean, std);
    LAUNCH_OK();
}

struct SynthTensor {
    char name[96];
    size_t numel;
    int norm;  // gamma: 1 + N(0, gamma_std)
};

static int synth_tensor_list(const Config *cfg, SynthTensor *list) {
    const int H = cfg->hidden_size, D = cfg->head_dim, I = cfg->intermediate_size;
    const size_t q_dim = (size_t)cfg->n_heads * D, kv_dim = (size_t)cfg->n_kv_heads * D;
    int n = 0;
    auto add = [&](const char *name, size_t numel, int norm) {
        if (list) {
            snprintf(list[n].name, sizeof list[n].name, "%s", name);
            list[n].numel = numel;
            list[n].norm = norm;
        }
        n++;
    };
    char name[96];
    add("model.embed_tokens.weight", (size_t)cfg->vocab_size * H, 0);
    for (int l = 0; l < cfg->n_layers; l++) {
        const struct {
            const char *suffix;
            size_t numel;
            int norm;
        } parts[] = {{"input_layernorm.weight", (size_t)H, 1},
                     {"self_attn.q_proj.weight", q_dim * H, 0},
                     {"self_attn.k_proj.weight", kv_dim * H, 0},
                     {"self_attn.v_proj.weight", kv_dim * H, 0},
                     {"self_attn.q_norm.weight", (size_t)D, 1},
                     {"self_attn.k_norm.weight", (size_t)D, 1},
                     {"self_attn.o_proj.weight", (size_t)H * q_dim, 0},
                     {"post_attention_layernorm.weight", (size_t)H, 1},
                     {"mlp.gate_proj.weight", (size_t)I * H, 0},
                     {"mlp.up_proj.weight", (size_t)I * H, 0},
                     {"mlp.down_proj.weight", (size_t)H * I, 0}};
        for (const auto &p : parts) {
            snprintf(name, sizeof name, "model.layers.%d.%s", l, p.suffix);
            add(name, p.numel, p.norm);
        }
    }
    add("model.norm.weight", (size_t)H, 1);
    return n;
}

extern "C" void synth_weights(const Config *cfg, Weights *w, uint64_t seed, float std,
                              float gamma_std) {
    memset(w, 0, sizeof *w);
    const int n = synth_tensor_list(cfg, nullptr);
    SynthTensor *list = (SynthTensor *)calloc(n, sizeof(SynthTensor));
    w->tensors = (TensorRef *)calloc(n, sizeof(TensorRef));
    w->layers = (LayerWeights *)calloc(cfg->n_layers, sizeof(LayerWeights));
    if (!list || !w->tensors || !w->layers) {
        free(list);
        llm_fail("synth_weights: out of memory");
        return;
    }
    synth_tensor_list(cfg, list);
    // every tensor on a 256-byte boundary inside one allocation
    size_t total = 0;
    for (int i = 0; i < n; i++) total += (list[i].numel * 2 + 255) & ~(size_t)255;
    char *base = nullptr;
    if (!HIP_OK(hipMalloc((void **)&base, total))) {
        free(list);
        return;
    }
    size_t off = 0;
    for (int i = 0; i < n; i++) {
        bf16 *p = (bf16 *)(base + off);
        off += (list[i].numel * 2 + 255) & ~(size_t)255;
        synth_fill(p, list[i].numel, seed, (uint64_t)i, list[i].norm ? 1.0f : 0.0f,
                   list[i].norm ? gamma_std : std, nullptr);
        TensorRef *t = &w->tensors[i];
        snprintf(t->name, sizeof t->name, "%s", list[i].name);
        t->data = p;
        t->numel = list[i].numel;
    }
    w->n_tensors = n;
    w->embed = w->tensors[0].data;
    for (int l = 0; l < cfg->n_layers; l++) {
        const TensorRef *t = &w->tensors[1 + 11 * l];
        LayerWeights *L = &w->layers[l];
        L->attn_norm = t[0].data;
        L->wq = t[1].data;
        L->wk = t[2].data;
        L->wv = t[3].data;
        L->q_norm = t[4].data;
        L->k_norm = t[5].data;
        L->wo = t[6].data;
        L->mlp_norm = t[7].data;
        L->w_gate = t[8].data;
        L->w_up = t[9].data;
        L->w_down = t[10].data;
    }
    w->final_norm = w->tensors[n - 1].data;
    w->lm_head = w->embed;
    w->gpu_buffers[0] = base;
    w->n_buffers = 1;
    w->gpu_bytes = total;
    free(list);
    HIP_OK(hipDeviceSynchronize());
}
