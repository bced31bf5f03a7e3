// The whole decode step as one persistent kernel for gfx950: one workgroup of 8 waves per CU,
// all resident at once (the grid is the CU count, one workgroup per CU), with no grid barrier. Each phase
// computes exactly what the standalone kernels compute (same per-row, per-head and per-block
// arithmetic), so the step is bit-identical to the multi-kernel step it replaces
// (src/forward.cu:118-193 order):
//
//   per layer:  rmsnorm + q/k/v rows | QK-norm + RoPE + KV write + attention, one workgroup
//               per query head | o rows + residual | rmsnorm + gate/up rows + SwiGLU |
//               down rows + residual
//   final:      rmsnorm + LM-head rows + per-workgroup argmax, published as tagged words;
//               one workgroup polls them, reduces the argmax, records the token, advances the
//               position and publishes the token to the others
//
// Activations cross workgroups (and XCDs, whose L2s are not coherent) as tagged vectors:
// element i is the 32-bit word (bf16 bits << 16) | tag, stored and loaded with agent-scope
// atomics (global_store/load ... sc1). The tag names the phase that wrote the value, so a
// consumer workgroup polls exactly the words it needs until every tag is the expected one,
// copying them into LDS; the data is its own ready signal and no phase waits for a barrier,
// for its stores to complete, or for workgroups it does not depend on. A writer of a vector's
// next version always depends (through the phases between) on every reader of its previous
// version, so no value is overwritten before it has been read. Weights and the KV history are
// read with plain non-temporal loads, requested a phase or more ahead. Every wait is bounded:
// on timeout the step sets an error flag and later waits give up at once, so the grid drains.
#include <limits.h>
#include <string.h>

#include <type_traits>

#include "common.h"
#include "internal.h"
#include "rope.h"
#include "step.h"

using namespace llm;

namespace {

constexpr int WAVES = 8;                   // waves per workgroup
constexpr int THREADS = 64 * WAVES;
constexpr long long SPIN_LIMIT = 1 << 22;  // polls before a wait gives up (~ seconds)
// Pause between polls (s_sleep units of 64 clocks). None: at 0.6B polling without a pause
// measured 0.3% faster than 64 clocks and 1% faster than 128.
constexpr int POLL_SLEEP = 0;
constexpr int PHASES = 5;                  // tagged vectors written per layer

// ---------------------------------------------------------------- coherent access

__device__ __forceinline__ uint64_t ld_coh64(const void *p) {
    return __hip_atomic_load(gptr((uint64_t *)p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- arguments

typedef const __attribute__((address_space(4))) StepArgs KArgs;
typedef const __attribute__((address_space(4))) LayerDev KLayer;

// The launch's arguments, read where they are used: scalar loads from the kernel-argument
// segment (StepArgs is the only explicit argument, at offset 0). The empty asm makes the
// segment pointer opaque, so the loads stay at their uses instead of being hoisted to the
// kernel entry, where dozens of pointers would occupy SGPRs for the whole step.
// The segment pointer exists only in the kernel function itself (in a called function the
// builtin yields 0), so every function that calls kargs() is force-inlined and the compiled
// step kernel must contain no calls.
__device__ __forceinline__ KArgs &kargs() {
    auto p = __builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(p));
    return *(KArgs *)p;
}

// A uniform value the compiler must treat as recomputed here: what is derived from it inside
// the layer loop (per-slot masks, offsets) is then recomputed per layer instead of being
// hoisted out of the loop and held in registers for the whole step.
__device__ __forceinline__ int opaque(int v) {
    asm volatile("" : "+s"(v));
    return v;
}

// Layer l's weight pointers. The table is written before the launch and never during it, so
// it is read through the constant address space (scalar loads), at each use.
__device__ __forceinline__ KLayer &klayer(KArgs &a, int l) {
    KLayer *t = (KLayer *)a.layers + l;
    asm volatile("" : "+s"(t));
    return *t;
}

// ---------------------------------------------------------------- tagged vectors

// Tag of the seq-th tagged phase since the workspace was zeroed: 1..65535, never 0 (the
// zeroed state). A word is rewritten every layer, so values 65535 phases apart never meet.
__device__ __forceinline__ uint32_t tag_of(unsigned seq) { return 1u + seq % 65535u; }

__device__ __forceinline__ void put_tagged(uint32_t *v, int i, uint32_t bits, uint32_t tag) {
    __hip_atomic_store(gptr(v + i), (bits << 16) | tag, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Element i of a replicated tagged vector of n elements, into each of its first COPIES copies
// (at most STEP_REPLICAS; the workgroups read only those).
template <int N, int COPIES>
__device__ __forceinline__ void put_tagged_all(uint32_t *v, int i, uint32_t bits, uint32_t tag) {
    static_assert(COPIES >= 1 && COPIES <= STEP_REPLICAS, "copies");
    constexpr int STRIDE = (int)step_replica_stride(N);
#pragma unroll
    for (int q = 0; q < COPIES; q++) put_tagged(v + q * STRIDE, i, bits, tag);
}

// Rows [r0, r1) of a replicated tagged vector, staged in LDS as tagged words by the waves that
// computed them, written to every copy by one wave: consecutive lanes on consecutive words of a
// copy, so each copy's run of rows goes out in one store instruction instead of one single-lane
// store per row and copy.
template <int N, int COPIES>
__device__ __forceinline__ void publish_rows(uint32_t *v, const uint32_t *stage, int r0, int r1) {
    static_assert(COPIES >= 1 && COPIES <= STEP_REPLICAS, "copies");
    constexpr int STRIDE = (int)step_replica_stride(N);
    const int n = r1 - r0;
    for (int idx = tid_x() & 63; idx < n * COPIES; idx += 64) {
        const int q = idx / n, r = idx - q * n;
        __hip_atomic_store(gptr(v + q * STRIDE + r0 + r), stage[r], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The copy of a replicated tagged vector of n elements, written in COPIES copies, that this
// workgroup reads.
template <int N, int COPIES>
__device__ __forceinline__ const uint32_t *my_copy(const uint32_t *v) {
    return v + (blockIdx.x % COPIES) * (int)step_replica_stride(N);
}

// Polls the 64-bit words src(p) (two tagged elements each) for pairs p < PAIRS until both tags
// equal `tag`, and writes the bf16 pairs to dst[p] (LDS). With ONE_WAVE only wave 0 polls (pair
// p = lane + 64 j): a wave with weight loads in flight would see the data only after them, since
// vector loads complete in order, so the workgroups that prefetch weights leave polling to a
// wave that has none. Otherwise every thread polls (p = threadIdx.x + THREADS j). The workgroup
// syncs before (the previous contents of dst have been read) and after. Bounded: once the error
// flag is set (an earlier error, or another wait that timed out), or when its own polls run out
// (the flag then becomes 2 unless already set), it goes on with what it read. With IDLE_OUT,
// waves wholly past the pairs (a wave-uniform test) stay out of the poll instead of re-reading
// the last pair.
template <int PAIRS, bool ONE_WAVE, bool IDLE_OUT = false, class Src>
__device__ __forceinline__ void stage_pairs(Src src, uint32_t tag, uint32_t *dst, int *err) {
    constexpr int STEP = ONE_WAVE ? 64 : THREADS;
    constexpr int P = (PAIRS + STEP - 1) / STEP;
    __syncthreads();
    if (ONE_WAVE ? wave_id() == 0 : !IDLE_OUT || wave_id() * 64 < PAIRS) {
        const int t0 = ONE_WAVE ? (tid_x() & 63) : (int)threadIdx.x;
        // Every lane issues every poll (a lane past the pairs re-reads the last one), so no
        // branch surrounds a load.
        uint64_t w[P];
        long long spins = 0;
        for (;;) {
            bool fresh = true;
#pragma unroll
            for (int j = 0; j < P; j++) {
                w[j] = ld_coh64(src(min(t0 + STEP * j, PAIRS - 1)));
                fresh &= (uint32_t)(w[j] & 0xffffu) == tag &&
                         (uint32_t)((w[j] >> 32) & 0xffffu) == tag;
            }
            if (fresh) break;
            if ((++spins & 63) == 0 && wait_gives_up(spins, SPIN_LIMIT, err)) break;
            if constexpr (POLL_SLEEP > 0) __builtin_amdgcn_s_sleep(POLL_SLEEP);
        }
#pragma unroll
        for (int j = 0; j < P; j++) {
            const int p = t0 + STEP * j;
            if (p < PAIRS)
                dst[p] = (uint32_t)((w[j] >> 16) & 0xffffu) | ((uint32_t)(w[j] >> 48) << 16);
        }
    }
    __syncthreads();
}

// Elements [0, N) of tagged vector v into LDS as plain bf16 (N even).
template <int N, bool ONE_WAVE>
__device__ __forceinline__ void stage_vector(const uint32_t *v, uint32_t tag, uint32_t *dst,
                                             int *err) {
    stage_pairs<N / 2, ONE_WAVE>([=](int p) { return v + 2 * p; }, tag, dst, err);
}

// The embedding row as the first layer's input (read-only: nothing to wait for).
template <int N>
__device__ __forceinline__ void stage_plain(const bf16 *row, uint32_t *dst) {
    __syncthreads();
    for (int c = threadIdx.x; c < N / 8; c += THREADS) ((u32x4 *)dst)[c] = ld16(row + 8 * c);
    __syncthreads();
}

// ---------------------------------------------------------------- wave building blocks

// The input vector of a GEMV as this lane's chunks (chunk lane + 64k), from LDS.
template <int NC>
__device__ __forceinline__ void lds_chunks(const uint32_t *vec, u32x4 (&out)[NC]) {
    const int lane = tid_x() & 63;
#pragma unroll
    for (int k = 0; k < NC; k++) out[k] = ((const u32x4 *)vec)[lane + 64 * k];
}

// Norm weights of the elements this thread normalises in wg_rmsnorm: i = threadIdx.x +
// THREADS * j.
template <int N>
struct NormW {
    static constexpr int E = (N + THREADS - 1) / THREADS;
    // the raw bf16 bits, widened where they are used: converting at the load would make the
    // wave wait for this load, and with it for every weight request issued before it
    uint32_t w[E];
    __device__ __forceinline__ void load(const bf16 *g) {
        const uint16_t *g16 = (const uint16_t *)g;
#pragma unroll
        for (int j = 0; j < E; j++) {
            const int i = threadIdx.x + THREADS * j;
            if constexpr (N % THREADS == 0) w[j] = gptr(g16)[i];
            else w[j] = i < N ? (uint32_t)gptr(g16)[i] : 0u;
        }
    }
    __device__ __forceinline__ float operator[](int j) const { return bf2f((bf16)w[j]); }
};

// RMSNorm of the staged vector (LDS, bf16), in place, once per workgroup with the arithmetic of
// rmsnorm_wave_kernel: wave 0 forms the sum of squares (lane l: chunks l + 64k in order, then the
// wave tree), every thread then normalises its elements as bf16(bf16(x * inv) * gamma). Ends with
// a workgroup sync.
template <int N>
__device__ __forceinline__ void wg_rmsnorm(uint32_t *vec, const NormW<N> &nw, float eps,
                                           float *inv_slot) {
    constexpr int NC = N / 512;
    if (wave_id() == 0) {
        u32x4 x[NC];
        lds_chunks<NC>(vec, x);
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < NC; k++) acc = dot8(x[k], x[k], acc);
        const float total = wave_sum(acc);
        if ((tid_x() & 63) == 0) *inv_slot = 1.0f / sqrtf(total / (float)N + eps);
    }
    __syncthreads();
    const float inv = *inv_slot;
    uint16_t *v16 = (uint16_t *)vec;
#pragma unroll
    for (int j = 0; j < NormW<N>::E; j++) {
        const int i = threadIdx.x + THREADS * j;
        if (i < N) v16[i] = (uint16_t)f2bf(round_bf(bf2f((bf16)v16[i]) * inv) * nw[j]);
    }
    __syncthreads();
}

// B rows of NC chunks each, held in registers: lane l has chunk l + 64k of every row. `rowp`
// maps a row index to its data, so a batch can straddle the q/k/v matrices.
// Declare them value-initialised (`Rows<..> r{};`) inside loops: a batch loaded only on some
// paths is otherwise carried from the previous iteration (in SSA form a variable declared in a
// loop body is one value across iterations), which holds its registers through the whole
// loop. The zero fill survives only on the paths that do not load.
template <int NC, int B>
struct Rows {
    u32x4 w[B][NC];
    // Rows at or past r1 (a short last batch, or a wave without rows: r = r1) read as zeros
    // with no memory access: each row is a buffer whose size is zero when the row is absent,
    // and buffer loads past the end return 0. The request is thus made on every path, with no
    // branch around it (see the step kernel).
    template <class RowP>
    __device__ __forceinline__ void load(RowP rowp, int r, int r1) {
        const int lane = tid_x() & 63;
#pragma unroll
        for (int i = 0; i < B; i++) {
            const bool in = r + i < r1;
            const bf16 *row = rowp(in ? r + i : 0);
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                (void *)row, (short)0, in ? NC * 1024 : 0, BUFFER_FLAGS);
#pragma unroll
            for (int k = 0; k < NC; k++)
                w[i][k] = __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * (lane + 64 * k), 0,
                                                                BUFFER_NT);
        }
    }
};

// The staged input vector read from LDS chunk by chunk where a dot product uses it (lane l's
// chunk k: 16 bytes at l + 64 k, as lds_chunks loads them), instead of NC registers held for
// the whole phase: for long rows (the down rows' 6144 or 9728 columns) those registers would
// otherwise spill.
struct LdsX {
    const u32x4 *v;
    __device__ __forceinline__ u32x4 operator[](int k) const { return v[(tid_x() & 63) + 64 * k]; }
};

// The B row sums of a batch against xin (gemv_kernel arithmetic: per-lane fma over the chunks
// in order, then the wave tree); lane l gets row scatter_row<B>(l) of the batch. BANK: the
// reduce-scatter's xor-4 and xor-8 steps without per-lane selects (the split instance: 0.6B
// after 8192 positions 1215 -> 1227 tokens/s; the one-head-per-workgroup instance at 0.6B
// measured 0.3% slower with it, at 1.7B and 4B the same).
template <bool BANK = false, int NC, int B, class X>
__device__ __forceinline__ float batch_sums(const Rows<NC, B> &b, const X &xin) {
    float part[B];
#pragma unroll
    for (int i = 0; i < B; i++) part[i] = 0.0f;
    if constexpr (std::is_same_v<X, LdsX>) {
        // each chunk read from LDS once for the batch's rows (same per-row order)
#pragma unroll
        for (int k = 0; k < NC; k++) {
            const u32x4 xk = xin[k];
#pragma unroll
            for (int i = 0; i < B; i++) part[i] = dot8(b.w[i][k], xk, part[i]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < B; i++)
#pragma unroll
            for (int k = 0; k < NC; k++) part[i] = dot8(b.w[i][k], xin[k], part[i]);
    }
    return wave_sum_scatter<B, false, BANK>(part);
}


// Rows [r0, r1) against xin, B rows per batch, the first batch already in `cur` (requested a
// phase ahead). With STREAM the next batch is requested before the current one is reduced
// (two batches in flight), else after. epi(row, sum, v) runs in one of lanes 0..B-1 and
// returns bf16 bits; v is `own` of lane row - r0. `own` is a per-row value the wave keeps
// (lane j: row r0 + j, at most 64 rows): with KEEP it is replaced by epi's result for the row,
// so a wave carries the residual rows it updates from one phase to the next. Lane
// scatter_row<B>(k) computes batch row k, and scatter_row<B> is its own inverse.
template <int NC, int B, bool STREAM, bool KEEP = false, bool BANK = false, class RowP, class X,
          class Epi>
__device__ __forceinline__ void wave_gemv(RowP rowp, int r0, int r1, const X &xin,
                                          Rows<NC, B> &cur, Epi epi, uint32_t *own = nullptr) {
    const int lane = tid_x() & 63;
    auto finish = [&](float t, int r) {
        const int row = r + scatter_row<B>(lane);
        const uint32_t v = KEEP ? (uint32_t)__shfl((int)*own, min(row - r0, 63)) : 0u;
        uint32_t res = 0;
        if (lane < B && row < r1) res = epi(row, t, v);
        if constexpr (KEEP) {
            const int k = r0 + lane - r;  // batch index of this lane's own row
            const bool in = k >= 0 && k < B && r0 + lane < r1;
            const uint32_t got = (uint32_t)__shfl((int)res, in ? scatter_row<B>(k) : 0);
            if (in) *own = got;
        }
    };
    if constexpr (STREAM) {
        Rows<NC, B> nxt;
        for (int r = r0; r < r1; r += 2 * B) {
            if (r + B < r1) nxt.load(rowp, r + B, r1);
            finish(batch_sums<BANK>(cur, xin), r);
            if (r + B >= r1) break;
            if (r + 2 * B < r1) cur.load(rowp, r + 2 * B, r1);
            finish(batch_sums<BANK>(nxt, xin), r + B);
        }
    } else {
        // the first batch outside the loop: a loop head would merge this batch's (long
        // complete) registers with the loads of the loop's back edge, and the wait placed there
        // would then also wait for every request issued since the prefetch
        if (r0 < r1) finish(batch_sums<BANK>(cur, xin), r0);
        for (int r = r0 + B; r < r1; r += B) {
            cur.load(rowp, r, r1);
            finish(batch_sums<BANK>(cur, xin), r);
        }
    }
}

// gate and up rows together (gate_up_kernel arithmetic); first batch preloaded. With STREAM the
// next batch is requested before the current one is computed (two batches in flight), else
// after.
template <int NC, int B, bool STREAM, bool BANK = false, class Epi>
__device__ __forceinline__ void wave_gemv2(const bf16 *Wg, const bf16 *Wu, int r0, int r1,
                                           const u32x4 (&xin)[NC], Rows<NC, B> &gb,
                                           Rows<NC, B> &ub, Epi epi) {
    const int lane = tid_x() & 63;
    constexpr int COLS = 512 * NC;
    auto g_row = [&](int rr) { return Wg + (size_t)rr * COLS; };
    auto u_row = [&](int rr) { return Wu + (size_t)rr * COLS; };
    auto finish = [&](const Rows<NC, B> &g, const Rows<NC, B> &u, int r) {
        const float tg = batch_sums<BANK>(g, xin), tu = batch_sums<BANK>(u, xin);
        const int row = r + scatter_row<B>(lane);
        if (lane < B && row < r1) epi(row, tg, tu);
    };
    if constexpr (STREAM) {
        Rows<NC, B> gn, un;
        for (int r = r0; r < r1; r += 2 * B) {
            if (r + B < r1) {
                gn.load(g_row, r + B, r1);
                un.load(u_row, r + B, r1);
            }
            finish(gb, ub, r);
            if (r + B >= r1) break;
            if (r + 2 * B < r1) {
                gb.load(g_row, r + 2 * B, r1);
                ub.load(u_row, r + 2 * B, r1);
            }
            finish(gn, un, r + B);
        }
    } else {
        if (r0 < r1) finish(gb, ub, r0);  // outside the loop, as in wave_gemv
        for (int r = r0 + B; r < r1; r += B) {
            gb.load(g_row, r, r1);
            ub.load(u_row, r, r1);
            finish(gb, ub, r);
        }
    }
}

// Optional wall-clock stamps (trace != NULL). stamp: by thread 0 of the first matrix
// workgroup, at index i. stamp_wg: for layer TRACE_LAYER only, by thread 0 of every
// workgroup, at index 4 * n_layers + 3 + 8 * workgroup + k, with k = 2 * phase (input
// staged) or 2 * phase + 1 (results stored); phase 0 is q/k/v (or a head's attention), then
// o, gate/up, down.
constexpr int TRACE_LAYER = 1;
// Only the first token of a launch is traced (step 0).
template <class S>
__device__ __forceinline__ void stamp(int i, int step) {
    if (step == 0 && blockIdx.x == S::HQ && threadIdx.x == 0) {
        long long *trace = kargs().trace;
        if (trace) gptr(trace)[i] = wall_clock64();
    }
}
__device__ __forceinline__ void stamp_wg(int l, int n_layers, int k, int step) {
    if (step == 0 && l == TRACE_LAYER) {
        long long *trace = kargs().trace;
        if (trace) {
            if (k & 1) __syncthreads();  // "stored": when every wave has issued its stores
            if (threadIdx.x == 0) gptr(trace)[4 * n_layers + 3 + 8 * blockIdx.x + k] = wall_clock64();
        }
    }
}

// ---------------------------------------------------------------- attention

constexpr int PV_ROUND = 4;     // 64-position blocks per PV round (two per wave)
constexpr int SCORE_LOADS = 8;  // keys per lane per scores round (8 * 4 * WAVES positions)

// History keys and values (positions < pos, written by earlier steps) of the first scores and
// PV rounds of one head, requested before its q/k/v are polled, and this lane's RoPE table entry
// at pos. Slots at or beyond pos hold zeros; attention_head substitutes the current position's
// key and value.
struct AttnPrefetch {
    u32x4 k[SCORE_LOADS];
    u32x4 v[PV_ROUND / 2][4];
    float cs[1], sn[1];  // RoPE table entry `lane` (rotation pair lane, lane + 64)
    uint32_t w0, w1;     // waves 0/1: q/k norm weights (bf16 bits) of elements lane, lane + 64
};

template <class S>
struct AttnSmem {
    static constexpr int D = 128;
    uint32_t raw[3][D / 2];         // the head's q, k and v rows as polled (bf16 pairs)
    u32x4 q[D / 8];                 // roped query head
    u32x4 k[D / 8];                 // roped key of the current position
    u32x4 v[D / 8];                 // value of the current position
    float sc[S::NMAX];              // scores, then probabilities
    float st[S::NMAX / 64][2];      // block max, block sum
    float gm[2];                    // global max, sum
    float quarter[PV_ROUND][4][D];  // PV partial of each (block, quarter) of a round
};

// One lane's 16 bytes of a KV-cache row. Rows written earlier in this launch (t >= pos0) were
// stored by another workgroup, possibly on another XCD, so they are read coherently; older rows
// come from earlier launches and stream non-temporally.
__device__ __forceinline__ u32x4 ld_kv(const bf16 *p, int t, int pos0) {
    if (t >= pos0) {
        const uint64_t a = ld_coh64(p), b = ld_coh64((const char *)p + 8);
        return u32x4{(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)};
    }
    return ld16_nt(p);
}
__device__ __forceinline__ void st_kv(bf16 *p, uint32_t v) {
    __hip_atomic_store(gptr((uint16_t *)p), (uint16_t)v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Position of key slot u of this lane in the scores round starting at `base`, and of value
// slot (j, it) in the PV round starting at block c0 (16 lanes per position, 8 waves).
__device__ __forceinline__ int key_slot(int base, int u) {
    return base + u * 4 * WAVES + (tid_x() >> 6) * 4 + ((tid_x() & 63) >> 4);
}
__device__ __forceinline__ int value_slot(int c0, int j, int it) {
    const int w = tid_x() >> 6;
    return (c0 + (w >> 2) + 2 * j) * 64 + (w & 3) * 16 + it * 4 + ((tid_x() & 63) >> 4);
}

// QK-RMSNorm + RoPE of one 128-element head by one wave (qk_norm_rope_kernel arithmetic): lane
// i holds elements i and i + 64 of x16 (bf16 bits), the pair RoPE rotates with table entry i
// (c, sn), w0 / w1 the norm weights of those elements; lanes 0-7 form the sum of squares in the
// order of the standalone kernel (elements 8L.. then 64+8L.., then the 8-lane tree). oa / ob:
// the rotated elements i and i + 64 (bf16 bits).
__device__ __forceinline__ void wave_qk_norm_rope(const uint16_t *x16, uint32_t w0, uint32_t w1,
                                                  float c, float sn, float eps, uint32_t &oa,
                                                  uint32_t &ob) {
    constexpr int D = 128;
    const int lane = tid_x() & 63;
    const uint32_t xi = x16[lane], xj = x16[64 + lane];
    float acc = 0.0f;
    {
        const int L8 = (lane & 7) * 8;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float v = bf2f((bf16)x16[L8 + e]);
            acc = fmaf(v, v, acc);
        }
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float v = bf2f((bf16)x16[64 + L8 + e]);
            acc = fmaf(v, v, acc);
        }
    }
    const float total = __uint_as_float(
        __builtin_amdgcn_readfirstlane(__float_as_uint(group_sum<8>(acc))));
    const float inv = 1.0f / sqrtf(total / (float)D + eps);
    const float ya = round_bf(round_bf(bf2f((bf16)xi) * inv) * bf2f((bf16)w0));
    const float yb = round_bf(round_bf(bf2f((bf16)xj) * inv) * bf2f((bf16)w1));
    const float a_cos = round_bf(ya * c), b_sin = round_bf(yb * sn);
    const float b_cos = round_bf(yb * c), a_sin = round_bf(ya * sn);
    oa = f2bf(a_cos - b_sin);
    ob = f2bf(b_cos + a_sin);
}

template <class S>
__device__ __forceinline__ void attention_prefetch(KArgs &a, KLayer &L, int h, int pos, int pos0,
                                                   int layer, AttnPrefetch &p) {
    constexpr int D = 128, REP = S::HQ / S::HKV, KVD = S::HKV * D;
    const int g = h / REP, Lp = tid_x() & 15;
    {
        const int lane = tid_x() & 63;
        const uint16_t *nw = (const uint16_t *)(wave_id() == 1 ? L.k_norm : L.q_norm);
        p.w0 = gptr(nw)[lane];
        p.w1 = gptr(nw)[64 + lane];
    }
    const bf16 *kc = a.key_cache + (size_t)layer * a.max_seq * KVD + g * D + 8 * Lp;
#pragma unroll
    for (int u = 0; u < SCORE_LOADS; u++) {
        const int t = key_slot(0, u);
        p.k[u] = t < pos ? ld_kv(kc + (size_t)t * KVD, t, pos0) : u32x4{0, 0, 0, 0};
    }
    const bf16 *vc = a.value_cache + (size_t)layer * a.max_seq * KVD + g * D + 8 * Lp;
#pragma unroll
    for (int j = 0; j < PV_ROUND / 2; j++)
#pragma unroll
        for (int it = 0; it < 4; it++) {
            const int t = value_slot(0, j, it);
            p.v[j][it] = t < pos ? ld_kv(vc + (size_t)t * KVD, t, pos0) : u32x4{0, 0, 0, 0};
        }
    rope_table<D>(pos, a.inv_freq, p.cs, p.sn);
    // computed here, before the workgroup waits for its q/k/v, not sunk to the first use
    asm volatile("" : "+v"(p.cs[0]), "+v"(p.sn[0]));
}

// One query head's attention at `pos` (attn_scores/pv/combine arithmetic, one workgroup): the
// head's q and its group's k and v rows are polled (tag `tag_in`) into LDS; wave 0 normalises
// and rotates q and k (the workgroup that owns the group writes k' and v into the cache);
// then scores, block statistics, the global max/sum, probabilities, PV per 64-position block in
// four quarters, and the in-order combine; the head's output is published with `tag_out`.
template <class S>
__device__ __forceinline__ void attention_head(KArgs &a, KLayer &L, int h, int pos, int pos0,
                                               int layer, AttnSmem<S> &sm, AttnPrefetch &pre,
                                               uint32_t tag_in, uint32_t tag_out, int n_layers,
                                               int step, float eps) {
    constexpr int D = 128, REP = S::HQ / S::HKV, QD = S::HQ * D, KVD = S::HKV * D;
    const int lane = tid_x() & 63, w = wave_id();
    const int g = h / REP;
    const bool owner = (h % REP) == 0;  // writes k', v into the cache
    bf16 *kc = a.key_cache + (size_t)layer * a.max_seq * KVD;
    bf16 *vc = a.value_cache + (size_t)layer * a.max_seq * KVD;
    const int n = pos + 1;
    const int nb = (n + 63) / 64;
    const u32x4 zero{0, 0, 0, 0};

    {
        const uint32_t *qkv = a.tqkv;
        const int qo = h * D, ko = QD + g * D, vo = QD + KVD + g * D;
        // the waves past the 192 pairs stay out of the poll where two query heads share a kv
        // head (0.6B 2436.8 -> 2446.0 tokens/s, 1.7B 1140.6 -> 1145.3); at 4B they poll too
        // (612.8 against 599.6 without them)
        stage_pairs<3 * D / 2, false, S::H <= 2048>(
            [=](int p) {
                // segment p / 64: q, k or v (arithmetic, not a select chain, which the compiler
                // turns into a table in scratch memory)
                const int seg = p / (D / 2), i = 2 * (p % (D / 2));
                return qkv + qo + (seg >= 1) * (ko - qo) + (seg >= 2) * (vo - ko) + i;
            },
            tag_in, &sm.raw[0][0], a.error_flag);
    }
    stamp_wg(layer, n_layers, 0, step);

    // history values of a PV round (the first one prefetched)
    u32x4 vv[PV_ROUND / 2][4];
#pragma unroll
    for (int j = 0; j < PV_ROUND / 2; j++)
#pragma unroll
        for (int it = 0; it < 4; it++) vv[j][it] = pre.v[j][it];
    auto load_v = [&](int c0) {
        const int Lq = tid_x() & 15;
#pragma unroll
        for (int j = 0; j < PV_ROUND / 2; j++)
#pragma unroll
            for (int it = 0; it < 4; it++) {
                const int t = value_slot(c0, j, it);
                vv[j][it] = t < pos ? ld_kv(vc + (size_t)t * KVD + g * D + 8 * Lq, t, pos0) : zero;
            }
    };

    // QK-norm + RoPE (qk_norm_rope_kernel arithmetic): wave 0 the query head, wave 1 the key
    // head, wave 2 copies the value row. Lane i holds elements i and i + 64, the pair RoPE
    // rotates with table entry i; lanes 0-7 form the sum of squares in the order of the
    // standalone kernel (elements 8L.. then 64+8L.., then the 8-lane tree).
    if (w < 3) {
        const uint16_t *x16 = (const uint16_t *)sm.raw[w];
        const uint32_t xi = x16[lane], xj = x16[64 + lane];
        const size_t row = (size_t)pos * KVD + g * D;
        if (w < 2) {
            uint32_t oa, ob;
            wave_qk_norm_rope(x16, pre.w0, pre.w1, pre.cs[0], pre.sn[0],
                              S::H <= 1024 ? eps : a.eps, oa, ob);
            uint16_t *dst = (uint16_t *)(w == 0 ? sm.q : sm.k);
            dst[lane] = (uint16_t)oa;
            dst[64 + lane] = (uint16_t)ob;
            if (w == 1 && owner) {
                st_kv(kc + row + lane, oa);
                st_kv(kc + row + 64 + lane, ob);
            }
        } else {
            uint16_t *dst = (uint16_t *)sm.v;
            dst[lane] = (uint16_t)xi;
            dst[64 + lane] = (uint16_t)xj;
            if (owner) {
                st_kv(vc + row + lane, xi);
                st_kv(vc + row + 64 + lane, xj);
            }
        }
    }
    __syncthreads();

    const int G = lane >> 4, Lp = lane & 15, qtr = w & 3;
    // scores: 16 lanes per position; a round is SCORE_LOADS keys per lane
    {
        const u32x4 qv = sm.q[Lp];
        const u32x4 kcur = sm.k[Lp];
        // the 16 lanes of a position reduce the round's SCORE_LOADS dot products together
        // (reduce-scatter, each total bit-identical to group_sum<16>): lane Lp < SCORE_LOADS
        // ends with the key slot scatter_row(Lp)
        const int us = scatter_row<SCORE_LOADS>(Lp);
        for (int base = 0; base < n; base += SCORE_LOADS * 4 * WAVES) {
            u32x4 kv[SCORE_LOADS];  // keys of a later round, all requested before the first use
            if (base > 0) {
#pragma unroll
                for (int u = 0; u < SCORE_LOADS; u++) {
                    const int t = key_slot(base, u);
                    kv[u] = t < pos ? ld_kv(kc + (size_t)t * KVD + g * D + 8 * Lp, t, pos0)
                                    : (t == pos ? kcur : zero);
                }
            }
            float part[SCORE_LOADS];
#pragma unroll
            for (int u = 0; u < SCORE_LOADS; u++) {
                part[u] = 0.0f;
                if (base + u * 4 * WAVES >= n) continue;  // the slot's 32 positions are past pos
                const int t = key_slot(base, u);
                part[u] = dot8(qv, base == 0 ? (t == pos ? kcur : pre.k[u]) : kv[u], 0.0f);
            }
            const float d = group_sum_scatter<16, SCORE_LOADS, false, true>(part);
            const int t = key_slot(base, us);
            if (Lp < SCORE_LOADS && t < n) sm.sc[t] = round_bf(round_bf(d) * a.scale);
        }
    }
    __syncthreads();
    if (nb == 1) {
        // one block: its max and sum are the global ones (its weight exp(0) is exactly 1), so
        // wave 0 finishes the softmax alone
        if (w == 0) {
            const bool v = lane < n;
            const float s = v ? sm.sc[lane] : -__builtin_huge_valf();
            const float M = wave_max(s);
            const float e = v ? exp_f32(s - M) : 0.0f;
            const float sum = wave_sum(e);
            if (v) sm.sc[lane] = round_bf(e / sum);
        }
        __syncthreads();
    } else if (nb <= WAVES) {
        // up to 8 blocks: wave b takes block b's statistics; after one sync every wave forms
        // the global max and sum from the nb pairs (lane b: block b, the order of the general
        // path below) and writes its block's probabilities
        const bool v = w < nb && w * 64 + lane < n;
        const float s = v ? sm.sc[w * 64 + lane] : -__builtin_huge_valf();
        if (w < nb) {
            const float m = wave_max(s);
            const float e = v ? exp_f32(s - m) : 0.0f;
            const float Ssum = wave_sum(e);
            if (lane == 0) {
                sm.st[w][0] = m;
                sm.st[w][1] = Ssum;
            }
        }
        __syncthreads();
        if (w < nb) {
            // lanes 0..7 hold the blocks (the rest would add -inf to the max and 0 to the sum,
            // so the 8-lane trees give the 64-lane results)
            const int b = lane & 7;
            const float M = group_max<8>(b < nb ? sm.st[b][0] : -__builtin_huge_valf());
            const float sum = group_sum<8>(b < nb ? sm.st[b][1] * exp_f32(sm.st[b][0] - M) : 0.0f);
            if (v) sm.sc[w * 64 + lane] = round_bf(exp_f32(s - M) / sum);
        }
        __syncthreads();
    } else {
    // block statistics
    for (int b = w; b < nb; b += WAVES) {
        const bool v = b * 64 + lane < n;
        const float s = v ? sm.sc[b * 64 + lane] : -__builtin_huge_valf();
        const float m = wave_max(s);
        const float e = v ? exp_f32(s - m) : 0.0f;
        const float Ssum = wave_sum(e);
        if (lane == 0) {
            sm.st[b][0] = m;
            sm.st[b][1] = Ssum;
        }
    }
    __syncthreads();
    if (w == 0) {
        float M = -__builtin_huge_valf();
        for (int c0 = 0; c0 < nb; c0 += 64) {
            const int bi = c0 + lane;
            M = fmaxf(M, wave_max(bi < nb ? sm.st[bi][0] : -__builtin_huge_valf()));
        }
        float sum = 0.0f;
        for (int c0 = 0; c0 < nb; c0 += 64) {
            const int bi = c0 + lane;
            const float term = bi < nb ? sm.st[bi][1] * exp_f32(sm.st[bi][0] - M) : 0.0f;
            const float cs = wave_sum(term);
            sum = c0 == 0 ? cs : sum + cs;
        }
        if (lane == 0) {
            sm.gm[0] = M;
            sm.gm[1] = sum;
        }
    }
    __syncthreads();
    {
        const float M = sm.gm[0], sum = sm.gm[1];
        for (int t = threadIdx.x; t < n; t += THREADS) sm.sc[t] = round_bf(exp_f32(sm.sc[t] - M) / sum);
    }
    __syncthreads();
    }
    // PV in rounds of PV_ROUND blocks: wave w takes blocks c0 + w/4 + 2j and quarter w % 4 of
    // each (slots quarter*16 + it*4 + G); the quarters meet in order, the blocks are added in order
    // by thread d < D, which keeps element d's running sum in a register
    const u32x4 vcur = sm.v[Lp];
    float out_d = 0.0f;
    for (int c0 = 0; c0 < nb; c0 += PV_ROUND) {
        if (c0 > 0) load_v(c0);
#pragma unroll
        for (int j = 0; j < PV_ROUND / 2; j++) {
            if (c0 + (w >> 2) + 2 * j >= nb) break;  // block past pos
            // every slot of the block, with no branch around the probability reads: a slot past
            // pos has value zeros and probability 0, and fma(0, 0, acc) is acc (acc starts at +0
            // and an exact zero sum is +0, so acc is never -0)
            float p[4];
#pragma unroll
            for (int it = 0; it < 4; it++) {
                const int t = value_slot(c0, j, it);
                const float pt = sm.sc[t];
                p[it] = t < n ? pt : 0.0f;
            }
            float acc[8];
#pragma unroll
            for (int e = 0; e < 8; e++) acc[e] = 0.0f;
#pragma unroll
            for (int it = 0; it < 4; it++) {
                const int t = value_slot(c0, j, it);
                const u32x4 vt = t == pos ? vcur : vv[j][it];
#pragma unroll
                for (int e = 0; e < 8; e++) acc[e] = fmaf(p[it], elem(vt, e), acc[e]);
            }
            // the four slot groups (lanes 16 apart) summed with the pairing of butterfly_sum<16,
            // 64> (xor 16, then xor 32), reduce-scattered: the lane ends with elements d0, d0 + 1
            float two[2];
            scatter_keep<8, 16, 64>(acc, two);
            const int d0 = ((G & 1) ? 4 : 0) + ((G & 2) ? 2 : 0);
            float *qd = &sm.quarter[(w >> 2) + 2 * j][qtr][8 * Lp + d0];
            qd[0] = two[0];
            qd[1] = two[1];
        }
        const bool last = c0 + PV_ROUND >= nb;
        // in the last round, the KV row this workgroup stored is complete before the sync, so
        // before the output that later steps depend on is published (a later token of the
        // launch reads the row from another workgroup)
        if (last) __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x < D) {
            const int d = threadIdx.x;
            for (int bi = 0; bi < PV_ROUND && c0 + bi < nb; bi++) {
                const float part = ((sm.quarter[bi][0][d] + sm.quarter[bi][1][d]) +
                                    sm.quarter[bi][2][d]) +
                                   sm.quarter[bi][3][d];
                out_d = c0 + bi == 0 ? part : out_d + part;
            }
        }
        if (!last) __syncthreads();  // the quarters are read before the next round rewrites them
    }
    if (threadIdx.x < D) put_tagged_all<QD, S::REPLICAS>(a.tattn, h * D + threadIdx.x, f2bf(out_d), tag_out);
}

// ---------------------------------------------------------------- split attention

// Long histories: attention split over (kv head g, 64-position block b) items, each run by half
// a workgroup (waves 4h..4h+3, 256 threads) with the lane layout and arithmetic of the
// multi-kernel step's passes (attn_scores_kernel, pv_item, the block-order combine), so the
// results are those of that step bit for bit. Half-slot s (split_items) takes kv head s % HKV
// and blocks s / HKV + k * SPG, k < SPLIT_ITEMS (SPG = 2 * grid / HKV half-slots per kv head;
// the host checks that the history fits). An item publishes its query heads' block statistics
// (max, sum of exp(s - max)) and, once every block's statistics of its kv head are in, its
// heads' block partials of p v, as tagged 64-bit words (float bits << 32 | tag); the attention
// workgroups and the last workgroups of the grid then each add the partials of a quarter of a
// head's columns in block order and publish them. Every workgroup takes part: its items' key
// and value rows are requested before it polls the q/k/v vector, so the history streams on
// every CU at once.
constexpr int SPLIT_ITEMS = 3;   // items of a half-slot at most
constexpr int SPLIT_MAXB = 192;  // blocks of 64 positions at most (3 chunks of 64 statistics)
constexpr int COMB_COLS = 32;    // columns of a head one workgroup combines

template <class S>
struct SplitSmem {
    static constexpr int REP = S::HQ / S::HKV, D = 128;
    uint32_t raw[2][REP + 2][D / 2];    // each half's q heads, k and v as polled (bf16 pairs)
    u32x4 q[2][REP][D / 8];             // roped query heads
    u32x4 k[2][D / 8];                  // roped key at pos
    float sc[2][SPLIT_ITEMS][REP][64];  // scores, then probabilities
    float gst[2][REP][2];               // each head's global max and sum
    float red[2][4][REP][D];            // the four waves' PV partials
    float comb[SPLIT_MAXB][COMB_COLS];  // a combine's staged block partials
};

// The key and value history rows of a half-slot's items, this lane's chunks (rows at or past
// pos read as zeros), requested a phase ahead of their use.
struct SplitKV {
    u32x4 k[SPLIT_ITEMS][4], v[SPLIT_ITEMS][4];
};

// Where a half-slot's items lie: kv head g, first block j0, SPG blocks apart; n_it items for the
// workgroup's loop (half 0 has at least as many as half 1). Half h of workgroup w is half-slot
// h * grid + w, so where some half-slots take one item more than the others (histories of
// more than 2 SPG blocks), those are half 0 of as many workgroups, not both halves of half as
// many: a CU then has one item less to compute.
struct SplitItems {
    int g, j0, spg, n_it;
};
template <class S>
__device__ __forceinline__ SplitItems split_items(int nb) {
    SplitItems it;
    it.spg = 2 * (int)gridDim.x / S::HKV;
    const int hslot = (wave_id() >> 2) * (int)gridDim.x + (int)blockIdx.x;
    it.g = hslot % S::HKV;
    it.j0 = hslot / S::HKV;
    const int j00 = (int)blockIdx.x / S::HKV;
    it.n_it = j00 < nb ? min(SPLIT_ITEMS, (nb - 1 - j00) / it.spg + 1) : 0;
    return it;
}

// Requests the history rows of this workgroup's items of layer `layer` at `pos` (slot
// w4 * 16 + it * 4 + G of each block, lane chunk Lk); rows written during this launch
// (t >= pos0) coherently.
template <class S>
__device__ __forceinline__ void split_request(KArgs &a, int pos, int pos0, int layer, SplitKV &kv) {
    constexpr int D = 128, KVD = S::HKV * D;
    const int nb = (pos + 64) / 64;
    const SplitItems si = split_items<S>(nb);
    const int lane = tid_x() & 63, w4 = wave_id() & 3, G = lane >> 4, Lk = lane & 15;
    const bf16 *kc = a.key_cache + (size_t)layer * a.max_seq * KVD;
    const bf16 *vc = a.value_cache + (size_t)layer * a.max_seq * KVD;
    const u32x4 zero{0, 0, 0, 0};
#pragma unroll
    for (int k = 0; k < SPLIT_ITEMS; k++)
#pragma unroll
        for (int it = 0; it < 4; it++) {
            const int t = (si.j0 + k * si.spg) * 64 + w4 * 16 + it * 4 + G;
            const bool in = k < si.n_it && t < pos;
            const size_t off = (size_t)t * KVD + si.g * D + 8 * Lk;
            kv.k[k][it] = in ? ld_kv(kc + off, t, pos0) : zero;
            kv.v[k][it] = in ? ld_kv(vc + off, t, pos0) : zero;
        }
}

__device__ __forceinline__ void put_tagged64(unsigned long long *p, float v, uint32_t tag) {
    __hip_atomic_store(gptr(p), ((unsigned long long)__float_as_uint(v) << 32) | tag,
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The split attention of layer `layer` at `pos` (n = pos + 1 > 0 positions, at most
// SPLIT_ITEMS * SPG blocks): q/k/v polled with tag `tag_in`; statistics, partials and, on the
// combining workgroups, the output published with `tag_out`. cs / sn: this lane's RoPE table
// entry at pos.
template <class S>
__device__ __forceinline__ void split_attention(KArgs &a, KLayer &L, int pos, int layer,
                                                SplitSmem<S> &sm, SplitKV &kv,
                                                uint32_t tag_in, uint32_t tag_out, float cs,
                                                float sn, int n_layers, int step, float eps) {
    constexpr int D = 128, REP = S::HQ / S::HKV, QD = S::HQ * D, KVD = S::HKV * D;
    static_assert(REP >= 1 && REP <= 4, "query heads per kv head");
    const int n = pos + 1, nb = (n + 63) / 64, mb = a.max_blocks;
    const int lane = tid_x() & 63, hf = wave_id() >> 2, w4 = wave_id() & 3;
    const int ht = tid_x() & 255;  // thread of the half
    const int G = lane >> 4, Lk = lane & 15;
    const SplitItems si = split_items<S>(nb);
    const int spg = si.spg, g = si.g, j0 = si.j0, n_it = si.n_it;
    bf16 *kc = a.key_cache + (size_t)layer * a.max_seq * KVD;
    bf16 *vc = a.value_cache + (size_t)layer * a.max_seq * KVD;
    if (n_it > 0) {
        // (the items' history rows were requested with split_request; loads complete in order,
        // so the q/k/v poll below lands once they have)
        uint32_t qn0, qn1, kn0, kn1;
        {
            const uint16_t *qn = (const uint16_t *)L.q_norm, *kn = (const uint16_t *)L.k_norm;
            qn0 = gptr(qn)[lane];
            qn1 = gptr(qn)[64 + lane];
            kn0 = gptr(kn)[lane];
            kn1 = gptr(kn)[64 + lane];
        }
        // the half's q heads, k and v (every half polls its own kv head's words)
        __syncthreads();
        {
            constexpr int PAIRS = (REP + 2) * D / 2, PP = (PAIRS + 255) / 256;
            const uint32_t *tq = a.tqkv;
            uint32_t *dst = &sm.raw[hf][0][0];
            uint64_t wd[PP];
            long long spins = 0;
            for (;;) {
                bool fresh = true;
#pragma unroll
                for (int j = 0; j < PP; j++) {
                    const int p = min(ht + 256 * j, PAIRS - 1);
                    const int seg = p / (D / 2), i = 2 * (p % (D / 2));
                    const int off = seg < REP ? (g * REP + seg) * D
                                              : QD + (seg - REP) * KVD + g * D;
                    wd[j] = ld_coh64(tq + off + i);
                    fresh &= (uint32_t)(wd[j] & 0xffffu) == tag_in &&
                             (uint32_t)((wd[j] >> 32) & 0xffffu) == tag_in;
                }
                if (fresh) break;
                if ((++spins & 63) == 0 && wait_gives_up(spins, SPIN_LIMIT, a.error_flag)) break;
            }
#pragma unroll
            for (int j = 0; j < PP; j++) {
                const int p = ht + 256 * j;
                if (p < PAIRS)
                    dst[p] = (uint32_t)((wd[j] >> 16) & 0xffffu) | ((uint32_t)(wd[j] >> 48) << 16);
            }
        }
        __syncthreads();
        if (blockIdx.x < S::HQ) stamp_wg(layer, n_layers, 0, step);
        // QK-norm + RoPE of the query heads (wave r of the half: head r) and, in the half whose
        // items hold pos, of the key, which that half writes with the value into row pos
        const int pb = nb - 1;  // the block holding pos
        const bool has_pos = pb >= j0 && (pb - j0) % spg == 0;
        for (int hh = w4; hh < REP + (has_pos ? 1 : 0); hh += 4) {
            const bool is_k = hh == REP;
            uint32_t oa, ob;
            wave_qk_norm_rope((const uint16_t *)sm.raw[hf][hh], is_k ? kn0 : qn0,
                              is_k ? kn1 : qn1, cs, sn, S::H <= 1024 ? eps : a.eps, oa, ob);
            uint16_t *dst = (uint16_t *)(is_k ? sm.k[hf] : sm.q[hf][hh]);
            dst[lane] = (uint16_t)oa;
            dst[64 + lane] = (uint16_t)ob;
            if (is_k) {
                const size_t row = (size_t)pos * KVD + g * D;
                st_kv(kc + row + lane, oa);
                st_kv(kc + row + 64 + lane, ob);
            }
        }
        if (has_pos && w4 == 3) {
            const uint16_t *v16 = (const uint16_t *)sm.raw[hf][REP + 1];
            const size_t row = (size_t)pos * KVD + g * D;
            st_kv(vc + row + lane, v16[lane]);
            st_kv(vc + row + 64 + lane, v16[64 + lane]);
        }
        __syncthreads();
        // the item holding pos takes its key and value (row pos of the caches, just written)
        // into the slot of pos, once, instead of a select in every slot of every item
        if (has_pos) {
            const u32x4 kcur = sm.k[hf][Lk];
            const u32x4 vcur = ((const u32x4 *)sm.raw[hf][REP + 1])[Lk];
#pragma unroll
            for (int k = 0; k < SPLIT_ITEMS; k++)
                if (j0 + k * spg == pb) {
#pragma unroll
                    for (int it = 0; it < 4; it++) {
                        const bool at = pb * 64 + w4 * 16 + it * 4 + G == pos;
                        kv.k[k][it] = at ? kcur : kv.k[k][it];
                        kv.v[k][it] = at ? vcur : kv.v[k][it];
                    }
                }
        }
        // scores s = bf16(bf16(q.k) * scale) of each item (attn_scores_kernel layout: slot
        // w4 * 16 + it * 4 + G, 16 lanes per position, reduce-scattered)
        {
            constexpr int NP = 4 * REP, SL = NP < 16 ? NP : 16;
            // the query heads' chunks as fp32 once (bf16 -> fp32 is exact, so each product and
            // the order of the fmas are those of dot8)
            float qf[REP][8];
#pragma unroll
            for (int r = 0; r < REP; r++) {
                const u32x4 qv = sm.q[hf][r][Lk];
#pragma unroll
                for (int e = 0; e < 8; e++) qf[r][e] = elem(qv, e);
            }
#pragma unroll
            for (int k = 0; k < SPLIT_ITEMS; k++) {
                const int b = j0 + k * spg;
                if (k >= n_it) break;
                if (b >= nb) continue;
                float part[NP];
#pragma unroll
                for (int it = 0; it < 4; it++) {
                    const u32x4 kt = kv.k[k][it];
                    float kf[8];
#pragma unroll
                    for (int e = 0; e < 8; e++) kf[e] = elem(kt, e);
#pragma unroll
                    for (int r = 0; r < REP; r++) {
                        float d = 0.0f;
#pragma unroll
                        for (int e = 0; e < 8; e++) d = fmaf(qf[r][e], kf[e], d);
                        part[it * REP + r] = d;
                    }
                }
#pragma unroll
                for (int s0 = 0; s0 < NP; s0 += SL) {
                    float slice[SL];
#pragma unroll
                    for (int j = 0; j < SL; j++) slice[j] = part[s0 + j];
                    const float d = group_sum_scatter<16, SL, false, true>(slice);
                    const int j = s0 + scatter_row<SL>(Lk), it = j / REP, r = j - it * REP;
                    if (Lk < SL)
                        sm.sc[hf][k][r][w4 * 16 + it * 4 + G] = round_bf(round_bf(d) * a.scale);
                }
            }
        }
        __syncthreads();
        // block statistics (wave r of the half: head r), published
        if (w4 < REP) {
            const int h = g * REP + w4;
#pragma unroll
            for (int k = 0; k < SPLIT_ITEMS; k++) {
                const int b = j0 + k * spg;
                if (k >= n_it) break;
                if (b >= nb) continue;
                const bool v = b * 64 + lane < n;
                const float sv = v ? sm.sc[hf][k][w4][lane] : -__builtin_huge_valf();
                const float m = wave_max<S::SPLIT_STATS_LDS>(sv);
                const float e = v ? exp_f32(sv - m) : 0.0f;
                const float ssum = wave_sum<S::SPLIT_STATS_LDS>(e);
                if (lane == 0) {
                    unsigned long long *st = a.tstat + ((size_t)h * mb + b) * 2;
                    put_tagged64(st, m, tag_out);
                    put_tagged64(st + 1, ssum, tag_out);
                }
            }
        }
        // every block's statistics of the head: global max M (exact in any order) and sum (the
        // chunks of 64 blocks tree-summed, S_b exp(m_b - M), added in order)
        if (w4 < REP && j0 < nb) {
            constexpr int MAXC = SPLIT_MAXB / 64;
            const unsigned long long *st = a.tstat + (size_t)(g * REP + w4) * mb * 2;
            float mv[MAXC], sv[MAXC];
            uint64_t wm[MAXC], ws[MAXC];
            long long spins = 0;
            for (;;) {
                bool fresh = true;
#pragma unroll
                for (int c = 0; c < MAXC; c++) {
                    const int bi = min(c * 64 + lane, nb - 1);
                    wm[c] = ld_coh64(st + 2 * bi);
                    ws[c] = ld_coh64(st + 2 * bi + 1);
                    fresh &= (uint32_t)wm[c] == tag_out && (uint32_t)ws[c] == tag_out;
                }
                if (fresh) break;
                if ((++spins & 63) == 0 && wait_gives_up(spins, SPIN_LIMIT, a.error_flag)) break;
            }
#pragma unroll
            for (int c = 0; c < MAXC; c++) {
                mv[c] = __uint_as_float((uint32_t)(wm[c] >> 32));
                sv[c] = __uint_as_float((uint32_t)(ws[c] >> 32));
            }
            float ml = -__builtin_huge_valf();
#pragma unroll
            for (int c = 0; c < MAXC; c++) ml = c * 64 + lane < nb ? fmaxf(ml, mv[c]) : ml;
            const float M = wave_max<S::SPLIT_STATS_LDS>(ml);
            float sum = 0.0f;
#pragma unroll
            for (int c = 0; c < MAXC; c++) {
                if (c * 64 >= nb) break;
                const float cs_ = wave_sum<S::SPLIT_STATS_LDS>(c * 64 + lane < nb ? sv[c] * exp_f32(mv[c] - M) : 0.0f);
                sum = c == 0 ? cs_ : sum + cs_;
            }
            if (lane == 0) {
                sm.gst[hf][w4][0] = M;
                sm.gst[hf][w4][1] = sum;
            }
        }
        __syncthreads();
        // probabilities p = bf16(exp(s - M) / sum)
        if (w4 < REP) {
            const float M = sm.gst[hf][w4][0], sum = sm.gst[hf][w4][1];
#pragma unroll
            for (int k = 0; k < SPLIT_ITEMS; k++) {
                const int b = j0 + k * spg;
                if (k >= n_it) break;
                if (b >= nb) continue;
                const float sv = sm.sc[hf][k][w4][lane];
                sm.sc[hf][k][w4][lane] = b * 64 + lane < n ? round_bf(exp_f32(sv - M) / sum) : 0.0f;
            }
        }
        __syncthreads();
        // PV of each item (pv_item layout: per lane over its slots in order, the position
        // groups reduce-scattered with the butterfly's pairing, the four waves added in order),
        // published per head and element
        // the KV row this workgroup may have stored is complete before any partial that later
        // steps depend on is published
        __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
        for (int k = 0; k < SPLIT_ITEMS; k++) {
            if (k >= n_it) break;
            const int b = j0 + k * spg;
            if (b < nb) {
                float acc[REP][8];
#pragma unroll
                for (int r = 0; r < REP; r++)
#pragma unroll
                    for (int e = 0; e < 8; e++) acc[r][e] = 0.0f;
#pragma unroll
                for (int it = 0; it < 4; it++) {
                    const int slot = w4 * 16 + it * 4 + G;
                    const int t = b * 64 + slot;
                    if (t < n) {
                        const u32x4 vt = kv.v[k][it];
#pragma unroll
                        for (int r = 0; r < REP; r++) {
                            const float p = sm.sc[hf][k][r][slot];
#pragma unroll
                            for (int e = 0; e < 8; e++) acc[r][e] = fmaf(p, elem(vt, e), acc[r][e]);
                        }
                    }
                }
                constexpr int NV = REP * 8, KEEP = NV / 4;
                float flat[NV], kept[KEEP];
#pragma unroll
                for (int r = 0; r < REP; r++)
#pragma unroll
                    for (int e = 0; e < 8; e++) flat[r * 8 + e] = acc[r][e];
                scatter_keep<NV, 16, 64>(flat, kept);
                int off = 0;
#pragma unroll
                for (int q = 0, m = NV; (16 << q) < 64; q++, m >>= 1)
                    if ((lane >> q) & 16) off += m / 2;
#pragma unroll
                for (int j = 0; j < KEEP; j++) {
                    const int idx = off + j, r = idx / 8, e = idx % 8;
                    sm.red[hf][w4][r][8 * Lk + e] = kept[j];
                }
            }
            __syncthreads();
            if (b < nb) {
                for (int i = ht; i < REP * D; i += 256) {
                    const int r = i / D, d = i - r * D;
                    const float v = ((sm.red[hf][0][r][d] + sm.red[hf][1][r][d]) +
                                     sm.red[hf][2][r][d]) +
                                    sm.red[hf][3][r][d];
                    put_tagged64(a.tpart + ((size_t)(g * REP + r) * mb + b) * D + d, v, tag_out);
                }
            }
            __syncthreads();  // red is rewritten by the next item
        }
    }
    // NT = HQ D / COMB_COLS combining tasks: columns [c0, c0 + COMB_COLS) of query head h, out =
    // bf16(block partials added in block order). Tasks 0..HQ-1 run on the attention
    // workgroups, the others on the last workgroups of the grid: workgroups that own no o rows,
    // whose weight requests (made after this) the o phase would wait for.
    constexpr int NT = S::HQ * (D / COMB_COLS);
    const int tail0 = (int)gridDim.x - (NT - S::HQ);
    const int task = (int)blockIdx.x < S::HQ ? (int)blockIdx.x
                     : (int)blockIdx.x >= tail0 ? S::HQ + (int)blockIdx.x - tail0 : -1;
    if (task >= 0) {
        const int h = task / (D / COMB_COLS), c0 = (task % (D / COMB_COLS)) * COMB_COLS;
        // thread t reads column t % 64 of blocks t / 64 + 8 j, as buffer loads with one lane
        // offset (the block stride in the scalar offset) and the coherence of ld_coh64 (sc1);
        // blocks past the history read as 0 and are not waited for
        constexpr int BPJ = THREADS / COMB_COLS, P = SPLIT_MAXB / BPJ;
        const int tb = tid_x() / COMB_COLS, tc = tid_x() % COMB_COLS;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(a.tpart + (size_t)h * mb * D + c0), (short)0, nb * D * 8, BUFFER_FLAGS);
        const int voff = (tb * D + tc) * 8;
        __syncthreads();
        // first the column-c0 word of every block (one per thread; an item stores all its words
        // at once), then every partial in one read: re-reading all of them while most are still
        // being written streams the whole set once per poll round (4B at 8192 positions: 409
        // tokens/s with two threads per block polling its 32 words each; 427 with eight
        // threads per block in passes of 64 blocks; 438 as here)
        if ((int)threadIdx.x < nb) {
            const unsigned long long *w0 = a.tpart + ((size_t)h * mb + threadIdx.x) * D + c0;
            long long spins = 0;
            while ((uint32_t)ld_coh64(w0) != tag_out)
                if ((++spins & 63) == 0 && wait_gives_up(spins, SPIN_LIMIT, a.error_flag)) break;
        }
        __syncthreads();
        {
            uint64_t w[P];
            long long spins = 0;
            for (;;) {
                bool fresh = true;
#pragma unroll
                for (int j = 0; j < P; j++) {
                    const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, voff, j * BPJ * D * 8,
                                                                        BUFFER_SC1);
                    w[j] = ((uint64_t)v[1] << 32) | v[0];
                    fresh &= tb + BPJ * j >= nb || (uint32_t)w[j] == tag_out;
                }
                if (fresh) break;
                if ((++spins & 63) == 0 && wait_gives_up(spins, SPIN_LIMIT, a.error_flag)) break;
            }
#pragma unroll
            for (int j = 0; j < P; j++)
                if (tb + BPJ * j < nb)
                    sm.comb[tb + BPJ * j][tc] = __uint_as_float((uint32_t)(w[j] >> 32));
        }
        __syncthreads();
        if (threadIdx.x < COMB_COLS) {
            const int c = threadIdx.x;
            float acc = sm.comb[0][c];
            int j = 1;
            for (; j + 16 <= nb; j += 16) {  // 16 LDS reads in flight, then the adds
                float v[16];
#pragma unroll
                for (int u = 0; u < 16; u++) v[u] = sm.comb[j + u][c];
#pragma unroll
                for (int u = 0; u < 16; u++) acc += v[u];
            }
            for (; j < nb; j++) acc += sm.comb[j][c];
            put_tagged_all<QD, S::REPLICAS>(a.tattn, h * D + c0 + c, f2bf(acc), tag_out);
        }
    }
}

// ---------------------------------------------------------------- argmax partials

// A workgroup's argmax partial as one tagged 64-bit word: the value's bits << 32, the row index
// << 14 (18 bits; AMAX_NO_ROW for a workgroup without rows, which loses every tie as INT_MAX
// does), and the token's 14-bit tag (never 0, so a zeroed word never matches).
constexpr int AMAX_NO_ROW = 0x3ffff;
__device__ __forceinline__ unsigned long long amax_word(float v, int i, uint32_t tag) {
    const uint32_t ix = i >= 0 && i < AMAX_NO_ROW ? (uint32_t)i : (uint32_t)AMAX_NO_ROW;
    return ((unsigned long long)__float_as_uint(v) << 32) | (ix << 14) | tag;
}

// ---------------------------------------------------------------- the step

// Rows [r0, r1) of a phase with R rows owned by wave w of this workgroup, the rows spread in
// order over waves FIRST_W..7 of workgroups first_wg.. (so a workgroup owns rows iff its wave
// FIRST_W does, and few workgroups take part in a small phase: each one polls the phase's
// input, and fewer pollers see a written vector sooner). A wave takes at least min_per rows.
// Waves below FIRST_W own none; an empty range is [R, R).
__host__ __device__ constexpr int rows_per_wave(int R, int n_waves) { return (R + n_waves - 1) / n_waves; }
template <int FIRST_W>
__device__ __forceinline__ void phase_rows(int R, int first_wg, int w, int &r0, int &r1,
                                           int min_per = 1) {
    constexpr int RW = WAVES - FIRST_W;
    const int per = max(rows_per_wave(R, ((int)gridDim.x - first_wg) * RW), min_per);
    const int gw = ((int)blockIdx.x - first_wg) * RW + w - FIRST_W;
    const bool none = (int)blockIdx.x < first_wg || w < FIRST_W;
    r0 = none ? R : min(R, gw * per);
    r1 = none ? R : min(R, r0 + per);
}
template <int FIRST_W>
__device__ __forceinline__ void phase_rows(int R, int first_wg, int &r0, int &r1,
                                           int min_per = 1) {
    phase_rows<FIRST_W>(R, first_wg, __builtin_amdgcn_readfirstlane(tid_x() >> 6), r0, r1,
                        min_per);
}
template <int FIRST_W>
__device__ __forceinline__ bool workgroup_has_rows(int R, int first_wg, int min_per = 1) {
    int r0, r1;
    phase_rows<FIRST_W>(R, first_wg, FIRST_W, r0, r1, min_per);
    return r0 < r1;
}

// The first workgroup with q/k/v rows: the one after the attention workgroups, or with
// S::QKV_AT_END the first of the last workgroups of the grid that hold them at
// S::QKV_PER_WAVE rows per matrix wave (the host checks that these lie past the attention
// workgroups).
template <class S>
__host__ __device__ constexpr int qkv_first_wg(int grid) {
    constexpr int rows = (S::HQ + 2 * S::HKV) * 128;
    constexpr int per_wg = (WAVES - (S::POLLER ? 1 : 0)) * S::QKV_PER_WAVE;
    return S::QKV_AT_END ? grid - (rows + per_wg - 1) / per_wg : S::HQ;
}

// When a matrix workgroup requests the down rows (PF_D) and the next layer's q/k/v rows
// (PF_QKV). Loads complete in order, so a request placed before a poll holds the poll until it
// lands, and weights streaming during a handoff slow it: at 0.6B both go out while attention
// runs (the q/k/v rows after the gate/up poll measured 7% slower, after the down rows 1.4%).
enum {
    PF_WITH_ATTENTION = 0,  // with the o and gate/up rows, while attention runs
    PF_AFTER_POLL = 1,      // down rows once the o input is staged, q/k/v once gate/up's is
    PF_AFTER_COMPUTE = 2,   // down rows after the gate/up rows, q/k/v after the down rows
};

// The roles a token loop is compiled for.
enum { ROLE_ATTN = 0, ROLE_MATRIX = 1, ROLE_EITHER = 2 };

// SPLIT: the instance for long histories, whose attention runs split over (kv head, block)
// items on every workgroup (split_attention); otherwise one workgroup per query head.
template <class S, bool SPLIT>
__global__ __launch_bounds__(THREADS) void step_kernel(StepArgs) {
    constexpr int H = S::H, I = S::I, D = 128, QD = S::HQ * D, KVD = S::HKV * D;
    constexpr int NCH = H / 512, NCO = QD / 512, NCI = I / 512;
    constexpr int VEC_WORDS = (I > QD ? (I > H ? I : H) : (QD > H ? QD : H)) / 2;
    __shared__ union Smem {
        AttnSmem<S> attn;
        std::conditional_t<SPLIT, SplitSmem<S>, char> split;  // the split instance's only
        uint32_t vec[VEC_WORDS];  // the staged input vector of a matrix phase (bf16 pairs)
    } sm;
    __shared__ float red_v[WAVES];
    __shared__ int red_i[WAVES];
    __shared__ uint32_t out_stage[WAVES * 64];  // a workgroup's x rows as tagged words
    __shared__ float norm_inv;

    int token, pos, n_layers, n_tokens;
    float eps_k = 0.0f;  // the RMSNorm epsilon (0.6B: read once, below)
    unsigned seq0;  // tagged phases before this launch
    {
        KArgs &a = kargs();
        seq0 = *gptr(a.epoch);
        token = *gptr(a.next_token);
        pos = *gptr(a.pos);
        n_layers = a.n_layers;
        if constexpr (S::H <= 1024) eps_k = a.eps;
        n_tokens = a.n_tokens;
        // one workgroup per query head holds at most NMAX positions; the split attention at
        // most SPLIT_ITEMS items per half-slot and the blocks the workspace holds
        const int last_nb = (pos + n_tokens + 63) / 64;
        if (pos < 0 || n_tokens < 1 || pos + n_tokens > a.max_seq || token < 0 ||
            token >= a.vocab ||
            (SPLIT ? last_nb > a.max_blocks || last_nb > SPLIT_MAXB ||
                         (2 * (int)gridDim.x) % S::HKV != 0 ||
                         last_nb > SPLIT_ITEMS * (2 * (int)gridDim.x / S::HKV)
                   : pos + n_tokens > S::NMAX)) {
            if (blockIdx.x == 0 && threadIdx.x == 0) *gptr(a.error_flag) = 1;
            return;  // every workgroup reads the same values and leaves at once
        }
    }
    // 0.6B: the RMSNorm epsilon held in an SGPR for the launch instead of loaded where the
    // RMSNorm's lane 0 uses it (2431.4 against 2425.7 tokens/s; at 4B 596.3 against 597.3, so
    // larger shapes read it at each use)
    if constexpr (S::H <= 1024) asm volatile("" : "+s"(eps_k));
    auto eps_now = [&]() __attribute__((always_inline)) {
        if constexpr (S::H <= 1024) return eps_k;
        else return kargs().eps;
    };
    const int pos0 = pos;  // KV rows from pos0 on are written during this launch
    const unsigned seq_step = PHASES * n_layers + 1;  // tags per token: 5 per layer + the token

    // Workgroups 0..HQ-1 run one query head's attention each and own no matrix rows; the
    // others own the matrix rows and, while attention runs, load the weights of the o,
    // gate/up and down rows. The o and down phases share the row partition, so the residual
    // rows a wave updates are its own (at most 64 per wave, checked by the host). A
    // workgroup reads a vector only when it owns rows that use it: then it produces part of
    // what every later writer of that vector waits for, so it never sees a value overwritten.
    const bool attn_wg = (int)blockIdx.x < S::HQ;
    int q0, q1, o0, o1, g0, g1;
    constexpr int FW = S::POLLER ? 1 : 0;  // first wave with matrix rows
    constexpr bool OW = S::POLLER;         // staging by wave 0 alone
    // a wave takes at least one prefetched batch of q/k/v rows (at 0.6B 4 rows on 1024 waves
    // instead of 3 on 1366: +0.8%), placed after the attention workgroups or, with
    // S::QKV_AT_END, on the last workgroups of the grid
    const int q_first = qkv_first_wg<S>((int)gridDim.x);
    constexpr int BQ = SPLIT ? S::B_QKV_SPLIT : S::B_QKV;  // q/k/v rows per batch
    constexpr int Q_MIN = S::QKV_AT_END ? 1 : BQ;  // rows per wave at least
    phase_rows<FW>(QD + 2 * KVD, q_first, q0, q1, Q_MIN);
    phase_rows<FW>(H, S::HQ, o0, o1);
    phase_rows<FW>(I, S::HQ, g0, g1);
    const bool wg_q = workgroup_has_rows<FW>(QD + 2 * KVD, q_first, Q_MIN);
    const bool wg_o = workgroup_has_rows<FW>(H, S::HQ);
    const bool wg_g = workgroup_has_rows<FW>(I, S::HQ);

    auto qkv_row = [](KLayer &L) {
        const bf16 *wq = L.wq, *wk = L.wk, *wv = L.wv;
        return [=](int r) -> const bf16 * {
            return r < QD ? wq + (size_t)r * H
                          : r < QD + KVD ? wk + (size_t)(r - QD) * H : wv + (size_t)(r - QD - KVD) * H;
        };
    };
    auto o_row = [](KLayer &L) {
        const bf16 *wo = L.wo;
        return [=](int r) { return wo + (size_t)r * QD; };
    };
    auto d_row = [](KLayer &L) {
        const bf16 *wd = L.w_down;
        return [=](int r) { return wd + (size_t)r * I; };
    };
    // A workgroup's new x rows (o and down phases) are staged in LDS as tagged words (row r at
    // out_stage[r - wr0]) and written out by publish_rows: one store instruction per copy
    // instead of a single-lane store per row and copy made the two x handoffs ~1 µs faster
    // (staging the SwiGLU and q/k/v outputs the same way measured slower).
    int wr0, wr1, dummy;  // this workgroup's o/down rows
    phase_rows<FW>(H, S::HQ, FW, wr0, dummy);
    phase_rows<FW>(H, S::HQ, WAVES - 1, dummy, wr1);
    auto residual = [](uint32_t *stage, int r_first, uint32_t tag) {
        return [=](int r, float y, uint32_t xr) {
            const uint32_t nb = f2bf(bf2f((bf16)xr) + bf2f((bf16)f2bf(y)));
            stage[r - r_first] = (nb << 16) | tag;
            return nb;
        };
    };

    // Weight requests are unconditional: a wave without rows in a phase has the empty range
    // [R, R) and loads row R - 1 (a cache hit after its owner's load). A request made on some
    // paths only would leave the registers to be merged where the paths join, and the copy
    // made there waits for the load (and, loads completing in order, for every earlier one).
    //
    // The token loop is instantiated per role: ROLE_ATTN (the attention workgroups),
    // ROLE_MATRIX, or ROLE_EITHER (one loop for both, the role a run-time branch). With
    // S::SPLIT_ROLES the two roles get their own loops, so the matrix role's loop-carried q/k/v
    // prefetch is not live through the attention code.
    auto run = [&](auto role) __attribute__((always_inline)) {
    constexpr int ROLE = decltype(role)::value;
    const bool attn = ROLE == ROLE_ATTN || (ROLE == ROLE_EITHER && attn_wg);
    // The first layer's q/k/v rows of the next token, requested before the token is known
    // (by the last layer of the previous token after the first).
    Rows<NCH, BQ> pf_qkv;
    NormW<H> nq;  // attn_norm weights of the coming q/k/v phase
    if (ROLE != ROLE_ATTN) {
        nq.load(klayer(kargs(), 0).attn_norm);
        pf_qkv.load(qkv_row(klayer(kargs(), 0)), q0, q1);
    }

    for (int step = 0; step < n_tokens; step++, pos++) {
    const unsigned sq0 = seq0 + step * seq_step;  // this token's first tag
    stamp<S>(0, step);
    // tags of layer l: seq q|k|v, seq+1 attention, seq+2 x after o, seq+3 SwiGLU, seq+4 x
    // after down, with seq = sq0 + PHASES * l; the next token: sq0 + PHASES * n_layers
    if (attn) {
        // ---- QK-norm + RoPE + KV write + attention, one query head per workgroup
        float rope_c = 0.0f, rope_s = 0.0f;  // this lane's RoPE table entry at pos (split)
        if constexpr (SPLIT) {
            float cs[1], sn[1];
            rope_table<D>(pos, kargs().inv_freq, cs, sn);
            rope_c = cs[0];
            rope_s = sn[0];
        }
        for (int l = 0; l < n_layers; l++) {
            const unsigned seq = sq0 + PHASES * l;
            if constexpr (SPLIT) {
                KArgs &a = kargs();
                SplitKV kv;
                split_request<S>(a, opaque(pos), opaque(pos0), l, kv);
                split_attention<S>(a, klayer(a, l), opaque(pos), l, sm.split, kv, tag_of(seq),
                                   tag_of(seq + 1), rope_c, rope_s, n_layers, step, eps_k);
                stamp_wg(l, n_layers, 1, step);
                continue;
            }
            for (int h = blockIdx.x; h < S::HQ; h += gridDim.x) {
                KArgs &a = kargs();
                AttnPrefetch pre;
                attention_prefetch<S>(a, klayer(a, l), h, opaque(pos), opaque(pos0), l, pre);
                attention_head<S>(a, klayer(a, l), h, opaque(pos), opaque(pos0), l, sm.attn, pre,
                                  tag_of(seq), tag_of(seq + 1), n_layers, step, eps_k);
                stamp_wg(l, n_layers, 1, step);
            }
        }
    } else {
        float rope_c = 0.0f, rope_s = 0.0f;  // this lane's RoPE table entry at pos (split)
        if constexpr (SPLIT) {
            float cs[1], sn[1];
            rope_table<D>(pos, kargs().inv_freq, cs, sn);
            rope_c = cs[0];
            rope_s = sn[0];
        }
        // the wave's residual rows of x (lane j: row o0 + j), starting as the embedding row
        uint32_t xown = 0;
        if (o0 < o1) {
            const int lane = tid_x() & 63;
            const uint16_t *erow = (const uint16_t *)(kargs().embed + (size_t)token * H);
            xown = o0 + lane < o1 ? (uint32_t)gptr(erow)[o0 + lane] : 0u;
        }
        for (int l = 0; l < n_layers; l++) {
            const int ln = l + 1 < n_layers ? l + 1 : 0;  // the layer whose q/k/v rows come next
            const unsigned seq = sq0 + PHASES * l;
            // ---- rmsnorm + q/k/v rows (weights requested a phase ahead)
            if (wg_q) {
                if (l == 0) {
                    stage_plain<H>(kargs().embed + (size_t)token * H, sm.vec);
                } else {
                    stage_vector<H, OW>(my_copy<H, S::REPLICAS>(kargs().tx), tag_of(seq - 1), sm.vec,
                                        kargs().error_flag);
                }
            }
            stamp<S>(1 + 4 * l, step);
            stamp_wg(l, n_layers, 0, step);
            // long histories: this workgroup's key and value rows of the split attention, which
            // stream during the q/k/v rows (its q/k/v stores then complete after them)
            SplitKV kv;
            if constexpr (SPLIT) split_request<S>(kargs(), opaque(pos), opaque(pos0), l, kv);
            if (wg_q) wg_rmsnorm<H>(sm.vec, nq, eps_now(), &norm_inv);
            if (q0 < q1) {
                KArgs &a = kargs();
                KLayer &L = klayer(a, l);
                u32x4 xb[NCH];
                lds_chunks<NCH>(sm.vec, xb);
                uint32_t *out = a.tqkv;
                const uint32_t tag = tag_of(seq);
                wave_gemv<NCH, BQ, false, false, SPLIT>(qkv_row(L), q0, q1, xb, pf_qkv,
                                                [=](int r, float y, uint32_t) {
                                                    const uint32_t b = f2bf(y);
                                                    put_tagged(out, r, b, tag);
                                                    return b;
                                                });
            }
            stamp_wg(l, n_layers, 1, step);
            // weights of the next phases, loaded while attention runs
            Rows<NCO, S::B_O> pf_o{};
            Rows<NCH, S::B_GU> pf_g{}, pf_u{};
            Rows<NCI, S::B_DOWN> pf_d{};
            NormW<H> ng{};  // mlp_norm weights
            if constexpr (SPLIT) {
                // long histories: this workgroup's share of the split attention first; the
                // weights after it (requested once the block statistics were out, they held the
                // issuing waves: 4B at 8192 positions, statistics published at 16.1 us against
                // 12.8 on the workgroups without weights; 0.6B at 4096 positions 1180 against
                // 1418 tokens/s; requested after the o poll, the o rows then waited for them:
                // 0.6B 1177 tokens/s; the gate/up rows alone after the o poll: 0.6B 1299, 4B at
                // 8192 positions 419 against 428)
                KArgs &a = kargs();
                split_attention<S>(a, klayer(a, l), opaque(pos), l, sm.split, kv, tag_of(seq),
                                   tag_of(seq + 1), rope_c, rope_s, n_layers, step, eps_k);
            }
            pf_o.load(o_row(klayer(kargs(), l)), o0, o1);
            ng.load(klayer(kargs(), l).mlp_norm);
            {
                KLayer &L = klayer(kargs(), l);
                const bf16 *wg = L.w_gate, *wu = L.w_up;
                pf_g.load([=](int r) { return wg + (size_t)r * H; }, g0, g1);
                pf_u.load([=](int r) { return wu + (size_t)r * H; }, g0, g1);
            }
            if constexpr (S::PF_D == PF_WITH_ATTENTION) pf_d.load(d_row(klayer(kargs(), l)), o0, o1);
            if constexpr (S::PF_QKV == PF_WITH_ATTENTION) {
                nq.load(klayer(kargs(), ln).attn_norm);
                pf_qkv.load(qkv_row(klayer(kargs(), ln)), q0, q1);
            }
            // ---- o rows + residual
            if (wg_o)
                stage_vector<QD, OW>(my_copy<QD, S::REPLICAS>(kargs().tattn), tag_of(seq + 1), sm.vec,
                                     kargs().error_flag);

            stamp<S>(2 + 4 * l, step);
            stamp_wg(l, n_layers, 2, step);
            if constexpr (S::PF_D == PF_AFTER_POLL) pf_d.load(d_row(klayer(kargs(), l)), o0, o1);
            if (wg_o) {
                if (o0 < o1) {
                    u32x4 in[NCO];
                    lds_chunks<NCO>(sm.vec, in);
                    wave_gemv<NCO, S::B_O, S::O_STREAM, true, SPLIT>(
                        o_row(klayer(kargs(), l)), o0, o1, in, pf_o,
                        residual(out_stage, wr0, tag_of(seq + 2)), &xown);
                }
                __syncthreads();
                if ((tid_x() >> 6) == FW) publish_rows<H, S::REPLICAS>(kargs().tx, out_stage, wr0, wr1);
            }
            stamp_wg(l, n_layers, 3, step);
            // ---- rmsnorm + gate/up rows + SwiGLU
            if (wg_g)
                stage_vector<H, OW>(my_copy<H, S::REPLICAS>(kargs().tx), tag_of(seq + 2), sm.vec,
                                    kargs().error_flag);
            stamp<S>(3 + 4 * l, step);
            stamp_wg(l, n_layers, 4, step);
            if constexpr (S::PF_QKV == PF_AFTER_POLL) {
                // the next layer's q/k/v rows stream during gate/up, down and their handoffs
                nq.load(klayer(kargs(), ln).attn_norm);
                pf_qkv.load(qkv_row(klayer(kargs(), ln)), q0, q1);
            }
            if (wg_g) wg_rmsnorm<H>(sm.vec, ng, eps_now(), &norm_inv);
            if (g0 < g1) {
                KArgs &a = kargs();
                KLayer &L = klayer(a, l);
                u32x4 xb[NCH];
                lds_chunks<NCH>(sm.vec, xb);
                uint32_t *hb = a.thb;
                const uint32_t tag = tag_of(seq + 3);
                wave_gemv2<NCH, S::B_GU, S::GU_STREAM, SPLIT>(L.w_gate, L.w_up, g0, g1, xb, pf_g, pf_u,
                                         [=](int r, float g, float u) {
                    const bf16 gb = (bf16)f2bf(g), ub = (bf16)f2bf(u);
                    const float s = round_bf(silu_f32(bf2f(gb)));
                    put_tagged_all<I, S::REPLICAS>(hb, r, f2bf(s * bf2f(ub)), tag);
                });
            }
            stamp_wg(l, n_layers, 5, step);
            if constexpr (S::PF_D == PF_AFTER_COMPUTE) pf_d.load(d_row(klayer(kargs(), l)), o0, o1);
            // ---- down rows + residual
            if (wg_o)
                stage_vector<I, OW>(my_copy<I, S::REPLICAS>(kargs().thb), tag_of(seq + 3), sm.vec,
                                    kargs().error_flag);
            stamp<S>(4 + 4 * l, step);
            stamp_wg(l, n_layers, 6, step);
            if (wg_o) {
                if (o0 < o1) {
                    if constexpr (S::X_LDS_DOWN) {
                        wave_gemv<NCI, S::B_DOWN, S::D_STREAM, true, SPLIT>(
                            d_row(klayer(kargs(), l)), o0, o1, LdsX{(const u32x4 *)sm.vec}, pf_d,
                            residual(out_stage, wr0, tag_of(seq + 4)), &xown);
                    } else {
                        u32x4 in[NCI];
                        lds_chunks<NCI>(sm.vec, in);
                        wave_gemv<NCI, S::B_DOWN, S::D_STREAM, true, SPLIT>(
                            d_row(klayer(kargs(), l)), o0, o1, in, pf_d,
                            residual(out_stage, wr0, tag_of(seq + 4)), &xown);
                    }
                }
                __syncthreads();
                if ((tid_x() >> 6) == FW) publish_rows<H, S::REPLICAS>(kargs().tx, out_stage, wr0, wr1);
            }
            stamp_wg(l, n_layers, 7, step);
            if constexpr (S::PF_QKV == PF_AFTER_COMPUTE) {
                nq.load(klayer(kargs(), ln).attn_norm);
                pf_qkv.load(qkv_row(klayer(kargs(), ln)), q0, q1);
            }
        }
    }

    // ---- final rmsnorm + LM head + argmax over every workgroup (two batches of LM-head rows
    // in flight; the first is requested before the residual stream is polled)
    {
        const unsigned seq_end = sq0 + PHASES * n_layers;  // the next token's tag
        int r0, r1;
        phase_rows<FW>(kargs().vocab, 0, r0, r1);
        const bf16 *lm = kargs().lm_head;
        auto lm_row = [=](int r) { return lm + (size_t)r * H; };
        Rows<NCH, S::B_LM> batch{};
        NormW<H> nf{};  // final_norm weights
        nf.load(kargs().final_norm);
        batch.load(lm_row, r0, r1);
        stage_vector<H, OW>(my_copy<H, S::REPLICAS>(kargs().tx), tag_of(seq_end - 1), sm.vec,
                            kargs().error_flag);
        stamp<S>(1 + 4 * n_layers, step);
        wg_rmsnorm<H>(sm.vec, nf, eps_now(), &norm_inv);
        float best = -__builtin_huge_valf();
        int bidx = INT_MAX;
        if (r0 < r1) {
            KArgs &a = kargs();
            u32x4 xb[NCH];
            lds_chunks<NCH>(sm.vec, xb);
            bf16 *logits = a.logits;
            wave_gemv<NCH, S::B_LM, true, false, SPLIT>(lm_row, r0, r1, xb, batch,
                                          [&](int r, float y, uint32_t) {
                const uint32_t yb = f2bf(y);
                gptr(logits)[r] = (bf16)yb;
                amax_pair(best, bidx, bf2f((bf16)yb), r);
                return yb;
            });
        }
        wave_amax(best, bidx);
        const int lane = tid_x() & 63, w = wave_id();
        if (lane == 0) {
            red_v[w] = best;
            red_i[w] = bidx;
        }
        __syncthreads();
        // this token's tag for the argmax partials (1..16383, 14 bits; consecutive tokens differ)
        const uint32_t ptag = 1u + tag_of(seq_end) % 16383u;
        if (threadIdx.x == 0) {
            KArgs &a = kargs();
            for (int k = 1; k < WAVES; k++) amax_pair(best, bidx, red_v[k], red_i[k]);
            __hip_atomic_store(gptr(a.amax + AMAX_STRIDE * blockIdx.x), amax_word(best, bidx, ptag),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // the workgroup that reduces the partials and publishes the token
        const int reducer = S::ARGMAX_FIRST_WG ? 0 : (int)gridDim.x - 1;
        int chosen = 0;  // the reducer's wave 0: this step's token
        if ((int)blockIdx.x == reducer && w == 0) {
            // the reducer polls every workgroup's partial (its own included) until each carries
            // this token's tag, then reduces them in the order k = lane, lane + 64, ...; every
            // partial of a round of 256 is requested before any is compared, and a lane past
            // the grid reads partial 0 and ignores it
            KArgs &a = kargs();
            float v = -__builtin_huge_valf();
            int idx = INT_MAX;
            for (int k0 = 0; k0 < (int)gridDim.x; k0 += 4 * 64) {
                unsigned long long p[4];
                long long spins = 0;
                for (;;) {
                    bool fresh = true;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int k = k0 + lane + 64 * j, kk = k < (int)gridDim.x ? k : 0;
                        p[j] = __hip_atomic_load(gptr(a.amax + AMAX_STRIDE * kk), __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
                        fresh &= (uint32_t)(p[j] & 0x3fffu) == ptag;
                    }
                    if (fresh) break;
                    if ((++spins & 63) == 0 && wait_gives_up(spins, SPIN_LIMIT, a.error_flag))
                        break;
                }
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int i = (int)((p[j] >> 14) & AMAX_NO_ROW);
                    if (k0 + lane + 64 * j < (int)gridDim.x)
                        amax_pair(v, idx, __uint_as_float((uint32_t)(p[j] >> 32)),
                                  i == AMAX_NO_ROW ? INT_MAX : i);
                }
            }
            wave_amax(v, idx);
            chosen = idx;
            if (lane == 0) {
                if (step + 1 < n_tokens) {
                    // the next token for every workgroup
                    __hip_atomic_store(gptr(a.token_word),
                                       ((unsigned long long)(unsigned)idx << 32) | tag_of(seq_end),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                *gptr(a.next_token) = idx;
                if (a.advance) {
                    const int i = pos - *gptr(a.pos_base);
                    if (i >= 0 && i < a.token_capacity) gptr(a.token_out)[i] = idx;
                    *gptr(a.pos) = pos + 1;
                }
                if (step + 1 >= n_tokens) {
                    *gptr(a.epoch) = seq0 + n_tokens * seq_step;
                    if (a.trace) gptr(a.trace)[2 + 4 * n_layers] = wall_clock64();
                }
            }
        }
        if (step + 1 < n_tokens) {
            // wait for the token this step chose (bounded like every other wait)
            __shared__ int next_tok;
            if (threadIdx.x == 0 && (int)blockIdx.x == reducer) {
                next_tok = chosen;  // the workgroup that chose it
            } else if (threadIdx.x == 0) {
                KArgs &a = kargs();
                unsigned long long tw = 0;
                long long spins = 0;
                for (;;) {
                    tw = __hip_atomic_load(gptr(a.token_word), __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                    if ((uint32_t)tw == tag_of(seq_end)) break;
                    if ((++spins & 63) == 0 && wait_gives_up(spins, SPIN_LIMIT, a.error_flag))
                        break;
                    __builtin_amdgcn_s_sleep(1);
                }
                const int t = (int)(tw >> 32);
                next_tok = t >= 0 && t < a.vocab ? t : 0;
            }
            __syncthreads();
            token = next_tok;
        }
    }
    }
    };
    if constexpr (S::SPLIT_ROLES || SPLIT) {
        if (attn_wg)
            run(std::integral_constant<int, ROLE_ATTN>{});
        else
            run(std::integral_constant<int, ROLE_MATRIX>{});
    } else {
        run(std::integral_constant<int, ROLE_EITHER>{});
    }
}

}  // namespace

// ------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------

// Compile-time shapes with the per-phase rows-per-batch choices (VGPR budget of 2 waves/SIMD)
// for a grid of 256 workgroups: the matrix rows spread over (256 - HQ) * 8 waves. PF: when
// the down rows and the next layer's q/k/v rows are requested (the o and gate/up rows always
// go out while attention runs).
template <int H_, int I_, int HQ_, int HKV_>
struct Shape {
    static constexpr int H = H_, I = I_, HQ = HQ_, HKV = HKV_;
    static constexpr int NMAX = 8192;  // positions a query head attends over (LDS scores)
    // Blocks of 64 positions of history from which attention runs split over (kv head, block)
    // items (the split instance): the crossover of the two attention forms' per-token time,
    // measured on MI355X (64 greedy tokens after an N(0, 1) cache; one workgroup per head /
    // split, tokens/s): 0.6B 384 1778 / 1713, 448 1693 / 1707, 512 1480 / 1683; 1.7B 320 1016 /
    // 993, 384 987 / 990, 448 958 / 985; 4B 448 517 / 504, 512 488 / 511.
    static constexpr int SPLIT_BLOCKS = H <= 1024 ? 8 : H <= 2048 ? 7 : 9;
    // STEP_AUTO's switch to the hipGraph step (at most the kernel's longest history), from the
    // split instance's and the graph's per-token times on MI355X (64 greedy tokens after an
    // N(0, 1) cache; split / graph tokens/s): 0.6B 4096 1450 / 1138, 8128 1213 / 1032; 1.7B
    // 4096 865 / 826, 5120 792 / 809, 6144 791 / 792, 7168 790 / 779, 8128 802 / 766; 4B 4096
    // 467-477 / 464-467, 5120 442 / 460, 6144 448 / 449, 7168 438 / 444, 8192 432-438 / 433-434.
    // The graph leads by at most 4%, between ~5000 and ~7500 positions at 1.7B and 4B, so the
    // kernel runs every position it holds (one launch per generate call). The small test shape
    // keeps a switch (736) so that a generate_greedy crossing it is exercised.
    static constexpr int SWITCH_POS = H < 1024 ? 736 : 1 << 30;
    // The split attention's statistics (block and global max and sum) reduce with their xor-4
    // and xor-8 steps through ds_swizzle (LDS8) where two query heads share a kv head, through
    // DPP at 4B (four): 0.6B after 8192 positions 1235-1237 tokens/s against 1185-1194 with DPP;
    // 4B 441.8-441.9 against 439.0-439.1 with the swizzle (the scores' reduce-scatter through
    // bank_pair_sum in both; alternating runs on one box).
    static constexpr bool SPLIT_STATS_LDS = H <= 2048;
    // q/k/v rows per wave (a prefetched batch; 4B with batches of 2: 575.4-575.9 tokens/s, of 1
    // row 544.7) and
    // where they go. A CU's vector-memory requests complete in order, so a workgroup's poll
    // lands only after every weight request it made before the poll. At 0.6B every matrix
    // workgroup requests its o, gate/up and down rows and the next layer's q/k/v rows while
    // attention runs; the o rows' workgroups (16-143) also held q/k/v rows, 208 KB in all, and
    // their poll of the attention output landed 0.9-2.1 us after the output existed. With the
    // q/k/v rows on the last workgroups, which own no o/down rows, that spread is 0.2 us and
    // the layer ~1 us shorter, less 0.3 us for the longer q/k/v GEMV. 8 rows per wave on the
    // last 64: 2300-2323 against 2282-2292 tokens/s (alternating runs on four boxes); 6 per
    // wave (one batch of 8 with two empty rows) on the last 86, so that the 38 of them that also
    // own gate/up rows request 160 KB instead of 192 KB before their gate/up poll: 2316-2333
    // against 2294-2313 (two boxes; 5 per wave +0.2%, 7 +0.5%). After the reductions' lane
    // exchanges were shortened, 7 per wave on the last 74 measured 2428.4-2428.9 against
    // 2425.0-2425.9 for 6 and 2421.5-2423.9 for 5 (alternating runs on one box), so 7 is kept.
    // Spreading the o/down or gate/up rows over more workgroups instead measured 1-3.5% slower
    // (more pollers per copy).
    // 4B: the wave's 4 rows in one prefetched batch, 592.0-592.3 tokens/s against 581.4-582.5
    // with two batches of 2 (the second requested once the first is computed) and 579.6 with
    // the second requested before it (alternating runs on one box); the split instance keeps
    // batches of 2 (4 spill 156 bytes there)
    static constexpr int B_QKV = H == 1024 ? 8 : H < 1024 ? 4 : H > 2048 ? 4 : 2;
    static constexpr int B_QKV_SPLIT = H > 2048 ? 2 : B_QKV;
    static constexpr bool QKV_AT_END = H == 1024;
    static constexpr int QKV_PER_WAVE = H == 1024 ? 7 : B_QKV;
    static constexpr int B_O = H <= 1024 ? 1 : (HQ * 128 <= 2048 ? 2 : 1);
    static constexpr int B_GU = H <= 1024 ? 2 : 1;
    static constexpr int B_DOWN = 1;
    // 0.6B: 4 rows +0.4% over 8, 16 spills; 4B: 4 rows spill (156 bytes), 561.1 against 575.4
    static constexpr int B_LM = H <= 2048 ? 4 : 2;
    // copies of x, the attention output and the SwiGLU output (at most STEP_REPLICAS), each
    // 1 KB off the 4 KB grid (step_replica_stride). 0.6B: 8 with the q/k/v rows at the end of the
    // grid (2339-2342 tokens/s against 2332-2335 with 4, five alternating rounds on two boxes;
    // 2 copies 2258); before that layout 4 measured faster (2291-2294 against 2280-2282 with 8,
    // 2301 against 2221 with 2 and 2067 with 3). 1.7B and 4B: 4 (1.7B 1115 against 1074 with 8).
    static constexpr int REPLICAS = H == 1024 ? 8 : 4;
    // which workgroup reduces the argmax partials: the first (an attention workgroup) at 4B,
    // 615.2-616.0 tokens/s against 598.9-599.7 for the last one and for a counter of the
    // workgroups done (the last to arrive reducing); the last at 0.6B and 1.7B (0.6B 2472.1,
    // first 2470.0, counter 2473.2; 1.7B 1143.3, first 1136.9, counter 1139.7; alternating
    // runs on one box)
    static constexpr bool ARGMAX_FIRST_WG = H > 2048;
    // 1.7B: the down rows with attention 1050 -> 1075 tokens/s, the q/k/v rows too 1005; 4B
    // (5-token prompt): 575.8-576.4 as below, the q/k/v rows after the gate/up poll 572.6-572.8,
    // the down rows after the o poll 466.2-466.3
    static constexpr int PF_D = H <= 2048 ? PF_WITH_ATTENTION : PF_AFTER_COMPUTE;
    static constexpr int PF_QKV = H <= 1024 ? PF_WITH_ATTENTION : PF_AFTER_COMPUTE;
    // separate token loops for the two roles: 0.6B +1.7%; 1.7B -1.8% (its one shared loop
    // spills the q/k/v prefetch to scratch memory, yet measures faster; measured again after
    // the split instance's change below: 1056 against 1110 tokens/s). The split instance
    // always separates them (1.7B: 208 -> 52 bytes of scratch, 905 -> 979 tokens/s at 512
    // positions, 767 -> 802 at 8128).
    static constexpr bool SPLIT_ROLES = H != 2048;
    // wave 0 of every workgroup stages the vectors and owns no matrix rows (so no weight load
    // is in flight in the polling wave); the larger shapes' vectors need every wave to poll
    static constexpr bool POLLER = false;
    static constexpr bool O_STREAM = H > 1024;
    static constexpr bool D_STREAM = H > 1024;
    // 4B: the gate/up rows (6 per wave) with two batches in flight: 577.7 tokens/s against 570.5
    // with one (alternating runs on one box, 5-token prompt then 256 tokens)
    static constexpr bool GU_STREAM = H > 2048;
    // the down rows read the SwiGLU output from LDS (LdsX) instead of 19 chunk registers per
    // lane, which spilled to scratch memory (95 VGPRs; the reloads queued behind the weight
    // requests): 4B 363 -> 572 tokens/s. At 1.7B (12 chunks) the registers measure 4% faster.
    static constexpr bool X_LDS_DOWN = H > 2048;
};

using Qwen3_06B = Shape<1024, 3072, 16, 8>;
using Qwen3_17B = Shape<2048, 6144, 16, 8>;
using Qwen3_4B = Shape<2560, 9728, 32, 8>;
using SmallTest = Shape<512, 1024, 8, 4>;

// The instance for these shapes: with `split`, the one whose attention runs split over
// (kv head, block) items.
static const void *step_kernel_for(const Config *c, bool split = false) {
    if (c->head_dim != 128) return nullptr;
#define MATCH(S)                                                                            \
    if (c->hidden_size == S::H && c->intermediate_size == S::I && c->n_heads == S::HQ &&    \
        c->n_kv_heads == S::HKV)                                                           \
        return split ? (const void *)step_kernel<S, true> : (const void *)step_kernel<S, false>;
    MATCH(Qwen3_06B) MATCH(Qwen3_17B) MATCH(Qwen3_4B) MATCH(SmallTest)
#undef MATCH
    return nullptr;
}

// The kernel's layout needs workgroups beyond the attention ones (at least as many again) and
// at most 64 residual rows per matrix wave (7 matrix waves per workgroup when wave 0 polls).
static bool step_grid_fits(const Config *c, int grid) {
    // (the split attention's combining workgroups, D / COMB_COLS per query head, are the last
    // ones of the grid)
    if (grid <= 0 || grid > 1024 || grid < 2 * c->n_heads ||
        grid < (128 / COMB_COLS) * c->n_heads)
        return false;
#define QKV_FITS(S)                                                                         \
    if (step_kernel_for(c) == (const void *)step_kernel<S, false> && qkv_first_wg<S>(grid) < S::HQ)   \
        return false;
    QKV_FITS(Qwen3_06B) QKV_FITS(Qwen3_17B) QKV_FITS(Qwen3_4B) QKV_FITS(SmallTest)
#undef QKV_FITS
    // a wave keeps its residual rows of x in one register (lane j: its row j)
    return rows_per_wave(c->hidden_size, (grid - c->n_heads) * WAVES) <= 64;
}

// The tagged vectors' words (each 4 bytes) after the StepWorkspace header.
static size_t step_vector_words(const Config *c) {
    const size_t qd = (size_t)c->n_heads * c->head_dim, kvd = (size_t)c->n_kv_heads * c->head_dim;
    return STEP_REPLICAS * step_replica_stride(c->hidden_size) +
           step_replica_stride(qd + 2 * kvd) + STEP_REPLICAS * step_replica_stride(qd) +
           STEP_REPLICAS * step_replica_stride(c->intermediate_size);
}

int step_split_max_blocks(const Config *c, int max_seq) {
    const int mb = (max_seq + 63) / 64;
    return mb < SPLIT_MAXB ? mb : SPLIT_MAXB;
}

// Offsets (bytes from the workspace start, 256-byte aligned) of the split attention's tagged
// statistics and partials.
static size_t step_stat_offset(const Config *c) {
    return (sizeof(StepWorkspace) + 4 * step_vector_words(c) + 255) / 256 * 256;
}
static size_t step_part_offset(const Config *c, int max_seq) {
    return step_stat_offset(c) + (size_t)c->n_heads * step_split_max_blocks(c, max_seq) * 2 * 8;
}

size_t step_workspace_bytes(const Config *c, int max_seq) {
    return step_part_offset(c, max_seq) +
           (size_t)c->n_heads * step_split_max_blocks(c, max_seq) * c->head_dim * 8;
}

void step_split_buffers(const Config *c, int max_seq, void *ws, unsigned long long **tstat,
                        unsigned long long **tpart) {
    *tstat = (unsigned long long *)((char *)ws + step_stat_offset(c));
    *tpart = (unsigned long long *)((char *)ws + step_part_offset(c, max_seq));
}

bool step_kernel_available(const Config *cfg) {
    // (the argmax partials carry a row index in 18 bits)
    return step_kernel_for(cfg) != nullptr && cfg->vocab_size > 0 && cfg->vocab_size < 0x3ffff &&
           step_grid_fits(cfg, step_kernel_grid());
}

int step_kernel_max_seq(const Config *cfg) {
    const int grid = step_kernel_grid();
    if (!step_kernel_available(cfg) || (2 * grid) % cfg->n_kv_heads != 0) return 0;
    int blocks = SPLIT_ITEMS * (2 * grid / cfg->n_kv_heads);
    if (blocks > SPLIT_MAXB) blocks = SPLIT_MAXB;
    return blocks * 64;
}

bool step_kernel_supported(const Config *cfg, int max_seq) {
    return step_kernel_available(cfg) && max_seq <= step_kernel_max_seq(cfg);
}

int step_kernel_split_blocks(const Config *cfg) {
#define SPLIT(S)                                                                            \
    if (step_kernel_for(cfg) == (const void *)step_kernel<S, false>) return S::SPLIT_BLOCKS;
    SPLIT(Qwen3_06B) SPLIT(Qwen3_17B) SPLIT(Qwen3_4B) SPLIT(SmallTest)
#undef SPLIT
    return 0;
}

// Measured on MI355X, 5-token prompt then 128-256 tokens: 0.6B 2356 tokens/s (step kernel)
// against 1278 (hipGraph), 1.7B 1121 against 893, 4B 578 against 492.
int step_kernel_switch_pos(const Config *cfg) {
    int sw = 0;
#define SWITCH(S)                                                                           \
    if (step_kernel_for(cfg) == (const void *)step_kernel<S, false>) sw = S::SWITCH_POS;
    SWITCH(Qwen3_06B) SWITCH(Qwen3_17B) SWITCH(Qwen3_4B) SWITCH(SmallTest)
#undef SWITCH
    const int longest = step_kernel_max_seq(cfg);
    return sw < longest ? sw : longest;
}

int step_kernel_grid() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    return cus > 1024 ? 1024 : cus;
}

// The workgroups wait for each other's tagged words, so all of them must be resident at once.
// The grid is the CU count and one workgroup fits a CU (checked here with the runtime's
// occupancy query), so a launch on an otherwise idle device places every workgroup at once; the
// step's stream runs nothing beside it. Should a workgroup still start late (another process
// holding CUs), the others' bounded waits let it catch up or end the step with the error flag
// set, never a hang. A plain launch is used, not hipLaunchCooperativeKernel: its co-residency
// check is the one made here, and under rocprofv3 the HIP runtime's exit-time release of the
// cooperative launch's resources ran after the profiler had shut its HSA runtime down and
// faulted (SIGSEGV in libhsa-runtime64, called from libamdhip64's exit handler, on a
// device-mapped page), after every result had been written.
bool step_kernel_launch(const Config *cfg, const StepArgs &args, bool split, int grid,
                        hipStream_t stream) {
    const void *fn = step_kernel_for(cfg, split);
    if (!fn) return llm_fail("step kernel: no specialisation for these shapes");
    if (!step_grid_fits(cfg, grid)) return llm_fail("step kernel: grid of %d does not fit", grid);
    int per_cu = 0, dev = 0, cus = 0;
    if (!HIP_OK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, THREADS, 0)) ||
        !HIP_OK(hipGetDevice(&dev)) ||
        !HIP_OK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)))
        return false;
    if ((long)per_cu * cus < grid)
        return llm_fail("step kernel: %d workgroups cannot all be resident (%d per CU, %d CUs)",
                        grid, per_cu, cus);
    StepArgs a = args;
    void *params[] = {&a};
    return HIP_OK(hipLaunchKernel(fn, dim3(grid), dim3(THREADS), params, 0, stream));
}
