// The whole decode step as one persistent kernel for gfx950: one workgroup of 8 waves per CU,
// cooperatively launched, phases separated by grid barriers. Each phase computes exactly what
// the standalone kernels compute (same per-row, per-head and per-block arithmetic), so the
// step is bit-identical to the multi-kernel step it replaces (src/forward.cu:118-193 order):
//
//   per layer:  rmsnorm + q/k/v rows | QK-norm + RoPE + KV write + attention, one workgroup
//               per query head | o rows + residual | rmsnorm + gate/up rows + SwiGLU |
//               down rows + residual
//   final:      rmsnorm + LM-head rows + per-workgroup argmax; the last workgroup to finish
//               reduces the argmax, records the token and advances the position
//
// Activations cross workgroups (and XCDs, whose L2s are not coherent) only through
// agent-scope atomic loads/stores (global_load/store ... sc1); weights and the KV history are
// read with plain non-temporal loads. A grid barrier is: every thread waits for its own
// stores (s_waitcnt), the workgroup syncs, thread 0 adds to one of 16 counters (one per
// 128-byte line), and wave 0 polls the 16 counters until each has its expected count. Every
// wait is bounded: on timeout the step sets an error flag and all later waits fall through, so
// the grid always drains.
#include <limits.h>
#include <string.h>

#include "common.h"
#include "internal.h"
#include "rope.h"
#include "step.h"

using namespace llm;

namespace {

constexpr int WAVES = 8;                 // waves per workgroup
constexpr int THREADS = 64 * WAVES;
constexpr int BAR_GROUPS = 16;           // barrier counter lines
constexpr long long SPIN_LIMIT = 1 << 22;  // polls before a wait gives up (~ seconds)

// ---------------------------------------------------------------- coherent access

__device__ __forceinline__ uint64_t ld_coh64(const void *p) {
    return __hip_atomic_load(gptr((uint64_t *)p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coh64(void *p, uint64_t v) {
    __hip_atomic_store(gptr((uint64_t *)p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u32x4 ld_coh16(const void *p) {
    const uint64_t a = ld_coh64(p), b = ld_coh64((const char *)p + 8);
    return u32x4{(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)};
}
__device__ __forceinline__ void st_coh_bf16(bf16 *p, uint32_t v) {
    __hip_atomic_store(gptr((unsigned short *)p), (unsigned short)v, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_coh_bf16(const bf16 *p) {
    return __hip_atomic_load(gptr((unsigned short *)p), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_coh_u32(const unsigned *p) {
    return __hip_atomic_load(gptr((unsigned *)p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

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

// ---------------------------------------------------------------- grid barrier

struct Barrier {
    unsigned epoch;  // barriers completed since the counters were zero
    int n;           // barriers passed in this launch

    __device__ __forceinline__ void init(unsigned base) {
        epoch = base;
        n = 0;
        stamp();
    }

    // optional wall-clock stamps (workgroup 0, thread 0)
    __device__ __forceinline__ void stamp() {
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            long long *trace = kargs().trace;
            if (trace) gptr(trace)[n] = wall_clock64();
        }
    }

    // Arrival: this thread's coherent stores are complete (s_waitcnt), the workgroup has
    // synced, and thread 0 adds to its counter line. Loads issued between arrive() and wait()
    // (the next phase's weights) overlap the wait.
    __device__ __forceinline__ void arrive() {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        epoch++;
        if (threadIdx.x == 0)
            __hip_atomic_fetch_add(gptr(&kargs().bar[(blockIdx.x % BAR_GROUPS) * 32]), 1u,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // Wave 0 polls the counter lines until each holds epoch x its member count.
    __device__ __forceinline__ void wait() {
        if (threadIdx.x < 64) {
            unsigned *ctr = kargs().bar;
            int *err = kargs().error_flag;
            const int g = threadIdx.x;
            // workgroups b with b % BAR_GROUPS == g
            const unsigned members = (unsigned)(((int)gridDim.x - g + BAR_GROUPS - 1) / BAR_GROUPS);
            const unsigned need = g < BAR_GROUPS ? epoch * members : 0u;
            long long spins = 0;
            for (;;) {
                const unsigned c = g < BAR_GROUPS
                                       ? __hip_atomic_load(gptr(&ctr[g * 32]), __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT)
                                       : 0u;
                if (__all((int)(c - need) >= 0)) break;
                if (++spins > SPIN_LIMIT ||
                    __hip_atomic_load(gptr(err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                    if (threadIdx.x == 0)
                        __hip_atomic_store(gptr(err), 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
            }
        }
        __syncthreads();
        n++;
        stamp();
    }

    __device__ __forceinline__ void sync() {
        arrive();
        wait();
    }
};

// ---------------------------------------------------------------- wave building blocks

// The input vector of a GEMV as this lane's chunks: chunk lane + 64k of the vector.
template <int NC>
__device__ __forceinline__ void load_vec_coh(const bf16 *v, u32x4 (&out)[NC]) {
    const int lane = tid_x() & 63;
#pragma unroll
    for (int k = 0; k < NC; k++) out[k] = ld_coh16(v + 8 * (lane + 64 * k));
}

// RMSNorm of a row of 512*NC elements held as chunks (rmsnorm_wave_kernel arithmetic).
template <int NC>
__device__ __forceinline__ void wave_rmsnorm(const u32x4 (&x)[NC], const bf16 *w, float eps,
                                             u32x4 (&out)[NC]) {
    const int lane = tid_x() & 63;
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < NC; k++) acc = dot8(x[k], x[k], acc);
    const float total = wave_sum(acc);
    const float inv = 1.0f / sqrtf(total / (float)(512 * NC) + eps);
#pragma unroll
    for (int k = 0; k < NC; k++) {
        const u32x4 wv = ld16(w + 8 * (lane + 64 * k));
        float r[8];
#pragma unroll
        for (int e = 0; e < 8; e++) r[e] = round_bf(elem(x[k], e) * inv) * elem(wv, e);
        out[k] = u32x4{pack2(r[0], r[1]), pack2(r[2], r[3]), pack2(r[4], r[5]), pack2(r[6], r[7])};
    }
}

// B rows of NC chunks each, held in registers: lane l has chunk l + 64k of every row. `rowp`
// maps a row index to its data, so a batch can straddle the q/k/v matrices.
template <int NC, int B>
struct Rows {
    u32x4 w[B][NC];
    template <class RowP>
    __device__ __forceinline__ void load(RowP rowp, int r, int r1) {
        const int lane = tid_x() & 63;
#pragma unroll
        for (int i = 0; i < B; i++) {
            const bf16 *row = rowp(min(r + i, r1 - 1));
#pragma unroll
            for (int k = 0; k < NC; k++) w[i][k] = ld16_nt(row + 8 * (lane + 64 * k));
        }
    }
};

// Rows [r0, r1) against xin, B rows per batch, the first batch already in `batch` (loaded
// before the barrier that precedes this phase); epi(row, sum) runs in one of lanes 0..B-1
// (gemv_kernel arithmetic: per-lane fma over the chunks in order, then the wave tree).
template <int NC, int B, class RowP, class Epi>
__device__ __forceinline__ void wave_gemv(RowP rowp, int r0, int r1, const u32x4 (&xin)[NC],
                                          Rows<NC, B> &batch, Epi epi, uint32_t lane_val = 0) {
    const int lane = tid_x() & 63;
    for (int r = r0; r < r1; r += B) {
        if (r != r0) batch.load(rowp, r, r1);
        float part[B];
#pragma unroll
        for (int i = 0; i < B; i++) {
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < NC; k++) acc = dot8(batch.w[i][k], xin[k], acc);
            part[i] = acc;
        }
        const float t = wave_sum_scatter<B>(part);
        const int row = r + scatter_row<B>(lane);
        // lane_val of lane (row - r0): a per-row value the caller loaded beforehand
        const uint32_t v = (uint32_t)__shfl((int)lane_val, min(row - r0, 63));
        if (lane < B && row < r1) epi(row, t, v);
    }
}

// Lane l < r1 - r0 (at most 64 rows): the bf16 bits of x[r0 + l], read coherently.
__device__ __forceinline__ uint32_t load_rows_coh(const bf16 *x, int r0, int r1) {
    const int lane = tid_x() & 63;
    return r0 + lane < r1 ? ld_coh_bf16(x + r0 + lane) : 0u;
}

// The residual rows [r0, r1) of this wave before layer l's o rows. Layer 0 reads them from the
// embedding row (the value workgroup 0 copies into x, which other workgroups may only read
// after a completed barrier); later layers read x, whose rows this wave itself wrote last.
__device__ __forceinline__ uint32_t residual_rows(KArgs &a, int l, int token, int H, int r0,
                                                  int r1) {
    if (l == 0) {
        const int lane = tid_x() & 63;
        const uint16_t *erow = (const uint16_t *)(a.embed + (size_t)token * H);
        return r0 + lane < r1 ? (uint32_t)gptr(erow)[r0 + lane] : 0u;
    }
    return load_rows_coh(a.x, r0, r1);
}

// gate and up rows together (gate_up_kernel arithmetic); first batch preloaded.
template <int NC, int B, class Epi>
__device__ __forceinline__ void wave_gemv2(const bf16 *Wg, const bf16 *Wu, int r0, int r1,
                                           const u32x4 (&xin)[NC], Rows<NC, B> &gb,
                                           Rows<NC, B> &ub, Epi epi) {
    const int lane = tid_x() & 63;
    constexpr int COLS = 512 * NC;
    for (int r = r0; r < r1; r += B) {
        if (r != r0) {
            gb.load([&](int rr) { return Wg + (size_t)rr * COLS; }, r, r1);
            ub.load([&](int rr) { return Wu + (size_t)rr * COLS; }, r, r1);
        }
        float pg[B], pu[B];
#pragma unroll
        for (int i = 0; i < B; i++) {
            float ag = 0.0f, au = 0.0f;
#pragma unroll
            for (int k = 0; k < NC; k++) {
                ag = dot8(gb.w[i][k], xin[k], ag);
                au = dot8(ub.w[i][k], xin[k], au);
            }
            pg[i] = ag;
            pu[i] = au;
        }
        const float tg = wave_sum_scatter<B>(pg), tu = wave_sum_scatter<B>(pu);
        const int row = r + scatter_row<B>(lane);
        if (lane < B && row < r1) epi(row, tg, tu);
    }
}


constexpr int PV_ROUND = 4;     // 64-position blocks per PV round (two per wave)
constexpr int SCORE_LOADS = 8;  // keys per lane per scores round (8 * 4 * WAVES positions)

// History keys (positions < pos, written by earlier steps) of the first scores round of one
// head, loaded before the barrier that precedes attention. Slots at or beyond pos hold zeros;
// attention_head substitutes the current position's key.
struct AttnPrefetch {
    u32x4 k[SCORE_LOADS];
};

template <class S>
struct AttnSmem {
    static constexpr int D = 128;
    u32x4 q[D / 8];                 // roped query head
    u32x4 k[D / 8];                 // roped key of the current position
    u32x4 v[D / 8];                 // value of the current position
    float sc[S::NMAX];              // scores, then probabilities
    float st[S::NMAX / 64][2];      // block max, block sum
    float gm[2];                    // global max, sum
    float quarter[PV_ROUND][4][D];  // PV partial of each (block, quarter) of a round
    float out[D];                   // running sum over blocks
};

// One query head's attention at `pos` (attn_scores/pv/combine arithmetic, one workgroup):
// wave 0 normalises and rotates q (and k, v for the workgroup that owns the cache write),
// then scores, block statistics, the global max/sum, probabilities, PV per 64-position block
// in four quarters, and the in-order combine.
// Position of key slot u of this lane in the scores round starting at `base`, and of value
// slot (j, it) in the PV round starting at block c0 (16 lanes per position, 8 waves).
__device__ __forceinline__ int key_slot(int base, int u) {
    return base + u * 4 * WAVES + (tid_x() >> 6) * 4 + ((tid_x() & 63) >> 4);
}
__device__ __forceinline__ int value_slot(int c0, int j, int it) {
    const int w = tid_x() >> 6;
    return (c0 + (w >> 2) + 2 * j) * 64 + (w & 3) * 16 + it * 4 + ((tid_x() & 63) >> 4);
}

template <class S>
__device__ __forceinline__ void attention_prefetch(KArgs &a, int h, int pos, int layer,
                                                   AttnPrefetch &p) {
    constexpr int D = 128, REP = S::HQ / S::HKV, KVD = S::HKV * D;
    const int g = h / REP, Lp = tid_x() & 15;
    const bf16 *kc = a.key_cache + (size_t)layer * a.max_seq * KVD + g * D + 8 * Lp;
#pragma unroll
    for (int u = 0; u < SCORE_LOADS; u++) {
        const int t = key_slot(0, u);
        p.k[u] = t < pos ? ld16_nt(kc + (size_t)t * KVD) : u32x4{0, 0, 0, 0};
    }
}

template <class S>
__device__ __forceinline__ void attention_head(KArgs &a, KLayer &L, int h, int pos, int layer,
                               AttnSmem<S> &sm, AttnPrefetch &pre, bool prefetched) {
    constexpr int D = 128, REP = S::HQ / S::HKV, KVD = S::HKV * D;
    const int lane = tid_x() & 63, w = tid_x() >> 6;
    const int g = h / REP;
    const bool owner = (h % REP) == 0;  // writes k', v into the cache
    bf16 *kc = a.key_cache + (size_t)layer * a.max_seq * KVD;
    bf16 *vc = a.value_cache + (size_t)layer * a.max_seq * KVD;
    const int n = pos + 1;
    const int nb = (n + 63) / 64;
    if (!prefetched) attention_prefetch<S>(a, h, pos, layer, pre);
    const u32x4 zero{0, 0, 0, 0};
    // history values of the first PV round, requested now so their latency overlaps the
    // prologue, the scores and the softmax
    u32x4 vv[PV_ROUND / 2][4];
    auto load_v = [&](int c0) {
        const int Lq = tid_x() & 15;
#pragma unroll
        for (int j = 0; j < PV_ROUND / 2; j++)
#pragma unroll
            for (int it = 0; it < 4; it++) {
                const int t = value_slot(c0, j, it);
                vv[j][it] = t < pos ? ld16_nt(vc + (size_t)t * KVD + g * D + 8 * Lq) : zero;
            }
    };
    load_v(0);

    if (w == 0) {
        // lanes 0-7: the query head, 8-15: the key head, 16-23: the value (copy only)
        const int slot = lane >> 3, Lh = lane & 7;
        float cs[1], sn[1];
        rope_table<D>(pos, a.inv_freq, cs, sn);
        const bf16 *src = slot == 1 ? a.k + g * D : slot == 2 ? a.v + g * D : a.q + h * D;
        const bf16 *nw = slot == 1 ? L.k_norm : L.q_norm;
        const u32x4 xa = ld_coh16(src + 8 * Lh), xb = ld_coh16(src + 64 + 8 * Lh);
        const u32x4 wa = ld16(nw + 8 * Lh), wb = ld16(nw + 64 + 8 * Lh);
        u32x4 ya, yb, oa, ob;
        norm_rope<D>(xa, xb, wa, wb, a.eps, cs, sn, Lh, ya, yb, oa, ob);
        const size_t row = (size_t)pos * KVD + g * D;
        if (slot == 0) {
            sm.q[Lh] = oa;
            sm.q[8 + Lh] = ob;
        } else if (slot == 1) {
            sm.k[Lh] = oa;
            sm.k[8 + Lh] = ob;
            if (owner) {
                st16(kc + row + 8 * Lh, oa);
                st16(kc + row + 64 + 8 * Lh, ob);
            }
        } else if (slot == 2) {
            sm.v[Lh] = xa;
            sm.v[8 + Lh] = xb;
            if (owner) {
                st16(vc + row + 8 * Lh, xa);
                st16(vc + row + 64 + 8 * Lh, xb);
            }
        }
    }
    __syncthreads();

    const int G = lane >> 4, Lp = lane & 15, qtr = w & 3;
    // scores: 16 lanes per position; a round is SCORE_LOADS keys per lane
    {
        const u32x4 qv = sm.q[Lp];
        const u32x4 kcur = sm.k[Lp];
        for (int base = 0; base < n; base += SCORE_LOADS * 4 * WAVES) {
            u32x4 kv[SCORE_LOADS];
#pragma unroll
            for (int u = 0; u < SCORE_LOADS; u++) {
                const int t = key_slot(base, u);
                if (base == 0) kv[u] = t == pos ? kcur : pre.k[u];
                else kv[u] = t < pos ? ld16_nt(kc + (size_t)t * KVD + g * D + 8 * Lp)
                                     : (t == pos ? kcur : zero);
            }
#pragma unroll
            for (int u = 0; u < SCORE_LOADS; u++) {
                const int t = key_slot(base, u);
                const float d = group_sum<16>(dot8(qv, kv[u], 0.0f));
                const float s = round_bf(round_bf(d) * a.scale);
                if (Lp == 0 && t < n) sm.sc[t] = s;
            }
        }
    }
    __syncthreads();
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
    // PV in rounds of PV_ROUND blocks: wave w takes blocks c0 + w/4 + 2j and quarter w % 4 of
    // each (slots quarter*16 + it*4 + G); the quarters meet in order, the blocks are added in order
    const u32x4 vcur = sm.v[Lp];
    for (int c0 = 0; c0 < nb; c0 += PV_ROUND) {
        if (c0 > 0) load_v(c0);
#pragma unroll
        for (int j = 0; j < PV_ROUND / 2; j++) {
            float acc[8];
#pragma unroll
            for (int e = 0; e < 8; e++) acc[e] = 0.0f;
#pragma unroll
            for (int it = 0; it < 4; it++) {
                const int t = value_slot(c0, j, it);
                if (t < n) {
                    const float p = sm.sc[t];
                    const u32x4 vt = t == pos ? vcur : vv[j][it];
#pragma unroll
                    for (int e = 0; e < 8; e++) acc[e] = fmaf(p, elem(vt, e), acc[e]);
                }
            }
#pragma unroll
            for (int e = 0; e < 8; e++) acc[e] = butterfly_sum<16, 64>(acc[e]);
            if (G == 0)
#pragma unroll
                for (int e = 0; e < 8; e++) sm.quarter[(w >> 2) + 2 * j][qtr][8 * Lp + e] = acc[e];
        }
        __syncthreads();
        if (threadIdx.x < D) {
            const int d = threadIdx.x;
            for (int bi = 0; bi < PV_ROUND && c0 + bi < nb; bi++) {
                const float part = ((sm.quarter[bi][0][d] + sm.quarter[bi][1][d]) +
                                    sm.quarter[bi][2][d]) +
                                   sm.quarter[bi][3][d];
                sm.out[d] = c0 + bi == 0 ? part : sm.out[d] + part;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x < D) st_coh_bf16(a.attn_out + h * D + threadIdx.x, f2bf(sm.out[threadIdx.x]));
}

// ---------------------------------------------------------------- the step

// Rows [r0, r1) of a phase with R rows owned by this wave. Wave 0 of each workgroup polls the
// grid barrier and owns no rows: vector loads return in order, so a poller with weight loads
// in flight would see the barrier only once they had landed.
__device__ __forceinline__ void phase_rows(int R, int &r0, int &r1) {
    const int w = __builtin_amdgcn_readfirstlane(tid_x() >> 6);
    const int nw = gridDim.x * (WAVES - 1);
    const int per = (R + nw - 1) / nw;
    const int gw = blockIdx.x * (WAVES - 1) + w - 1;
    r0 = w == 0 ? R : min(R, gw * per);
    r1 = w == 0 ? R : min(R, r0 + per);
}

template <class S>
__global__ __launch_bounds__(THREADS) void step_kernel(StepArgs) {
    constexpr int H = S::H, I = S::I, D = 128, QD = S::HQ * D, KVD = S::HKV * D;
    constexpr int NCH = H / 512, NCO = QD / 512, NCI = I / 512;
    __shared__ AttnSmem<S> sm;
    __shared__ float red_v[WAVES];
    __shared__ int red_i[WAVES];
    __shared__ int last_wg;
    const int lane = tid_x() & 63, w = tid_x() >> 6;

    Barrier bar;
    int token, pos, n_layers;
    {
        KArgs &a = kargs();
        bar.init(*gptr(a.epoch));
        token = *gptr(a.next_token);
        pos = *gptr(a.pos);
        n_layers = a.n_layers;
        if (pos < 0 || pos >= a.max_seq || token < 0 || token >= a.vocab) {
            if (blockIdx.x == 0 && threadIdx.x == 0) *gptr(a.error_flag) = 1;
            return;  // every workgroup reads the same values and leaves before any barrier
        }
        if (blockIdx.x == 0) {  // the residual stream starts as the embedding row
            const bf16 *erow = a.embed + (size_t)token * H;
            for (int c = threadIdx.x; c < H / 8; c += THREADS) {
                const u32x4 v = ld16(erow + 8 * c);
                st_coh64(a.x + 8 * c, (uint64_t)v.x | ((uint64_t)v.y << 32));
                st_coh64(a.x + 8 * c + 4, (uint64_t)v.z | ((uint64_t)v.w << 32));
            }
        }
    }

    // rows of each phase owned by this wave; o and down share the partition, so the residual
    // rows a wave updates are its own (at most 64 per wave, checked by the host)
    int q0, q1, o0, o1, g0, g1;
    phase_rows(QD + 2 * KVD, q0, q1);
    phase_rows(H, o0, o1);
    phase_rows(I, g0, g1);

    auto qkv_row = [](KLayer &L) {
        const bf16 *wq = L.wq, *wk = L.wk, *wv = L.wv;
        return [=](int r) -> const bf16 * {
            return r < QD ? wq + (size_t)r * H
                          : r < QD + KVD ? wk + (size_t)(r - QD) * H : wv + (size_t)(r - QD - KVD) * H;
        };
    };
    auto residual = [](bf16 *x) {
        return [=](int r, float y, uint32_t xr) {
            st_coh_bf16(x + r, f2bf(bf2f((bf16)xr) + bf2f((bf16)f2bf(y))));
        };
    };

    Rows<NCH, S::B_QKV> pf_qkv;
    if (q0 < q1) pf_qkv.load(qkv_row(klayer(kargs(), 0)), q0, q1);

    for (int l = 0;; l++) {
        // ---- rmsnorm + q/k/v rows (weights prefetched during the previous barrier)
        if (q0 < q1) {
            KArgs &a = kargs();
            KLayer &L = klayer(a, l);
            u32x4 x[NCH], xb[NCH];
            if (l == 0) {
                const bf16 *erow = a.embed + (size_t)token * H;
#pragma unroll
                for (int k = 0; k < NCH; k++) x[k] = ld16(erow + 8 * (lane + 64 * k));
            } else {
                load_vec_coh<NCH>(a.x, x);
            }
            wave_rmsnorm<NCH>(x, L.attn_norm, a.eps, xb);
            bf16 *q = a.q, *k = a.k, *v = a.v;
            wave_gemv<NCH, S::B_QKV>(qkv_row(L), q0, q1, xb, pf_qkv, [=](int r, float y, uint32_t) {
                bf16 *dst = r < QD ? q + r : r < QD + KVD ? k + (r - QD) : v + (r - QD - KVD);
                st_coh_bf16(dst, f2bf(y));
            });
        }
        // ---- QK-norm + RoPE + KV write + attention, one workgroup per query head. Attention
        // workgroups load their first K/V history rounds during the barrier and the o weights
        // after attention; the others load the o weights at once. Both paths pass two barriers.
        Rows<NCO, S::B_O> pf_o;
        auto o_row = [](KLayer &L) {
            const bf16 *wo = L.wo;
            return [=](int r) { return wo + (size_t)r * QD; };
        };
        uint32_t xres;
        if (blockIdx.x < S::HQ) {
            AttnPrefetch pre;
            bar.arrive();
            attention_prefetch<S>(kargs(), blockIdx.x, opaque(pos), l, pre);
            bar.wait();
            for (int h = blockIdx.x; h < S::HQ; h += gridDim.x) {
                KArgs &a = kargs();
                attention_head<S>(a, klayer(a, l), h, opaque(pos), l, sm, pre,
                                  h == (int)blockIdx.x);
            }
            bar.arrive();
            if (o0 < o1) pf_o.load(o_row(klayer(kargs(), l)), o0, o1);
            xres = residual_rows(kargs(), l, token, H, o0, o1);
            bar.wait();
        } else {
            bar.arrive();
            if (o0 < o1) pf_o.load(o_row(klayer(kargs(), l)), o0, o1);
            xres = residual_rows(kargs(), l, token, H, o0, o1);
            bar.wait();
            bar.arrive();
            bar.wait();
        }
        // ---- o rows + residual
        if (o0 < o1) {
            u32x4 in[NCO];
            load_vec_coh<NCO>(kargs().attn_out, in);
            wave_gemv<NCO, S::B_O>(o_row(klayer(kargs(), l)), o0, o1, in, pf_o,
                                   residual(kargs().x), xres);
        }
        Rows<NCH, S::B_GU> pf_g, pf_u;
        bar.arrive();
        if (g0 < g1) {
            KLayer &L = klayer(kargs(), l);
            const bf16 *wg = L.w_gate, *wu = L.w_up;
            pf_g.load([=](int r) { return wg + (size_t)r * H; }, g0, g1);
            pf_u.load([=](int r) { return wu + (size_t)r * H; }, g0, g1);
        }
        bar.wait();
        // ---- rmsnorm + gate/up rows + SwiGLU
        if (g0 < g1) {
            KArgs &a = kargs();
            KLayer &L = klayer(a, l);
            u32x4 x[NCH], xb[NCH];
            load_vec_coh<NCH>(a.x, x);
            wave_rmsnorm<NCH>(x, L.mlp_norm, a.eps, xb);
            bf16 *hb = a.hb;
            wave_gemv2<NCH, S::B_GU>(L.w_gate, L.w_up, g0, g1, xb, pf_g, pf_u,
                                     [=](int r, float g, float u) {
                const bf16 gb = (bf16)f2bf(g), ub = (bf16)f2bf(u);
                const float s = round_bf(silu_f32(bf2f(gb)));
                st_coh_bf16(hb + r, f2bf(s * bf2f(ub)));
            });
        }
        Rows<NCI, S::B_DOWN> pf_d;
        auto d_row = [](KLayer &L) {
            const bf16 *wd = L.w_down;
            return [=](int r) { return wd + (size_t)r * I; };
        };
        bar.arrive();
        if (o0 < o1) pf_d.load(d_row(klayer(kargs(), l)), o0, o1);
        xres = load_rows_coh(kargs().x, o0, o1);
        bar.wait();
        // ---- down rows + residual
        if (o0 < o1) {
            u32x4 in[NCI];
            load_vec_coh<NCI>(kargs().hb, in);
            wave_gemv<NCI, S::B_DOWN>(d_row(klayer(kargs(), l)), o0, o1, in, pf_d,
                                      residual(kargs().x), xres);
        }
        if (l + 1 == n_layers) break;
        bar.arrive();
        if (q0 < q1) pf_qkv.load(qkv_row(klayer(kargs(), l + 1)), q0, q1);
        bar.wait();
    }

    // ---- final rmsnorm + LM head + argmax (the first batch of LM-head rows is loaded during
    // the last barrier)
    {
        int r0, r1;
        phase_rows(kargs().vocab, r0, r1);
        const bf16 *lm = kargs().lm_head;
        auto lm_row = [=](int r) { return lm + (size_t)r * H; };
        Rows<NCH, S::B_LM> batch;
        bar.arrive();
        if (r0 < r1) batch.load(lm_row, r0, r1);
        bar.wait();
        float best = -__builtin_huge_valf();
        int bidx = INT_MAX;
        if (r0 < r1) {
            KArgs &a = kargs();
            u32x4 x[NCH], xb[NCH];
            load_vec_coh<NCH>(a.x, x);
            wave_rmsnorm<NCH>(x, a.final_norm, a.eps, xb);
            bf16 *logits = a.logits;
            wave_gemv<NCH, S::B_LM>(lm_row, r0, r1, xb, batch, [&](int r, float y, uint32_t) {
                const uint32_t yb = f2bf(y);
                gptr(logits)[r] = (bf16)yb;
                amax_pair(best, bidx, bf2f((bf16)yb), r);
            });
        }
        wave_amax(best, bidx);
        if (lane == 0) {
            red_v[w] = best;
            red_i[w] = bidx;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            KArgs &a = kargs();
            for (int k = 1; k < WAVES; k++) amax_pair(best, bidx, red_v[k], red_i[k]);
            __hip_atomic_store(gptr((unsigned *)&a.amax_val[blockIdx.x]), __float_as_uint(best),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(gptr(&a.amax_idx[blockIdx.x]), bidx, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0);
            const unsigned done = __hip_atomic_fetch_add(gptr(a.final_ctr), 1u, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            last_wg = done == gridDim.x - 1;
        }
        __syncthreads();
        if (last_wg && w == 0) {
            // the last workgroup: every partial is complete; the wave reduces them in parallel
            KArgs &a = kargs();
            float v = -__builtin_huge_valf();
            int idx = INT_MAX;
            for (int k = lane; k < (int)gridDim.x; k += 64)
                amax_pair(v, idx,
                          __uint_as_float(__hip_atomic_load(gptr((unsigned *)&a.amax_val[k]),
                                                            __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT)),
                          __hip_atomic_load(gptr(&a.amax_idx[k]), __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT));
            wave_amax(v, idx);
            if (lane == 0) {
                *gptr(a.next_token) = idx;
                if (a.advance) {
                    const int i = pos - *gptr(a.pos_base);
                    if (i >= 0 && i < a.token_capacity) gptr(a.token_out)[i] = idx;
                    *gptr(a.pos) = pos + 1;
                }
                *gptr(a.final_ctr) = 0;
                *gptr(a.epoch) = bar.epoch;
                if (a.trace) gptr(a.trace)[bar.n + 1] = wall_clock64();
            }
        }
    }
}

}  // namespace

// ------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------

// Compile-time shapes with the per-phase rows-per-batch choices (VGPR budget of 2 waves/SIMD).
template <int H_, int I_, int HQ_, int HKV_>
struct Shape {
    static constexpr int H = H_, I = I_, HQ = HQ_, HKV = HKV_;
    static constexpr int NMAX = 8192;  // positions a query head attends over (LDS scores)
    static constexpr int B_QKV = H <= 1024 ? 4 : 2;
    static constexpr int B_O = HQ * 128 <= 2048 ? 2 : 1;
    static constexpr int B_GU = H <= 1024 ? 2 : 1;
    static constexpr int B_DOWN = 1;
    static constexpr int B_LM = H <= 1024 ? 8 : (H <= 2048 ? 4 : 2);
};

using Qwen3_06B = Shape<1024, 3072, 16, 8>;
using Qwen3_17B = Shape<2048, 6144, 16, 8>;
using Qwen3_4B = Shape<2560, 9728, 32, 8>;
using SmallTest = Shape<512, 1024, 8, 4>;

static const void *step_kernel_for(const Config *c) {
    if (c->head_dim != 128) return nullptr;
#define MATCH(S)                                                                            \
    if (c->hidden_size == S::H && c->intermediate_size == S::I && c->n_heads == S::HQ &&    \
        c->n_kv_heads == S::HKV)                                                           \
        return (const void *)step_kernel<S>;
    MATCH(Qwen3_06B) MATCH(Qwen3_17B) MATCH(Qwen3_4B) MATCH(SmallTest)
#undef MATCH
    return nullptr;
}

bool step_kernel_supported(const Config *cfg, int max_seq) {
    return step_kernel_for(cfg) != nullptr && max_seq <= 8192 && cfg->vocab_size > 0;
}

int step_kernel_grid() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    return cus;
}

bool step_kernel_launch(const Config *cfg, const StepArgs &args, int grid, hipStream_t stream) {
    const void *fn = step_kernel_for(cfg);
    if (!fn) return llm_fail("step kernel: no specialisation for these shapes");
    StepArgs a = args;
    void *params[] = {&a};
    return HIP_OK(hipLaunchCooperativeKernel(fn, dim3(grid), dim3(THREADS), params, 0, stream));
}
