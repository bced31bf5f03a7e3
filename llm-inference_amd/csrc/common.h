// Shared host/device helpers of the gfx950 decode library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "errors.h"
#include "llm_amd/kernels.h"

namespace llm {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Every buffer the library touches is device (global) memory. Pointers that the compiler
// cannot trace to a kernel argument (fields of structs in memory) would otherwise be accessed
// with FLAT instructions, which also count against lgkmcnt, so every later LDS or scalar wait
// would wait for them too; the casts make them global_load/global_store.
#define LLM_GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ LLM_GLOBAL T *gptr(T *p) {
    return (LLM_GLOBAL T *)p;
}
template <class T>
__device__ __forceinline__ const LLM_GLOBAL T *gptr(const T *p) {
    return (const LLM_GLOBAL T *)p;
}

__device__ __forceinline__ u32x4 ld16(const void *p) { return *gptr((const u32x4 *)p); }
// Streamed operands (weights, KV cache) are read non-temporally so they do not evict the
// small reused vectors from L2.
__device__ __forceinline__ u32x4 ld16_nt(const void *p) {
    return __builtin_nontemporal_load(gptr((const u32x4 *)p));
}
__device__ __forceinline__ void st16(void *p, u32x4 v) { *gptr((u32x4 *)p) = v; }

// Word 3 of a raw buffer descriptor (CDNA): 32-bit data format, no swizzle, no stride; loads at
// offsets past the descriptor's size return zero without a memory access.
constexpr int BUFFER_FLAGS = 0x00020000;
// Cache policy operand of a buffer load: non-temporal, as ld16_nt.
constexpr int BUFFER_NT = 2;
// Cache policy operand of a buffer load with the coherence of an agent-scope atomic load (sc1).
constexpr int BUFFER_SC1 = 16;

// bf16 element e of a packed 16-byte chunk (element 0 in the low half of dword 0).
__device__ __forceinline__ float lo_f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// fp32 -> bf16 round to nearest even; NaN stays NaN with the quiet bit set (the upper half of
// the fp32 pattern | 0x40), denormals rounded like normals: the arithmetic of the integer form
// (u + 0x7fff + ((u >> 16) & 1)) >> 16 for non-NaN u. gfx950 does it in one instruction
// (v_cvt_pk_bf16_f32, two values at once), which gives the same bits for every input class.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f2bf(float f) {
    const __bf16 b = (__bf16)f;
    uint16_t u;
    __builtin_memcpy(&u, &b, 2);
    return u;
}
__device__ __forceinline__ float round_bf(float f) { return __uint_as_float(f2bf(f) << 16); }
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    uint32_t u;
    __builtin_memcpy(&u, &v, 4);
    return u;
}

// Element e (0..7) of a chunk as fp32.
__device__ __forceinline__ float elem(const u32x4 &v, int e) {
    uint32_t w = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
    return (e & 1) ? hi_f(w) : lo_f(w);
}

// acc += a[e] * b[e] for e = 0..7 in order (products of bf16 are exact in fp32).
__device__ __forceinline__ float dot8(const u32x4 &a, const u32x4 &b, float acc) {
    acc = fmaf(lo_f(a.x), lo_f(b.x), acc);
    acc = fmaf(hi_f(a.x), hi_f(b.x), acc);
    acc = fmaf(lo_f(a.y), lo_f(b.y), acc);
    acc = fmaf(hi_f(a.y), hi_f(b.y), acc);
    acc = fmaf(lo_f(a.z), lo_f(b.z), acc);
    acc = fmaf(hi_f(a.z), hi_f(b.z), acc);
    acc = fmaf(lo_f(a.w), lo_f(b.w), acc);
    acc = fmaf(hi_f(a.w), hi_f(b.w), acc);
    return acc;
}

// threadIdx.x, opaque to the optimiser: lane-derived values (offsets, masks) are recomputed
// where they are used instead of being hoisted out of long loops and held in registers.
__device__ __forceinline__ int tid_x() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// The wave's index in the workgroup as a wave-uniform (scalar) value, so branches on it are
// scalar branches and not per-lane masks.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(tid_x() >> 6); }

// The value of lane (lane ^ S), S a power of two below 64, without an LDS address: DPP
// quad_perm for 1 and 2; for 4 two DPP moves into one register, row_shl:4 (lane l reads
// l + 4) into banks 0 and 2 (lanes 0-3 and 8-11 of each 16-lane row) and row_shr:4 (l - 4)
// into banks 1 and 3; DPP row_ror:8 for 8 (a rotation by 8 within a row); v_permlane16_swap /
// v_permlane32_swap of the register with itself for 16 / 32 (afterwards the first result holds
// the even rows / the low half in both rows / halves of each pair and the second the odd rows /
// the high half). With LDS8 the xor-4 and xor-8 steps are ds_swizzles (bitmask mode: and 0x1f,
// xor S): they then run on the LDS unit beside the VALU, which pays where many reductions run
// side by side (the DPP forms need wait states and VALU moves of their own), while the DPP forms
// are shorter on a single dependent chain.
template <int S, bool LDS8 = false>
__device__ __forceinline__ int xor_lane(int x) {
    static_assert(S > 0 && S < 64 && (S & (S - 1)) == 0, "xor distance");
    if constexpr (S == 1) {
        return __builtin_amdgcn_mov_dpp(x, 0xB1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
    } else if constexpr (S == 2) {
        return __builtin_amdgcn_mov_dpp(x, 0x4E, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
    } else if constexpr (S == 4 && !LDS8) {
        const int t = __builtin_amdgcn_update_dpp(x, x, 0x104, 0xf, 0x5, false);  // row_shl:4
        return __builtin_amdgcn_update_dpp(t, x, 0x114, 0xf, 0xA, false);         // row_shr:4
    } else if constexpr (S == 8 && !LDS8) {
        return __builtin_amdgcn_mov_dpp(x, 0x128, 0xf, 0xf, false);  // row_ror:8
    } else if constexpr (S < 16) {
        return __builtin_amdgcn_ds_swizzle(x, 0x1f | (S << 10));
    } else if constexpr (S == 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        return (tid_x() & 16) ? (int)p[0] : (int)p[1];
    } else {
        const auto p = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        return (tid_x() & 32) ? (int)p[0] : (int)p[1];
    }
}
template <int S, bool LDS8 = false>
__device__ __forceinline__ float xor_lane(float v) {
    return __int_as_float(xor_lane<S, LDS8>(__float_as_int(v)));
}

// The two values a butterfly step at xor distance S (16 or 32) combines, own and partner in an
// order that differs between the lanes of a pair: the swapped halves of the register with
// itself, so no per-lane select picks the partner's value. Used with a commutative combine
// (+, max), the result is that of own combined with partner in every lane.
template <int S>
__device__ __forceinline__ void swap_pair(float v, float &a, float &b) {
    static_assert(S == 16 || S == 32, "swap distance");
    const unsigned u = __float_as_uint(v);
    const auto p = S == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                           : __builtin_amdgcn_permlane32_swap(u, u, false, false);
    a = __uint_as_float(p[0]);
    b = __uint_as_float(p[1]);
}

// The partner value of the xor-4 step of a butterfly that began at xor 1: every aligned quad
// then holds one value, so lane l ^ 7 (DPP row_half_mirror, a register move instead of an LDS
// swizzle) holds the same value as lane l ^ 4.
__device__ __forceinline__ float quad_partner(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xf, 0xf, false));
}

// Steps xor S, 2S, ..., N/2 of the butterfly sum. UNI: the butterfly began at xor 1 (each
// aligned group of S lanes holds one value), which lets the xor-4 step take quad_partner.
template <int S, int N, bool LDS8 = false, bool UNI = false>
__device__ __forceinline__ float butterfly_sum(float v) {
    if constexpr (S < N) {
        if constexpr (S >= 16) {
            float a, b;
            swap_pair<S>(v, a, b);
            return butterfly_sum<2 * S, N, LDS8, UNI>(a + b);
        } else if constexpr (S == 4 && UNI && !LDS8) {
            return butterfly_sum<2 * S, N, LDS8, UNI>(v + quad_partner(v));
        } else {
            return butterfly_sum<2 * S, N, LDS8, UNI>(v + xor_lane<S, LDS8>(v));
        }
    } else {
        return v;
    }
}

// Sum over aligned groups of N lanes by xor butterfly: lane l adds lane l^s for s = 1, 2, ...,
// N/2, i.e. the balanced pairwise tree in lane order; every lane of a group ends with the sum.
template <int N, bool LDS8 = false>
__device__ __forceinline__ float group_sum(float v) {
    return butterfly_sum<1, N, LDS8, true>(v);
}
template <bool LDS8 = false>
__device__ __forceinline__ float wave_sum(float v) { return group_sum<64, LDS8>(v); }

template <int S, int N = 64, bool LDS8 = false, bool UNI = false>
__device__ __forceinline__ float butterfly_max(float v) {
    if constexpr (S < N) {
        if constexpr (S >= 16) {
            float a, b;
            swap_pair<S>(v, a, b);
            return butterfly_max<2 * S, N, LDS8, UNI>(fmaxf(a, b));
        } else if constexpr (S == 4 && UNI && !LDS8) {
            return butterfly_max<2 * S, N, LDS8, UNI>(fmaxf(v, quad_partner(v)));
        } else {
            return butterfly_max<2 * S, N, LDS8, UNI>(fmaxf(v, xor_lane<S, LDS8>(v)));
        }
    } else {
        return v;
    }
}
template <int N, bool LDS8 = false>
__device__ __forceinline__ float group_max(float v) { return butterfly_max<1, N, LDS8, true>(v); }
template <bool LDS8 = false>
__device__ __forceinline__ float wave_max(float v) { return butterfly_max<1, 64, LDS8, true>(v); }

// One reduce-scatter step at xor S = 4 or 8 (lanes whose bit S is clear keep lo, the others
// hi), with no per-lane select: two DPP moves fill one register with the partner's copy of the
// value each lane keeps, selecting by bank (4 lanes) which lanes each move writes: at S = 4
// row_shl:4 (lane l reads l + 4) into banks 0 and 2 over the lane's own hi, and row_shr:4 (l - 4)
// into banks 1 and 3 over its own lo; at S = 8 row_ror:8 into banks 0-1, then into banks 2-3.
// The sum is own + partner (in an order that differs between the two lanes of a pair).
template <int S>
__device__ __forceinline__ float bank_pair_sum(float lo, float hi) {
    static_assert(S == 4 || S == 8, "bank-selected exchange");
    constexpr int LOW = S == 4 ? 0x5 : 0x3, HIGH = S == 4 ? 0xA : 0xC;
    constexpr int FROM_UP = S == 4 ? 0x104 : 0x128, FROM_DOWN = S == 4 ? 0x114 : 0x128;
    const int l = __float_as_int(lo), h = __float_as_int(hi);
    // banks of the lower lanes: the partner's lo; the upper lanes: their own hi
    const int a = __builtin_amdgcn_update_dpp(h, l, FROM_UP, 0xf, LOW, false);
    // banks of the upper lanes: the partner's hi; the lower lanes: their own lo
    const int b = __builtin_amdgcn_update_dpp(l, h, FROM_DOWN, 0xf, HIGH, false);
    return __int_as_float(a) + __int_as_float(b);
}

// Wave sums of B rows (B a power of two up to 64) with the pairing of wave_sum, so each total
// is bit-identical to wave_sum of that row, but scattered: at step xor 2^k for k < log2(B) a
// lane keeps half of its rows (the upper half when bit k of its lane index is set) and adds
// its partner's values of those rows; the remaining steps are the plain butterfly. Lane l ends
// with the total of row scatter_row<B>(l); B - 1 + 6 - log2(B) exchanges instead of 6 B.
template <int B>
__device__ __forceinline__ int scatter_row(int lane) {
    int row = 0;
#pragma unroll
    for (int k = 0; (1 << k) < B; k++)
        if ((lane >> k) & 1) row += B >> (k + 1);
    return row;
}
template <int M, int S, int N = 64, bool LDS8 = false, bool BANK = false>
__device__ __forceinline__ float scatter_sum_step(const float *v) {
    if constexpr (M == 1) {
        return butterfly_sum<S, N, LDS8, S == 1>(v[0]);
    } else {
        const bool up = (tid_x() & S) != 0;
        float keep[M / 2];
#pragma unroll
        for (int j = 0; j < M / 2; j++) {
            const float lo = v[j], hi = v[j + M / 2];
            if constexpr ((S == 4 || S == 8) && BANK && !LDS8) {
                keep[j] = bank_pair_sum<S>(lo, hi);
            } else {
                const float recv = xor_lane<S, LDS8>(up ? lo : hi);
                keep[j] = (up ? hi : lo) + recv;
            }
        }
        return scatter_sum_step<M / 2, 2 * S, N, LDS8, BANK>(keep);
    }
}
// BANK: the xor-4 and xor-8 steps through bank_pair_sum (no per-lane select).
template <int B, bool LDS8 = false, bool BANK = false>
__device__ __forceinline__ float wave_sum_scatter(const float (&v)[B]) {
    static_assert(B >= 1 && B <= 64 && (B & (B - 1)) == 0, "rows per batch");
    return scatter_sum_step<B, 1, 64, LDS8, BANK>(v);
}
// The same over aligned groups of N lanes: each total is bit-identical to group_sum<N> of that
// row, and lane l ends with row scatter_row<B>(l) (B <= N).
template <int N, int B, bool LDS8 = false, bool BANK = false>
__device__ __forceinline__ float group_sum_scatter(const float (&v)[B]) {
    static_assert(B >= 1 && B <= N && N <= 64 && (B & (B - 1)) == 0, "rows per group");
    return scatter_sum_step<B, 1, N, LDS8, BANK>(v);
}

// Reduce-scatter of M values per lane over aligned lane groups of N, from xor distance S on:
// at each step a lane keeps half of its values (the upper half when bit S of its lane index is
// set) and adds its partner's copies of them, so every total has the pairing of the butterfly
// sum; `out` receives the M * S / N values left.
// From S = 16 on, the step swaps the rows (16) or halves (32) of values j and j + M/2 with
// v_permlane16_swap / v_permlane32_swap: each lane receives the value it keeps and its partner's
// copy of it, in an order that differs between the two lanes (a + b = b + a), with no select.
template <int M, int S, int N>
__device__ __forceinline__ void scatter_keep(const float *v, float *out) {
    if constexpr (S >= N) {
#pragma unroll
        for (int j = 0; j < M; j++) out[j] = v[j];
    } else if constexpr (S >= 16) {
        float keep[M / 2];
#pragma unroll
        for (int j = 0; j < M / 2; j++) {
            const unsigned a = __float_as_uint(v[j]), b = __float_as_uint(v[j + M / 2]);
            const auto p = S == 16 ? __builtin_amdgcn_permlane16_swap(a, b, false, false)
                                   : __builtin_amdgcn_permlane32_swap(a, b, false, false);
            keep[j] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
        }
        scatter_keep<M / 2, 2 * S, N>(keep, out);
    } else {
        const bool up = (tid_x() & S) != 0;
        float keep[M / 2];
#pragma unroll
        for (int j = 0; j < M / 2; j++)
            keep[j] = (up ? v[j + M / 2] : v[j]) + xor_lane<S>(up ? v[j] : v[j + M / 2]);
        scatter_keep<M / 2, 2 * S, N>(keep, out);
    }
}

// Error flag of the bounded waits between workgroups: 0 none, 1 a token or position out of
// range, 2 a wait that ran out of polls. A wait that sees the flag set stops at once and leaves
// the code as it is; a wait that runs out sets 2 only if no earlier error set the flag.
__device__ __forceinline__ bool wait_error_set(const int *err) {
    return __hip_atomic_load(gptr((int *)err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}
__device__ __forceinline__ void wait_timed_out(int *err) {
    int expected = 0;
    __hip_atomic_compare_exchange_strong(gptr(err), &expected, 2, __ATOMIC_RELAXED,
                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// One check of a bounded wait, every few polls: true once the wait must stop.
__device__ __forceinline__ bool wait_gives_up(long long spins, long long limit, int *err) {
    if (wait_error_set(err)) return true;
    if (spins > limit) {
        wait_timed_out(err);
        return true;
    }
    return false;
}

// Larger value wins, equal values keep the lower index; NaN is never taken.
__device__ __forceinline__ void amax_pair(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

// (max, lowest index of the max) over the wave; every lane ends with the result.
template <int S = 1>
__device__ __forceinline__ void wave_amax(float &v, int &i) {
    if constexpr (S < 64) {
        const float v2 = xor_lane<S>(v);
        const int i2 = xor_lane<S>(i);
        amax_pair(v, i, v2, i2);
        wave_amax<2 * S>(v, i);
    }
}


// exp in fp32: k = rint(x log2 e); r = x - k ln2 (16-bit head of ln2 so k*hi and x - k*hi are
// exact, then the tail); e^r by the degree-7 Taylor series as 1 + (r + r^2 q(r)); scaled by
// 2^k with one rounding (v_ldexp_f32; the same bits as p * 2^(k/2) * 2^(k - k/2), whose first
// product is exact, so gradual underflow rounds once either way). Within 1 ulp of the correctly rounded
// value for every fp32 input (checked exhaustively on the CPU against libm).
__device__ __forceinline__ float exp_f32(float x) {
    if (x != x) return x;
    if (x > 89.0f) return __builtin_huge_valf();
    if (x < -104.0f) return 0.0f;
    float k = rintf(x * 0x1.715476p+0f);
    float r = fmaf(k, -0x1.62e400p-1f, x);
    r = fmaf(k, -0x1.7f7d1cp-20f, r);
    float q = 0x1.a01a02p-13f;
    q = fmaf(q, r, 0x1.6c16c2p-10f);
    q = fmaf(q, r, 0x1.111112p-7f);
    q = fmaf(q, r, 0x1.555556p-5f);
    q = fmaf(q, r, 0x1.555556p-3f);
    q = fmaf(q, r, 0x1.000000p-1f);
    float r2 = r * r;
    float t = fmaf(r2, q, r);
    float p = 1.0f + t;
    return __builtin_amdgcn_ldexpf(p, (int)k);
}

// sin and cos in double: k = rint(x 2/pi), r = x - k pi/2 with pi/2 in two 33-bit heads and a
// tail, Taylor series to x^17 / x^18 on |r| <= pi/4 (Horner, fma), quadrant from k mod 4.
// Rounded to fp32 it matches libm at every RoPE angle checked.
__device__ __forceinline__ void sincos_d(double x, double *s_out, double *c_out) {
    double k = rint(x * 0x1.45f306dc9c883p-1);
    double r = fma(-k, 0x1.921fb54400000p+0, x);
    r = fma(-k, 0x1.0b4611a600000p-34, r);
    r = fma(-k, 0x1.3198a2e037073p-69, r);
    double z = r * r;
    double ps = 0x1.952c77030ad4ap-49;
    ps = fma(ps, z, -0x1.ae7f3e733b81fp-41);
    ps = fma(ps, z, 0x1.6124613a86d09p-33);
    ps = fma(ps, z, -0x1.ae64567f544e4p-26);
    ps = fma(ps, z, 0x1.71de3a556c734p-19);
    ps = fma(ps, z, -0x1.a01a01a01a01ap-13);
    ps = fma(ps, z, 0x1.1111111111111p-7);
    ps = fma(ps, z, -0x1.5555555555555p-3);
    double sr = fma(r * z, ps, r);
    double pc = -0x1.6827863b97d97p-53;
    pc = fma(pc, z, 0x1.ae7f3e733b81fp-45);
    pc = fma(pc, z, -0x1.93974a8c07c9dp-37);
    pc = fma(pc, z, 0x1.1eed8eff8d898p-29);
    pc = fma(pc, z, -0x1.27e4fb7789f5cp-22);
    pc = fma(pc, z, 0x1.a01a01a01a01ap-16);
    pc = fma(pc, z, -0x1.6c16c16c16c17p-10);
    pc = fma(pc, z, 0x1.5555555555555p-5);
    pc = fma(pc, z, -0x1.0000000000000p-1);
    double cr = fma(z, pc, 1.0);
    int quadrant = (int)((long long)k & 3);
    double s, c;
    switch (quadrant) {
    case 0: s = sr; c = cr; break;
    case 1: s = cr; c = -sr; break;
    case 2: s = -sr; c = -cr; break;
    default: s = -cr; c = sr; break;
    }
    *s_out = s;
    *c_out = c;
}

// silu in fp32 as HF evaluates it for bf16 inputs: g / (1 + exp(-g)).
__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + exp_f32(-g)); }

// round_bf(silu_f32(g)) for the 8 values of a chunk, cheaper: an estimate from the hardware
// exp2 and reciprocal (within ~13 fp32 ulps of silu_f32 for |g| <= 8), rounded to bf16. Two
// fp32 values closer than the band round to the same bf16 unless a rounding midpoint (low 16
// bits 0x8000) lies between them, so the estimate is kept when its low 16 bits are more than
// 64 from 0x8000 and |g| <= 8; otherwise (and for inf and NaN) silu_f32 itself is rounded. The
// result is silu_f32's rounding for every bf16 g (checked exhaustively on the GPU).
__device__ __forceinline__ void silu_bf16x8(const float (&g)[8], float (&out)[8]) {
    unsigned redo = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float ex = __builtin_amdgcn_exp2f(g[e] * -0x1.715476p+0f);
        const float y = g[e] * __builtin_amdgcn_rcpf(1.0f + ex);
        const uint32_t low = __float_as_uint(y) & 0xffffu;
        out[e] = round_bf(y);
        if (!(fabsf(g[e]) <= 8.0f) || low - 0x7fc0u <= 0x80u) redo |= 1u << e;
    }
    if (redo) {
#pragma unroll
        for (int e = 0; e < 8; e++)
            if (redo & (1u << e)) out[e] = round_bf(silu_f32(g[e]));
    }
}

}  // namespace llm
