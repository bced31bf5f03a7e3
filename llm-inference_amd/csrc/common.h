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

__device__ __forceinline__ u32x4 ld16(const void *p) { return *(const u32x4 *)p; }
// Streamed operands (weights, KV cache) are read non-temporally so they do not evict the
// small reused vectors from L2.
__device__ __forceinline__ u32x4 ld16_nt(const void *p) {
    return __builtin_nontemporal_load((const u32x4 *)p);
}
__device__ __forceinline__ void st16(void *p, u32x4 v) { *(u32x4 *)p = v; }

// bf16 element e of a packed 16-byte chunk (element 0 in the low half of dword 0).
__device__ __forceinline__ float lo_f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// fp32 -> bf16 round to nearest even; NaN stays NaN with the quiet bit set.
__device__ __forceinline__ uint32_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float round_bf(float f) { return __uint_as_float(f2bf(f) << 16); }
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return f2bf(lo) | (f2bf(hi) << 16);
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

// Sum over aligned groups of N lanes by xor butterfly: lane l adds lane l^s for s = 1, 2, ...,
// N/2, i.e. the balanced pairwise tree in lane order; every lane of a group ends with the sum.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int s = 1; s < N; s <<= 1) v += __shfl_xor(v, s);
    return v;
}
__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) v = fmaxf(v, __shfl_xor(v, s));
    return v;
}

// 2^n for n in [-126, 127].
__device__ __forceinline__ float pow2i(int n) { return __uint_as_float((uint32_t)(n + 127) << 23); }

// exp in fp32: k = rint(x log2 e); r = x - k ln2 (16-bit head of ln2 so k*hi and x - k*hi are
// exact, then the tail); e^r by the degree-7 Taylor series as 1 + (r + r^2 q(r)); scaled by
// 2^k in two steps so gradual underflow rounds once. Within 1 ulp of the correctly rounded
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
    int ki = (int)k;
    int k1 = ki / 2;
    int k2 = ki - k1;
    return p * pow2i(k1) * pow2i(k2);
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

}  // namespace llm
