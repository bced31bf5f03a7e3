// Per-lane QK-RMSNorm + RoPE of one head, shared by the standalone kernel and the persistent
// step so both compute it from the same code (src/kernels.cu:323-380 rounding points).
//
// Lane layout: a head of D elements is a group of D/16 lanes; lane L of the group holds the
// chunk [8L, 8L+8) and its rotation partner [D/2+8L, D/2+8L+8). Sum of squares: fma over the
// first chunk then the second, then the xor tree over the D/16 lanes.
#pragma once

#include "common.h"

namespace llm {

template <int D>
struct RopeShape {
    static constexpr int LH = D / 16;             // lanes per head
    static constexpr int HALF = D / 2;            // rotation pairs
    static constexpr int NJ = (HALF + 63) / 64;   // table entries held per lane
};

// Entry j = lane + 64m of the RoPE table at `pos`: angle = fp32(pos * inv_freq_j); cos and sin
// in double (sincos_d), rounded to fp32 and then to bf16 as HF's emb.cos().to(bf16).
template <int D, class Table>
__device__ __forceinline__ void rope_table(int pos, Table inv_freq,
                                           float (&cs)[RopeShape<D>::NJ],
                                           float (&sn)[RopeShape<D>::NJ]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int m = 0; m < RopeShape<D>::NJ; m++) {
        const int j = lane + 64 * m;
        cs[m] = sn[m] = 0.0f;
        if (j < RopeShape<D>::HALF) {
            const float angle = (float)pos * inv_freq[j];
            double s, c;
            sincos_d((double)angle, &s, &c);
            cs[m] = round_bf((float)c);
            sn[m] = round_bf((float)s);
        }
    }
}

// The table entries of rotation pairs 8L .. 8L+7 (a lane's chunk), fetched from the lanes that
// computed them. Every lane of the wave must call this (it shuffles).
template <int D>
__device__ __forceinline__ void rope_fetch(const float (&cs)[RopeShape<D>::NJ],
                                           const float (&sn)[RopeShape<D>::NJ], int L,
                                           float (&c)[8], float (&s)[8]) {
    constexpr int NJ = RopeShape<D>::NJ;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const int j = 8 * L + e;
        c[e] = __shfl(cs[0], j & 63);
        s[e] = __shfl(sn[0], j & 63);
#pragma unroll
        for (int m = 1; m < NJ; m++) {
            const float cm = __shfl(cs[m], j & 63), sm = __shfl(sn[m], j & 63);
            if ((j >> 6) == m) {
                c[e] = cm;
                s[e] = sm;
            }
        }
    }
}

// RMSNorm of the head (weight chunks wa/wb), then the rotation with the lane's table entries
// c/s (rope_fetch). Outputs: the normed chunks (ya/yb, for taps) and the rotated chunks
// (oa/ob). The lanes of a head must call this together (the sum of squares is a lane tree);
// lanes of an absent head pass zeros and ignore the results.
template <int D>
__device__ __forceinline__ void norm_rope_with(const u32x4 &xa, const u32x4 &xb, const u32x4 &wa,
                                               const u32x4 &wb, float eps, const float (&c)[8],
                                               const float (&s)[8], u32x4 &ya_out, u32x4 &yb_out,
                                               u32x4 &oa_out, u32x4 &ob_out) {
    constexpr int LH = RopeShape<D>::LH;
    float acc = dot8(xa, xa, 0.0f);
    acc = dot8(xb, xb, acc);
    const float total = group_sum<LH>(acc);
    const float inv = 1.0f / sqrtf(total / (float)D + eps);
    float ya[8], yb[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        ya[e] = round_bf(round_bf(elem(xa, e) * inv) * elem(wa, e));
        yb[e] = round_bf(round_bf(elem(xb, e) * inv) * elem(wb, e));
    }
    float oa[8], ob[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float a_cos = round_bf(ya[e] * c[e]);
        const float b_sin = round_bf(yb[e] * s[e]);
        const float b_cos = round_bf(yb[e] * c[e]);
        const float a_sin = round_bf(ya[e] * s[e]);
        oa[e] = a_cos - b_sin;
        ob[e] = b_cos + a_sin;
    }
    ya_out = u32x4{pack2(ya[0], ya[1]), pack2(ya[2], ya[3]), pack2(ya[4], ya[5]), pack2(ya[6], ya[7])};
    yb_out = u32x4{pack2(yb[0], yb[1]), pack2(yb[2], yb[3]), pack2(yb[4], yb[5]), pack2(yb[6], yb[7])};
    oa_out = u32x4{pack2(oa[0], oa[1]), pack2(oa[2], oa[3]), pack2(oa[4], oa[5]), pack2(oa[6], oa[7])};
    ob_out = u32x4{pack2(ob[0], ob[1]), pack2(ob[2], ob[3]), pack2(ob[4], ob[5]), pack2(ob[6], ob[7])};
}

// rope_fetch + norm_rope_with. Every lane of the wave must call this (it shuffles).
template <int D>
__device__ __forceinline__ void norm_rope(const u32x4 &xa, const u32x4 &xb, const u32x4 &wa,
                                          const u32x4 &wb, float eps,
                                          const float (&cs)[RopeShape<D>::NJ],
                                          const float (&sn)[RopeShape<D>::NJ], int L, u32x4 &ya_out,
                                          u32x4 &yb_out, u32x4 &oa_out, u32x4 &ob_out) {
    float c[8], s[8];
    rope_fetch<D>(cs, sn, L, c, s);
    norm_rope_with<D>(xa, xb, wa, wb, eps, c, s, ya_out, yb_out, oa_out, ob_out);
}

}  // namespace llm
