// Decode kernels for gfx950 (MI355X), behind the launcher names of the reference's
// src/kernels.cuh. Wave64 throughout: a GEMV row is one wave whose lanes stream 16-byte chunks
// (global_load_dwordx4, non-temporal for weights and the KV cache) and meet in an xor-butterfly
// tree; RMSNorm rows up to 8192 wide are one wave held in registers; a RoPE head is a group of
// D/16 lanes that each hold the chunk [8L, 8L+8) and its rotation partner [D/2+8L, ...), so the
// rotation is lane-local. Arithmetic is fp32 with bf16 stores at the reference's rounding points
// (src/kernels.cu), in the summation orders the CPU oracle restates.
#include <limits.h>
#include <math.h>
#include <stdarg.h>
#include <string.h>

#include <mutex>

#include "common.h"
#include "internal.h"
#include "rope.h"

using namespace llm;

// ------------------------------------------------------------------------------------------
// error handling (src/common.cuh:11-22 semantics, switchable to recording)
// ------------------------------------------------------------------------------------------

static int g_exit_on_error = 1;
static thread_local char g_err[1024];
static thread_local bool g_has_err = false;

bool llm_fail(const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (g_exit_on_error) {
        fprintf(stderr, "%s\n", buf);
        exit(EXIT_FAILURE);
    }
    if (!g_has_err) {  // keep the first error until it is cleared
        strncpy(g_err, buf, sizeof g_err - 1);
        g_err[sizeof g_err - 1] = 0;
        g_has_err = true;
    }
    return false;
}

bool llm_has_error() { return g_has_err; }

extern "C" int llm_set_exit_on_error(int enable) {
    int old = g_exit_on_error;
    g_exit_on_error = enable ? 1 : 0;
    return old;
}
extern "C" const char *llm_last_error(void) { return g_has_err ? g_err : nullptr; }
extern "C" void llm_clear_error(void) {
    g_has_err = false;
    g_err[0] = 0;
}

static bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// ------------------------------------------------------------------------------------------
// embedding (src/kernels.cu:7-23)
// ------------------------------------------------------------------------------------------

// One workgroup copies the row in 16-byte chunks. With vocab > 0 a token outside [0, vocab)
// sets *err and copies nothing (the step uses this for tokens fed back on the device).
__global__ __launch_bounds__(256) void embedding_kernel(bf16 *out, const bf16 *table,
                                                        const int *d_token, int hidden, int vocab,
                                                        int *err) {
    const int token = *d_token;
    if (vocab > 0 && (token < 0 || token >= vocab)) {
        if (err && threadIdx.x == 0) *err = 1;
        return;
    }
    const bf16 *row = table + (size_t)token * hidden;
    if ((hidden & 7) == 0) {
        for (int c = threadIdx.x; c < hidden / 8; c += blockDim.x) st16(out + 8 * c, ld16(row + 8 * c));
    } else {
        for (int i = threadIdx.x; i < hidden; i += blockDim.x) out[i] = row[i];
    }
}

static void launch_embedding(bf16 *out, const bf16 *table, const int *d_token, int hidden,
                             int vocab, int *err, hipStream_t stream) {
    if (hidden <= 0) {
        llm_fail("embedding: hidden %d must be positive", hidden);
        return;
    }
    if ((hidden & 7) == 0 && (!aligned16(out) || !aligned16(table))) {
        llm_fail("embedding: out and table must be 16-byte aligned");
        return;
    }
    embedding_kernel<<<1, 256, 0, stream>>>(out, table, d_token, hidden, vocab, err);
    LAUNCH_OK();
}

extern "C" void embedding_forward(bf16 *out, const bf16 *table, const int *d_token, int hidden,
                                  hipStream_t stream) {
    launch_embedding(out, table, d_token, hidden, 0, nullptr, stream);
}

// Used by the step for device-fed tokens.
void embedding_checked(bf16 *out, const bf16 *table, const int *d_token, int hidden, int vocab,
                       int *err, hipStream_t stream) {
    launch_embedding(out, table, d_token, hidden, vocab, err, stream);
}

// ------------------------------------------------------------------------------------------
// RMSNorm (src/kernels.cu:25-71)
// ------------------------------------------------------------------------------------------

// One wave per row, the row in registers: lane l holds chunks l, l+64, ... (NC of them).
// sum of squares: per-lane fma in chunk/element order, then the wave tree. The row, its output
// and the weights are buffers: chunks past the end read as zeros and are not written, with no
// branch around the loads and stores (with per-chunk bounds branches and plain loads the
// 4096 x 2560 sweep took 10.5 us instead of 7.3; two or four rows per wave with the next row
// requested early measured slower still).
template <int NC>
__global__ __launch_bounds__(256) void rmsnorm_wave_kernel(bf16 *out, const bf16 *in,
                                                           const bf16 *weight, int rows, int dim,
                                                           float eps) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (row >= rows) return;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(in + (size_t)row * dim), (short)0, dim * 2, BUFFER_FLAGS);
    const __amdgpu_buffer_rsrc_t wr =
        __builtin_amdgcn_make_buffer_rsrc((void *)weight, (short)0, dim * 2, BUFFER_FLAGS);
    const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(out + (size_t)row * dim), (short)0, dim * 2, BUFFER_FLAGS);
    u32x4 xv[NC], wv[NC];
#pragma unroll
    for (int k = 0; k < NC; k++)
        xv[k] = __builtin_amdgcn_raw_buffer_load_b128(xr, 16 * (lane + 64 * k), 0, BUFFER_NT);
#pragma unroll
    for (int k = 0; k < NC; k++)
        wv[k] = __builtin_amdgcn_raw_buffer_load_b128(wr, 16 * (lane + 64 * k), 0, 0);
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < NC; k++) acc = dot8(xv[k], xv[k], acc);
    const float total = wave_sum(acc);
    const float inv = 1.0f / sqrtf(total / (float)dim + eps);
#pragma unroll
    for (int k = 0; k < NC; k++) {
        float r[8];
#pragma unroll
        for (int e = 0; e < 8; e++) r[e] = round_bf(elem(xv[k], e) * inv) * elem(wv[k], e);
        __builtin_amdgcn_raw_buffer_store_b128(
            u32x4{pack2(r[0], r[1]), pack2(r[2], r[3]), pack2(r[4], r[5]), pack2(r[6], r[7])}, yr,
            16 * (lane + 64 * k), 0, BUFFER_NT);
    }
}

// Any dim: W waves per row (W = max(1, min(16, ceil(chunks / 1024)))), thread t takes chunks
// t, t + 64W, ... element by element; wave trees, then the waves added in order through LDS.
__global__ __launch_bounds__(1024) void rmsnorm_generic_kernel(bf16 *out, const bf16 *in,
                                                               const bf16 *weight, int dim,
                                                               float eps) {
    __shared__ float part[16];
    const int row = blockIdx.x;
    const int T = blockDim.x;
    const bf16 *x = in + (size_t)row * dim;
    const int n_chunks = (dim + 7) / 8;
    float acc = 0.0f;
    for (int c = threadIdx.x; c < n_chunks; c += T)
        for (int e = 0; e < 8; e++) {
            const int i = 8 * c + e;
            if (i < dim) {
                const float v = bf2f(x[i]);
                acc = fmaf(v, v, acc);
            }
        }
    const float ws = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ws;
    __syncthreads();
    float total = part[0];
    for (int w = 1; w < T / 64; w++) total = total + part[w];
    const float inv = 1.0f / sqrtf(total / (float)dim + eps);
    bf16 *y = out + (size_t)row * dim;
    for (int i = threadIdx.x; i < dim; i += T)
        y[i] = f2bf(round_bf(bf2f(x[i]) * inv) * bf2f(weight[i]));
}

static int rms_waves(int dim) {
    int n_chunks = (dim + 7) / 8;
    int w = (n_chunks + 64 * 16 - 1) / (64 * 16);
    return w < 1 ? 1 : (w > 16 ? 16 : w);
}

extern "C" void rmsnorm_forward(bf16 *out, const bf16 *in, const bf16 *weight, int rows, int dim,
                                float eps, hipStream_t stream) {
    if (rows <= 0 || dim <= 0) {
        llm_fail("rmsnorm: rows %d and dim %d must be positive", rows, dim);
        return;
    }
    const int per_lane = (dim / 8 + 63) / 64;
    const bool fast = (dim & 7) == 0 && per_lane <= 16 && aligned16(out) && aligned16(in) &&
                      aligned16(weight);
    if (fast) {
        const int blocks = (rows + 3) / 4;
#define RMS(NC_)                                                                            \
    if (per_lane <= NC_) {                                                                  \
        rmsnorm_wave_kernel<NC_><<<blocks, 256, 0, stream>>>(out, in, weight, rows, dim, eps); \
        LAUNCH_OK();                                                                        \
        return;                                                                             \
    }
        RMS(1) RMS(2) RMS(3) RMS(4) RMS(5) RMS(6) RMS(8) RMS(12) RMS(16)
#undef RMS
    }
    rmsnorm_generic_kernel<<<rows, 64 * rms_waves(dim), 0, stream>>>(out, in, weight, dim, eps);
    LAUNCH_OK();
}

// ------------------------------------------------------------------------------------------
// GEMV family (src/kernels.cu:79-212, :215-298)
// ------------------------------------------------------------------------------------------

// A launch covers up to three weight matrices against one input vector (qkv stacks
// [wq; wk; wv]); each segment owns a contiguous range of waves.
struct GemvSeg {
    const bf16 *w;
    bf16 *out;
    int rows;
    int wave_begin;
};

struct GemvArgs {
    GemvSeg seg[3];
    int n_seg;
    const bf16 *x;
    int cols;
    bf16 *tap;             // residual epilogue: optional copy of y
    const bf16 *norm_w;    // fused RMSNorm prologue: gamma (NORM kernels only)
    float eps;
};

// The fused RMSNorm prologue of a one-panel GEMV: the wave's input chunks (lane l: chunks
// l + 64k, the layout of rmsnorm_wave_kernel<NC>) normalised in registers with that kernel's
// arithmetic, so the GEMV sees exactly the bf16 vector rmsnorm_forward would have written. The
// gamma chunks are requested with the input, before the weight rows, and the arithmetic runs
// after the weight requests: loads complete in order, so it waits for the input and gamma only.
template <int NC>
__device__ __forceinline__ void norm_gamma_load(const bf16 *gamma, int cols, u32x4 (&gv)[NC]) {
    const int lane = tid_x() & 63;
    const __amdgpu_buffer_rsrc_t gr =
        __builtin_amdgcn_make_buffer_rsrc((void *)gamma, (short)0, cols * 2, BUFFER_FLAGS);
#pragma unroll
    for (int k = 0; k < NC; k++) gv[k] = __builtin_amdgcn_raw_buffer_load_b128(gr, 16 * (lane + 64 * k), 0, 0);
}
template <int NC>
__device__ __forceinline__ void norm_apply(u32x4 (&xv)[NC], const u32x4 (&gv)[NC], int cols, float eps) {
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < NC; k++) acc = dot8(xv[k], xv[k], acc);
    const float total = wave_sum(acc);
    const float inv = 1.0f / sqrtf(total / (float)cols + eps);
#pragma unroll
    for (int k = 0; k < NC; k++) {
        float r[8];
#pragma unroll
        for (int e = 0; e < 8; e++) r[e] = round_bf(elem(xv[k], e) * inv) * elem(gv[k], e);
        xv[k] = u32x4{pack2(r[0], r[1]), pack2(r[2], r[3]), pack2(r[4], r[5]), pack2(r[6], r[7])};
    }
}

enum { EPI_PLAIN = 0, EPI_RESID = 1 };

// Wave `wave` computes RPW consecutive rows. Lane l streams chunks l, l+64, ... of each row
// (NC per lane per panel, panels until the row ends), fma-accumulating in order; the wave tree
// then gives every lane each row's sum and lane i stores row row0+i.
template <int NC, int RPW, int EPI, bool NORM = false>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
    // Wide rows (NC >= 10: over 4096 columns) take the input through LDS: the workgroup loads
    // each panel of x once instead of once per wave, which at one row per wave would double the
    // L2-to-CU traffic of the weight stream.
    constexpr bool XLDS = NC >= 10 && !NORM;
    constexpr int XT = XLDS ? (64 * NC + 255) / 256 : 1;  // x chunks per thread and panel
    __shared__ u32x4 xs[XLDS ? 64 * NC : 1];
    const int lane = threadIdx.x & 63;
    // wave-uniform (scalar), so the per-row buffer descriptors below are scalar too
    const int wave = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int si = (a.n_seg > 2 && wave >= a.seg[2].wave_begin)   ? 2
                   : (a.n_seg > 1 && wave >= a.seg[1].wave_begin) ? 1
                                                                  : 0;
    const bf16 *w = si == 0 ? a.seg[0].w : si == 1 ? a.seg[1].w : a.seg[2].w;
    bf16 *out = si == 0 ? a.seg[0].out : si == 1 ? a.seg[1].out : a.seg[2].out;
    const int rows = si == 0 ? a.seg[0].rows : si == 1 ? a.seg[1].rows : a.seg[2].rows;
    const int wb = si == 0 ? a.seg[0].wave_begin : si == 1 ? a.seg[1].wave_begin : a.seg[2].wave_begin;
    const int row0 = (wave - wb) * RPW;
    // with XLDS every wave takes part in the workgroup's syncs; a wave without rows loads
    // nothing (zero-size row buffers) and stores nothing
    const bool active = row0 < rows;
    if (!XLDS && !active) return;
    const int cols = a.cols;
    const int n_chunks = cols >> 3;
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.x, (short)0, cols * 2, BUFFER_FLAGS);
    float acc[RPW];
#pragma unroll
    for (int i = 0; i < RPW; i++) acc[i] = 0.0f;
    for (int c0 = 0; c0 < n_chunks; c0 += 64 * NC) {
        u32x4 wv[RPW][NC];
        u32x4 xv[NC];
        u32x4 xt[XT];
        if constexpr (XLDS) {
#pragma unroll
            for (int j = 0; j < XT; j++)
                xt[j] = __builtin_amdgcn_raw_buffer_load_b128(
                    xr, 16 * (c0 + (int)threadIdx.x + 256 * j), 0, 0);
        } else {
#pragma unroll
            for (int k = 0; k < NC; k++)
                xv[k] = __builtin_amdgcn_raw_buffer_load_b128(xr, 16 * (c0 + lane + 64 * k), 0, 0);
        }
        u32x4 gm[NC];  // one panel when NORM (host check)
        if constexpr (NORM) norm_gamma_load<NC>(a.norm_w, cols, gm);
#pragma unroll
        for (int i = 0; i < RPW; i++) {
            // the row as a buffer: chunks past its end read as zeros with no branch around the
            // loads, so each chunk's FMAs wait only for that chunk's load
            const int r = min(row0 + i, rows - 1);
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                (void *)(w + (size_t)r * cols), (short)0, active ? cols * 2 : 0, BUFFER_FLAGS);
#pragma unroll
            for (int k = 0; k < NC; k++)
                wv[i][k] = __builtin_amdgcn_raw_buffer_load_b128(rs, 16 * (c0 + lane + 64 * k), 0,
                                                                 BUFFER_NT);
        }
        if constexpr (XLDS) {
            if (c0 > 0) __syncthreads();  // every wave has read the previous panel
#pragma unroll
            for (int j = 0; j < XT; j++)
                if ((int)threadIdx.x + 256 * j < 64 * NC) xs[threadIdx.x + 256 * j] = xt[j];
            __syncthreads();
#pragma unroll
            for (int k = 0; k < NC; k++) xv[k] = xs[lane + 64 * k];
        }
        if constexpr (NORM) norm_apply<NC>(xv, gm, cols, a.eps);
#pragma unroll
        for (int i = 0; i < RPW; i++)
#pragma unroll
            for (int k = 0; k < NC; k++) acc[i] = dot8(wv[i][k], xv[k], acc[i]);
    }
    if (!active) return;
    float mine = 0.0f;
#pragma unroll
    for (int i = 0; i < RPW; i++) {
        const float t = wave_sum(acc[i]);
        if (lane == i) mine = t;
    }
    const int r = row0 + lane;
    if (lane < RPW && r < rows) {
        const uint32_t y = f2bf(mine);
        if (EPI == EPI_PLAIN) {
            out[r] = (bf16)y;
        } else {
            if (a.tap) a.tap[r] = (bf16)y;
            out[r] = (bf16)f2bf(bf2f(out[r]) + bf2f((bf16)y));
        }
    }
}

// gate and up rows together: g = bf16(wg[r].x), u = bf16(wu[r].x),
// act = bf16(bf16(silu(g)) * u) (src/kernels.cu:276-287).
template <int NC, int RPW, bool NORM = false>
__global__ __launch_bounds__(256) void gate_up_kernel(bf16 *act, const bf16 *wg, const bf16 *wu,
                                                      const bf16 *x, int rows, int cols,
                                                      bf16 *gate_tap, bf16 *up_tap,
                                                      const bf16 *norm_w = nullptr,
                                                      float eps = 0.0f) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = wave * RPW;
    if (row0 >= rows) return;
    const int n_chunks = cols >> 3;
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc((void *)x, (short)0, cols * 2, BUFFER_FLAGS);
    float ag[RPW], au[RPW];
#pragma unroll
    for (int i = 0; i < RPW; i++) ag[i] = au[i] = 0.0f;
    for (int c0 = 0; c0 < n_chunks; c0 += 64 * NC) {
        u32x4 xv[NC];
        u32x4 gv[RPW][NC], uv[RPW][NC];
#pragma unroll
        for (int k = 0; k < NC; k++)
            xv[k] = __builtin_amdgcn_raw_buffer_load_b128(xr, 16 * (c0 + lane + 64 * k), 0, 0);
        u32x4 gm[NC];  // one panel when NORM (host check)
        if constexpr (NORM) norm_gamma_load<NC>(norm_w, cols, gm);
#pragma unroll
        for (int i = 0; i < RPW; i++) {
            const size_t r = (size_t)min(row0 + i, rows - 1);
            const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
                (void *)(wg + r * cols), (short)0, cols * 2, BUFFER_FLAGS);
            const __amdgpu_buffer_rsrc_t ru = __builtin_amdgcn_make_buffer_rsrc(
                (void *)(wu + r * cols), (short)0, cols * 2, BUFFER_FLAGS);
#pragma unroll
            for (int k = 0; k < NC; k++) {
                const int off = 16 * (c0 + lane + 64 * k);
                gv[i][k] = __builtin_amdgcn_raw_buffer_load_b128(rg, off, 0, BUFFER_NT);
                uv[i][k] = __builtin_amdgcn_raw_buffer_load_b128(ru, off, 0, BUFFER_NT);
            }
        }
        if constexpr (NORM) norm_apply<NC>(xv, gm, cols, eps);
#pragma unroll
        for (int i = 0; i < RPW; i++)
#pragma unroll
            for (int k = 0; k < NC; k++) {
                ag[i] = dot8(gv[i][k], xv[k], ag[i]);
                au[i] = dot8(uv[i][k], xv[k], au[i]);
            }
    }
    float g_mine = 0.0f, u_mine = 0.0f;
#pragma unroll
    for (int i = 0; i < RPW; i++) {
        const float g = wave_sum(ag[i]);
        const float u = wave_sum(au[i]);
        if (lane == i) {
            g_mine = g;
            u_mine = u;
        }
    }
    const int r = row0 + lane;
    if (lane < RPW && r < rows) {
        const bf16 g = (bf16)f2bf(g_mine);
        const bf16 u = (bf16)f2bf(u_mine);
        if (gate_tap) gate_tap[r] = g;
        if (up_tap) up_tap[r] = u;
        const float s = round_bf(silu_f32(bf2f(g)));
        act[r] = (bf16)f2bf(s * bf2f(u));
    }
}

// Per-lane chunk capacity of one panel.
static int pick_nc(int n_chunks) {
    const int per_lane = (n_chunks + 63) / 64;
    static const int ncs[] = {1, 2, 3, 4, 5, 6, 8, 10, 12, 16, 20};
    for (int v : ncs)
        if (v >= per_lane) return v;
    return 20;
}

// Rows per wave: enough loads in flight per lane (RPW*NC ~ 8-16) while keeping at least ~2048
// waves (8 per CU) when the matrix has the rows for it.
static int pick_rpw(int nc, long total_rows, int pairs) {
    int rpw = nc <= 2 ? 8 : nc <= 4 ? 4 : nc <= 8 ? 2 : 1;
    if (pairs) rpw = rpw > 1 ? rpw / 2 : 1;
    while (rpw > 1 && total_rows / rpw < 2048) rpw /= 2;
    return rpw;
}

static bool check_gemv(const char *name, const void *w, const void *x, int rows, int cols) {
    if (cols % 8 != 0) return llm_fail("%s: cols %d is not a multiple of 8", name, cols);
    if (rows <= 0 || cols <= 0) return llm_fail("%s: rows %d and cols %d must be positive", name, rows, cols);
    if (!aligned16(w) || !aligned16(x))
        return llm_fail("%s: weight and input must be 16-byte aligned", name);
    return true;
}

#define GEMV_CASES(X) \
    X(1, 1) X(1, 2) X(1, 4) X(1, 8) X(2, 1) X(2, 2) X(2, 4) X(2, 8) X(3, 1) X(3, 2) X(3, 4) \
    X(4, 1) X(4, 2) X(4, 4) X(5, 1) X(5, 2) X(6, 1) X(6, 2) X(8, 1) X(8, 2) X(10, 1)    \
    X(12, 1) X(16, 1) X(20, 1)

template <int EPI>
static bool dispatch_gemv(const GemvArgs &a, int nc, int rpw, int blocks, hipStream_t st) {
#define X(NC_, RPW_)                                                         \
    if (nc == NC_ && rpw == RPW_) {                                          \
        if (EPI == EPI_PLAIN && a.norm_w)                                    \
            gemv_kernel<NC_, RPW_, EPI_PLAIN, true><<<blocks, 256, 0, st>>>(a); \
        else                                                                 \
            gemv_kernel<NC_, RPW_, EPI><<<blocks, 256, 0, st>>>(a);          \
        return LAUNCH_OK();                                                  \
    }
    GEMV_CASES(X)
#undef X
    return llm_fail("gemv: no kernel for nc %d rpw %d", nc, rpw);
}

static void launch_gemv(GemvArgs &a, int epi, hipStream_t stream) {
    long total_rows = 0;
    for (int i = 0; i < a.n_seg; i++) total_rows += a.seg[i].rows;
    const int nc = pick_nc(a.cols / 8);
    const int rpw = pick_rpw(nc, total_rows, 0);
    int waves = 0;
    for (int i = 0; i < a.n_seg; i++) {
        a.seg[i].wave_begin = waves;
        waves += (a.seg[i].rows + rpw - 1) / rpw;
    }
    const int blocks = (waves + 3) / 4;
    if (epi == EPI_PLAIN)
        dispatch_gemv<EPI_PLAIN>(a, nc, rpw, blocks, stream);
    else
        dispatch_gemv<EPI_RESID>(a, nc, rpw, blocks, stream);
}

extern "C" void gemv_forward(bf16 *out, const bf16 *w, const bf16 *x, int rows, int cols,
                             hipStream_t stream) {
    if (!check_gemv("gemv", w, x, rows, cols)) return;
    GemvArgs a = {};
    a.seg[0] = {w, out, rows, 0};
    a.n_seg = 1;
    a.x = x;
    a.cols = cols;
    launch_gemv(a, EPI_PLAIN, stream);
}

extern "C" void gemv_residual_forward(bf16 *x, const bf16 *w, const bf16 *in, int rows, int cols,
                                      bf16 *tap, hipStream_t stream) {
    if (!check_gemv("gemv_residual", w, in, rows, cols)) return;
    if (x == in) {
        llm_fail("gemv_residual: in must not alias x");
        return;
    }
    GemvArgs a = {};
    a.seg[0] = {w, x, rows, 0};
    a.n_seg = 1;
    a.x = in;
    a.cols = cols;
    a.tap = tap;
    launch_gemv(a, EPI_RESID, stream);
}

extern "C" void qkv_forward(bf16 *q, bf16 *k, bf16 *v, const bf16 *wq, const bf16 *wk,
                            const bf16 *wv, const bf16 *x, int q_rows, int kv_rows, int cols,
                            hipStream_t stream) {
    if (!check_gemv("qkv", wq, x, q_rows, cols) || !check_gemv("qkv", wk, x, kv_rows, cols) ||
        !check_gemv("qkv", wv, x, kv_rows, cols))
        return;
    GemvArgs a = {};
    a.seg[0] = {wq, q, q_rows, 0};
    a.seg[1] = {wk, k, kv_rows, 0};
    a.seg[2] = {wv, v, kv_rows, 0};
    a.n_seg = 3;
    a.x = x;
    a.cols = cols;
    launch_gemv(a, EPI_PLAIN, stream);
}

#define GATE_UP_CASES(X) \
    X(1, 1) X(1, 2) X(1, 4) X(2, 1) X(2, 2) X(2, 4) X(3, 1) X(3, 2) X(4, 1) X(4, 2) X(5, 1) \
    X(6, 1) X(8, 1) X(10, 1) X(12, 1) X(16, 1) X(20, 1)

static void launch_gate_up(bf16 *act, const bf16 *w_gate, const bf16 *w_up, const bf16 *x,
                           int rows, int cols, bf16 *gate_tap, bf16 *up_tap, const bf16 *norm_w,
                           float eps, hipStream_t stream) {
    const int nc = pick_nc(cols / 8);
    const int rpw = pick_rpw(nc, rows, 1);
    const int waves = (rows + rpw - 1) / rpw;
    const int blocks = (waves + 3) / 4;
#define X(NC_, RPW_)                                                                       \
    if (nc == NC_ && rpw == RPW_) {                                                        \
        if (norm_w)                                                                        \
            gate_up_kernel<NC_, RPW_, true><<<blocks, 256, 0, stream>>>(                   \
                act, w_gate, w_up, x, rows, cols, gate_tap, up_tap, norm_w, eps);          \
        else                                                                               \
            gate_up_kernel<NC_, RPW_><<<blocks, 256, 0, stream>>>(act, w_gate, w_up, x,    \
                                                                 rows, cols, gate_tap, up_tap); \
        LAUNCH_OK();                                                                       \
        return;                                                                            \
    }
    GATE_UP_CASES(X)
#undef X
    llm_fail("gate_up: no kernel for nc %d rpw %d", nc, rpw);
}

extern "C" void gate_up_forward(bf16 *act, const bf16 *w_gate, const bf16 *w_up, const bf16 *x,
                                int rows, int cols, bf16 *gate_tap, bf16 *up_tap,
                                hipStream_t stream) {
    if (!check_gemv("gate_up", w_gate, x, rows, cols) || !check_gemv("gate_up", w_up, x, rows, cols))
        return;
    launch_gate_up(act, w_gate, w_up, x, rows, cols, gate_tap, up_tap, nullptr, 0.0f, stream);
}

// The fused forms: RMSNorm of x (one row) as the GEMV's prologue, summing the squares in the
// order of rmsnorm_wave_kernel (lane l: chunks l, l+64, ..., then the wave tree), so the result
// is rmsnorm_forward's. That kernel covers rows of up to 64 * 16 chunks (8192 columns), which
// also fit one GEMV panel.
static bool check_norm_fused(const char *name, const bf16 *norm_w, int cols) {
    if (!norm_w) return llm_fail("%s: norm weights are NULL", name);
    if (!aligned16(norm_w)) return llm_fail("%s: norm weights must be 16-byte aligned", name);
    if ((cols / 8 + 63) / 64 > 16 || cols / 8 > 64 * pick_nc(cols / 8))
        return llm_fail("%s: %d columns do not fit one panel (at most 8192)", name, cols);
    return true;
}

extern "C" void rmsnorm_qkv_forward(bf16 *q, bf16 *k, bf16 *v, const bf16 *wq, const bf16 *wk,
                                    const bf16 *wv, const bf16 *x, const bf16 *norm_w, float eps,
                                    int q_rows, int kv_rows, int cols, hipStream_t stream) {
    if (!check_gemv("rmsnorm_qkv", wq, x, q_rows, cols) ||
        !check_gemv("rmsnorm_qkv", wk, x, kv_rows, cols) ||
        !check_gemv("rmsnorm_qkv", wv, x, kv_rows, cols) ||
        !check_norm_fused("rmsnorm_qkv", norm_w, cols))
        return;
    GemvArgs a = {};
    a.seg[0] = {wq, q, q_rows, 0};
    a.seg[1] = {wk, k, kv_rows, 0};
    a.seg[2] = {wv, v, kv_rows, 0};
    a.n_seg = 3;
    a.x = x;
    a.cols = cols;
    a.norm_w = norm_w;
    a.eps = eps;
    launch_gemv(a, EPI_PLAIN, stream);
}

extern "C" void rmsnorm_gemv_forward(bf16 *out, const bf16 *w, const bf16 *x, const bf16 *norm_w,
                                     float eps, int rows, int cols, hipStream_t stream) {
    if (!check_gemv("rmsnorm_gemv", w, x, rows, cols) ||
        !check_norm_fused("rmsnorm_gemv", norm_w, cols))
        return;
    GemvArgs a = {};
    a.seg[0] = {w, out, rows, 0};
    a.n_seg = 1;
    a.x = x;
    a.cols = cols;
    a.norm_w = norm_w;
    a.eps = eps;
    launch_gemv(a, EPI_PLAIN, stream);
}

extern "C" void rmsnorm_gate_up_forward(bf16 *act, const bf16 *w_gate, const bf16 *w_up,
                                        const bf16 *x, const bf16 *norm_w, float eps, int rows,
                                        int cols, hipStream_t stream) {
    if (!check_gemv("rmsnorm_gate_up", w_gate, x, rows, cols) ||
        !check_gemv("rmsnorm_gate_up", w_up, x, rows, cols) ||
        !check_norm_fused("rmsnorm_gate_up", norm_w, cols))
        return;
    launch_gate_up(act, w_gate, w_up, x, rows, cols, nullptr, nullptr, norm_w, eps, stream);
}

// ------------------------------------------------------------------------------------------
// SwiGLU elementwise (src/kernels.cu:283-286 over arrays)
// ------------------------------------------------------------------------------------------

__device__ __forceinline__ u32x4 swiglu8(const u32x4 &g, const u32x4 &u) {
    float gv[8], s[8], r[8];
#pragma unroll
    for (int e = 0; e < 8; e++) gv[e] = elem(g, e);
    silu_bf16x8(gv, s);
#pragma unroll
    for (int e = 0; e < 8; e++) r[e] = s[e] * elem(u, e);
    return u32x4{pack2(r[0], r[1]), pack2(r[2], r[3]), pack2(r[4], r[5]), pack2(r[6], r[7])};
}

// Grid-stride over 16-byte chunks, U chunks per thread per step. One chunk per thread and a grid
// of up to 80 workgroups per CU (every chunk of a 4096 x 9728 call in one pass) measured fastest:
// 38.7 us against 47.5 with 4 chunks per thread and 8 workgroups per CU.
constexpr int SWIGLU_U = 1;
constexpr int SWIGLU_BLOCKS_PER_CU = 80;
__global__ __launch_bounds__(256) void swiglu_kernel(bf16 *act, const bf16 *gate, const bf16 *up,
                                                     size_t n) {
    constexpr int U = SWIGLU_U;
    const size_t n_chunks = n / 8;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; c + (U - 1) * stride < n_chunks; c += U * stride) {
        u32x4 g[U], u[U];
#pragma unroll
        for (int i = 0; i < U; i++) {
            g[i] = ld16_nt(gate + 8 * (c + i * stride));
            u[i] = ld16_nt(up + 8 * (c + i * stride));
        }
#pragma unroll
        for (int i = 0; i < U; i++)
            __builtin_nontemporal_store(swiglu8(g[i], u[i]), (u32x4 *)(act + 8 * (c + i * stride)));
    }
    for (; c < n_chunks; c += stride)
        __builtin_nontemporal_store(swiglu8(ld16_nt(gate + 8 * c), ld16_nt(up + 8 * c)),
                                    (u32x4 *)(act + 8 * c));
    if (blockIdx.x == 0)
        for (size_t i = n_chunks * 8 + threadIdx.x; i < n; i += blockDim.x)
            act[i] = (bf16)f2bf(round_bf(silu_f32(bf2f(gate[i]))) * bf2f(up[i]));
}

// Scalar variant for buffers that are not 16-byte aligned.
__global__ __launch_bounds__(256) void swiglu_scalar_kernel(bf16 *act, const bf16 *gate,
                                                            const bf16 *up, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        act[i] = (bf16)f2bf(round_bf(silu_f32(bf2f(gate[i]))) * bf2f(up[i]));
}

static int device_cus() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
    }
    return cus;
}

extern "C" void swiglu_forward(bf16 *act, const bf16 *gate, const bf16 *up, size_t n,
                               hipStream_t stream) {
    if (n == 0) return;
    const size_t chunks = (n + 7) / 8;
    size_t blocks = (chunks + 255) / 256;
    const size_t cap = (size_t)device_cus() * SWIGLU_BLOCKS_PER_CU;
    if (blocks > cap) blocks = cap;
    if (aligned16(act) && aligned16(gate) && aligned16(up))
        swiglu_kernel<<<(unsigned)blocks, 256, 0, stream>>>(act, gate, up, n);
    else
        swiglu_scalar_kernel<<<(unsigned)blocks, 256, 0, stream>>>(act, gate, up, n);
    LAUNCH_OK();
}

// ------------------------------------------------------------------------------------------
// QK-norm + RoPE + KV-cache write (src/kernels.cu:301-403)
// ------------------------------------------------------------------------------------------

struct RopeArgs {
    bf16 *q;
    bf16 *k;
    const bf16 *v;
    const bf16 *qn;
    const bf16 *kn;
    bf16 *kc;
    bf16 *vc;
    const int *positions;
    bf16 *q_tap;
    bf16 *k_tap;
    int n_tokens, n_heads, n_kv_heads;
    float eps;
    int qg, kg, vg;  // waves per token: q head groups, k head groups, v copy groups
    float inv_freq[128];
};

// A wave handles 64/(D/16) heads of one token: lane L of a head holds [8L, 8L+8) and
// [D/2+8L, D/2+8L+8). Sum of squares: fma over the first chunk then the second, tree over the
// D/16 lanes. The RoPE table (cos/sin of pos*inv_freq_j in double, rounded to fp32 then bf16)
// is computed one entry per lane and fetched by lane shuffles.
template <int D>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(RopeArgs a) {
    constexpr int LH = D / 16;
    constexpr int HPW = 64 / LH;
    constexpr int HALF = D / 2;
    constexpr int NJ = (HALF + 63) / 64;
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int per_token = a.qg + a.kg + a.vg;
    const int t = wave / per_token;
    if (t >= a.n_tokens) return;
    const int item = wave - t * per_token;
    const int pos = a.positions[t];
    const int hg = lane / LH, L = lane % LH;
    const int q_dim = a.n_heads * D, kv_dim = a.n_kv_heads * D;
    const size_t slot = (size_t)pos * kv_dim;

    if (item >= a.qg + a.kg) {  // value rows into the cache
        const int h = (item - a.qg - a.kg) * HPW + hg;
        if (h < a.n_kv_heads) {
            const bf16 *src = a.v + (size_t)t * kv_dim + h * D;
            bf16 *dst = a.vc + slot + h * D;
            st16(dst + 8 * L, ld16(src + 8 * L));
            st16(dst + HALF + 8 * L, ld16(src + HALF + 8 * L));
        }
        return;
    }
    const bool is_k = item >= a.qg;
    // the wave's heads h0 .. h0 + HPW - 1 (those that exist) as one buffer, so the descriptor is
    // wave-uniform: loads past the last head read zeros and stores there are dropped; the
    // loads go out before the RoPE table is computed, which then overlaps them
    const int h0 = (is_k ? item - a.qg : item) * HPW;
    const int n_h = min(HPW, (is_k ? a.n_kv_heads : a.n_heads) - h0);
    const size_t off = (size_t)t * (is_k ? kv_dim : q_dim) + (size_t)h0 * D;
    bf16 *tap = is_k ? a.k_tap : a.q_tap;
    auto heads = [&](bf16 *base) {
        return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, n_h * D * 2, BUFFER_FLAGS);
    };
    const __amdgpu_buffer_rsrc_t xr = heads((is_k ? a.k : a.q) + off);
    const int oa = hg * D * 2 + 16 * L, ob = oa + 2 * HALF;
    const u32x4 xa = __builtin_amdgcn_raw_buffer_load_b128(xr, oa, 0, BUFFER_NT);
    const u32x4 xb = __builtin_amdgcn_raw_buffer_load_b128(xr, ob, 0, BUFFER_NT);
    const bf16 *w = is_k ? a.kn : a.qn;
    const u32x4 wa = ld16(w + 8 * L), wb = ld16(w + HALF + 8 * L);
    float cs[NJ], sn[NJ];
    rope_table<D>(pos, a.inv_freq, cs, sn);
    u32x4 ya, yb, va, vb;
    norm_rope<D>(xa, xb, wa, wb, a.eps, cs, sn, L, ya, yb, va, vb);
    if (tap) {
        const __amdgpu_buffer_rsrc_t tr = heads(tap + off);
        __builtin_amdgcn_raw_buffer_store_b128(ya, tr, oa, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(yb, tr, ob, 0, 0);
    }
    __builtin_amdgcn_raw_buffer_store_b128(va, xr, oa, 0, BUFFER_NT);
    __builtin_amdgcn_raw_buffer_store_b128(vb, xr, ob, 0, BUFFER_NT);
    if (is_k) {
        const __amdgpu_buffer_rsrc_t cr = heads(a.kc + slot + (size_t)h0 * D);
        __builtin_amdgcn_raw_buffer_store_b128(va, cr, oa, 0, BUFFER_NT);
        __builtin_amdgcn_raw_buffer_store_b128(vb, cr, ob, 0, BUFFER_NT);
    }
}

// inv_freq_j = 1 / fp32(pow(theta, fp32(2j / D))) as HF computes it (modeling_qwen3.py:121),
// cached per (theta, D).
void rope_inv_freq_table(float theta, int D, float *out) {
    static std::mutex mu;
    static float cached_theta = -1.0f;
    static int cached_d = -1;
    static float table[128];
    std::lock_guard<std::mutex> lock(mu);
    if (cached_theta != theta || cached_d != D) {
        for (int j = 0; j < D / 2; j++) {
            const float e = (float)(2 * j) / (float)D;
            table[j] = 1.0f / (float)pow((double)theta, (double)e);
        }
        cached_theta = theta;
        cached_d = D;
    }
    memcpy(out, table, sizeof(float) * (D / 2));
}

static void launch_qk_norm_rope(bf16 *q, bf16 *k, const bf16 *v, const bf16 *q_norm_w,
                                const bf16 *k_norm_w, bf16 *key_cache, bf16 *value_cache,
                                const int *positions, int n_tokens, int n_heads, int n_kv_heads,
                                int head_dim, float eps, float theta, bf16 *q_tap, bf16 *k_tap,
                                hipStream_t stream) {
    if (head_dim != 64 && head_dim != 128 && head_dim != 256) {
        llm_fail("qk_norm_rope: head_dim %d is not 64, 128 or 256", head_dim);
        return;
    }
    if (n_tokens <= 0 || n_heads <= 0 || n_kv_heads <= 0) {
        llm_fail("qk_norm_rope: n_tokens %d, n_heads %d, n_kv_heads %d must be positive",
                 n_tokens, n_heads, n_kv_heads);
        return;
    }
    const void *ptrs[] = {q, k, v, q_norm_w, k_norm_w, key_cache, value_cache, q_tap, k_tap};
    for (const void *p : ptrs)
        if (p && !aligned16(p)) {
            llm_fail("qk_norm_rope: tensors must be 16-byte aligned");
            return;
        }
    RopeArgs a;
    memset(&a, 0, sizeof a);
    a.q = q;
    a.k = k;
    a.v = v;
    a.qn = q_norm_w;
    a.kn = k_norm_w;
    a.kc = key_cache;
    a.vc = value_cache;
    a.positions = positions;
    a.q_tap = q_tap;
    a.k_tap = k_tap;
    a.n_tokens = n_tokens;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.eps = eps;
    const int hpw = 64 / (head_dim / 16);
    a.qg = (n_heads + hpw - 1) / hpw;
    a.kg = (n_kv_heads + hpw - 1) / hpw;
    a.vg = a.kg;
    rope_inv_freq_table(theta, head_dim, a.inv_freq);
    const long waves = (long)n_tokens * (a.qg + a.kg + a.vg);
    const unsigned blocks = (unsigned)((waves + 3) / 4);
    if (head_dim == 64)
        qk_norm_rope_kernel<64><<<blocks, 256, 0, stream>>>(a);
    else if (head_dim == 128)
        qk_norm_rope_kernel<128><<<blocks, 256, 0, stream>>>(a);
    else
        qk_norm_rope_kernel<256><<<blocks, 256, 0, stream>>>(a);
    LAUNCH_OK();
}

extern "C" void qk_norm_rope_forward(bf16 *q, bf16 *k, const bf16 *v, const bf16 *q_norm_w,
                                     const bf16 *k_norm_w, bf16 *key_cache, bf16 *value_cache,
                                     const int *d_pos, int n_heads, int n_kv_heads, int head_dim,
                                     float eps, float theta, bf16 *q_tap, bf16 *k_tap,
                                     hipStream_t stream) {
    launch_qk_norm_rope(q, k, v, q_norm_w, k_norm_w, key_cache, value_cache, d_pos, 1, n_heads,
                        n_kv_heads, head_dim, eps, theta, q_tap, k_tap, stream);
}

extern "C" void qk_norm_rope_rows(bf16 *q, bf16 *k, const bf16 *v, const bf16 *q_norm_w,
                                  const bf16 *k_norm_w, bf16 *key_cache, bf16 *value_cache,
                                  const int *d_positions, int n_tokens, int n_heads,
                                  int n_kv_heads, int head_dim, float eps, float theta,
                                  bf16 *q_tap, bf16 *k_tap, hipStream_t stream) {
    launch_qk_norm_rope(q, k, v, q_norm_w, k_norm_w, key_cache, value_cache, d_positions,
                        n_tokens, n_heads, n_kv_heads, head_dim, eps, theta, q_tap, k_tap, stream);
}

// ------------------------------------------------------------------------------------------
// decode attention, split softmax (src/kernels.cu:439-497)
// ------------------------------------------------------------------------------------------

constexpr int ATT_B = 64;  // positions per block

struct AttnArgs {
    bf16 *out;
    const bf16 *q;
    const bf16 *kc;
    const bf16 *vc;
    float *scores;   // [n_heads, max_seq]
    float *stats;    // [n_heads, max_blocks, 2]: block max, block sum of exp(s - max)
    float *partial;  // [n_heads, max_blocks, D]: block sums of p v
    const int *d_pos;
    int n_heads, n_kv_heads, max_seq, max_blocks;
    float scale;
};

static size_t ceil_div(size_t a, size_t b) { return (a + b - 1) / b; }

// Workspace layout: scores [n_heads, max_seq], stats [n_heads, max_blocks, 2], then (from a
// 16-byte boundary) partials [n_heads, max_blocks, D].
static size_t attention_partial_offset(int n_heads, int max_seq) {
    const size_t mb = ceil_div((size_t)max_seq, ATT_B);
    return ceil_div((size_t)n_heads * max_seq + (size_t)n_heads * mb * 2, 4) * 4;
}

extern "C" size_t attention_workspace_floats(int n_heads, int head_dim, int max_seq) {
    const size_t mb = ceil_div((size_t)max_seq, ATT_B);
    return attention_partial_offset(n_heads, max_seq) + (size_t)n_heads * mb * head_dim;
}

// Pass 1, per (block of 64 positions, kv head): scores of the REP query heads sharing the kv
// head, s = bf16(bf16(q.k) * scale) with q.k over D/8 lanes; then per head the block max and
// the block's tree sum of exp(s - max). Work items are strided over a fixed grid because the
// position count is only known on the device.
template <int D, int REP>
__global__ __launch_bounds__(256) void attn_scores_kernel(AttnArgs a) {
    constexpr int LP = D / 8, PPW = 64 / LP, PER_WAVE = ATT_B / 4, ITERS = PER_WAVE / PPW;
    __shared__ float sc[REP][ATT_B];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int G = lane / LP, L = lane % LP;
    const int n = *a.d_pos + 1;
    const int nb = (n + ATT_B - 1) / ATT_B;
    const int kv_dim = a.n_kv_heads * D;
    for (int item = blockIdx.x; item < nb * a.n_kv_heads; item += gridDim.x) {
        const int b = item / a.n_kv_heads, g = item - b * a.n_kv_heads;
        u32x4 qv[REP];
#pragma unroll
        for (int r = 0; r < REP; r++) qv[r] = ld16(a.q + (size_t)(g * REP + r) * D + 8 * L);
        u32x4 kv[ITERS];
#pragma unroll
        for (int it = 0; it < ITERS; it++) {
            const int t = b * ATT_B + w * PER_WAVE + it * PPW + G;
            kv[it] = t < n ? ld16_nt(a.kc + (size_t)t * kv_dim + g * D + 8 * L) : u32x4{0, 0, 0, 0};
        }
        // the ITERS * REP dot products of a lane, reduced over the LP lanes of its position group
        // LP at a time by reduce-scatter (each total bit-identical to group_sum<LP>): lane L of a
        // slice ends with product scatter_row(L) of that slice
        constexpr int NP = ITERS * REP, SL = NP < LP ? NP : LP;
        float part[NP];
#pragma unroll
        for (int it = 0; it < ITERS; it++)
#pragma unroll
            for (int r = 0; r < REP; r++) part[it * REP + r] = dot8(qv[r], kv[it], 0.0f);
#pragma unroll
        for (int s0 = 0; s0 < NP; s0 += SL) {
            float slice[SL];
#pragma unroll
            for (int j = 0; j < SL; j++) slice[j] = part[s0 + j];
            const float d = group_sum_scatter<LP, SL>(slice);
            const int j = s0 + scatter_row<SL>(L), it = j / REP, r = j - it * REP;
            const int slot = w * PER_WAVE + it * PPW + G;
            const int t = b * ATT_B + slot;
            const float s = round_bf(round_bf(d) * a.scale);
            if (L < SL) {
                sc[r][slot] = s;
                if (t < n) a.scores[(size_t)(g * REP + r) * a.max_seq + t] = s;
            }
        }
        __syncthreads();
        for (int r = w; r < REP; r += 4) {
            const bool v = b * ATT_B + lane < n;
            const float s = v ? sc[r][lane] : -__builtin_huge_valf();
            const float m = wave_max(s);
            const float e = v ? exp_f32(s - m) : 0.0f;
            const float S = wave_sum(e);
            if (lane == 0) {
                float *st = a.stats + ((size_t)(g * REP + r) * a.max_blocks + b) * 2;
                st[0] = m;
                st[1] = S;
            }
        }
        __syncthreads();
    }
}

// Pass 1 with the QK-norm + RoPE of the position folded in (qk_norm_rope_forward followed by
// attn_scores_kernel, the same bits): an item requests its key history rows (positions < pos)
// first, then normalises and rotates its kv head's REP query heads (waves 0 .. QWAVES-1, the
// qk_norm_rope_kernel lane layout) into LDS while they stream; the item of the block holding
// pos also rotates the key (next wave), which it uses for position pos and writes, with the
// value row, into the caches' row pos. Every item of a kv head computes the same roped query
// heads; nothing waits for another workgroup.
struct AttnRopeArgs {
    AttnArgs at;
    const bf16 *k, *v, *qn, *kn;  // at.q is the query before QK-norm + RoPE
    bf16 *kc_w, *vc_w;            // the caches, writable (row pos)
    const float *table;           // the RoPE table at *d_pos (rope_table_kernel), or NULL
    float eps;
    float inv_freq[128];
};

// The RoPE table at *d_pos, once for every layer of a step: table[j] = cos and table[D/2 + j] =
// sin of fp32(pos * inv_freq_j) as rope_table computes them (double sincos, rounded to fp32 and
// then to bf16), j < D/2.
struct RopeFreqArgs {
    float inv_freq[128];
};
__global__ __launch_bounds__(128) void rope_table_kernel(float *table, const int *d_pos,
                                                         RopeFreqArgs f, int half) {
    const int j = threadIdx.x;
    if (j < half) {
        const float angle = (float)*d_pos * f.inv_freq[j];
        double sn, cs;
        sincos_d((double)angle, &sn, &cs);
        table[j] = round_bf((float)cs);
        table[half + j] = round_bf((float)sn);
    }
}

bool rope_table_launch(float *table, const int *d_pos, int head_dim, float theta,
                       hipStream_t stream) {
    if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return llm_fail("rope_table: head_dim %d is not 64, 128 or 256", head_dim);
    RopeFreqArgs f;
    rope_inv_freq_table(theta, head_dim, f.inv_freq);
    rope_table_kernel<<<1, 128, 0, stream>>>(table, d_pos, f, head_dim / 2);
    return LAUNCH_OK();
}

// The rope inputs of one wave (the raw head rows and norm weights), requested before the key
// rows so that they are not behind them (loads complete in order), and the RoPE table.
template <int D>
struct RopeIn {
    u32x4 xa, xb, wa, wb;
    float cs[RopeShape<D>::NJ], sn[RopeShape<D>::NJ];
};

// This lane's RoPE frequencies inv_freq[lane + 64 m], m < NJ, picked out of the argument table
// with scalar loads and selects. Indexed per lane, the table would be read with a vector load,
// which the compiler places at its use, after the key rows requested before it; the wait for it
// would then wait for all of those rows.
template <int D>
struct LaneFreq {
    float f[RopeShape<D>::NJ];
    __device__ float operator[](int j) const { return f[j >> 6]; }  // j = lane + 64 m
};
template <int D>
__device__ __forceinline__ LaneFreq<D> lane_freq(const float (&table)[128]) {
    constexpr int NJ = RopeShape<D>::NJ, HALF = RopeShape<D>::HALF;
    const int lane = threadIdx.x & 63;
    LaneFreq<D> out;
#pragma unroll
    for (int m = 0; m < NJ; m++) {
        float f = 0.0f;
#pragma unroll
        for (int k = 0; k < 64 && 64 * m + k < HALF; k++) f = lane == k ? table[64 * m + k] : f;
        out.f[m] = f;
    }
    return out;
}

// Waves 0 .. QWAVES-1 take the kv head's REP query heads (HPW per wave, the qk_norm_rope_kernel
// lane layout); wave QWAVES the key head when `key`. Returns whether this wave has rope work.
template <int D, int REP>
__device__ __forceinline__ bool rope_request(const AttnRopeArgs &r, int g, int pos, bool key,
                                             RopeIn<D> &in) {
    constexpr int LH = D / 16, HPW = 64 / LH, HALF = D / 2;
    constexpr int QWAVES = (REP + HPW - 1) / HPW;
    static_assert(QWAVES < 4 && HPW >= 2, "rope waves");
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (w > QWAVES || (w == QWAVES && !key)) return false;
    const int lane = threadIdx.x & 63, hg = lane / LH, L = lane % LH;
    const bool is_k = w == QWAVES;
    const int hl0 = is_k ? 0 : w * HPW;
    const int n_h = is_k ? 1 : min(HPW, REP - hl0);
    const bf16 *src = is_k ? r.k + (size_t)g * D : r.at.q + ((size_t)g * REP + hl0) * D;
    // the wave's heads as one wave-uniform buffer: loads past the last head read zeros
    const __amdgpu_buffer_rsrc_t xr =
        __builtin_amdgcn_make_buffer_rsrc((void *)src, (short)0, n_h * D * 2, BUFFER_FLAGS);
    const int oa = hg * D * 2 + 16 * L, ob = oa + 2 * HALF;
    in.xa = __builtin_amdgcn_raw_buffer_load_b128(xr, oa, 0, 0);
    in.xb = __builtin_amdgcn_raw_buffer_load_b128(xr, ob, 0, 0);
    const bf16 *nw = is_k ? r.kn : r.qn;
    in.wa = ld16(nw + 8 * L);
    in.wb = ld16(nw + HALF + 8 * L);
    return true;
}

// QK-norm + RoPE of the requested heads into q_out / k_out (LDS); the key wave also writes k'
// and (its next group of lanes) the value row into the caches' row pos.
template <int D, int REP>
__device__ __forceinline__ void rope_finish(const AttnRopeArgs &r, int g, int pos,
                                            const RopeIn<D> &in, u32x4 *q_out, u32x4 *k_out) {
    constexpr int LH = D / 16, HPW = 64 / LH, HALF = D / 2;
    constexpr int QWAVES = (REP + HPW - 1) / HPW;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, hg = lane / LH, L = lane % LH;
    const bool is_k = w == QWAVES;
    const int hl0 = is_k ? 0 : w * HPW;
    const int n_h = is_k ? 1 : min(HPW, REP - hl0);
    const size_t kv_dim = (size_t)r.at.n_kv_heads * D;
    u32x4 ya, yb, va, vb;
    norm_rope<D>(in.xa, in.xb, in.wa, in.wb, r.eps, in.cs, in.sn, L, ya, yb, va, vb);
    if (hg < n_h) {
        u32x4 *dst = is_k ? k_out : q_out + (hl0 + hg) * (D / 8);
        dst[L] = va;
        dst[HALF / 8 + L] = vb;
        if (is_k) {
            bf16 *row = r.kc_w + (size_t)pos * kv_dim + (size_t)g * D;
            st16(row + 8 * L, va);
            st16(row + HALF + 8 * L, vb);
        }
    } else if (is_k && hg == 1) {  // the next group of lanes copies the value row
        const bf16 *vsrc = r.v + (size_t)g * D;
        bf16 *row = r.vc_w + (size_t)pos * kv_dim + (size_t)g * D;
        st16(row + 8 * L, ld16(vsrc + 8 * L));
        st16(row + HALF + 8 * L, ld16(vsrc + HALF + 8 * L));
    }
}

// TABLE: the RoPE table comes from r.table (a small load issued with the rope inputs) instead of
// being computed in double precision by every item. The kernel then fits 96 registers without
// spills for D <= 128 and REP <= 4 (five workgroups per CU instead of four: Qwen3-4B's 1056 items
// at 8448 positions are resident in one wave of 1280 slots) and its items' rope chain is shorter.
template <int D, int REP, bool TABLE>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(TABLE && D <= 128 && REP <= 4 ? 5 : 1)))
void attn_rope_scores_kernel(AttnRopeArgs r) {
    constexpr int LP = D / 8, PPW = 64 / LP, PER_WAVE = ATT_B / 4, ITERS = PER_WAVE / PPW;
    const AttnArgs &a = r.at;
    __shared__ float sc[REP][ATT_B];
    __shared__ u32x4 qk_s[(REP + 1) * (D / 8)];  // the roped query heads, then the key
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int G = lane / LP, L = lane % LP;
    const int pos = *a.d_pos;
    const int n = pos + 1;
    const int nb = (n + ATT_B - 1) / ATT_B;
    const int kv_dim = a.n_kv_heads * D;
    for (int item = blockIdx.x; item < nb * a.n_kv_heads; item += gridDim.x) {
        const int b = item / a.n_kv_heads, g = item - b * a.n_kv_heads;
        const bool last = b == nb - 1;
        RopeIn<D> in;
        const bool roper = rope_request<D, REP>(r, g, pos, last, in);
        LaneFreq<D> freq{};
        if constexpr (TABLE) {
            constexpr int HALF = D / 2;
            const __amdgpu_buffer_rsrc_t tr = __builtin_amdgcn_make_buffer_rsrc(
                (void *)r.table, (short)0, 2 * HALF * 4, BUFFER_FLAGS);
#pragma unroll
            for (int m = 0; m < RopeShape<D>::NJ; m++) {
                const int j = lane + 64 * m;  // entries past HALF read as zeros
                in.cs[m] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                    tr, 4 * (j < HALF ? j : 2 * HALF), 0, 0));
                in.sn[m] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                    tr, 4 * (j < HALF ? HALF + j : 2 * HALF), 0, 0));
            }
            __builtin_amdgcn_sched_barrier(0);  // ahead of the key rows
        } else {
            freq = lane_freq<D>(r.inv_freq);
        }
        u32x4 kv[ITERS];
#pragma unroll
        for (int it = 0; it < ITERS; it++) {
            const int t = b * ATT_B + w * PER_WAVE + it * PPW + G;
            kv[it] = t < pos ? ld16_nt(a.kc + (size_t)t * kv_dim + g * D + 8 * L) : u32x4{0, 0, 0, 0};
        }
        // the table while the rows stream (arithmetic only)
        if (!TABLE && roper) rope_table<D>(pos, freq, in.cs, in.sn);
        __syncthreads();  // qk_s of the previous item has been read
        if (roper) rope_finish<D, REP>(r, g, pos, in, qk_s, qk_s + REP * (D / 8));
        __syncthreads();
#pragma unroll
        for (int it = 0; it < ITERS; it++)
            if (b * ATT_B + w * PER_WAVE + it * PPW + G == pos) kv[it] = qk_s[REP * (D / 8) + L];
        // the scores of attn_scores_kernel
        constexpr int NP = ITERS * REP, SL = NP < LP ? NP : LP;
        float part[NP];
#pragma unroll
        for (int it = 0; it < ITERS; it++)
#pragma unroll
            for (int q = 0; q < REP; q++) part[it * REP + q] = dot8(qk_s[q * (D / 8) + L], kv[it], 0.0f);
#pragma unroll
        for (int s0 = 0; s0 < NP; s0 += SL) {
            float slice[SL];
#pragma unroll
            for (int j = 0; j < SL; j++) slice[j] = part[s0 + j];
            const float d = group_sum_scatter<LP, SL>(slice);
            const int j = s0 + scatter_row<SL>(L), it = j / REP, q = j - it * REP;
            const int slot = w * PER_WAVE + it * PPW + G;
            const int t = b * ATT_B + slot;
            const float s = round_bf(round_bf(d) * a.scale);
            if (L < SL) {
                sc[q][slot] = s;
                if (t < n) a.scores[(size_t)(g * REP + q) * a.max_seq + t] = s;
            }
        }
        __syncthreads();
        for (int q = w; q < REP; q += 4) {
            const bool v = b * ATT_B + lane < n;
            const float s = v ? sc[q][lane] : -__builtin_huge_valf();
            const float m = wave_max(s);
            const float e = v ? exp_f32(s - m) : 0.0f;
            const float S = wave_sum(e);
            if (lane == 0) {
                float *st = a.stats + ((size_t)(g * REP + q) * a.max_blocks + b) * 2;
                st[0] = m;
                st[1] = S;
            }
        }
    }
}

// Pass 2, per (block, kv head): each query head's global max M and sum (chunks of 64 block
// statistics: tree sum of S_b exp(m_b - M), chunks added in order), the block's probabilities
// p = bf16(exp(s - M) / sum), then p v accumulated per lane over its positions, tree over the
// position groups of a wave, waves added in order 0..3.
// One item of pass 2, block b of kv head g: the probabilities of the block's positions for the
// REP query heads, and the block's partial output sum p v of each head, handed over as
// store(index into the [n_heads, max_blocks, D] partials, value).
template <int D, int REP, class Store>
__device__ __forceinline__ void pv_item(const AttnArgs &a, int b, int g, int n, int nb,
                                        float (&p_s)[REP][ATT_B], float (&red)[4][REP][D],
                                        Store store) {
    constexpr int LP = D / 8, PPW = 64 / LP, PER_WAVE = ATT_B / 4, ITERS = PER_WAVE / PPW;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int G = lane / LP, L = lane % LP;
    const int kv_dim = a.n_kv_heads * D;
    // The first head of this wave (r = w): its score and block statistics are requested
    // before the values. Loads complete in order, so the statistics chain then waits only
    // for them and runs while the values stream. Unconditional (clamped indices), so no
    // branch joins before the value requests.
    constexpr int MAXC = 4;  // chunks of 64 block statistics held in registers
    const int r_first = w < REP ? w : 0;
    float mv0[MAXC], sv0[MAXC], s_t0;
    {
        const int h = g * REP + r_first;
        const float *st = a.stats + (size_t)h * a.max_blocks * 2;
        s_t0 = a.scores[(size_t)h * a.max_seq + min(b * ATT_B + lane, n - 1)];
#pragma unroll
        for (int c = 0; c < MAXC; c++) {
            const int bi = min(c * 64 + lane, nb - 1);
            mv0[c] = st[2 * bi];
            sv0[c] = st[2 * bi + 1];
        }
    }
    // every lane requests a value row (positions past n clamped to n - 1: the PV loop skips
    // those slots), so no load sits on some paths only and no wait is made conservative
    u32x4 vv[ITERS];
#pragma unroll
    for (int it = 0; it < ITERS; it++) {
        const int t = min(b * ATT_B + w * PER_WAVE + it * PPW + G, n - 1);
        vv[it] = ld16_nt(a.vc + (size_t)t * kv_dim + g * D + 8 * L);
    }
    // The first head's probabilities from those statistics (nb <= 64 * MAXC: the max is exact
    // in any order, so over the lane's chunks first and then one wave_max; the chunk sums
    // added in order), computed by every wave with no branch, so the requests above are not
    // moved below the value requests. Kept only by a wave that has a head, for nb <= 64 MAXC.
    float p0;
    {
        float ml = -__builtin_huge_valf();
#pragma unroll
        for (int c = 0; c < MAXC; c++) ml = c * 64 + lane < nb ? fmaxf(ml, mv0[c]) : ml;
        const float M = wave_max(ml);
        float cs[MAXC];
#pragma unroll
        for (int c = 0; c < MAXC; c++)
            cs[c] = wave_sum(c * 64 + lane < nb ? sv0[c] * exp_f32(mv0[c] - M) : 0.0f);
        float sum = cs[0];
#pragma unroll
        for (int c = 1; c < MAXC; c++) sum = c * 64 < nb ? sum + cs[c] : sum;
        p0 = b * ATT_B + lane < n ? round_bf(exp_f32(s_t0 - M) / sum) : 0.0f;
    }
    for (int r = w; r < REP; r += 4) {
        if (r == w && nb <= 64 * MAXC) {
            p_s[r][lane] = p0;
            continue;
        }
        // a second head of the wave (REP = 8), or more than 64 * MAXC blocks
        const int h = g * REP + r;
        const float *st = a.stats + (size_t)h * a.max_blocks * 2;
        const int t = b * ATT_B + lane;
        const float s_t = a.scores[(size_t)h * a.max_seq + min(t, n - 1)];
        float M = -__builtin_huge_valf(), sum = 0.0f;
        if (nb <= 64 * MAXC) {
            // every statistic requested at once (clamped indices, no branch around the
            // loads), then the same max and in-order chunk sums as p0's
            float mv[MAXC], sv[MAXC];
#pragma unroll
            for (int c = 0; c < MAXC; c++) {
                const int bi = min(c * 64 + lane, nb - 1);
                mv[c] = st[2 * bi];
                sv[c] = st[2 * bi + 1];
            }
            float ml = -__builtin_huge_valf();
#pragma unroll
            for (int c = 0; c < MAXC; c++)
                if (c * 64 + lane < nb) ml = fmaxf(ml, mv[c]);
            M = wave_max(ml);
#pragma unroll
            for (int c = 0; c < MAXC; c++)
                if (c * 64 < nb) {
                    const float term = c * 64 + lane < nb ? sv[c] * exp_f32(mv[c] - M) : 0.0f;
                    const float cs = wave_sum(term);
                    sum = c == 0 ? cs : sum + cs;
                }
        } else {
            for (int c0 = 0; c0 < nb; c0 += 64) {
                const int bi = c0 + lane;
                M = fmaxf(M, wave_max(bi < nb ? st[2 * bi] : -__builtin_huge_valf()));
            }
            for (int c0 = 0; c0 < nb; c0 += 64) {
                const int bi = c0 + lane;
                const float term = bi < nb ? st[2 * bi + 1] * exp_f32(st[2 * bi] - M) : 0.0f;
                const float cs = wave_sum(term);
                sum = c0 == 0 ? cs : sum + cs;
            }
        }
        p_s[r][lane] = t < n ? round_bf(exp_f32(s_t - M) / sum) : 0.0f;
    }
    __syncthreads();
    float acc[REP][8];
#pragma unroll
    for (int r = 0; r < REP; r++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[r][e] = 0.0f;
#pragma unroll
    for (int it = 0; it < ITERS; it++) {
        const int slot = w * PER_WAVE + it * PPW + G;
        if (b * ATT_B + slot < n) {
#pragma unroll
            for (int r = 0; r < REP; r++) {
                const float p = p_s[r][slot];
#pragma unroll
                for (int e = 0; e < 8; e++) acc[r][e] = fmaf(p, elem(vv[it], e), acc[r][e]);
            }
        }
    }
    // the position groups (lanes LP apart) summed with the pairing of butterfly_sum<LP, 64>,
    // reduce-scattered: each lane keeps REP * 8 / (64 / LP) of the values, at offset `off`
    constexpr int NV = REP * 8, NG = 64 / LP, KEEP = NV / NG;
    float flat[NV], kept[KEEP];
#pragma unroll
    for (int r = 0; r < REP; r++)
#pragma unroll
        for (int e = 0; e < 8; e++) flat[r * 8 + e] = acc[r][e];
    scatter_keep<NV, LP, 64>(flat, kept);
    int off = 0;
#pragma unroll
    for (int k = 0, m = NV; (LP << k) < 64; k++, m >>= 1)
        if ((lane >> k) & LP) off += m / 2;
#pragma unroll
    for (int j = 0; j < KEEP; j++) {
        const int idx = off + j, r = idx / 8, e = idx % 8;
        red[w][r][8 * L + e] = kept[j];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < REP * D; i += 256) {
        const int r = i / D, d = i - r * D;
        const float v = ((red[0][r][d] + red[1][r][d]) + red[2][r][d]) + red[3][r][d];
        store(((size_t)(g * REP + r) * a.max_blocks + b) * D + d, v);
    }
    __syncthreads();
}

template <int D, int REP>
__global__ __launch_bounds__(256) void attn_pv_kernel(AttnArgs a) {
    __shared__ float p_s[REP][ATT_B];
    __shared__ float red[4][REP][D];
    const int n = *a.d_pos + 1;
    const int nb = (n + ATT_B - 1) / ATT_B;
    for (int item = blockIdx.x; item < nb * a.n_kv_heads; item += gridDim.x) {
        const int b = item / a.n_kv_heads, g = item - b * a.n_kv_heads;
        pv_item<D, REP>(a, b, g, n, nb, p_s, red,
                        [&](size_t i, float v) { a.partial[i] = v; });
    }
}

// Pass 3: out = bf16(block partials added in block order). A workgroup takes COMBINE_COLS
// columns of one query head (D / COMBINE_COLS workgroups per head, so the loads spread over
// more CUs). The additions are sequential, the loads are not: the columns' partials are staged
// in LDS by all 256 threads (every 16-byte load of a chunk of CB blocks in flight at once), then
// thread c adds column c in block order, 16 LDS reads at a time.
constexpr int COMBINE_COLS = 32;
template <int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
    constexpr int CC = COMBINE_COLS, Q = CC / 4;  // columns; 16-byte loads per block row
    constexpr int CB = 256;                      // blocks per LDS chunk (32 KB, 16384 positions)
    static_assert(D % CC == 0, "columns per workgroup");
    __shared__ float part[CB * CC];
    const int h = blockIdx.x / (D / CC), c0 = (blockIdx.x % (D / CC)) * CC;
    const float *src = a.partial + (size_t)h * a.max_blocks * D + c0;
    float acc = 0.0f;
    // Each chunk's loads cover min(CB, max_blocks - b0) blocks, whatever the history, and the
    // position is read after them (a per-lane load: as a uniform value it would be loaded, and
    // waited for, before them): one round trip instead of two. Blocks past the history are
    // loaded and not added.
    for (int b0 = 0; b0 < a.max_blocks; b0 += CB) {
        if (b0 > 0) __syncthreads();  // the previous chunk has been added
        constexpr int PER = CB * Q / 256;  // 16-byte loads per thread for a full chunk
        const int n4 = min(CB, a.max_blocks - b0) * Q;
        u32x4 v4[PER];
#pragma unroll
        for (int j = 0; j < PER; j++) {
            // load i: block b0 + i / Q, columns c0 + 4 (i % Q) .. + 3
            const int i = min((int)threadIdx.x + 256 * j, n4 - 1);
            v4[j] = *(const u32x4 *)(src + (size_t)(b0 + i / Q) * D + 4 * (i % Q));
        }
        const int n = a.d_pos[tid_x() >> 31] + 1;
        // staged before the history is looked at, so the loads above cannot be moved past it
#pragma unroll
        for (int j = 0; j < PER; j++)
            if ((int)threadIdx.x + 256 * j < n4) ((u32x4 *)part)[threadIdx.x + 256 * j] = v4[j];
        const int nb = __builtin_amdgcn_readfirstlane((n + ATT_B - 1) / ATT_B);
        if (b0 >= nb) break;
        const int cnt = min(CB, nb - b0);
        __syncthreads();
        if (threadIdx.x < CC) {
            // 16 LDS reads in flight, then their additions in order
            const int c = threadIdx.x;
            for (int j0 = 0; j0 < cnt; j0 += 16) {
                float v[16];
#pragma unroll
                for (int j = 0; j < 16; j++) v[j] = part[min(j0 + j, cnt - 1) * CC + c];
#pragma unroll
                for (int j = 0; j < 16; j++)
                    if (j0 + j < cnt) acc = (b0 + j0 + j == 0) ? v[j] : acc + v[j];
            }
        }
    }
    if (threadIdx.x < CC) a.out[(size_t)h * D + c0 + threadIdx.x] = (bf16)f2bf(acc);
}

// ------------------------------------------------------------------------------------------
// One-pass attention of the step: QK-norm + RoPE, the scores, the split softmax, PV and the
// combine in ONE launch, with the arithmetic of qk_norm_rope_kernel followed by
// attn_scores/pv/combine (the same bits; blocks of 64 positions as there). Workgroup (g, i), i
// < ipk, of kv head g takes the blocks i, i + ipk, i + 2 ipk, ... of the history. The split
// softmax has two global steps: every block's statistics before any probability, every block's
// partial output before the combine. They are handoffs between the ipk workgroups of a kv head,
// as tagged 64-bit words (float bits << 32 | tag, agent-scope atomic stores and loads; the tag
// names the launch), so the data is its own ready signal: no counter, no fence, no grid
// barrier. The combine is split by columns: workgroup i adds, in block order, the partials of
// its columns of the kv head's query heads. Each workgroup counts its launches in a word of
// its own (one cache line each: the count every wave reads at the start is not one line that
// the whole grid queues on), so the tag is that count + 1.
//
// Workgroups wait for each other, so all must be resident: the grid never exceeds the CU count
// (one 512-thread workgroup per CU fits), and every wait is bounded (on timeout the error flag
// is set and the kernel finishes with what it read).
// ------------------------------------------------------------------------------------------

constexpr int OP_WAVES = 8, OP_THREADS = 64 * OP_WAVES;
constexpr int OP_PRE = 3;          // rounds (two blocks each) whose K/V rows are requested first
constexpr int OP_MAXJ = 16;        // blocks of one workgroup (scores and probabilities in LDS)
constexpr int OP_MAXB = 512;       // blocks of the history (32768 positions)
constexpr int OP_MAXCPI = 32;      // combine columns of one workgroup
constexpr int OP_STAGE = 8192;     // floats staged: statistics, or a chunk of combine partials
constexpr long long OP_SPIN_LIMIT = 1 << 22;
constexpr int OP_MAXGRID = 1024;   // workgroups (launch counters in the workspace)
constexpr int OP_CTR_STRIDE = 16;  // 8-byte words between two counters (128 bytes)
constexpr size_t OP_HEADER = (size_t)OP_MAXGRID * OP_CTR_STRIDE * 8;

struct OnePassArgs {
    AttnRopeArgs r;                  // r.at.q: the query before QK-norm + RoPE; r.at.out: output
    unsigned long long *tstats;      // [n_heads, max_blocks, 2] tagged block max, block sum
    unsigned long long *tpart;       // [n_heads, max_blocks, D] tagged block partial outputs
    unsigned long long *launches;    // per workgroup (OP_CTR_STRIDE words apart): its launches
    int *err;                        // set to 2 when a wait times out
    int ipk;                         // workgroups per kv head
    int cpi;                         // combine columns per workgroup
};

__device__ __forceinline__ unsigned long long op_ld(const unsigned long long *p) {
    return __hip_atomic_load(gptr((unsigned long long *)p), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void op_st(unsigned long long *p, float v, uint32_t tag) {
    __hip_atomic_store(gptr(p), ((unsigned long long)__float_as_uint(v) << 32) | tag,
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Polls the tagged words addr(idx), idx = threadIdx.x + NT k < total (NT threads in the
// workgroup, K words of a thread in flight), until every tag is `tag`, and hands each value to
// put(idx, value). Bounded: once *err is set (by another wait or an earlier error), or when its
// own polls run out (then *err = 2 unless already set), it goes on with what it read.
template <int NT = OP_THREADS, int K = 8, class Addr, class Put>
__device__ __forceinline__ void op_poll(int total, uint32_t tag, int *err, Addr addr, Put put) {
    for (int base = 0; base < total; base += NT * K) {
        unsigned long long wv[K];
        long long spins = 0;
        for (;;) {
            bool fresh = true;
#pragma unroll
            for (int k = 0; k < K; k++) {
                const int idx = base + (int)threadIdx.x + NT * k;
                wv[k] = idx < total ? op_ld(addr(idx)) : 0ull;
                fresh &= idx >= total || (uint32_t)wv[k] == tag;
            }
            if (fresh) break;
            if ((++spins & 15) == 0 && wait_gives_up(spins, OP_SPIN_LIMIT, err)) break;
        }
#pragma unroll
        for (int k = 0; k < K; k++) {
            const int idx = base + (int)threadIdx.x + NT * k;
            if (idx < total) put(idx, __uint_as_float((uint32_t)(wv[k] >> 32)));
        }
    }
}

template <int REP>
__global__ __launch_bounds__(OP_THREADS) void attn_one_pass_kernel(OnePassArgs o) {
    constexpr int D = 128, LP = D / 8, PPW = 64 / LP, ITERS = ATT_B / 4 / PPW;
    static_assert(ITERS == 4, "a wave takes a quarter (16 positions) of a block");
    constexpr int MAXC = 4;  // chunks of 64 block statistics held in registers
    const AttnRopeArgs &r = o.r;
    const AttnArgs &a = r.at;
    __shared__ u32x4 qk_s[(REP + 1) * (D / 8)];  // the roped query heads, then the key
    __shared__ float sc[REP][OP_MAXJ][ATT_B];    // scores, then probabilities
    __shared__ float red[2][4][REP][D];          // PV quarters of a round's two blocks
    __shared__ float stage[OP_STAGE];            // statistics / a chunk of combine partials
    __shared__ float gstat[REP][2];              // each head's global max and sum
    __shared__ unsigned long long launch_s;

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int half = w >> 2, qtr = w & 3;  // block of a round, quarter of the block
    const int G = lane / LP, L = lane % LP;
    const int ipk = o.ipk;
    const int g = blockIdx.x / ipk, i = blockIdx.x - g * ipk;
    const int pos = *a.d_pos;
    if (pos < 0 || pos >= a.max_seq) {  // every workgroup reads the same pos: all return
        if (threadIdx.x == 0) *o.err = 1;
        return;
    }
    const int n = pos + 1;
    const int nb = (n + ATT_B - 1) / ATT_B;
    const int nj = nb > i ? (nb - i + ipk - 1) / ipk : 0;  // blocks of this workgroup
    const bool owner = (pos / ATT_B) % ipk == i;            // holds the block of pos
    const int row_bytes = a.n_kv_heads * D * 2;
    auto slot_pos = [&](int j, int it) {  // position of this lane's slot `it` in block j
        return (i + ipk * j) * ATT_B + qtr * 16 + it * PPW + G;
    };
    // The kv head's K and V history as buffers over rows 0..pos-1: a lane's load of a row at or
    // past pos, or of a block this workgroup does not have (offset past the end), returns zeros
    // without a memory access. Every load is then unconditional, so each wait below waits
    // exactly for the rows it needs (loads complete in order).
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a.kc + g * D), (short)0, pos * row_bytes, BUFFER_FLAGS);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a.vc + g * D), (short)0, pos * row_bytes, BUFFER_FLAGS);
    auto off = [&](int j, int it) { return (uint32_t)(slot_pos(j, it) * row_bytes + 16 * L); };
    auto rows_of = [&](const __amdgpu_buffer_rsrc_t &all, const bf16 *base, int j) {
        return j < nj ? all : __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, 0,
                                                                BUFFER_FLAGS);
    };

    // Every request is unconditional (absent data: empty buffers), issued in the order of use:
    // the launch counter, the rope inputs (wave 0: the query heads; wave 1 of the workgroup
    // holding pos: the key head, and the value row for the cache and PV), this lane's RoPE
    // frequency, then the K and V rows of the first rounds.
    const unsigned long long launches = op_ld(o.launches + (size_t)blockIdx.x * OP_CTR_STRIDE);
    constexpr int LH = D / 16, HALF = D / 2;
    static_assert(REP <= 64 / LH, "a kv head's query heads in one wave");
    const bool rq_q = w == 0, rq_k = w == 1 && owner;
    const int hg = lane / LH, Lr = lane % LH;
    RopeIn<D> in;
    {
        const bf16 *src = rq_k ? r.k + (size_t)g * D : a.q + (size_t)g * REP * D;
        const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
            (void *)src, (short)0, rq_q ? REP * D * 2 : rq_k ? D * 2 : 0, BUFFER_FLAGS);
        in.xa = __builtin_amdgcn_raw_buffer_load_b128(xr, hg * D * 2 + 16 * Lr, 0, 0);
        in.xb = __builtin_amdgcn_raw_buffer_load_b128(xr, hg * D * 2 + 16 * Lr + D, 0, 0);
        const __amdgpu_buffer_rsrc_t nr = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(rq_k ? r.kn : r.qn), (short)0, rq_q || rq_k ? D * 2 : 0, BUFFER_FLAGS);
        in.wa = __builtin_amdgcn_raw_buffer_load_b128(nr, 16 * Lr, 0, 0);
        in.wb = __builtin_amdgcn_raw_buffer_load_b128(nr, 16 * Lr + D, 0, 0);
    }
    // the value row of pos: every lane of the workgroup holding pos (PV), lanes L of wave 1's
    // second head group write it to the cache
    const __amdgpu_buffer_rsrc_t vrow = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(r.v + (size_t)g * D), (short)0, owner ? D * 2 : 0, BUFFER_FLAGS);
    const u32x4 vcur = __builtin_amdgcn_raw_buffer_load_b128(vrow, 16 * L, 0, 0);
    const u32x4 vcp_a = __builtin_amdgcn_raw_buffer_load_b128(vrow, 16 * Lr, 0, 0);
    const u32x4 vcp_b = __builtin_amdgcn_raw_buffer_load_b128(vrow, 16 * Lr + D, 0, 0);
    const LaneFreq<D> freq = lane_freq<D>(r.inv_freq);
    // the small requests stay ahead of the rows (the compiler would otherwise move them after,
    // and every wait for them would wait for all the rows too)
    __builtin_amdgcn_sched_barrier(0);
    u32x4 kpre[OP_PRE][ITERS], vpre[OP_PRE][ITERS];
#pragma unroll
    for (int rd = 0; rd < OP_PRE; rd++) {
        const __amdgpu_buffer_rsrc_t kr = rows_of(krs, a.kc, 2 * rd + half);
#pragma unroll
        for (int it = 0; it < ITERS; it++)
            kpre[rd][it] = __builtin_amdgcn_raw_buffer_load_b128(kr, off(2 * rd + half, it), 0,
                                                                 BUFFER_NT);
    }
#pragma unroll
    for (int rd = 0; rd < OP_PRE; rd++) {
        const __amdgpu_buffer_rsrc_t vr = rows_of(vrs, a.vc, 2 * rd + half);
#pragma unroll
        for (int it = 0; it < ITERS; it++)
            vpre[rd][it] = __builtin_amdgcn_raw_buffer_load_b128(vr, off(2 * rd + half, it), 0,
                                                                 BUFFER_NT);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (rq_q || rq_k) rope_table<D>(pos, freq, in.cs, in.sn);  // while the rows stream
    if (threadIdx.x == 0) launch_s = launches;
    __syncthreads();
    const uint32_t tag = (uint32_t)(launch_s % 0xffffffffull) + 1u;
    // QK-norm + RoPE (qk_norm_rope_kernel lane layout): the roped query heads and key into
    // LDS; the workgroup holding pos writes k' and v into the caches' row pos
    if (rq_q || rq_k) {
        u32x4 ya, yb, va, vb;
        norm_rope<D>(in.xa, in.xb, in.wa, in.wb, r.eps, in.cs, in.sn, Lr, ya, yb, va, vb);
        const size_t row = (size_t)pos * a.n_kv_heads * D + (size_t)g * D;
        if (rq_q && hg < REP) {
            qk_s[hg * (D / 8) + Lr] = va;
            qk_s[hg * (D / 8) + HALF / 8 + Lr] = vb;
        } else if (rq_k && hg == 0) {
            qk_s[REP * (D / 8) + Lr] = va;
            qk_s[REP * (D / 8) + HALF / 8 + Lr] = vb;
            st16(r.kc_w + row + 8 * Lr, va);
            st16(r.kc_w + row + HALF + 8 * Lr, vb);
        } else if (rq_k && hg == 1) {
            st16(r.vc_w + row + 8 * Lr, vcp_a);
            st16(r.vc_w + row + HALF + 8 * Lr, vcp_b);
        }
    }
    __syncthreads();

    // scores (attn_scores_kernel): block j's quarter qtr, 16 lanes per position
    auto scores = [&](int j, const u32x4 (&kr)[ITERS]) {
        const u32x4 kcur = qk_s[REP * (D / 8) + L];
        u32x4 qv[REP];
#pragma unroll
        for (int q = 0; q < REP; q++) qv[q] = qk_s[q * (D / 8) + L];
        constexpr int NP = ITERS * REP, SL = NP < LP ? NP : LP;
        float part[NP];
#pragma unroll
        for (int it = 0; it < ITERS; it++) {
            const u32x4 kk = slot_pos(j, it) == pos ? kcur : kr[it];
#pragma unroll
            for (int q = 0; q < REP; q++) part[it * REP + q] = dot8(qv[q], kk, 0.0f);
        }
#pragma unroll
        for (int s0 = 0; s0 < NP; s0 += SL) {
            float slice[SL];
#pragma unroll
            for (int u = 0; u < SL; u++) slice[u] = part[s0 + u];
            const float d = group_sum_scatter<LP, SL>(slice);
            const int u = s0 + scatter_row<SL>(L), it = u / REP, q = u - it * REP;
            if (L < SL) sc[q][j][qtr * 16 + it * PPW + G] = round_bf(round_bf(d) * a.scale);
        }
    };
#pragma unroll
    for (int rd = 0; rd < OP_PRE; rd++)
        if (2 * rd + half < nj) scores(2 * rd + half, kpre[rd]);
    for (int j = 2 * OP_PRE + half; j < nj; j += 2) {
        u32x4 kr[ITERS];
#pragma unroll
        for (int it = 0; it < ITERS; it++)
            kr[it] = __builtin_amdgcn_raw_buffer_load_b128(rows_of(krs, a.kc, j), off(j, it), 0,
                                                           BUFFER_NT);
        scores(j, kr);
    }
    __syncthreads();

    // block statistics (max, tree sum of exp(s - max)), published tagged; two (head, block)
    // pairs per wave at a time
    for (int p0 = w; p0 < REP * nj; p0 += 2 * OP_WAVES) {
        float s2[2], m2[2], e2[2], S2[2];
        bool v2[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int p = min(p0 + u * OP_WAVES, REP * nj - 1), q = p % REP, j = p / REP;
            v2[u] = (i + ipk * j) * ATT_B + lane < n;
            s2[u] = v2[u] ? sc[q][j][lane] : -__builtin_huge_valf();
        }
#pragma unroll
        for (int u = 0; u < 2; u++) m2[u] = wave_max(s2[u]);
#pragma unroll
        for (int u = 0; u < 2; u++) e2[u] = v2[u] ? exp_f32(s2[u] - m2[u]) : 0.0f;
#pragma unroll
        for (int u = 0; u < 2; u++) S2[u] = wave_sum(e2[u]);
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int p = p0 + u * OP_WAVES;
            if (p < REP * nj && lane < 2) {
                const int q = p % REP, j = p / REP, b = i + ipk * j;
                unsigned long long *st = o.tstats + ((size_t)(g * REP + q) * a.max_blocks + b) * 2;
                op_st(st + lane, lane == 0 ? m2[u] : S2[u], tag);
            }
        }
    }

    // every block's statistics of the kv head's query heads, then each head's global max and
    // sum (attn_pv_kernel order: max over all blocks; chunks of 64 blocks summed by the wave
    // tree, the chunk sums added in order)
    op_poll(REP * nb * 2, tag, o.err,
            [&](int idx) {
                const int q = idx / (2 * nb), rest = idx - q * 2 * nb;
                return o.tstats + ((size_t)(g * REP + q) * a.max_blocks) * 2 + rest;
            },
            [&](int idx, float v) { stage[idx] = v; });
    __syncthreads();
    if (w < REP) {
        const float *st = stage + w * 2 * nb;
        float M, sum;
        if (nb <= 64 * MAXC) {
            // the chunks' terms and wave sums side by side (independent chains)
            float mv[MAXC], sv[MAXC], cs[MAXC];
#pragma unroll
            for (int c = 0; c < MAXC; c++) {
                const int bi = min(c * 64 + lane, nb - 1);
                mv[c] = st[2 * bi];
                sv[c] = st[2 * bi + 1];
            }
            float ml = -__builtin_huge_valf();
#pragma unroll
            for (int c = 0; c < MAXC; c++) ml = c * 64 + lane < nb ? fmaxf(ml, mv[c]) : ml;
            M = wave_max(ml);
#pragma unroll
            for (int c = 0; c < MAXC; c++)
                cs[c] = wave_sum(c * 64 + lane < nb ? sv[c] * exp_f32(mv[c] - M) : 0.0f);
            sum = cs[0];
#pragma unroll
            for (int c = 1; c < MAXC; c++) sum = c * 64 < nb ? sum + cs[c] : sum;
        } else {
            float ml = -__builtin_huge_valf();
            for (int c0 = 0; c0 < nb; c0 += 64)
                if (c0 + lane < nb) ml = fmaxf(ml, st[2 * (c0 + lane)]);
            M = wave_max(ml);
            sum = 0.0f;
            for (int c0 = 0; c0 < nb; c0 += 64) {
                const int bi = c0 + lane;
                const float cs =
                    wave_sum(bi < nb ? st[2 * bi + 1] * exp_f32(st[2 * bi] - M) : 0.0f);
                sum = c0 == 0 ? cs : sum + cs;
            }
        }
        if (lane == 0) {
            gstat[w][0] = M;
            gstat[w][1] = sum;
        }
    }
    __syncthreads();

    // PV (attn_pv_kernel), per round of two blocks: each wave turns the scores of its quarter
    // into probabilities p = bf16(exp(s - M) / sum) (0 past the history; only this wave reads
    // them), lane (G, L) accumulates its 4 slots, the position groups meet in the butterfly's
    // pairing (reduce-scattered), the quarters are added in order 0..3, and each block's partial
    // output is published tagged
    auto pv_round = [&](int rd, const u32x4 (&vr)[ITERS]) {
        const int j = 2 * rd + half;
        if (j < nj) {
            const int b = i + ipk * j;
#pragma unroll
            for (int u = 0; u < (REP * 16 + 63) / 64; u++) {
                const int idx = lane + 64 * u, q = idx / 16, sl = qtr * 16 + idx % 16;
                if (idx < REP * 16) {
                    const float s = sc[q][j][sl];
                    sc[q][j][sl] =
                        b * ATT_B + sl < n ? round_bf(exp_f32(s - gstat[q][0]) / gstat[q][1]) : 0.0f;
                }
            }
            float acc[REP][8];
#pragma unroll
            for (int q = 0; q < REP; q++)
#pragma unroll
                for (int e = 0; e < 8; e++) acc[q][e] = 0.0f;
#pragma unroll
            for (int it = 0; it < ITERS; it++) {
                const int t = slot_pos(j, it);
                if (t < n) {
                    const u32x4 vt = t == pos ? vcur : vr[it];
#pragma unroll
                    for (int q = 0; q < REP; q++) {
                        const float p = sc[q][j][qtr * 16 + it * PPW + G];
#pragma unroll
                        for (int e = 0; e < 8; e++) acc[q][e] = fmaf(p, elem(vt, e), acc[q][e]);
                    }
                }
            }
            constexpr int NV = REP * 8, NG = 64 / LP, KEEP = NV / NG;
            float flat[NV], kept[KEEP];
#pragma unroll
            for (int q = 0; q < REP; q++)
#pragma unroll
                for (int e = 0; e < 8; e++) flat[q * 8 + e] = acc[q][e];
            scatter_keep<NV, LP, 64>(flat, kept);
            int off0 = 0;
#pragma unroll
            for (int k = 0, m = NV; (LP << k) < 64; k++, m >>= 1)
                if ((lane >> k) & LP) off0 += m / 2;
#pragma unroll
            for (int u = 0; u < KEEP; u++) {
                const int idx = off0 + u, q = idx / 8, e = idx % 8;
                red[half][qtr][q][8 * L + e] = kept[u];
            }
        }
        __syncthreads();
        for (int idx = threadIdx.x; idx < 2 * REP * D; idx += OP_THREADS) {
            const int h2 = idx / (REP * D), rest = idx - h2 * REP * D;
            const int q = rest / D, d = rest - q * D, jb = 2 * rd + h2;
            if (jb < nj) {
                const float v = ((red[h2][0][q][d] + red[h2][1][q][d]) + red[h2][2][q][d]) +
                                red[h2][3][q][d];
                const int b = i + ipk * jb;
                op_st(o.tpart + ((size_t)(g * REP + q) * a.max_blocks + b) * D + d, v, tag);
            }
        }
        __syncthreads();
    };
#pragma unroll
    for (int rd = 0; rd < OP_PRE; rd++)
        if (2 * rd < nj) pv_round(rd, vpre[rd]);
    for (int rd = OP_PRE; 2 * rd < nj; rd++) {
        u32x4 vr[ITERS];
#pragma unroll
        for (int it = 0; it < ITERS; it++)
            vr[it] = __builtin_amdgcn_raw_buffer_load_b128(rows_of(vrs, a.vc, 2 * rd + half),
                                                           off(2 * rd + half, it), 0, BUFFER_NT);
        pv_round(rd, vr);
    }

    // combine (attn_combine_kernel): columns [c0, c1) of the kv head's REP * D, each the
    // block partials added in block order, staged in chunks of the blocks
    const int c0 = i * o.cpi, c1 = min(REP * D, c0 + o.cpi), nc = c1 - c0;
    if (nc > 0) {
        const int cb = OP_STAGE / nc;  // blocks per chunk
        float acc = 0.0f;
        for (int b0 = 0; b0 < nb; b0 += cb) {
            const int cnt = min(cb, nb - b0);
            op_poll(cnt * nc, tag, o.err,
                    [&](int idx) {
                        const int bb = idx / nc, c = c0 + idx - bb * nc, q = c / D, d = c - q * D;
                        return o.tpart + ((size_t)(g * REP + q) * a.max_blocks + b0 + bb) * D + d;
                    },
                    [&](int idx, float v) { stage[idx] = v; });
            __syncthreads();
            if ((int)threadIdx.x < nc) {
                const int c = threadIdx.x;
                int j0 = 0;
                if (b0 == 0) {
                    acc = stage[c];
                    j0 = 1;
                }
                for (; j0 + 16 <= cnt; j0 += 16) {  // 16 LDS reads in flight, then the adds
                    float v[16];
#pragma unroll
                    for (int u = 0; u < 16; u++) v[u] = stage[(j0 + u) * nc + c];
#pragma unroll
                    for (int u = 0; u < 16; u++) acc += v[u];
                }
                for (; j0 < cnt; j0++) acc += stage[j0 * nc + c];
            }
            __syncthreads();
        }
        if ((int)threadIdx.x < nc) {
            const int c = c0 + threadIdx.x, q = c / D, d = c - q * D;
            a.out[(size_t)(g * REP + q) * D + d] = (bf16)f2bf(acc);
        }
    }
    if (threadIdx.x == 0)
        __hip_atomic_store(gptr(o.launches + (size_t)blockIdx.x * OP_CTR_STRIDE), launch_s + 1,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

extern "C" size_t attention_one_pass_bytes(int n_heads, int head_dim, int max_seq) {
    const size_t mb = ceil_div((size_t)max_seq, ATT_B);
    return OP_HEADER + (size_t)n_heads * mb * 2 * 8 + (size_t)n_heads * mb * head_dim * 8;
}

// The workgroups per kv head of the one-pass attention on this device (0: not supported).
static int one_pass_ipk(int n_heads, int n_kv_heads, int head_dim, int max_seq) {
    if (head_dim != 128 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0) return 0;
    const int rep = n_heads / n_kv_heads;
    if (rep != 1 && rep != 2 && rep != 4 && rep != 8) return 0;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    int ipk = (cus < OP_MAXGRID ? cus : OP_MAXGRID) / n_kv_heads;
    if (ipk > 64) ipk = 64;
    const int max_blocks = (int)ceil_div((size_t)max_seq, ATT_B);
    if ((size_t)max_seq * n_kv_heads * head_dim * 2 >= ((size_t)1 << 31)) return 0;
    if (ipk < 1 || max_blocks > OP_MAXB || max_blocks > ipk * OP_MAXJ ||
        (rep * head_dim + ipk - 1) / ipk > OP_MAXCPI)
        return 0;
    return ipk;
}

extern "C" int attention_one_pass_supported(int n_heads, int n_kv_heads, int head_dim,
                                            int max_seq) {
    return one_pass_ipk(n_heads, n_kv_heads, head_dim, max_seq) > 0;
}

bool attention_one_pass_launch(bf16 *out, const bf16 *q, const bf16 *k, const bf16 *v,
                               const bf16 *q_norm_w, const bf16 *k_norm_w, bf16 *key_cache,
                               bf16 *value_cache, void *ws, int *err, const int *d_pos,
                               int n_heads, int n_kv_heads, int head_dim, float eps, float theta,
                               int max_seq, float scale, hipStream_t stream) {
    const int ipk = one_pass_ipk(n_heads, n_kv_heads, head_dim, max_seq);
    if (ipk <= 0)
        return llm_fail("attention_one_pass: no one-pass attention for %d/%d heads of %d over %d "
                        "positions on this device", n_heads, n_kv_heads, head_dim, max_seq);
    const void *ptrs[] = {out, q, k, v, q_norm_w, k_norm_w, key_cache, value_cache, ws, err,
                          d_pos};
    for (const void *p : ptrs)
        if (!p) return llm_fail("attention_one_pass: null pointer argument");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(q_norm_w) ||
        !aligned16(k_norm_w) || !aligned16(key_cache) || !aligned16(value_cache) ||
        ((uintptr_t)ws & 255))
        return llm_fail("attention_one_pass: q, k, v, the norm weights and the caches must be "
                        "16-byte aligned and the workspace 256-byte aligned");
    OnePassArgs o;
    memset(&o, 0, sizeof o);
    AttnArgs &a = o.r.at;
    a.out = out;
    a.q = q;
    a.kc = key_cache;
    a.vc = value_cache;
    a.d_pos = d_pos;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.max_seq = max_seq;
    a.max_blocks = (int)ceil_div((size_t)max_seq, ATT_B);
    a.scale = scale;
    o.r.k = k;
    o.r.v = v;
    o.r.qn = q_norm_w;
    o.r.kn = k_norm_w;
    o.r.kc_w = key_cache;
    o.r.vc_w = value_cache;
    o.r.eps = eps;
    rope_inv_freq_table(theta, head_dim, o.r.inv_freq);
    o.launches = (unsigned long long *)ws;
    o.tstats = (unsigned long long *)((char *)ws + OP_HEADER);
    o.tpart = o.tstats + (size_t)n_heads * a.max_blocks * 2;
    o.err = err;
    o.ipk = ipk;
    const int rep = n_heads / n_kv_heads;
    o.cpi = (rep * head_dim + ipk - 1) / ipk;
    const int grid = n_kv_heads * ipk;
    switch (rep) {
    case 1: attn_one_pass_kernel<1><<<grid, OP_THREADS, 0, stream>>>(o); break;
    case 2: attn_one_pass_kernel<2><<<grid, OP_THREADS, 0, stream>>>(o); break;
    case 4: attn_one_pass_kernel<4><<<grid, OP_THREADS, 0, stream>>>(o); break;
    default: attn_one_pass_kernel<8><<<grid, OP_THREADS, 0, stream>>>(o); break;
    }
    return LAUNCH_OK();
}

extern "C" void qk_norm_rope_attention_one_pass(bf16 *out, const bf16 *q, const bf16 *k,
                                                const bf16 *v, const bf16 *q_norm_w,
                                                const bf16 *k_norm_w, bf16 *key_cache,
                                                bf16 *value_cache, void *ws, int *err,
                                                const int *d_pos, int n_heads, int n_kv_heads,
                                                int head_dim, float eps, float theta,
                                                int max_seq, float scale, hipStream_t stream) {
    attention_one_pass_launch(out, q, k, v, q_norm_w, k_norm_w, key_cache, value_cache, ws, err,
                              d_pos, n_heads, n_kv_heads, head_dim, eps, theta, max_seq, scale,
                              stream);
}

// ------------------------------------------------------------------------------------------
// Passes 2 and 3 in one launch (attn_pv_kernel followed by attn_combine_kernel, the same bits),
// for the step's attention. Every item publishes its block partials as tagged 64-bit words
// (float bits << 32 | tag; the tag is the workgroup's launch count + 1, counted in a word of
// its own as in the one-pass kernel), and the items of the T last blocks of each kv head then
// combine: item nb - T + j adds, in block order, the partials of columns [j C, (j + 1) C) of the
// kv head's REP * D (C = REP * D / T), once it has read every block's partial of them with the
// current tag. T is the largest power of two <= min(nb, REP * D / PVC_COLS). One workgroup per
// item of the longest history, so the items of a step are one wave of the grid; only the
// T * n_kv_heads combine items wait, every other item runs to its end, so the waits end. They
// are bounded all the same: a timeout sets *err, and the kernel finishes with what it read.
// ------------------------------------------------------------------------------------------

// fewest columns of a combine item (4B after 8192 positions: 431.2-431.8 tokens/s; 8 columns
// 428.5-428.8, 32 columns 418.5-418.6)
constexpr int PVC_COLS = 16;
constexpr int PVC_STRIDE = 16;      // 8-byte words between two workgroups' launch counters
constexpr int PVC_MAXGRID = 8192;   // items (blocks x kv heads) of the longest history

struct PvCombineArgs {
    AttnArgs a;
    unsigned long long *tpart;     // [n_heads, max_blocks, D] tagged block partials
    unsigned long long *launches;  // per workgroup, PVC_STRIDE words apart: its launches
    int *err;                      // set to 2 when a wait times out
};

template <int D, int REP>
__global__ __launch_bounds__(256) void attn_pv_combine_kernel(PvCombineArgs o) {
    constexpr int COLS = REP * D;
    constexpr int STAGE = 4 * REP * D > 4096 ? 4 * REP * D : 4096;  // floats
    constexpr int CPT = (COLS + 255) / 256;  // columns of a thread when one item combines all
    __shared__ float p_s[REP][ATT_B];
    __shared__ float stage[STAGE];  // the PV quarter sums, then the combine's staged partials
    float(&red)[4][REP][D] = *reinterpret_cast<float(*)[4][REP][D]>(stage);
    const AttnArgs &a = o.a;
    unsigned long long *ctr = o.launches + (size_t)blockIdx.x * PVC_STRIDE;
    const unsigned long long launches = op_ld(ctr);
    const uint32_t tag = (uint32_t)(launches % 0xffffffffull) + 1u;
    const int n = *a.d_pos + 1;
    const int nb = (n + ATT_B - 1) / ATT_B;
    if (n <= 0 || n > a.max_seq) {  // every workgroup reads the same position: all skip
        if (threadIdx.x == 0) {
            __hip_atomic_store(gptr(o.err), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(gptr(ctr), launches + 1, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    if ((int)blockIdx.x < nb * a.n_kv_heads) {  // the grid holds every item: one each
        const int b = blockIdx.x / a.n_kv_heads, g = blockIdx.x - b * a.n_kv_heads;
        pv_item<D, REP>(a, b, g, n, nb, p_s, red,
                        [&](size_t i, float v) { op_st(o.tpart + i, v, tag); });
        int T = 1;
        while (2 * T <= nb && 2 * T * PVC_COLS <= COLS) T *= 2;
        if (b >= nb - T) {
            const int nc = COLS / T, c0 = (b - (nb - T)) * nc;
            const int cb = STAGE / nc;  // blocks per staged chunk
            float acc[CPT];
#pragma unroll
            for (int k = 0; k < CPT; k++) acc[k] = 0.0f;
            for (int b0 = 0; b0 < nb; b0 += cb) {
                const int cnt = min(cb, nb - b0);
                op_poll<256, 16>(
                    cnt * nc, tag, o.err,
                    [&](int idx) {
                        const int bb = idx / nc, c = c0 + idx - bb * nc, q = c / D, d = c - q * D;
                        return o.tpart + ((size_t)(g * REP + q) * a.max_blocks + b0 + bb) * D + d;
                    },
                    [&](int idx, float v) { stage[idx] = v; });
                __syncthreads();
#pragma unroll
                for (int k = 0; k < CPT; k++) {
                    const int c = threadIdx.x + 256 * k;
                    if (c < nc) {
                        int j0 = 0;
                        if (b0 == 0) {
                            acc[k] = stage[c];
                            j0 = 1;
                        }
                        for (; j0 + 16 <= cnt; j0 += 16) {  // 16 LDS reads in flight, then adds
                            float v[16];
#pragma unroll
                            for (int u = 0; u < 16; u++) v[u] = stage[(j0 + u) * nc + c];
#pragma unroll
                            for (int u = 0; u < 16; u++) acc[k] += v[u];
                        }
                        for (; j0 < cnt; j0++) acc[k] += stage[j0 * nc + c];
                    }
                }
                __syncthreads();
            }
#pragma unroll
            for (int k = 0; k < CPT; k++) {
                const int c = c0 + threadIdx.x + 256 * k, q = c / D, d = c - q * D;
                if ((int)threadIdx.x + 256 * k < nc)
                    a.out[(size_t)(g * REP + q) * D + d] = (bf16)f2bf(acc[k]);
            }
        }
    }
    __syncthreads();  // every wave has its tag
    if (threadIdx.x == 0)
        __hip_atomic_store(gptr(ctr), launches + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Bytes of the attn_pv_combine_kernel workspace (the launch counters, then the tagged partials),
// or 0 where that kernel is not used: head_dim other than 128, or more than PVC_MAXGRID items.
size_t attention_pv_combine_bytes(int n_heads, int n_kv_heads, int head_dim, int max_seq) {
    if (head_dim != 128 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0 || max_seq <= 0) return 0;
    const int rep = n_heads / n_kv_heads;
    if (rep != 1 && rep != 2 && rep != 4 && rep != 8) return 0;
    const size_t mb = ceil_div((size_t)max_seq, ATT_B);
    if (mb * n_kv_heads > PVC_MAXGRID) return 0;
    return mb * n_kv_heads * PVC_STRIDE * 8 + (size_t)n_heads * mb * head_dim * 8;
}

// The second and third passes: attn_pv_combine_kernel on the workspace `pvc` where given (grid
// = every item of the longest history, as attention_pv_combine_bytes admits), else the PV and
// combine kernels.
template <int D, int REP>
static void launch_attention_t(const AttnArgs &a, int grid, hipStream_t stream,
                               const AttnRopeArgs *rope = nullptr, void *pvc = nullptr,
                               int *err = nullptr) {
    if (rope && rope->table)
        attn_rope_scores_kernel<D, REP, true><<<grid, 256, 0, stream>>>(*rope);
    else if (rope)
        attn_rope_scores_kernel<D, REP, false><<<grid, 256, 0, stream>>>(*rope);
    else
        attn_scores_kernel<D, REP><<<grid, 256, 0, stream>>>(a);
    if (!LAUNCH_OK()) return;
    if constexpr (D == 128) {
        if (pvc) {
            PvCombineArgs o;
            o.a = a;
            o.launches = (unsigned long long *)pvc;
            o.tpart = o.launches + (size_t)grid * PVC_STRIDE;
            o.err = err;
            attn_pv_combine_kernel<D, REP><<<grid, 256, 0, stream>>>(o);
            LAUNCH_OK();
            return;
        }
    }
    attn_pv_kernel<D, REP><<<grid, 256, 0, stream>>>(a);
    if (!LAUNCH_OK()) return;
    attn_combine_kernel<D><<<a.n_heads * (D / COMBINE_COLS), 256, 0, stream>>>(a);
    LAUNCH_OK();
}

// Block statistics and partial outputs of attention_forward for a caller whose `att` holds only
// the reference's [n_heads, max_seq] scores (src/forward.cu:10-51 sizes it so): a library-owned
// device array of 2^22 floats (16 MiB) per device, as argmax_forward keeps its partials. Every
// value a call reads from it was written earlier in the same call, so nothing is cleared; calls
// on one device that use it must not overlap.
constexpr size_t ATTN_BLOCK_FLOATS = (size_t)1 << 22;
static __device__ __align__(256) float g_attn_blocks[ATTN_BLOCK_FLOATS];

static float *attn_blocks_on_current_device() {
    static std::mutex mu;
    static float *addr[64];
    int dev = 0;
    if (!HIP_OK(hipGetDevice(&dev))) return nullptr;
    if (dev < 0 || dev >= 64) {
        llm_fail("attention: device %d out of range", dev);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        float *p = nullptr;
        if (!HIP_OK(hipGetSymbolAddress((void **)&p, HIP_SYMBOL(g_attn_blocks)))) return nullptr;
        addr[dev] = p;
    }
    return addr[dev];
}

// Where the split softmax keeps its block statistics and partial outputs. An `att` with room for
// attention_workspace_floats() floats holds them after the scores. An `att` sized the
// reference's way, [n_heads, max_seq] floats, holds the scores only, and the rest goes to the
// library's array. A smaller `att` is an error, not an overrun. The room is what the runtime
// knows of the allocation holding `att` (a buffer carved out of a larger allocation counts to
// that allocation's end); where it knows nothing, `att` is taken to hold the whole workspace.
static bool attention_blocks(float *att, int n_heads, int head_dim, int max_seq, float **stats,
                             float **partial) {
    *stats = att + (size_t)n_heads * max_seq;
    *partial = att + attention_partial_offset(n_heads, max_seq);
    hipDeviceptr_t base = nullptr;
    size_t bytes = 0;
    if (hipMemGetAddressRange(&base, &bytes, (hipDeviceptr_t)att) != hipSuccess || !base) {
        (void)hipGetLastError();  // not a runtime allocation: nothing to check against
        return true;
    }
    const size_t avail = bytes - (size_t)((const char *)att - (const char *)base);
    const size_t need = attention_workspace_floats(n_heads, head_dim, max_seq) * sizeof(float);
    if (avail >= need) return true;
    const size_t scores = (size_t)n_heads * max_seq * sizeof(float);
    if (avail < scores)
        return llm_fail("attention: att has room for %zu bytes, fewer than the %zu of its "
                        "[%d, %d] scores", avail, scores, n_heads, max_seq);
    const size_t mb = ceil_div((size_t)max_seq, ATT_B);
    const size_t stat_floats = ceil_div((size_t)n_heads * mb * 2, 4) * 4;
    const size_t block_floats = stat_floats + (size_t)n_heads * mb * head_dim;
    if (block_floats > ATTN_BLOCK_FLOATS)
        return llm_fail("attention: att holds the [%d, %d] scores only, and the %zu floats of "
                        "block statistics and partials exceed the library's %zu (give att "
                        "attention_workspace_floats(%d, %d, %d) floats)",
                        n_heads, max_seq, block_floats, ATTN_BLOCK_FLOATS, n_heads, head_dim,
                        max_seq);
    float *blocks = attn_blocks_on_current_device();
    if (!blocks) return false;
    *stats = blocks;
    *partial = blocks + stat_floats;
    return true;
}

static bool attention_args(AttnArgs &a, int &grid, bf16 *out, const bf16 *q,
                           const bf16 *key_cache, const bf16 *value_cache, float *att,
                           int n_heads, int n_kv_heads, int head_dim, const int *d_pos,
                           int max_seq, float scale) {
    if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return llm_fail("attention: head_dim %d is not 64, 128 or 256", head_dim);
    if (n_kv_heads <= 0 || n_heads % n_kv_heads != 0)
        return llm_fail("attention: n_heads %d is not a multiple of n_kv_heads %d", n_heads,
                        n_kv_heads);
    const int rep = n_heads / n_kv_heads;
    if (rep != 1 && rep != 2 && rep != 4 && rep != 8)
        return llm_fail("attention: n_heads / n_kv_heads = %d is not 1, 2, 4 or 8", rep);
    if (max_seq <= 0) return llm_fail("attention: max_seq %d must be positive", max_seq);
    if (!aligned16(q) || !aligned16(key_cache) || !aligned16(value_cache) || !aligned16(att))
        return llm_fail("attention: q, the caches and att must be 16-byte aligned");
    float *stats = nullptr, *partial = nullptr;
    if (!attention_blocks(att, n_heads, head_dim, max_seq, &stats, &partial)) return false;
    a.out = out;
    a.q = q;
    a.kc = key_cache;
    a.vc = value_cache;
    a.max_blocks = (int)ceil_div((size_t)max_seq, ATT_B);
    a.scores = att;
    a.stats = stats;
    a.partial = partial;
    a.d_pos = d_pos;
    a.n_heads = n_heads;
    a.n_kv_heads = n_kv_heads;
    a.max_seq = max_seq;
    a.scale = scale;
    // one workgroup per (block, kv head) of the longest history, so every item of a step runs in
    // the same wave of workgroups (a fixed cap made the last few items of a long history a second
    // wave that doubled the kernel time); items beyond the current history exit at once
    const long items = (long)a.max_blocks * n_kv_heads;
    grid = (int)(items < 8192 ? items : 8192);
    return true;
}

bool attention_launch(bf16 *out, const bf16 *q, const bf16 *key_cache, const bf16 *value_cache,
                      float *att, int n_heads, int n_kv_heads, int head_dim, const int *d_pos,
                      int max_seq, float scale, hipStream_t stream, void *pvc, int *err) {
    AttnArgs a;
    int grid = 0;
    if (!attention_args(a, grid, out, q, key_cache, value_cache, att, n_heads, n_kv_heads,
                        head_dim, d_pos, max_seq, scale))
        return false;
    if (pvc && (!err || !attention_pv_combine_bytes(n_heads, n_kv_heads, head_dim, max_seq)))
        return llm_fail("attention: no one-launch PV and combine for these shapes");
    const int rep = n_heads / n_kv_heads;
#define ATT(D_, R_)                                                        \
    if (head_dim == D_ && rep == R_) {                                     \
        launch_attention_t<D_, R_>(a, grid, stream, nullptr, pvc, err);    \
        return !llm_has_error();                                           \
    }
    ATT(64, 1) ATT(64, 2) ATT(64, 4) ATT(64, 8) ATT(128, 1) ATT(128, 2) ATT(128, 4) ATT(128, 8)
    ATT(256, 1) ATT(256, 2) ATT(256, 4) ATT(256, 8)
#undef ATT
    return false;
}

extern "C" void attention_forward(bf16 *out, const bf16 *q, const bf16 *key_cache,
                                  const bf16 *value_cache, float *att, int n_heads, int n_kv_heads,
                                  int head_dim, const int *d_pos, int max_seq, float scale,
                                  hipStream_t stream) {
    attention_launch(out, q, key_cache, value_cache, att, n_heads, n_kv_heads, head_dim, d_pos,
                     max_seq, scale, stream, nullptr, nullptr);
}

// Workspace of attention_forward_noalloc: a library-owned device array instead of the caller's
// `att`, for callers that cannot allocate. Each device holds its own copy until the process
// ends; it keeps the last call's scores, statistics and partial outputs (every value a call
// reads was written earlier in the same call, so nothing needs clearing). Calls that overlap on
// one device race on it.
constexpr size_t ATTN_SCRATCH_FLOATS = (size_t)1 << 20;  // 4 MiB
static __device__ __align__(256) float scratch[ATTN_SCRATCH_FLOATS];

// The device address of this device's copy of `scratch`, looked up once per device with that
// device current. In host code the array's name is only a host-side stand-in, never passed to a
// kernel.
static float *scratch_on_current_device() {
    static std::mutex mu;
    static float *addr[64];
    int dev = 0;
    if (!HIP_OK(hipGetDevice(&dev))) return nullptr;
    if (dev < 0 || dev >= 64) {
        llm_fail("attention_forward_noalloc: device %d out of range", dev);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        float *p = nullptr;
        if (!HIP_OK(hipGetSymbolAddress((void **)&p, HIP_SYMBOL(scratch)))) return nullptr;
        addr[dev] = p;
    }
    return addr[dev];
}

bool qk_norm_rope_attention_launch(bf16 *out, const bf16 *q, const bf16 *k, const bf16 *v,
                                   const bf16 *q_norm_w, const bf16 *k_norm_w, bf16 *key_cache,
                                   bf16 *value_cache, float *att, const int *d_pos, int n_heads,
                                   int n_kv_heads, int head_dim, float eps, float theta,
                                   int max_seq, float scale, hipStream_t stream,
                                   const float *rope_table, void *pvc, int *err) {
    AttnRopeArgs r;
    memset(&r, 0, sizeof r);
    int grid = 0;
    if (!attention_args(r.at, grid, out, q, key_cache, value_cache, att, n_heads, n_kv_heads,
                        head_dim, d_pos, max_seq, scale))
        return false;
    if (pvc && (!err || !attention_pv_combine_bytes(n_heads, n_kv_heads, head_dim, max_seq)))
        return llm_fail("qk_norm_rope_attention: no one-launch PV and combine for these shapes");
    const void *ptrs[] = {k, v, q_norm_w, k_norm_w};
    for (const void *p : ptrs)
        if (!p || !aligned16(p))
            return llm_fail("qk_norm_rope_attention: k, v and the norm weights must be non-null "
                            "and 16-byte aligned");
    r.k = k;
    r.v = v;
    r.qn = q_norm_w;
    r.kn = k_norm_w;
    r.kc_w = key_cache;
    r.vc_w = value_cache;
    r.table = rope_table;
    r.eps = eps;
    rope_inv_freq_table(theta, head_dim, r.inv_freq);
    const int rep = n_heads / n_kv_heads;
#define ATT(D_, R_)                                        \
    if (head_dim == D_ && rep == R_) {                     \
        launch_attention_t<D_, R_>(r.at, grid, stream, &r, pvc, err);\
        return !llm_has_error();                                     \
    }
    ATT(64, 1) ATT(64, 2) ATT(64, 4) ATT(64, 8) ATT(128, 1) ATT(128, 2) ATT(128, 4) ATT(128, 8)
    ATT(256, 1) ATT(256, 2) ATT(256, 4) ATT(256, 8)
#undef ATT
    return false;
}

extern "C" void qk_norm_rope_attention_forward(bf16 *out, const bf16 *q, const bf16 *k,
                                               const bf16 *v, const bf16 *q_norm_w,
                                               const bf16 *k_norm_w, bf16 *key_cache,
                                               bf16 *value_cache, float *att, const int *d_pos,
                                               int n_heads, int n_kv_heads, int head_dim,
                                               float eps, float theta, int max_seq, float scale,
                                               hipStream_t stream) {
    qk_norm_rope_attention_launch(out, q, k, v, q_norm_w, k_norm_w, key_cache, value_cache, att,
                                  d_pos, n_heads, n_kv_heads, head_dim, eps, theta, max_seq,
                                  scale, stream);
}

extern "C" void attention_forward_noalloc(bf16 *out, const bf16 *q, const bf16 *key_cache,
                                          const bf16 *value_cache, int n_heads, int n_kv_heads,
                                          int head_dim, const int *d_pos, int max_seq,
                                          float scale, hipStream_t stream) {
    if (n_heads <= 0 || head_dim <= 0 || max_seq <= 0) {
        llm_fail("attention_forward_noalloc: n_heads %d, head_dim %d and max_seq %d must be "
                 "positive", n_heads, head_dim, max_seq);
        return;
    }
    const size_t need = attention_workspace_floats(n_heads, head_dim, max_seq);
    if (need > ATTN_SCRATCH_FLOATS) {
        llm_fail("attention_forward_noalloc: %zu floats of workspace for %d heads of %d over %d "
                 "positions; the library's scratch holds %zu",
                 need, n_heads, head_dim, max_seq, ATTN_SCRATCH_FLOATS);
        return;
    }
    float *ws = scratch_on_current_device();
    if (!ws) return;
    attention_forward(out, q, key_cache, value_cache, ws, n_heads, n_kv_heads, head_dim, d_pos,
                      max_seq, scale, stream);
}

// ------------------------------------------------------------------------------------------
// temperature sampling (src/kernels.cu:546-597)
// ------------------------------------------------------------------------------------------

// Inverse-CDF sampling from softmax(x * inv_temp), one workgroup of SAMPLE_T threads. The
// additions keep the reference's order, so the chosen index follows from the weights alone: the
// row's max; thread t adds the weights exp((x - max) * inv_temp) of the contiguous chunk
// [t c, t c + c) in order (c = ceil(n / SAMPLE_T)); thread 0 adds the chunk sums in order for the
// total, walks them to the chunk holding u * total (never past the last) and then that chunk's
// elements to the first whose running sum passes it (-1 if none does). Not on the decode path.
constexpr int SAMPLE_T = 1024;

__global__ __launch_bounds__(SAMPLE_T) void sample_kernel(int *out, const bf16 *x, int n,
                                                          float inv_temp, float u) {
    __shared__ float sums[SAMPLE_T];
    __shared__ float wmax[SAMPLE_T / 64];
    const int t = threadIdx.x;
    float m = -__builtin_huge_valf();
    for (int i = t; i < n; i += SAMPLE_T) m = fmaxf(m, bf2f(x[i]));
    m = wave_max(m);
    if ((t & 63) == 0) wmax[t >> 6] = m;
    __syncthreads();
    float mx = wmax[0];
    for (int w = 1; w < SAMPLE_T / 64; w++) mx = fmaxf(mx, wmax[w]);  // max: any order
    const int chunk = (n + SAMPLE_T - 1) / SAMPLE_T;
    const int start = t * chunk, end = min(start + chunk, n);
    float acc = 0.0f;
    for (int i = start; i < end; i++) acc += exp_f32((bf2f(x[i]) - mx) * inv_temp);
    sums[t] = acc;
    __syncthreads();
    if (t != 0) return;
    float total = 0.0f;
    for (int k = 0; k < SAMPLE_T; k++) total += sums[k];
    const float target = u * total;
    float cdf = 0.0f;
    int k = 0;
    while (k < SAMPLE_T - 1 && cdf + sums[k] <= target) cdf += sums[k++];
    int chosen = -1;
    float run = 0.0f;
    for (int i = k * chunk; i < min(k * chunk + chunk, n); i++) {
        run += exp_f32((bf2f(x[i]) - mx) * inv_temp);
        if (cdf + run > target) {
            chosen = i;
            break;
        }
    }
    *out = chosen;
}

extern "C" void sample_forward(int *out, const bf16 *x, int n, float inv_temp, float u,
                               hipStream_t stream) {
    if (n <= 0) {
        llm_fail("sample: n %d must be positive", n);
        return;
    }
    sample_kernel<<<1, SAMPLE_T, 0, stream>>>(out, x, n, inv_temp, u);
    LAUNCH_OK();
}

// ------------------------------------------------------------------------------------------
// streaming ceiling probe (measurement helper)
// ------------------------------------------------------------------------------------------

// MODE 0: read n16 chunks of a (grid-stride, four 16-byte loads in flight per thread), each
// thread's xor of its chunks to dst (one word per thread); MODE 1: dst = a; MODE 2: dst = a ^ b
// (one chunk per thread). The shapes that measured fastest for plain reads and copies on MI355X.
template <int MODE>
__global__ __launch_bounds__(256) void stream_probe_kernel(u32x4 *dst, const u32x4 *a,
                                                           const u32x4 *b, size_t n16) {
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    if constexpr (MODE == 0) {
        // thread (block b, lane-in-block i) reads chunks b * 1024 + i + 256 u + stride j
        const size_t stride = (size_t)gridDim.x * 256 * 4;
        uint32_t acc = 0;
        for (size_t base = (size_t)blockIdx.x * 1024 + threadIdx.x; base < n16; base += stride) {
            u32x4 v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const size_t i = base + 256 * u;
                v[u] = i < n16 ? __builtin_nontemporal_load(a + i) : u32x4{0, 0, 0, 0};
            }
#pragma unroll
            for (int u = 0; u < 4; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
        }
        ((uint32_t *)dst)[t] = acc;
    } else {
        for (size_t i = t; i < n16; i += (size_t)gridDim.x * 256) {
            u32x4 v = __builtin_nontemporal_load(a + i);
            if constexpr (MODE == 2) v ^= __builtin_nontemporal_load(b + i);
            __builtin_nontemporal_store(v, dst + i);
        }
    }
}

extern "C" void hbm_stream_probe(void *dst, const void *a, const void *b, size_t n_bytes, int mode,
                                 hipStream_t stream) {
    if (mode < 0 || mode > 2 || n_bytes % 16 != 0 || !aligned16(dst) || !aligned16(a) ||
        (mode == 2 && !aligned16(b))) {
        llm_fail("hbm_stream_probe: mode %d, %zu bytes (a multiple of 16, 16-byte aligned)", mode,
                 n_bytes);
        return;
    }
    const size_t n16 = n_bytes / 16;
    if (n16 == 0) return;
    if (mode == 0) {
        stream_probe_kernel<0><<<1024, 256, 0, stream>>>((u32x4 *)dst, (const u32x4 *)a, nullptr, n16);
    } else {
        size_t blocks = (n16 + 255) / 256;
        const size_t cap = (size_t)device_cus() * 80;
        if (blocks > cap) blocks = cap;
        if (mode == 1)
            stream_probe_kernel<1><<<(unsigned)blocks, 256, 0, stream>>>((u32x4 *)dst,
                                                                        (const u32x4 *)a, nullptr, n16);
        else
            stream_probe_kernel<2><<<(unsigned)blocks, 256, 0, stream>>>(
                (u32x4 *)dst, (const u32x4 *)a, (const u32x4 *)b, n16);
    }
    LAUNCH_OK();
}

// The device read peak (bench/bandwidth.cu:25-116 read_kernel): 16-byte chunks, U non-temporal
// loads in flight per thread per round, either grid-stride over the whole buffer (CONTIG false,
// the reference's pattern) or over one contiguous range per workgroup (CONTIG true, as a GEMV's
// workgroups read their rows). The xor of the data is stored only in the unlikely case it equals
// a constant, so the loads are not removed.
template <int U, bool CONTIG>
__global__ __launch_bounds__(1024) void read_peak_kernel(const u32x4 *a, size_t n16,
                                                         uint32_t *out) {
    size_t first = 0, end = n16, stride = (size_t)gridDim.x * blockDim.x;
    size_t t0 = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if constexpr (CONTIG) {
        const size_t span = (n16 + gridDim.x - 1) / gridDim.x;
        first = min(n16, (size_t)blockIdx.x * span);
        end = min(n16, first + span);
        stride = blockDim.x;
        t0 = first + threadIdx.x;
    }
    uint32_t acc = 0;
    for (size_t base = t0; base < end; base += U * stride) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const size_t i = base + u * stride;
            v[u] = i < end ? __builtin_nontemporal_load(a + i) : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9e3779b9u) *out = acc;
}

extern "C" void hbm_read_peak_probe(unsigned *out, const void *a, size_t n_bytes, int blocks,
                                    int threads, int loads_in_flight, int contiguous,
                                    hipStream_t stream) {
    if (n_bytes % 16 != 0 || !aligned16(a) || out == nullptr || blocks < 1 ||
        blocks > (1 << 20) || (threads != 64 && threads != 128 && threads != 256 &&
                               threads != 512 && threads != 1024) ||
        (loads_in_flight != 4 && loads_in_flight != 8 && loads_in_flight != 16) ||
        (contiguous != 0 && contiguous != 1)) {
        llm_fail("hbm_read_peak_probe: %zu bytes (a multiple of 16, 16-byte aligned), %d blocks "
                 "of %d threads (64..1024, a power of two), %d loads in flight (4, 8 or 16), "
                 "layout %d (0 grid-stride, 1 a range per workgroup)",
                 n_bytes, blocks, threads, loads_in_flight, contiguous);
        return;
    }
    if (n_bytes == 0) return;
    const u32x4 *p = (const u32x4 *)a;
    const size_t n16 = n_bytes / 16;
#define PEAK(U, C) read_peak_kernel<U, C><<<blocks, threads, 0, stream>>>(p, n16, out)
    if (contiguous) {
        if (loads_in_flight == 4) PEAK(4, true);
        else if (loads_in_flight == 8) PEAK(8, true);
        else PEAK(16, true);
    } else {
        if (loads_in_flight == 4) PEAK(4, false);
        else if (loads_in_flight == 8) PEAK(8, false);
        else PEAK(16, false);
    }
#undef PEAK
    LAUNCH_OK();
}

// The device copy peak: a grid-stride copy, each thread requesting U non-temporal 16-byte loads
// (chunks blockDim apart) before it stores them. Every chunk index is checked against n16.
template <int U>
__global__ __launch_bounds__(1024) void copy_peak_kernel(u32x4 *__restrict__ d,
                                                         const u32x4 *__restrict__ a, size_t n16) {
    const size_t tile = (size_t)blockDim.x * U, stride = (size_t)gridDim.x * tile;
    for (size_t base = (size_t)blockIdx.x * tile + threadIdx.x; base < n16; base += stride) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const size_t i = base + (size_t)u * blockDim.x;
            v[u] = i < n16 ? __builtin_nontemporal_load(a + i) : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const size_t i = base + (size_t)u * blockDim.x;
            if (i < n16) __builtin_nontemporal_store(v[u], d + i);
        }
    }
}

extern "C" void hbm_copy_peak_probe(void *dst, const void *a, size_t n_bytes, int blocks,
                                    int threads, int chunks_in_flight, hipStream_t stream) {
    if (n_bytes % 16 != 0 || !aligned16(a) || !aligned16(dst) || blocks < 1 ||
        blocks > (1 << 20) || (threads != 64 && threads != 128 && threads != 256 &&
                               threads != 512 && threads != 1024) ||
        (chunks_in_flight != 1 && chunks_in_flight != 2 && chunks_in_flight != 4 &&
         chunks_in_flight != 8)) {
        llm_fail("hbm_copy_peak_probe: %zu bytes (a multiple of 16, 16-byte aligned), %d blocks "
                 "of %d threads (64..1024, a power of two), %d chunks in flight (1, 2, 4 or 8)",
                 n_bytes, blocks, threads, chunks_in_flight);
        return;
    }
    if (n_bytes == 0) return;
    u32x4 *d = (u32x4 *)dst;
    const u32x4 *p = (const u32x4 *)a;
    const size_t n16 = n_bytes / 16;
    if (chunks_in_flight == 1) copy_peak_kernel<1><<<blocks, threads, 0, stream>>>(d, p, n16);
    else if (chunks_in_flight == 2) copy_peak_kernel<2><<<blocks, threads, 0, stream>>>(d, p, n16);
    else if (chunks_in_flight == 4) copy_peak_kernel<4><<<blocks, threads, 0, stream>>>(d, p, n16);
    else copy_peak_kernel<8><<<blocks, threads, 0, stream>>>(d, p, n16);
    LAUNCH_OK();
}

// ------------------------------------------------------------------------------------------
// argmax (src/kernels.cu:499-544), two stages
// ------------------------------------------------------------------------------------------

constexpr int AMAX_GROUPS = 256;
// Library-owned partial results of argmax_forward (calls on one device must not overlap).
__device__ float g_amax_val[AMAX_GROUPS];
__device__ int g_amax_idx[AMAX_GROUPS];

__device__ __forceinline__ void block_amax(float &v, int &i, float *lv, int *li) {
    wave_amax(v, i);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        lv[w] = v;
        li[w] = i;
    }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int k = 1; k < (int)(blockDim.x >> 6); k++) amax_pair(v, i, lv[k], li[k]);
}

__global__ __launch_bounds__(256) void argmax_stage1_kernel(const bf16 *x, int n, int vec,
                                                            float *pv, int *pi) {
    __shared__ float lv[4];
    __shared__ int li[4];
    float v = -__builtin_huge_valf();
    int idx = INT_MAX;
    const int stride = gridDim.x * blockDim.x;
    const int t0 = blockIdx.x * blockDim.x + threadIdx.x;
    int done = 0;
    if (vec) {
        const int n_chunks = n / 8;
        for (int c = t0; c < n_chunks; c += stride) {
            const u32x4 ch = ld16(x + 8 * (size_t)c);
#pragma unroll
            for (int e = 0; e < 8; e++) amax_pair(v, idx, elem(ch, e), 8 * c + e);
        }
        done = n_chunks * 8;
    }
    for (int i = done + t0; i < n; i += stride) amax_pair(v, idx, bf2f(x[i]), i);
    block_amax(v, idx, lv, li);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = v;
        pi[blockIdx.x] = idx;
    }
}

__global__ __launch_bounds__(256) void argmax_stage2_kernel(const float *pv, const int *pi,
                                                            int groups, int *out) {
    __shared__ float lv[4];
    __shared__ int li[4];
    float v = -__builtin_huge_valf();
    int idx = INT_MAX;
    for (int k = threadIdx.x; k < groups; k += blockDim.x) amax_pair(v, idx, pv[k], pi[k]);
    block_amax(v, idx, lv, li);
    if (threadIdx.x == 0) *out = idx;
}

int argmax_partial_count() { return AMAX_GROUPS; }

static int argmax_groups(int n) {
    const int g = (n + 256 * 8 - 1) / (256 * 8);
    return g < 1 ? 1 : (g > AMAX_GROUPS ? AMAX_GROUPS : g);
}

// Shared by argmax_forward (library buffer) and the step (its own buffer).
void argmax_launch(int *out, const bf16 *x, int n, float *pv, int *pi, hipStream_t stream) {
    const int groups = argmax_groups(n);
    argmax_stage1_kernel<<<groups, 256, 0, stream>>>(x, n, aligned16(x) ? 1 : 0, pv, pi);
    if (!LAUNCH_OK()) return;
    argmax_stage2_kernel<<<1, 256, 0, stream>>>(pv, pi, groups, out);
    LAUNCH_OK();
}

extern "C" void argmax_forward(int *out, const bf16 *x, int n, hipStream_t stream) {
    if (n <= 0) {
        llm_fail("argmax: n %d must be positive", n);
        return;
    }
    // Each device holds its own copy of the partials; look their addresses up once per device.
    static std::mutex mu;
    static float *pv_dev[64];
    static int *pi_dev[64];
    int dev = 0;
    if (!HIP_OK(hipGetDevice(&dev))) return;
    if (dev < 0 || dev >= 64) {
        llm_fail("argmax: device %d out of range", dev);
        return;
    }
    float *pv;
    int *pi;
    {
        std::lock_guard<std::mutex> lock(mu);
        if (!pv_dev[dev]) {
            if (!HIP_OK(hipGetSymbolAddress((void **)&pv_dev[dev], HIP_SYMBOL(g_amax_val))) ||
                !HIP_OK(hipGetSymbolAddress((void **)&pi_dev[dev], HIP_SYMBOL(g_amax_idx)))) {
                pv_dev[dev] = nullptr;
                return;
            }
        }
        pv = pv_dev[dev];
        pi = pi_dev[dev];
    }
    argmax_launch(out, x, n, pv, pi, stream);
}
