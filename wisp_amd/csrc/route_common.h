/*
 * route_common.h — router dot products and the wave-level top-k selection
 * shared by the routing kernels and the fused decode prep (internal).
 *
 * Selection rule (csrc/core/wisp_engine.c:803-815, csrc/cuda/router.cu:
 * 118-130): k passes of "largest untaken score wins, ties to the lowest
 * index". Softmax and sigmoid are strictly increasing, so the selection
 * runs on the logit itself (plus bias where it enters before the
 * activation).
 */
#pragma once

#include "hip_common.h"

#define ROUTE_MAX_TOPK 64
#define ROUTE_MAX_EXPERTS 1024
#define ROUTE_TOK_PER_WG 4

template <typename XT>
__device__ __forceinline__ float xval(const XT* x, size_t i);
template <> __device__ __forceinline__ float xval<float>(const float* x, size_t i) { return x[i]; }
template <> __device__ __forceinline__ float xval<uint16_t>(const uint16_t* x, size_t i) {
    return half_bits_to_float(x[i]);
}

/* Eight consecutive activations starting at p (16-byte aligned) as fp32. */
__device__ __forceinline__ void load_x8(const uint16_t* p, float (&o)[8]) {
    const h8 v = *(const h8*)p;
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = (float)v[i];
}
__device__ __forceinline__ void load_x8(const float* p, float (&o)[8]) {
    const f4 a = *(const f4*)p, b = *(const f4*)(p + 4);
#pragma unroll
    for (int i = 0; i < 4; i++) { o[i] = a[i]; o[4 + i] = b[i]; }
}

/* acc[t] = sum_c row[c] * x[t * hidden + c] for t < nt (<= 4), reduced over
 * the wave: every lane returns the full sums. fp16 row, fp32 x (given as
 * fp16 or fp32), fp32 accumulate. Needs hidden % 8 == 0, row and x 16-byte
 * aligned; x is normally an LDS copy. A lane issues all its row loads of a
 * pass (up to ROUTE_UNROLL x 16 B) before it uses any of them. */
#define ROUTE_UNROLL 16
template <typename XT>
__device__ __forceinline__ void router_row_dot(const uint16_t* __restrict__ row,
                                               const XT* x, int nt, int hidden,
                                               int lane, float (&acc)[ROUTE_TOK_PER_WG]) {
#pragma unroll
    for (int t = 0; t < ROUTE_TOK_PER_WG; t++) acc[t] = 0.0f;
    const int n8 = hidden / 8;
    for (int base = 0; base < n8; base += ROUTE_UNROLL * WAVE) {
        u4 w[ROUTE_UNROLL];
#pragma unroll
        for (int i = 0; i < ROUTE_UNROLL; i++) {
            const int c8 = base + i * WAVE + lane;
            w[i] = c8 < n8 ? ((const u4*)row)[c8] : (u4){0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < ROUTE_UNROLL; i++) {
            const int c8 = base + i * WAVE + lane;
            if (c8 < n8) {
                const h8 wh = __builtin_bit_cast(h8, w[i]);
#pragma unroll
                for (int t = 0; t < ROUTE_TOK_PER_WG; t++) {
                    if (t < nt) {
                        float xv[8];
                        load_x8(x + (size_t)t * hidden + (size_t)c8 * 8, xv);
#pragma unroll
                        for (int e = 0; e < 8; e++) acc[t] = __builtin_fmaf((float)wh[e], xv[e], acc[t]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < ROUTE_TOK_PER_WG; t++) acc[t] = wave_sum(acc[t]);
}

/* Single-pass split of router_row_dot for hidden <= ROUTE_UNROLL * 512:
 * router_row_load issues a lane's row loads, router_row_fma consumes them
 * (x from LDS) and reduces over the wave. */
__device__ __forceinline__ void router_row_load(const uint16_t* __restrict__ row, int hidden,
                                                int lane, u4 (&w)[ROUTE_UNROLL]) {
    const int n8 = hidden / 8;
#pragma unroll
    for (int i = 0; i < ROUTE_UNROLL; i++) {
        const int c8 = i * WAVE + lane;
        w[i] = c8 < n8 ? ((const u4*)row)[c8] : (u4){0u, 0u, 0u, 0u};
    }
}

/* Lane 0 writes out[t * out_stride] = add + the dot of the loaded row with
 * token t's x row (x in LDS), for t < nt. Tokens are a runtime loop to keep
 * the code small. */
template <typename XT>
__device__ __forceinline__ void router_row_fma(const u4 (&w)[ROUTE_UNROLL], const XT* x, int nt,
                                               int hidden, int lane, float* out, int out_stride,
                                               float add) {
    const int n8 = hidden / 8;
#pragma unroll 1
    for (int t = 0; t < nt; t++) {
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < ROUTE_UNROLL; i++) {
            const int c8 = i * WAVE + lane;
            if (c8 < n8) {
                const h8 wh = __builtin_bit_cast(h8, w[i]);
                float xv[8];
                load_x8(x + (size_t)t * hidden + (size_t)c8 * 8, xv);
#pragma unroll
                for (int e = 0; e < 8; e++) a = __builtin_fmaf((float)wh[e], xv[e], a);
            }
        }
        a = wave_sum(a);
        if (lane == 0) out[(size_t)t * out_stride] = a + add;
    }
}

/* Copies nt rows of x [nt][hidden] (16-byte aligned, hidden % 8 == 0) to
 * LDS with 16-byte accesses, in the caller's type. */
template <typename XT>
__device__ __forceinline__ void stage_rows(XT* dst, const XT* __restrict__ src, int nt, int hidden) {
    constexpr int PER16 = 16 / sizeof(XT);
    const int n = nt * hidden / PER16;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ((u4*)dst)[i] = ((const u4*)src)[i];
}

/* a beats b: larger key, or equal key and lower index. NaN never wins. */
__device__ __forceinline__ bool route_beats(float av, int ai, float bv, int bi) {
    return av > bv || (av == bv && ai >= 0 && (bi < 0 || ai < bi));
}

/* One wave, one token. lg: the token's raw logits [n_experts] (global or
 * LDS; for SOFTMAX they already include the bias). s_key / s_sc: LDS
 * scratch of n_experts floats each; s_sc may alias lg (entry e is only
 * ever touched by lane e % 64). Writes the post-activation scores to
 * scores_out, and idx/w [top_k] (written by lane 0). For SIGMOID the bias
 * (if any) is added to the score for selection only; weights are the
 * selected unbiased scores renormalised to sum 1. Loops are runtime loops:
 * this runs once per token and its code size is what costs time. */
__device__ __noinline__ void topk_lds(const float* lg, const uint16_t* __restrict__ bias,
                                      float* s_key, float* s_sc, float* scores_out,
                                      int n_experts, int top_k, int kind, int* out_idx,
                                      float* out_w, int lane) {
    const bool sig = kind == WISP_ROUTER_SIGMOID;
    float mx = -INFINITY;
    for (int e = lane; e < n_experts; e += WAVE) {
        const float l = lg[e];
        float k = l;
        if (sig && bias) k = 1.0f / (1.0f + __expf(-l)) + half_bits_to_float(bias[e]);
        s_key[e] = k;
        s_sc[e] = l;
        mx = fmaxf(mx, l);
    }
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, WAVE));
    float denom = 0.0f;
    for (int e = lane; e < n_experts; e += WAVE) {
        const float l = s_sc[e];
        const float v = sig ? 1.0f / (1.0f + __expf(-l)) : __expf(l - mx);
        s_sc[e] = v;
        denom += v;
    }
    denom = wave_sum(denom);
    const float inv = 1.0f / (denom > 0.0f ? denom : 1.0f);
    for (int e = lane; e < n_experts; e += WAVE) {
        float v = s_sc[e];
        if (!sig) v *= inv;
        s_sc[e] = v;
        scores_out[e] = v;
    }
    float wsum = 0.0f;
    for (int k = 0; k < top_k; k++) {
        float bv = -INFINITY, bs = 0.0f;
        int bi = -1;
        for (int e = lane; e < n_experts; e += WAVE) {
            const float kv = s_key[e];
            if (route_beats(kv, e, bv, bi)) { bv = kv; bi = e; bs = s_sc[e]; }
        }
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off, WAVE);
            const int oi = __shfl_xor(bi, off, WAVE);
            const float os = __shfl_xor(bs, off, WAVE);
            if (route_beats(ov, oi, bv, bi)) { bv = ov; bi = oi; bs = os; }
        }
        if (bi >= 0 && (bi % WAVE) == lane) s_key[bi] = NAN;   /* taken: never wins again */
        if (lane == 0) {
            out_idx[k] = bi;
            const float w = bi >= 0 ? bs : 0.0f;
            out_w[k] = w;
            wsum += w;
        }
    }
    if (lane == 0 && wsum > 0.0f) {
        for (int k = 0; k < top_k; k++) out_w[k] /= wsum;
    }
}
