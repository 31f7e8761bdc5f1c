/*
 * route_common.h — router dot products and the workgroup top-k selection
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

/* Selection key of expert e as one unsigned 64-bit number: the high word
 * maps the float key to an unsigned integer of the same order (-0 as +0,
 * NaN to 0 below every number), the low word is ~e, so "a beats b"
 * (larger key, or equal key and lower index) is a single compare
 * composite(a) > composite(b). */
__device__ __forceinline__ uint64_t route_composite(float key, int e) {
    uint32_t u = __float_as_uint(key == 0.0f ? 0.0f : key);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    if (key != key) u = 0u;
    return ((uint64_t)u << 32) | (uint32_t)~(uint32_t)e;
}

typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint64_t readlane64(uint64_t v, int lane) {
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, lane);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
    return ((uint64_t)hi << 32) | lo;
}

/* One wave, n_experts <= 64, one token: the selection topk_block makes,
 * with the same arithmetic in the same order (so the same bits), but
 * every reduction in registers: no LDS and no barrier. lg: the token's raw
 * logits (LDS or global). Writes scores_out[e]; lane q < top_k returns the
 * q-th selection in sel_e (-1 past the candidates) and its renormalised
 * weight in sel_w. */
__device__ __forceinline__ void topk_wave_small(const float* lg, const uint16_t* __restrict__ bias,
                                                float* scores_out, int n_experts, int top_k,
                                                int kind, int& sel_e, float& sel_w) {
    const bool sig = kind == WISP_ROUTER_SIGMOID;
    const int lane = threadIdx.x & 63;
    const bool act = lane < n_experts;
    const float l = act ? lg[lane] : -INFINITY;
    float key = l;
    if (act && sig && bias) key = 1.0f / (1.0f + __expf(-l)) + half_bits_to_float(bias[lane]);
    const uint64_t ce = act ? route_composite(key, lane) : 0ull;
    float mx = l;
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, WAVE));
    const float v = act ? (sig ? 1.0f / (1.0f + __expf(-l)) : __expf(l - mx)) : 0.0f;
    const float denom = wave_sum(v);
    const float inv = 1.0f / (denom > 0.0f ? denom : 1.0f);
    const float score = sig ? v : v * inv;
    if (act) scores_out[lane] = score;
    int rank = 0;
    for (int j = 0; j < n_experts; j++) rank += readlane64(ce, j) > ce;
    const bool picked = act && (ce >> 32) != 0 && rank < top_k;
    /* lane q takes the expert of rank q */
    sel_e = -1;
    sel_w = 0.0f;
    for (int q = 0; q < top_k; q++) {
        const uint64_t m = __ballot(picked && rank == q);
        if (m) {
            const int src = __builtin_ctzll(m);
            const float sv = __shfl(score, src, WAVE);
            if (lane == q) {
                sel_e = src;
                sel_w = sv;
            }
        }
    }
    float wsum = 0.0f;
    for (int q = 0; q < top_k; q++) wsum += __shfl(sel_w, q, WAVE);
    if (wsum > 0.0f) sel_w /= wsum;
}

/* All threads of the workgroup, one token. lg: the token's raw logits
 * [n_experts] (LDS or global; for SOFTMAX they already include the bias).
 * s_ck: LDS scratch of n_experts uint64, 16-byte aligned; s_sc: LDS
 * scratch of n_experts floats (it may alias lg when lg is in LDS: every
 * entry is read by its own thread before it is written); s_red: LDS
 * scratch of 32 floats. Writes the post-activation scores to scores_out
 * and the selection to out_idx/out_w [top_k] (LDS or global). For SIGMOID
 * the bias (if any) is added to the score for selection only; weights are
 * the selected unbiased scores renormalised to sum 1.
 *
 * Selection by rank, not by k passes of an argmax: expert e's rank is the
 * number of experts whose composite key exceeds its own; ranks below top_k
 * are the selection in order, which is what k passes of "largest untaken,
 * ties to the lowest index" produce. Each expert is ranked by two half
 * waves (lanes l and l+32), each counting half the keys with branch-free
 * 64-bit compares on 16-byte broadcast LDS reads, then summed with one
 * cross-half shuffle. NaN keys are never selected; with fewer than top_k
 * candidates the rest are -1 with weight 0. */
__device__ __forceinline__ void topk_block(const float* lg, const uint16_t* __restrict__ bias,
                                           uint64_t* s_ck, float* s_sc, float* s_red,
                                           float* scores_out, int n_experts, int top_k,
                                           int kind, int* out_idx, float* out_w) {
    const bool sig = kind == WISP_ROUTER_SIGMOID;
    const int tid = threadIdx.x, nt = blockDim.x, lane = tid & 63, wv = tid >> 6;
    const int nw = (nt + 63) >> 6;
    float mx = -INFINITY;
    for (int e = tid; e < n_experts; e += nt) {
        const float l = lg[e];
        float k = l;
        if (sig && bias) k = 1.0f / (1.0f + __expf(-l)) + half_bits_to_float(bias[e]);
        s_ck[e] = route_composite(k, e);
        s_sc[e] = l;
        mx = fmaxf(mx, l);
    }
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, WAVE));
    if (lane == 0) s_red[wv] = mx;
    for (int q = tid; q < top_k; q += nt) {
        out_idx[q] = -1;
        out_w[q] = 0.0f;
    }
    __syncthreads();
    mx = s_red[0];
    for (int q = 1; q < nw; q++) mx = fmaxf(mx, s_red[q]);
    float denom = 0.0f;
    for (int e = tid; e < n_experts; e += nt) {
        const float l = s_sc[e];
        const float v = sig ? 1.0f / (1.0f + __expf(-l)) : __expf(l - mx);
        s_sc[e] = v;
        denom += v;
    }
    denom = wave_sum(denom);
    __syncthreads();   /* every thread has read s_red for the max */
    if (lane == 0) s_red[wv] = denom;
    __syncthreads();
    denom = 0.0f;
    for (int q = 0; q < nw; q++) denom += s_red[q];
    const float inv = 1.0f / (denom > 0.0f ? denom : 1.0f);
    for (int e = tid; e < n_experts; e += nt) {
        float v = s_sc[e];
        if (!sig) v *= inv;
        s_sc[e] = v;
        scores_out[e] = v;
    }
    /* ranks: half h of the wave counts key pairs [lo, hi) of its expert */
    const int n_pairs = n_experts >> 1;
    const int half_pairs = (n_pairs + 1) >> 1;
    const int h = lane >> 5;
    const int lo = h * half_pairs, hi = min(n_pairs, lo + half_pairs);
    const u64x2* ck2 = (const u64x2*)s_ck;
    for (int base = wv * 32; base < n_experts; base += nw * 32) {
        const int e = base + (lane & 31);
        const uint64_t ce = e < n_experts ? s_ck[e] : ~0ull;
        int rank = 0;
#pragma unroll 8
        for (int q = lo; q < hi; q++) {
            const u64x2 v = ck2[q];
            rank += (v.x > ce) + (v.y > ce);
        }
        if (h == 1 && (n_experts & 1)) rank += s_ck[n_experts - 1] > ce;
        rank += __shfl_xor(rank, 32, WAVE);
        if (h == 0 && e < n_experts && (ce >> 32) != 0 && rank < top_k) out_idx[rank] = e;
    }
    __syncthreads();   /* selection and final scores visible */
    if (wv == 0) {
        /* lane q gathers the q-th weight; the sum runs in rank order */
        float v = 0.0f;
        if (lane < top_k) {
            const int e = out_idx[lane];
            v = e >= 0 ? s_sc[e] : 0.0f;
        }
        float wsum = 0.0f;
        for (int q = 0; q < top_k; q++)
            wsum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), q));
        if (lane < top_k) out_w[lane] = wsum > 0.0f ? v / wsum : v;
    }
    __syncthreads();
}
