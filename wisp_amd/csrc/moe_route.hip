/*
 * moe_route.hip — device-side routing for the MoE expert path (gfx950):
 * router GEMV, top-k selection, the expert-offset builder, token
 * gather and the deterministic weighted combine.
 *
 * Selection rule (csrc/core/wisp_engine.c:803-815, csrc/cuda/router.cu:
 * 118-130): k passes of "largest untaken score wins, ties to the lowest
 * index". Softmax and sigmoid are strictly increasing, so the kernels
 * select on the logit itself (plus bias where it enters before the
 * activation); this is the reference's order without the ties that fp32
 * rounding of the probabilities can create.
 */
#include <mutex>

#include "route_common.h"

/* ======================================================================= */
/* router logits: one wave per expert row, up to 4 tokens per pass           */
/* ======================================================================= */

/* logits[t, e] = sum_c W[e, c] x[t, c] (+ bias[e] when add_bias). The
 * workgroup's token rows are staged in LDS first (dynamic LDS of
 * ROUTE_TOK_PER_WG * hidden * sizeof(XT) bytes); W rows need 16-byte
 * alignment, which the launchers check. */
template <typename XT>
__global__ __launch_bounds__(256) void router_logits_kernel(const uint16_t* __restrict__ W,
                                                            const uint16_t* __restrict__ bias,
                                                            const XT* __restrict__ x,
                                                            float* __restrict__ logits,
                                                            int n_tokens, int hidden,
                                                            int n_experts, int add_bias) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_raw[];
    XT* xs = (XT*)lds_raw;
    const int t0 = blockIdx.y * ROUTE_TOK_PER_WG;
    const int nt = min(ROUTE_TOK_PER_WG, n_tokens - t0);
    const int lane = threadIdx.x & 63;
    if (hidden <= ROUTE_UNROLL * WAVE * 8 && gridDim.x * 4 >= n_experts) {
        /* one row per wave: its loads go out before the token rows are
         * staged, so the kernel costs one memory round trip */
        const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
        u4 wrow[ROUTE_UNROLL];
        if (e < n_experts) router_row_load(W + (size_t)e * hidden, hidden, lane, wrow);
        stage_rows<XT>(xs, x + (size_t)t0 * hidden, nt, hidden);
        __syncthreads();
        if (e < n_experts) {
            const float b = (add_bias && bias) ? half_bits_to_float(bias[e]) : 0.0f;
            router_row_fma<XT>(wrow, xs, nt, hidden, lane, logits + (size_t)t0 * n_experts + e,
                               n_experts, b);
        }
        return;
    }
    stage_rows<XT>(xs, x + (size_t)t0 * hidden, nt, hidden);
    __syncthreads();
    for (int e = blockIdx.x * 4 + (threadIdx.x >> 6); e < n_experts; e += gridDim.x * 4) {
        float acc[ROUTE_TOK_PER_WG];
        router_row_dot<XT>(W + (size_t)e * hidden, xs, nt, hidden, lane, acc);
        const float b = (add_bias && bias) ? half_bits_to_float(bias[e]) : 0.0f;
#pragma unroll
        for (int t = 0; t < ROUTE_TOK_PER_WG; t++)
            if (lane == 0 && t < nt) logits[(size_t)(t0 + t) * n_experts + e] = acc[t] + b;
    }
}

/* Launch of router_logits_kernel; false when its requirements (16-byte
 * aligned W and x, hidden % 8 == 0, token rows fitting 64 KiB of LDS) are
 * not met. */
template <typename XT>
static bool launch_router_logits(const uint16_t* W, const uint16_t* bias, const XT* x,
                                 float* logits, int n_tokens, int hidden, int n_experts,
                                 int add_bias, hipStream_t s) {
    const size_t lds = (size_t)ROUTE_TOK_PER_WG * hidden * sizeof(XT);
    if (hidden % 8 || (uintptr_t)W % 16 || (uintptr_t)x % 16 || lds > 65536) return false;
    dim3 grid((n_experts + 3) / 4, (n_tokens + ROUTE_TOK_PER_WG - 1) / ROUTE_TOK_PER_WG);
    hipLaunchKernelGGL(router_logits_kernel<XT>, grid, dim3(256), lds, s, W, bias, x, logits,
                       n_tokens, hidden, n_experts, add_bias);
    return true;
}

/* Any alignment and hidden size: one wave per expert row, scalar loads
 * (the reference kernel's shape, csrc/cuda/router.cu:29-60). Only used when
 * router_logits_kernel's requirements are not met. */
template <typename XT>
__global__ __launch_bounds__(256) void router_logits_any_kernel(const uint16_t* __restrict__ W,
                                                                const uint16_t* __restrict__ bias,
                                                                const XT* __restrict__ x,
                                                                float* __restrict__ logits,
                                                                int n_tokens, int hidden,
                                                                int n_experts, int add_bias) {
    const int e = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int t0 = blockIdx.y * ROUTE_TOK_PER_WG;
    if (e >= n_experts) return;
    const int nt = min(ROUTE_TOK_PER_WG, n_tokens - t0);
    const uint16_t* row = W + (size_t)e * hidden;
    float acc[ROUTE_TOK_PER_WG] = {0.f, 0.f, 0.f, 0.f};
    for (int c = lane; c < hidden; c += WAVE) {
        const float w = half_bits_to_float(row[c]);
        for (int t = 0; t < nt; t++)
            acc[t] = __builtin_fmaf(w, xval<XT>(x, (size_t)(t0 + t) * hidden + c), acc[t]);
    }
    const float b = (add_bias && bias) ? half_bits_to_float(bias[e]) : 0.0f;
#pragma unroll
    for (int t = 0; t < ROUTE_TOK_PER_WG; t++) {
        const float v = wave_sum(acc[t]);
        if (lane == 0 && t < nt) logits[(size_t)(t0 + t) * n_experts + e] = v + b;
    }
}

template <typename XT>
static void router_logits(const uint16_t* W, const uint16_t* bias, const XT* x, float* logits,
                          int n_tokens, int hidden, int n_experts, int add_bias, hipStream_t s) {
    if (launch_router_logits<XT>(W, bias, x, logits, n_tokens, hidden, n_experts, add_bias, s))
        return;
    dim3 grid((n_experts + 3) / 4, (n_tokens + ROUTE_TOK_PER_WG - 1) / ROUTE_TOK_PER_WG);
    hipLaunchKernelGGL(router_logits_any_kernel<XT>, grid, dim3(256), 0, s, W, bias, x, logits,
                       n_tokens, hidden, n_experts, add_bias);
}

/* Raw logits for the fused layer decode when the router matrix is too large
 * for its single-workgroup prep (internal; declared in moe_decode.hip). */
hipError_t wisp_amd__router_logits(const wisp_half* W, const wisp_half* bias, const void* x,
                                   int x_dtype, int n_tokens, int hidden, int n_experts,
                                   int add_bias, float* logits, hipStream_t s) {
    if (x_dtype == WISP_DTYPE_F16)
        router_logits<uint16_t>(W, bias, (const uint16_t*)x, logits, n_tokens, hidden, n_experts,
                                add_bias, s);
    else
        router_logits<float>(W, bias, (const float*)x, logits, n_tokens, hidden, n_experts,
                             add_bias, s);
    return hipGetLastError();
}

/* ======================================================================= */
/* top-k: one wave per token                                                */
/* ======================================================================= */

/* scores_out[t, e] = softmax probability or sigmoid score; idx/w [t, k].
 * One workgroup of 256 per token; dynamic LDS of topk_lds_bytes. */
static inline size_t topk_lds_bytes(int n_experts) {
    return (size_t)((n_experts + 1) & ~1) * 8 + (size_t)n_experts * 4;
}

__global__ __launch_bounds__(256) void topk_kernel(const float* logits,
                                                   const uint16_t* __restrict__ bias,
                                                   float* scores_out,
                                                   int n_tokens, int n_experts, int top_k,
                                                   int kind, int* __restrict__ out_idx,
                                                   float* __restrict__ out_w) {
    extern __shared__ __attribute__((aligned(16))) uint64_t topk_buf[];
    __shared__ float s_red[32];
    const int t = blockIdx.x;
    if (t >= n_tokens) return;
    uint64_t* s_ck = topk_buf;
    float* s_sc = (float*)(topk_buf + ((n_experts + 1) & ~1));
    topk_block(logits + (size_t)t * n_experts, bias, s_ck, s_sc, s_red,
               scores_out + (size_t)t * n_experts, n_experts, top_k, kind,
               out_idx + (size_t)t * top_k, out_w + (size_t)t * top_k);
}

static hipError_t launch_topk(const float* d_logits, const uint16_t* d_bias, float* d_scores,
                              int n_tokens, int n_experts, int top_k, int kind,
                              int* d_idx, float* d_w, hipStream_t s) {
    hipLaunchKernelGGL(topk_kernel, dim3(n_tokens), dim3(256), topk_lds_bytes(n_experts), s,
                       d_logits, d_bias,
                       d_scores, n_tokens, n_experts, top_k, kind, d_idx, d_w);
    return hipGetLastError();
}

extern "C" hipError_t wisp_gpu_topk_from_logits(const float* d_logits, const wisp_half* d_bias,
                                                int n_tokens, int n_experts, int top_k, int kind,
                                                float* d_scores, int* d_topk_idx, float* d_topk_w,
                                                hipStream_t s) {
    if (n_tokens <= 0 || n_experts <= 0 || n_experts > ROUTE_MAX_EXPERTS || top_k <= 0 ||
        top_k > ROUTE_MAX_TOPK || (kind != WISP_ROUTER_SOFTMAX && kind != WISP_ROUTER_SIGMOID))
        return hipErrorInvalidValue;
    return launch_topk(d_logits, kind == WISP_ROUTER_SIGMOID ? d_bias : nullptr, d_scores,
                       n_tokens, n_experts, top_k, kind, d_topk_idx, d_topk_w, s);
}

extern "C" hipError_t wisp_gpu_moe_route(const wisp_half* d_router_w, const wisp_half* d_bias,
                                         const wisp_half* d_x, int n_tokens, int hidden,
                                         int n_experts, int top_k, int kind, float* d_logits,
                                         int* d_topk_idx, float* d_topk_w, hipStream_t s) {
    if (n_tokens <= 0 || hidden <= 0 || n_experts <= 0 || n_experts > ROUTE_MAX_EXPERTS ||
        top_k <= 0 || top_k > ROUTE_MAX_TOPK || top_k > n_experts ||
        (kind != WISP_ROUTER_SOFTMAX && kind != WISP_ROUTER_SIGMOID))
        return hipErrorInvalidValue;
    ev_before(EV_ROUTE, s);
    router_logits<uint16_t>(d_router_w, d_bias, d_x, d_logits, n_tokens, hidden, n_experts,
                            kind == WISP_ROUTER_SOFTMAX ? 1 : 0, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    /* the scores overwrite the logits in place: each wave reads its token's
     * row completely before writing it */
    e = launch_topk(d_logits, kind == WISP_ROUTER_SIGMOID ? d_bias : nullptr, d_logits,
                    n_tokens, n_experts, top_k, kind, d_topk_idx, d_topk_w, s);
    ev_after(EV_ROUTE, s);
    return e;
}

/* ======================================================================= */
/* reference-signature router (csrc/cuda/router.cu:140-171)                 */
/* ======================================================================= */

/* Per-device staging for the host copy of the selection. A file-scope
 * device array: no allocation, one copy per device. */
__device__ int g_route_stage_idx[ROUTE_MAX_TOPK];
__device__ float g_route_stage_w[ROUTE_MAX_TOPK];

#define ROUTE_MAX_DEVICES 64
static std::mutex g_stage_mu;
static void* g_stage_idx_ptr[ROUTE_MAX_DEVICES];
static void* g_stage_w_ptr[ROUTE_MAX_DEVICES];

static bool route_stage(void** pidx, void** pw) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= ROUTE_MAX_DEVICES) return false;
    std::lock_guard<std::mutex> lk(g_stage_mu);
    if (!g_stage_idx_ptr[dev]) {
        void *a = nullptr, *b = nullptr;
        if (hipGetSymbolAddress(&a, HIP_SYMBOL(g_route_stage_idx)) != hipSuccess) return false;
        if (hipGetSymbolAddress(&b, HIP_SYMBOL(g_route_stage_w)) != hipSuccess) return false;
        g_stage_idx_ptr[dev] = a;
        g_stage_w_ptr[dev] = b;
    }
    *pidx = g_stage_idx_ptr[dev];
    *pw = g_stage_w_ptr[dev];
    return true;
}

extern "C" void wisp_gpu_router_topk(const wisp_half* W, const wisp_half* bias, const float* x,
                                     float* logits_scratch, int n_experts, int hidden,
                                     int top_k, int* out_idx, float* out_w, hipStream_t s) {
    if (n_experts <= 0 || top_k <= 0) return;
    if (top_k > ROUTE_MAX_TOPK) top_k = ROUTE_MAX_TOPK;
    if (n_experts > ROUTE_MAX_EXPERTS || top_k > n_experts) return;
    void *didx, *dw;
    if (!route_stage(&didx, &dw)) return;
    router_logits<float>(W, bias, x, logits_scratch, 1, hidden, n_experts, 1, s);
    (void)launch_topk(logits_scratch, nullptr, logits_scratch, 1, n_experts, top_k,
                WISP_ROUTER_SOFTMAX, (int*)didx, (float*)dw, s);
    (void)hipMemcpyAsync(out_idx, didx, (size_t)top_k * sizeof(int), hipMemcpyDeviceToHost, s);
    (void)hipMemcpyAsync(out_w, dw, (size_t)top_k * sizeof(float), hipMemcpyDeviceToHost, s);
}

/* ======================================================================= */
/* expert-offset builder                                                    */
/* ======================================================================= */

#define EO_THREADS 1024
#define EO_WAVES (EO_THREADS / 64)
#define EO_BATCH 8     /* pairs per lane loaded before any is used */

/* Stable counting sort of the pairs by expert in one workgroup of 16 waves.
 * Wave w owns the contiguous chunk [w C, w C + C) of pairs, C = ceil(n / 16).
 * Pass 1 counts each wave's chunk into hist[w][e] (LDS atomics; the order
 * does not matter for counting). Then thread e turns its column into
 * running bases, hist[w][e] = number of e-pairs in chunks before w, and the
 * workgroup scans the totals into offsets. Pass 2: each wave walks its
 * chunk in order, 64 pairs at a time; lanes holding the same expert find
 * each other with one ballot per bit of the id, so a pair's position is
 * offsets[e] + hist[w][e] + the number of such lanes below it, and the
 * lowest of them advances hist[w][e] by their count (one wave's LDS
 * operations run in order, so the next group sees it). Flat pair order is
 * kept within every expert. Loads go out EO_BATCH per lane at a time. */
__global__ __launch_bounds__(EO_THREADS) void expert_offsets_kernel(
    const int* __restrict__ topk_idx, int n_pairs, int n_experts, int* __restrict__ counts,
    int* __restrict__ offsets, int* __restrict__ order, int* __restrict__ inv) {
    extern __shared__ int eo_lds[];   /* hist [EO_WAVES][E], then off [E] */
    __shared__ int s_wsum[EO_WAVES];
    const int E = n_experts;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    int* hist = eo_lds;
    int* off = eo_lds + EO_WAVES * E;
    for (int i = tid; i < EO_WAVES * E; i += EO_THREADS) hist[i] = 0;
    __syncthreads();
    const int C = (n_pairs + EO_WAVES - 1) / EO_WAVES;
    const int c0 = min(wv * C, n_pairs), c1 = min(c0 + C, n_pairs);
    for (int base = c0; base < c1; base += 64 * EO_BATCH) {
        int ev[EO_BATCH];
#pragma unroll
        for (int q = 0; q < EO_BATCH; q++) {
            const int p = base + 64 * q + lane;
            ev[q] = p < c1 ? topk_idx[p] : -1;
        }
#pragma unroll
        for (int q = 0; q < EO_BATCH; q++)
            if (ev[q] >= 0 && ev[q] < E) atomicAdd(&hist[wv * E + ev[q]], 1);
    }
    __syncthreads();
    /* column e: running bases over the waves, total in tot */
    const int e = tid;
    int tot = 0;
    if (e < E) {
        for (int w = 0; w < EO_WAVES; w++) {
            const int h = hist[w * E + e];
            hist[w * E + e] = tot;
            tot += h;
        }
    }
    /* exclusive scan of the totals (E <= EO_THREADS) */
    int incl = tot;
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(incl, d, 64);
        if (lane >= d) incl += y;
    }
    if (lane == 63) s_wsum[wv] = incl;
    __syncthreads();
    for (int w = 0; w < wv; w++) incl += s_wsum[w];
    if (e < E) {
        off[e] = incl - tot;
        offsets[e] = incl - tot;
        counts[e] = tot;
        if (e == E - 1) offsets[E] = incl;
    }
    __syncthreads();
    int nbits = 0;
    while ((1 << nbits) < E) nbits++;
    const uint64_t lt = (1ull << lane) - 1ull;
    for (int base = c0; base < c1; base += 64 * EO_BATCH) {
        int ev[EO_BATCH];
#pragma unroll
        for (int q = 0; q < EO_BATCH; q++) {
            const int p = base + 64 * q + lane;
            ev[q] = p < c1 ? topk_idx[p] : -1;
        }
#pragma unroll
        for (int q = 0; q < EO_BATCH; q++) {
            const int p = base + 64 * q + lane;
            if (base + 64 * q >= c1) break;           /* uniform: past the chunk */
            const bool valid = p < c1 && ev[q] >= 0 && ev[q] < E;
            const int ee = valid ? ev[q] : 0;
            uint64_t peers = __ballot(valid);
            for (int bit = 0; bit < nbits; bit++) {
                const bool set = (ee >> bit) & 1;
                const uint64_t m = __ballot(valid && set);
                peers &= set ? m : ~m;
            }
            if (valid) {
                const int pos = off[ee] + hist[wv * E + ee] + __popcll(peers & lt);
                order[pos] = p;
                inv[p] = pos;
            } else if (p < c1) {
                inv[p] = -1;
            }
            /* the lowest lane of each expert advances the wave's base */
            if (valid && (peers & lt) == 0) hist[wv * E + ee] += __popcll(peers);
        }
    }
}

extern "C" hipError_t wisp_gpu_expert_offsets(const int* d_topk_idx, int n_tokens, int top_k,
                                              int n_experts, int* d_counts, int* d_offsets,
                                              int* d_order, int* d_inv, hipStream_t s) {
    if (n_tokens <= 0 || top_k <= 0 || n_experts <= 0 || n_experts > ROUTE_MAX_EXPERTS)
        return hipErrorInvalidValue;
    const long n_pairs = (long)n_tokens * top_k;
    if (n_pairs > (1L << 30)) return hipErrorInvalidValue;
    /* hist [16][E] + off [E]: at most 68 KiB of LDS for 1024 experts */
    const size_t lds = (size_t)(EO_WAVES + 1) * n_experts * sizeof(int);
    if (lds > 65536)
        (void)hipFuncSetAttribute((const void*)expert_offsets_kernel,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    hipLaunchKernelGGL(expert_offsets_kernel, dim3(1), dim3(EO_THREADS), lds, s, d_topk_idx,
                       (int)n_pairs, n_experts, d_counts, d_offsets, d_order, d_inv);
    return hipGetLastError();
}

/* ======================================================================= */
/* gather / weighted combine                                                */
/* ======================================================================= */

__global__ void gather_kernel(const uint16_t* __restrict__ x, const int* __restrict__ order,
                              int n_pairs, int top_k, int hidden, uint16_t* __restrict__ xg) {
    const int p = blockIdx.x;
    if (order[p] < 0) return;
    const int tok = order[p] / top_k;
    const uint16_t* src = x + (size_t)tok * hidden;
    uint16_t* dst = xg + (size_t)p * hidden;
    if (hidden % 8 == 0 && ((uintptr_t)x % 16 == 0) && ((uintptr_t)xg % 16 == 0)) {
        for (int c = threadIdx.x; c < hidden / 8; c += blockDim.x)
            ((u4*)dst)[c] = ((const u4*)src)[c];
    } else {
        for (int c = threadIdx.x; c < hidden; c += blockDim.x) dst[c] = src[c];
    }
}

extern "C" hipError_t wisp_gpu_moe_gather(const wisp_half* d_x, const int* d_order, int n_pairs,
                                          int top_k, int hidden, wisp_half* d_xg, hipStream_t s) {
    if (n_pairs < 0 || top_k <= 0 || hidden <= 0) return hipErrorInvalidValue;
    if (n_pairs == 0) return hipSuccess;
    hipLaunchKernelGGL(gather_kernel, dim3(n_pairs), dim3(256), 0, s, d_x,
                       d_order, n_pairs, top_k, hidden, d_xg);
    return hipGetLastError();
}

__global__ void combine_kernel(const float* __restrict__ y, const int* __restrict__ inv,
                               const float* __restrict__ w, int top_k, int hidden,
                               int accumulate, float* __restrict__ out) {
    const int t = blockIdx.x;
    for (int c = threadIdx.x; c < hidden; c += blockDim.x) {
        float acc = accumulate ? out[(size_t)t * hidden + c] : 0.0f;
        for (int k = 0; k < top_k; k++) {
            int p = inv[(size_t)t * top_k + k];
            if (p >= 0) acc = __builtin_fmaf(w[(size_t)t * top_k + k], y[(size_t)p * hidden + c], acc);
        }
        out[(size_t)t * hidden + c] = acc;
    }
}

extern "C" hipError_t wisp_gpu_moe_scatter(const float* d_y, const int* d_inv,
                                           const float* d_topk_w, int n_tokens, int top_k,
                                           int hidden, int accumulate, float* d_out,
                                           hipStream_t s) {
    if (n_tokens < 0 || top_k <= 0 || hidden <= 0) return hipErrorInvalidValue;
    if (n_tokens == 0) return hipSuccess;
    hipLaunchKernelGGL(combine_kernel, dim3(n_tokens), dim3(256), 0, s, d_y, d_inv,
                       d_topk_w, top_k, hidden, accumulate, d_out);
    return hipGetLastError();
}
