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

#include "hip_common.h"

#define ROUTE_MAX_TOPK 64
#define ROUTE_MAX_EXPERTS 1024
#define ROUTE_TOK_PER_WG 4

/* ======================================================================= */
/* router logits: one wave per expert row, up to 4 tokens per pass           */
/* ======================================================================= */

template <typename XT>
__device__ __forceinline__ float xval(const XT* x, size_t i);
template <> __device__ __forceinline__ float xval<float>(const float* x, size_t i) { return x[i]; }
template <> __device__ __forceinline__ float xval<uint16_t>(const uint16_t* x, size_t i) {
    return half_bits_to_float(x[i]);
}

/* logits[t, e] = sum_c W[e, c] x[t, c] (+ bias[e] when add_bias). */
template <typename XT>
__global__ __launch_bounds__(256) void router_logits_kernel(const uint16_t* __restrict__ W,
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
    const bool vec = (hidden % 8 == 0) && ((uintptr_t)row % 16 == 0);
    if (vec) {
        for (int c8 = lane; c8 < hidden / 8; c8 += WAVE) {
            h8 w = __builtin_bit_cast(h8, ((const u4*)row)[c8]);
#pragma unroll
            for (int t = 0; t < ROUTE_TOK_PER_WG; t++) {
                if (t < nt) {
                    const XT* xr = x + (size_t)(t0 + t) * hidden + (size_t)c8 * 8;
#pragma unroll
                    for (int i = 0; i < 8; i++)
                        acc[t] = __builtin_fmaf((float)w[i], xval<XT>(xr, i), acc[t]);
                }
            }
        }
    } else {
        for (int c = lane; c < hidden; c += WAVE) {
            float w = half_bits_to_float(row[c]);
            for (int t = 0; t < nt; t++)
                acc[t] = __builtin_fmaf(w, xval<XT>(x, (size_t)(t0 + t) * hidden + c), acc[t]);
        }
    }
    float b = (add_bias && bias) ? half_bits_to_float(bias[e]) : 0.0f;
#pragma unroll
    for (int t = 0; t < ROUTE_TOK_PER_WG; t++) {
        float v = wave_sum(acc[t]);
        if (lane == 0 && t < nt) logits[(size_t)(t0 + t) * n_experts + e] = v + b;
    }
}

/* ======================================================================= */
/* top-k: one wave per token                                                */
/* ======================================================================= */

struct KeyIdx { float v; int i; };

/* a beats b: larger key, or equal key and lower index. NaN never wins. */
__device__ __forceinline__ bool beats(float av, int ai, float bv, int bi) {
    return av > bv || (av == bv && ai >= 0 && (bi < 0 || ai < bi));
}

/* scores_out[t, e] = softmax probability or sigmoid score; idx/w [t, k].
 * For SOFTMAX the logits already include the bias. For SIGMOID the bias
 * (if any) is added to the score for selection only. */
__global__ __launch_bounds__(64) void topk_kernel(const float* logits,
                                                  const uint16_t* __restrict__ bias,
                                                  float* scores_out,
                                                  int n_tokens, int n_experts, int top_k,
                                                  int kind, int* __restrict__ out_idx,
                                                  float* __restrict__ out_w) {
    const int t = blockIdx.x;
    const int lane = threadIdx.x;
    if (t >= n_tokens) return;
    const float* lg = logits + (size_t)t * n_experts;
    constexpr int PER = ROUTE_MAX_EXPERTS / WAVE;   /* keys per lane */
    float key[PER], lgt[PER];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        int e = lane + i * WAVE;
        float l = e < n_experts ? lg[e] : NAN;
        lgt[i] = l;
        float k = l;
        if (kind == WISP_ROUTER_SIGMOID && bias && e < n_experts)
            k = 1.0f / (1.0f + __expf(-l)) + half_bits_to_float(bias[e]);
        key[i] = e < n_experts ? k : NAN;
        if (e < n_experts) mx = fmaxf(mx, l);
    }
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, WAVE));
    /* denominators / scores */
    float denom = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        int e = lane + i * WAVE;
        if (e < n_experts) {
            float sc = (kind == WISP_ROUTER_SOFTMAX) ? __expf(lgt[i] - mx)
                                                     : 1.0f / (1.0f + __expf(-lgt[i]));
            lgt[i] = sc;
            denom += sc;
        }
    }
    denom = wave_sum(denom);
    const float inv = 1.0f / (denom > 0.0f ? denom : 1.0f);
#pragma unroll
    for (int i = 0; i < PER; i++) {
        int e = lane + i * WAVE;
        if (e < n_experts) {
            if (kind == WISP_ROUTER_SOFTMAX) lgt[i] = lgt[i] * inv;
            scores_out[(size_t)t * n_experts + e] = lgt[i];
        }
    }
    /* k passes of argmax */
    uint32_t taken = 0;
    float wsum = 0.0f;
    for (int k = 0; k < top_k; k++) {
        float bv = -INFINITY;
        int bi = -1;
        float bs = 0.0f;
#pragma unroll
        for (int i = 0; i < PER; i++) {
            int e = lane + i * WAVE;
            if (!(taken & (1u << i)) && beats(key[i], e, bv, bi)) {
                bv = key[i]; bi = e; bs = lgt[i];
            }
        }
        for (int off = 32; off > 0; off >>= 1) {
            float ov = __shfl_xor(bv, off, WAVE);
            int oi = __shfl_xor(bi, off, WAVE);
            float os = __shfl_xor(bs, off, WAVE);
            if (beats(ov, oi, bv, bi)) { bv = ov; bi = oi; bs = os; }
        }
        if (bi >= 0 && (bi % WAVE) == lane) taken |= 1u << (bi / WAVE);
        if (lane == 0) {
            out_idx[(size_t)t * top_k + k] = bi;
            float w = bi >= 0 ? bs : 0.0f;
            out_w[(size_t)t * top_k + k] = w;
            wsum += w;
        }
    }
    if (lane == 0 && wsum > 0.0f) {
        for (int k = 0; k < top_k; k++) out_w[(size_t)t * top_k + k] /= wsum;
    }
}

static hipError_t launch_topk(const float* d_logits, const uint16_t* d_bias, float* d_scores,
                              int n_tokens, int n_experts, int top_k, int kind,
                              int* d_idx, float* d_w, hipStream_t s) {
    hipLaunchKernelGGL(topk_kernel, dim3(n_tokens), dim3(64), 0, s, d_logits, d_bias,
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
    dim3 grid((n_experts + 3) / 4, (n_tokens + ROUTE_TOK_PER_WG - 1) / ROUTE_TOK_PER_WG);
    ev_before(EV_ROUTE, s);
    hipLaunchKernelGGL(router_logits_kernel<uint16_t>, grid, dim3(256), 0, s, d_router_w,
                       d_bias, d_x, d_logits, n_tokens, hidden, n_experts,
                       kind == WISP_ROUTER_SOFTMAX ? 1 : 0);
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
    hipLaunchKernelGGL(router_logits_kernel<float>, dim3((n_experts + 3) / 4, 1), dim3(256), 0,
                       s, W, bias, x, logits_scratch, 1, hidden, n_experts, 1);
    (void)launch_topk(logits_scratch, nullptr, logits_scratch, 1, n_experts, top_k,
                WISP_ROUTER_SOFTMAX, (int*)didx, (float*)dw, s);
    (void)hipMemcpyAsync(out_idx, didx, (size_t)top_k * sizeof(int), hipMemcpyDeviceToHost, s);
    (void)hipMemcpyAsync(out_w, dw, (size_t)top_k * sizeof(float), hipMemcpyDeviceToHost, s);
}

/* ======================================================================= */
/* expert-offset builder                                                    */
/* ======================================================================= */

/* One workgroup of T threads; thread t owns the contiguous pair chunk
 * [t*L, (t+1)*L). cnt[t][e] (u16, LDS) counts e in chunk t, then becomes
 * the number of e-pairs in chunks before t. Placement walks each chunk in
 * order, so the result is stable in flat pair order. */
__global__ void expert_offsets_kernel(const int* __restrict__ topk_idx, int n_pairs,
                                      int n_experts, int* __restrict__ counts,
                                      int* __restrict__ offsets, int* __restrict__ order,
                                      int* __restrict__ inv) {
    extern __shared__ uint16_t cnt[];            /* [T][n_experts] */
    __shared__ int s_off[ROUTE_MAX_EXPERTS + 1];
    const int T = blockDim.x;
    const int t = threadIdx.x;
    const int L = (n_pairs + T - 1) / T;
    const int p0 = min(t * L, n_pairs), p1 = min(p0 + L, n_pairs);
    for (int i = t; i < T * n_experts; i += T) cnt[i] = 0;
    __syncthreads();
    uint16_t* mine = cnt + (size_t)t * n_experts;
    for (int p = p0; p < p1; p++) {
        int e = topk_idx[p];
        if (e >= 0 && e < n_experts) mine[e]++;
    }
    __syncthreads();
    /* per-expert exclusive prefix over chunks; totals */
    for (int e = t; e < n_experts; e += T) {
        int run = 0;
        for (int c = 0; c < T; c++) {
            int v = cnt[(size_t)c * n_experts + e];
            cnt[(size_t)c * n_experts + e] = (uint16_t)run;
            run += v;
        }
        counts[e] = run;
        s_off[e + 1] = run;
    }
    __syncthreads();
    if (t == 0) {
        s_off[0] = 0;
        for (int e = 0; e < n_experts; e++) s_off[e + 1] += s_off[e];
    }
    __syncthreads();
    for (int e = t; e <= n_experts; e += T) offsets[e] = s_off[e];
    for (int p = p0; p < p1; p++) {
        int e = topk_idx[p];
        if (e >= 0 && e < n_experts) {
            int pos = s_off[e] + mine[e]++;
            order[pos] = p;
            inv[p] = pos;
        } else {
            inv[p] = -1;
        }
    }
}

extern "C" hipError_t wisp_gpu_expert_offsets(const int* d_topk_idx, int n_tokens, int top_k,
                                              int n_experts, int* d_counts, int* d_offsets,
                                              int* d_order, int* d_inv, hipStream_t s) {
    if (n_tokens <= 0 || top_k <= 0 || n_experts <= 0 || n_experts > ROUTE_MAX_EXPERTS)
        return hipErrorInvalidValue;
    long n_pairs = (long)n_tokens * top_k;
    /* chunks of at most 65535 pairs per thread (u16 counters) and a count
     * table of at most 64 KiB of LDS */
    int T = 256;
    while (T > 32 && (size_t)T * n_experts * 2 > 65536) T >>= 1;
    if ((n_pairs + T - 1) / T > 65535) return hipErrorInvalidValue;
    size_t lds = (size_t)T * n_experts * sizeof(uint16_t);
    hipLaunchKernelGGL(expert_offsets_kernel, dim3(1), dim3(T), lds, s, d_topk_idx,
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
