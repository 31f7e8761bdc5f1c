/*
 * moe_decode.hip — fused int4 MoE decode for M = 1..4 tokens on gfx950.
 *
 * Replaces the reference's per-expert chain (csrc/core/wisp_engine.c:
 * 1507-1531 and 1563-1674: 3 full-matrix dequants into fp16 scratch, a
 * fused gate/up GEMV, a down GEMV and a scale-accumulate, per expert) with
 * three launches per MoE layer:
 *
 *   prep    : unique-expert list of the M tokens (shared expert first, then
 *             first appearance in flat (token, slot) order), per-(expert,
 *             token) routing weights, and x permuted into the MFMA operand
 *             order of unpack8_magic.
 *   gate/up : grid (inter/32 row blocks) x (unique experts). Each wave owns a
 *             K range; per 128-element block it loads 16 B of packed nibbles
 *             per lane for 2 gate + 2 up row tiles (a lane's 16 B are 32
 *             consecutive elements of one row), unpacks them with 5 integer
 *             ops per 8 values and feeds v_mfma_f32_16x16x32_f16 with the
 *             activations as the A operand (M of its 16 rows used) and the
 *             weights as B. One extra MFMA per block against a constant
 *             operand yields the magic-number excess (a second one sum(x)
 *             when zero points are present); the group scale and zero are
 *             applied per block in fp32. The K split is
 *             reduced through LDS in a fixed order; the epilogue writes
 *             h' = w_route * silu(g) * u in fp16, already permuted for the
 *             down kernel.
 *   down    : grid (hidden/16 row blocks). The K range of a block is the
 *             concatenation of all unique experts' inter dimensions, so the
 *             routed sum happens inside the contraction; routing weights are
 *             folded into h'. Output fp32 and/or fp16.
 *
 * Weights are read once, in place, from the reference blob layout
 * (csrc/core/wisp_engine.h:214-238); nothing is dequantised to memory.
 */
#include "hip_common.h"

#define DEC_MAX_TOKENS 4
#define DEC_MAX_TOPK 64
#define DEC_MAX_WAVES 16
#define DEC_GU_TILES 1
#define DEC_GU_MAX_WAVES 8

struct DecodeParams {
    uint64_t p_off[3], s_off[3], z_off[3];
    int hidden, inter, gs, has_zeros;
    int max_u;
    int* n_unique;
    const uint8_t** ublob;
    float* uw;            /* [max_u][4] routing weight of each token     */
    uint16_t* xperm;      /* [M][hidden] permuted fp16 activations        */
    uint16_t* hperm;      /* [max_u][M][inter] permuted fp16 h'           */
};

/* ======================================================================= */
/* prep                                                                     */
/* ======================================================================= */

template <typename XT>
__device__ __forceinline__ float load_x(const XT* x, size_t i);
template <> __device__ __forceinline__ float load_x<float>(const float* x, size_t i) { return x[i]; }
template <> __device__ __forceinline__ float load_x<uint16_t>(const uint16_t* x, size_t i) {
    return half_bits_to_float(x[i]);
}

/* Writes one 8-element block of a permuted activation row: even elements
 * as fp16(v), odd elements as fp16(v / 16), in unpack8_magic slot order. */
__device__ __forceinline__ void store_perm8(uint16_t* dst, const float* v) {
    uint16_t o[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        f16 h = (f16)((e & 1) ? v[e] * 0.0625f : v[e]);
        o[perm_slot(e)] = __builtin_bit_cast(uint16_t, h);
    }
    u4 q;
    q.x = o[0] | ((uint32_t)o[1] << 16);
    q.y = o[2] | ((uint32_t)o[3] << 16);
    q.z = o[4] | ((uint32_t)o[5] << 16);
    q.w = o[6] | ((uint32_t)o[7] << 16);
    *(u4*)dst = q;
}

template <typename XT>
__global__ __launch_bounds__(256) void decode_prep_kernel(DecodeParams P,
                                                          const void* const* __restrict__ table,
                                                          const void* shared_blob,
                                                          const XT* __restrict__ x, int M,
                                                          const int* __restrict__ idx,
                                                          const float* __restrict__ w,
                                                          int top_k, int n_experts) {
    if (blockIdx.x == 0) {
        /* unique list: one thread per (token, slot) pair, <= 256 pairs */
        __shared__ int s_e[DEC_MAX_TOKENS * DEC_MAX_TOPK];
        __shared__ int s_wcount[4];
        const int n_pairs = M * top_k;
        const int p = threadIdx.x;
        const int lane = p & 63, wv = p >> 6;
        const int base = shared_blob ? 1 : 0;
        int e = -1;
        if (p < n_pairs) {
            e = idx[p];
            if (e < 0 || e >= n_experts) e = -1;
            s_e[p] = e;
        }
        __syncthreads();
        int first_p = -1;
        if (e >= 0) {
            for (int q = 0; q < p; q++)
                if (s_e[q] == e) { first_p = q; break; }
        }
        const bool is_first = (e >= 0 && first_p < 0);
        uint64_t m = __ballot(is_first);
        if (lane == 0) s_wcount[wv] = __popcll(m);
        __syncthreads();
        int before = base;
        for (int q = 0; q < wv; q++) before += s_wcount[q];
        if (is_first) {
            int slot = before + __popcll(m & ((1ull << lane) - 1ull));
            P.ublob[slot] = (const uint8_t*)table[e];
            /* weights of every token for this expert, in flat pair order */
            float acc[DEC_MAX_TOKENS] = {0.f, 0.f, 0.f, 0.f};
            for (int q = p; q < n_pairs; q++)
                if (s_e[q] == e) acc[q / top_k] += w[q];
            for (int v = 0; v < DEC_MAX_TOKENS; v++) P.uw[slot * 4 + v] = acc[v];
        }
        if (p == 0) {
            int total = base;
            for (int q = 0; q < 4; q++) total += (q * 64 < n_pairs) ? s_wcount[q] : 0;
            *P.n_unique = total;
            if (shared_blob) {
                P.ublob[0] = (const uint8_t*)shared_blob;
                for (int v = 0; v < DEC_MAX_TOKENS; v++) P.uw[v] = v < M ? 1.0f : 0.0f;
            }
        }
        return;
    }
    /* permuted activations: one 8-element block per thread */
    const int nb = M * (P.hidden / 8);
    for (int i = (blockIdx.x - 1) * blockDim.x + threadIdx.x; i < nb;
         i += (gridDim.x - 1) * blockDim.x) {
        const int v = i / (P.hidden / 8), b = i - v * (P.hidden / 8);
        float xv[8];
#pragma unroll
        for (int e = 0; e < 8; e++) xv[e] = load_x<XT>(x, (size_t)v * P.hidden + b * 8 + e);
        store_perm8(P.xperm + (size_t)v * P.hidden + b * 8, xv);
    }
}

/* ======================================================================= */
/* shared MFMA block step                                                   */
/* ======================================================================= */

/* One 128-element block for NT row tiles: xa[4] are this lane's activation
 * operands (token `col`, k-slice j), wv[s] the 16 B of nibbles of tile s.
 * Adds scale*(sum - excess) + zero*sum(x) into tot[s][v]. The excess and
 * sum(x) come from MFMAs against constant operands that are equal in every
 * column, so lane `col` holds them for its own tokens. */
template <int M, int NG, int NT>
__device__ __forceinline__ void block_step(const h8 (&xa)[4], const u4 (&wv)[NT], int gamma,
                                           const float (&sc)[NT][NG], const float (&zc)[NT][NG],
                                           bool has_zeros, float (&tot)[NT][M]) {
    const h8 bex = mfma_excess_operand();
    const h8 bsum = mfma_sum_operand();
#pragma unroll
    for (int g = 0; g < NG; g++) {
        h8 xg[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            if (NG == 1 || gamma == g) xg[t] = xa[t];
            else xg[t] = (h8){0, 0, 0, 0, 0, 0, 0, 0};
        }
        f4 ex = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; t++) ex = mfma16x16x32(xg[t], bex, ex);
        f4 xs = {0.f, 0.f, 0.f, 0.f};
        if (has_zeros) {
#pragma unroll
            for (int t = 0; t < 4; t++) xs = mfma16x16x32(xg[t], bsum, xs);
        }
        f4 acc[NT];
#pragma unroll
        for (int s = 0; s < NT; s++) {
            acc[s] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; t++) acc[s] = mfma16x16x32(xg[t], unpack8_magic(wv[s][t]), acc[s]);
        }
#pragma unroll
        for (int v = 0; v < M; v++) {
#pragma unroll
            for (int s = 0; s < NT; s++)
                tot[s][v] = __builtin_fmaf(sc[s][g], acc[s][v] - ex[v],
                                           __builtin_fmaf(zc[s][g], xs[v], tot[s][v]));
        }
    }
}

template <int M>
__device__ __forceinline__ void load_x4(h8 (&xa)[4], const uint16_t* p, bool valid) {
#pragma unroll
    for (int t = 0; t < 4; t++) {
        if (valid) xa[t] = *(const h8*)(p + 8 * t);
        else xa[t] = (h8){0, 0, 0, 0, 0, 0, 0, 0};
    }
}

/* ======================================================================= */
/* gate/up + SiLU                                                           */
/* ======================================================================= */

template <int M, int NG>
__global__ __launch_bounds__(64 * DEC_GU_MAX_WAVES) void gateup_kernel(const DecodeParams P) {
    constexpr int TILES = DEC_GU_TILES;
    constexpr int NT = 2 * TILES;
    __shared__ float red[DEC_GU_MAX_WAVES][NT][16][M];
    const int u = blockIdx.y;
    if (u >= *P.n_unique) return;
    const uint8_t* blob = P.ublob[u];
    const int K = P.hidden;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int col = lane & 15, j = lane >> 4;
    const int r0 = blockIdx.x * 16 * TILES;
    const int nblk = K >> 7;
    const int b0 = wave * nblk / nw, b1 = (wave + 1) * nblk / nw;
    const size_t row_bytes = (size_t)K / 2;
    const int gpr = K / P.gs;
    const int gamma = (NG == 1) ? 0 : (j * NG) / 4;

    const uint8_t* wp[NT];
    const uint16_t* sp[NT];
    const uint16_t* zp[NT];
#pragma unroll
    for (int s = 0; s < NT; s++) {
        const int mat = s < TILES ? 0 : 1;
        const int row = r0 + 16 * (s % TILES) + col;
        wp[s] = blob + P.p_off[mat] + (size_t)row * row_bytes + 16 * j;
        sp[s] = (const uint16_t*)(blob + P.s_off[mat]) + (size_t)row * gpr;
        zp[s] = (const uint16_t*)(blob + P.z_off[mat]) + (size_t)row * gpr;
    }
    const bool xvalid = col < M;
    const uint16_t* xp = P.xperm + (size_t)(xvalid ? col : 0) * K + 32 * j;

    float tot[NT][M];
#pragma unroll
    for (int s = 0; s < NT; s++)
#pragma unroll
        for (int v = 0; v < M; v++) tot[s][v] = 0.0f;

    if (b0 < b1) {
        u4 wv[NT];
        h8 xa[4];
#pragma unroll
        for (int s = 0; s < NT; s++) wv[s] = *(const u4*)(wp[s] + (size_t)b0 * 64);
        load_x4<M>(xa, xp + (size_t)b0 * 128, xvalid);
        for (int b = b0; b < b1; b++) {
            u4 wn[NT];
            h8 xn[4];
            const bool more = b + 1 < b1;
            if (more) {
#pragma unroll
                for (int s = 0; s < NT; s++) wn[s] = *(const u4*)(wp[s] + (size_t)(b + 1) * 64);
                load_x4<M>(xn, xp + (size_t)(b + 1) * 128, xvalid);
            }
            float sc[NT][NG], zc[NT][NG];
#pragma unroll
            for (int g = 0; g < NG; g++) {
                const int gi = (b * 128 + g * (128 / NG)) / P.gs;
#pragma unroll
                for (int s = 0; s < NT; s++) {
                    sc[s][g] = half_bits_to_float(sp[s][gi]);
                    zc[s][g] = P.has_zeros ? half_bits_to_float(zp[s][gi]) : 0.0f;
                }
            }
            block_step<M, NG, NT>(xa, wv, gamma, sc, zc, P.has_zeros != 0, tot);
            if (more) {
#pragma unroll
                for (int s = 0; s < NT; s++) wv[s] = wn[s];
#pragma unroll
                for (int t = 0; t < 4; t++) xa[t] = xn[t];
            }
        }
    }
    if (lane < 16) {
#pragma unroll
        for (int s = 0; s < NT; s++)
#pragma unroll
            for (int v = 0; v < M; v++) red[wave][s][col][v] = tot[s][v];
    }
    __syncthreads();
    for (int o = threadIdx.x; o < TILES * 16 * M; o += blockDim.x) {
        const int v = o % M, rc = o / M, q = rc / 16, c = rc % 16;
        float g = 0.0f, up = 0.0f;
        for (int ww = 0; ww < nw; ww++) {
            g += red[ww][q][c][v];
            up += red[ww][TILES + q][c][v];
        }
        const float h = silu_f(g) * up * P.uw[u * 4 + v];
        const int r = r0 + 16 * q + c;
        const int e = r & 7;
        f16 hv = (f16)((e & 1) ? h * 0.0625f : h);
        P.hperm[((size_t)u * M + v) * P.inter + (r & ~7) + perm_slot(e)] =
            __builtin_bit_cast(uint16_t, hv);
    }
}

/* ======================================================================= */
/* down + combine                                                           */
/* ======================================================================= */

template <int M, int NG, int TILES>
__global__ __launch_bounds__(1024) void down_kernel(const DecodeParams P, float* out32,
                                                    uint16_t* out16, int accumulate) {
    constexpr int NT = TILES;
    __shared__ float red[DEC_MAX_WAVES][NT][16][M];
    const int n_u = *P.n_unique;
    const int K = P.inter, H = P.hidden;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int col = lane & 15, j = lane >> 4;
    const int r0 = blockIdx.x * 16 * TILES;
    const int bpe = K >> 7;
    const int NB = n_u * bpe;
    const int b0 = wave * NB / nw, b1 = (wave + 1) * NB / nw;
    const size_t row_bytes = (size_t)K / 2;
    const int gpr = K / P.gs;
    const int gamma = (NG == 1) ? 0 : (j * NG) / 4;
    const bool xvalid = col < M;

    float tot[NT][M];
#pragma unroll
    for (int s = 0; s < NT; s++)
#pragma unroll
        for (int v = 0; v < M; v++) tot[s][v] = 0.0f;

    if (b0 < b1) {
        int cur_u = -1;
        const uint8_t* wp[NT];
        const uint16_t* sp[NT];
        const uint16_t* zp[NT];
        const uint16_t* xp = nullptr;
        u4 wv[NT];
        h8 xa[4];
        for (int gb = b0; gb < b1; gb++) {
            const int uu = gb / bpe, b = gb - uu * bpe;
            if (uu != cur_u) {
                cur_u = uu;
                const uint8_t* blob = P.ublob[uu];
#pragma unroll
                for (int s = 0; s < NT; s++) {
                    const int row = r0 + 16 * s + col;
                    wp[s] = blob + P.p_off[2] + (size_t)row * row_bytes + 16 * j;
                    sp[s] = (const uint16_t*)(blob + P.s_off[2]) + (size_t)row * gpr;
                    zp[s] = (const uint16_t*)(blob + P.z_off[2]) + (size_t)row * gpr;
                }
                xp = P.hperm + ((size_t)uu * M + (xvalid ? col : 0)) * K + 32 * j;
            }
#pragma unroll
            for (int s = 0; s < NT; s++) wv[s] = *(const u4*)(wp[s] + (size_t)b * 64);
            load_x4<M>(xa, xp + (size_t)b * 128, xvalid);
            float sc[NT][NG], zc[NT][NG];
#pragma unroll
            for (int g = 0; g < NG; g++) {
                const int gi = (b * 128 + g * (128 / NG)) / P.gs;
#pragma unroll
                for (int s = 0; s < NT; s++) {
                    sc[s][g] = half_bits_to_float(sp[s][gi]);
                    zc[s][g] = P.has_zeros ? half_bits_to_float(zp[s][gi]) : 0.0f;
                }
            }
            block_step<M, NG, NT>(xa, wv, gamma, sc, zc, P.has_zeros != 0, tot);
        }
    }
    if (lane < 16) {
#pragma unroll
        for (int s = 0; s < NT; s++)
#pragma unroll
            for (int v = 0; v < M; v++) red[wave][s][col][v] = tot[s][v];
    }
    __syncthreads();
    for (int o = threadIdx.x; o < TILES * 16 * M; o += blockDim.x) {
        const int v = o % M, rc = o / M, q = rc / 16, c = rc % 16;
        float y = 0.0f;
        for (int ww = 0; ww < nw; ww++) y += red[ww][q][c][v];
        const int r = r0 + 16 * q + c;
        const size_t oi = (size_t)v * H + r;
        if (out32) {
            if (accumulate) y += out32[oi];
            out32[oi] = y;
        }
        if (out16) out16[oi] = __builtin_bit_cast(uint16_t, (f16)y);
    }
}

/* ======================================================================= */
/* host side                                                                */
/* ======================================================================= */

extern "C" hipError_t wisp_expert_layout_check(const WispExpertLayout* L) {
    if (!L) return hipErrorInvalidValue;
    const uint64_t inter = L->rows[0], hidden = L->cols[0];
    if (L->rows[1] != inter || L->cols[1] != hidden || L->rows[2] != hidden ||
        L->cols[2] != inter)
        return hipErrorInvalidValue;
    if (inter == 0 || hidden == 0 || inter % 128 || hidden % 128) return hipErrorInvalidValue;
    const uint64_t gs = L->group_size;
    const bool gs_ok = gs == 32 || gs == 64 || (gs >= 128 && gs % 128 == 0);
    if (!gs_ok || hidden % gs || inter % gs) return hipErrorInvalidValue;
    for (int m = 0; m < 3; m++) {
        const uint64_t n = (uint64_t)L->rows[m] * L->cols[m];
        if ((L->packed_off[m] + 8) % 16) return hipErrorInvalidValue;
        if (L->scales_off[m] < L->packed_off[m] + n / 2) return hipErrorInvalidValue;
        if (L->scales_off[m] % 2 || L->zeros_off[m] % 2) return hipErrorInvalidValue;
        if (L->has_zeros && L->zeros_off[m] < L->scales_off[m] + n / gs * 2)
            return hipErrorInvalidValue;
    }
    return hipSuccess;
}

struct WsLayout {
    size_t nu, ublob, uw, xperm, hperm, total;
    int max_u;
};

static WsLayout ws_layout(const WispExpertLayout* L, int M, int top_k, int has_shared) {
    WsLayout w;
    w.max_u = (has_shared ? 1 : 0) + M * top_k;
    size_t off = 0;
    w.nu = off; off += 256;
    w.ublob = off; off = align_up(off + (size_t)w.max_u * sizeof(void*), 256);
    w.uw = off; off = align_up(off + (size_t)w.max_u * 4 * sizeof(float), 256);
    w.xperm = off; off = align_up(off + (size_t)M * L->cols[0] * 2, 256);
    w.hperm = off; off = align_up(off + (size_t)w.max_u * M * L->rows[0] * 2, 256);
    w.total = off;
    return w;
}

extern "C" size_t wisp_moe_decode_workspace_bytes(const WispExpertLayout* L, int n_tokens,
                                                  int top_k, int has_shared) {
    if (!L || n_tokens < 1 || n_tokens > DEC_MAX_TOKENS || top_k < 1 || top_k > DEC_MAX_TOPK)
        return 0;
    return ws_layout(L, n_tokens, top_k, has_shared).total;
}

template <int M, int NG>
static void launch_compute(const DecodeParams& P, int gu_waves, int dn_waves, float* out32,
                           uint16_t* out16, int accumulate, hipStream_t s) {
    ev_before(EV_GATEUP, s);
    hipLaunchKernelGGL((gateup_kernel<M, NG>), dim3(P.inter / (16 * DEC_GU_TILES), P.max_u),
                       dim3(64 * gu_waves), 0, s, P);
    ev_after(EV_GATEUP, s);
    ev_before(EV_DOWN, s);
    hipLaunchKernelGGL((down_kernel<M, NG, 1>), dim3(P.hidden / 16), dim3(64 * dn_waves), 0, s,
                       P, out32, out16, accumulate);
    ev_after(EV_DOWN, s);
}

template <int M>
static void launch_ng(int ng, const DecodeParams& P, int gw, int dw, float* o32, uint16_t* o16,
                      int acc, hipStream_t s) {
    if (ng == 1) launch_compute<M, 1>(P, gw, dw, o32, o16, acc, s);
    else if (ng == 2) launch_compute<M, 2>(P, gw, dw, o32, o16, acc, s);
    else launch_compute<M, 4>(P, gw, dw, o32, o16, acc, s);
}

/* Waves per workgroup for a K split: about 4 blocks of 128 per wave. */
static int clamp_waves(int blocks_total, int max_waves) {
    int w = blocks_total / 4;
    if (w < 1) w = 1;
    if (w > max_waves) w = max_waves;
    return w;
}

extern "C" hipError_t wisp_gpu_moe_decode_int4(const void* const* d_expert_table,
                                               const void* d_shared_blob,
                                               const WispExpertLayout* L, const void* d_x,
                                               int x_dtype, int n_tokens, const int* d_topk_idx,
                                               const float* d_topk_w, int top_k, int n_experts,
                                               void* d_workspace, size_t workspace_bytes,
                                               int accumulate, float* d_out_f32,
                                               wisp_half* d_out_f16, hipStream_t s) {
    if (n_tokens < 1 || n_tokens > DEC_MAX_TOKENS || top_k < 1 || top_k > DEC_MAX_TOPK ||
        n_experts < 1 || !d_expert_table || !d_x || !d_topk_idx || !d_topk_w || !d_workspace ||
        (!d_out_f32 && !d_out_f16) || (x_dtype != WISP_DTYPE_F16 && x_dtype != WISP_DTYPE_F32))
        return hipErrorInvalidValue;
    if (wisp_expert_layout_check(L) != hipSuccess) return hipErrorInvalidValue;
    const WsLayout w = ws_layout(L, n_tokens, top_k, d_shared_blob != nullptr);
    if (workspace_bytes < w.total) return hipErrorInvalidValue;

    DecodeParams P;
    for (int m = 0; m < 3; m++) {
        P.p_off[m] = L->packed_off[m];
        P.s_off[m] = L->scales_off[m];
        P.z_off[m] = L->zeros_off[m];
    }
    P.hidden = (int)L->cols[0];
    P.inter = (int)L->rows[0];
    P.gs = (int)L->group_size;
    P.has_zeros = L->has_zeros ? 1 : 0;
    P.max_u = w.max_u;
    char* ws = (char*)d_workspace;
    P.n_unique = (int*)(ws + w.nu);
    P.ublob = (const uint8_t**)(ws + w.ublob);
    P.uw = (float*)(ws + w.uw);
    P.xperm = (uint16_t*)(ws + w.xperm);
    P.hperm = (uint16_t*)(ws + w.hperm);

    const int prep_blocks = 1 + (n_tokens * (P.hidden / 8) + 255) / 256;
    ev_before(EV_PREP, s);
    if (x_dtype == WISP_DTYPE_F16)
        hipLaunchKernelGGL(decode_prep_kernel<uint16_t>, dim3(prep_blocks), dim3(256), 0, s, P,
                           d_expert_table, d_shared_blob, (const uint16_t*)d_x, n_tokens,
                           d_topk_idx, d_topk_w, top_k, n_experts);
    else
        hipLaunchKernelGGL(decode_prep_kernel<float>, dim3(prep_blocks), dim3(256), 0, s, P,
                           d_expert_table, d_shared_blob, (const float*)d_x, n_tokens,
                           d_topk_idx, d_topk_w, top_k, n_experts);
    ev_after(EV_PREP, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;

    const int gs = P.gs;
    const int ng = gs >= 128 ? 1 : 128 / gs;
    const int gu_waves = clamp_waves(P.hidden / 128, DEC_GU_MAX_WAVES);
    const int dn_waves = clamp_waves(w.max_u * (P.inter / 128), DEC_MAX_WAVES);
    switch (n_tokens) {
        case 1: launch_ng<1>(ng, P, gu_waves, dn_waves, d_out_f32, d_out_f16, accumulate, s); break;
        case 2: launch_ng<2>(ng, P, gu_waves, dn_waves, d_out_f32, d_out_f16, accumulate, s); break;
        case 3: launch_ng<3>(ng, P, gu_waves, dn_waves, d_out_f32, d_out_f16, accumulate, s); break;
        default: launch_ng<4>(ng, P, gu_waves, dn_waves, d_out_f32, d_out_f16, accumulate, s); break;
    }
    return hipGetLastError();
}
