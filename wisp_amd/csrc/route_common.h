/*
 * route_common.h — router dot products and the workgroup top-k selection
 * shared by the routing kernels and the fused decode prep (internal).
 *
 * Selection rule (csrc/core/wisp_engine.c:803-815, csrc/cuda/router.cu:
 * 118-130): k passes of "largest untaken score wins, ties to the lowest
 * index". The softmax selection runs on the logit (plus bias): exp is
 * increasing, and distinct logits give equal probabilities only at
 * near-ties. The sigmoid selection runs on the fp32 score (plus bias, if
 * any), which saturates to 1 for logits above about 16.6: saturated experts
 * tie and go to the lowest index, as the oracle's do.
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

/* DPP lane moves within rows of 16 lanes (gfx9 encodings). */
#define DPP_QUAD_XOR1 0xB1   /* quad_perm [1,0,3,2] */
#define DPP_QUAD_XOR2 0x4E   /* quad_perm [2,3,0,1] */
#define DPP_ROW_ROR4 0x124
#define DPP_ROW_ROR8 0x128

#define DPP_MOVE(v, ctrl) \
    __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), (ctrl), 0xF, 0xF, false))

/* Sum over the 64 lanes, the same value in every lane. Order: quads (lane
 * xor 1, xor 2), then within each row quad + quad rotated by 4, then by 8,
 * then the four row totals (r0 + r1) + (r2 + r3). DPP moves and readlanes
 * only: no LDS round trips. */
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += DPP_MOVE(v, DPP_QUAD_XOR1);
    v += DPP_MOVE(v, DPP_QUAD_XOR2);
    v += DPP_MOVE(v, DPP_ROW_ROR4);
    v += DPP_MOVE(v, DPP_ROW_ROR8);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

/* Maximum over the 64 lanes (NaN-ignoring fmaxf), in every lane. */
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, DPP_MOVE(v, DPP_QUAD_XOR1));
    v = fmaxf(v, DPP_MOVE(v, DPP_QUAD_XOR2));
    v = fmaxf(v, DPP_MOVE(v, DPP_ROW_ROR4));
    v = fmaxf(v, DPP_MOVE(v, DPP_ROW_ROR8));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

/* The dot of the loaded row with token t's x row (x in LDS), summed over
 * the wave: every lane returns it. Branch-free: past the row end a lane's
 * weights are zero (router_row_load) and its x operands are replaced by
 * zeros, so every LDS read of the unrolled loop can be in flight at once. */
template <typename XT>
__device__ __forceinline__ float router_row_dot1(const u4 (&w)[ROUTE_UNROLL], const XT* x, int t,
                                                 int hidden, int lane) {
    const int n8 = hidden / 8;
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < ROUTE_UNROLL; i++) {
        const int c8 = i * WAVE + lane;
        const bool in = c8 < n8;
        const h8 wh = __builtin_bit_cast(h8, w[i]);
        float xv[8];
        load_x8(x + (size_t)t * hidden + (size_t)(in ? c8 : 0) * 8, xv);
#pragma unroll
        for (int e = 0; e < 8; e++) a = __builtin_fmaf((float)wh[e], in ? xv[e] : 0.0f, a);
    }
    return wave_sum_dpp(a);
}

/* Lane 0 writes out[t * out_stride] = add + router_row_dot1(t), for t < nt.
 * Tokens are a runtime loop to keep the code small. */
template <typename XT>
__device__ __forceinline__ void router_row_fma(const u4 (&w)[ROUTE_UNROLL], const XT* x, int nt,
                                               int hidden, int lane, float* out, int out_stride,
                                               float add) {
#pragma unroll 1
    for (int t = 0; t < nt; t++) {
        const float a = router_row_dot1<XT>(w, x, t, hidden, lane);
        if (lane == 0) out[(size_t)t * out_stride] = a + add;
    }
}

/* Copies nt rows of x [nt][hidden] (16-byte aligned, hidden % 8 == 0) to
 * LDS with 16-byte accesses, in the caller's type. Up to 8 pieces per
 * thread are loaded before any is stored, so the copy costs one memory round
 * trip per 8 x blockDim pieces (a load-store loop would wait for each load,
 * and its first wait also for every load the caller issued before). */
template <typename XT>
__device__ __forceinline__ void stage_rows(XT* dst, const XT* __restrict__ src, int nt, int hidden) {
    constexpr int PER16 = 16 / sizeof(XT);
    constexpr int CAP = 8;
    const int n = nt * hidden / PER16;
    const int nthr = blockDim.x;
    for (int base = 0; base < n; base += CAP * nthr) {
        u4 v[CAP];
#pragma unroll
        for (int c = 0; c < CAP; c++) {
            const int i = base + (int)threadIdx.x + c * nthr;
            if (i < n) v[c] = ((const u4*)src)[i];
        }
#pragma unroll
        for (int c = 0; c < CAP; c++) {
            const int i = base + (int)threadIdx.x + c * nthr;
            if (i < n) ((u4*)dst)[i] = v[c];
        }
    }
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

/* Rank of `ce` among the 2 NP keys at keys[0..2 NP) in LDS (16-byte
 * aligned): the number of larger keys. Every lane reads the same 16 bytes
 * at a time (a broadcast), all reads unrolled, so they are in flight
 * together; a loop of v_readlane over the keys instead costs about a
 * hundred cycles per key in its register dependencies. */
template <int NP>
__device__ __forceinline__ int lds_rank(const uint64_t* keys, uint64_t ce) {
    const u64x2* k2 = (const u64x2*)keys;
    int rank = 0;
#pragma unroll
    for (int q = 0; q < NP; q++) {
        const u64x2 v = k2[q];
        rank += (v.x > ce) + (v.y > ce);
    }
    return rank;
}

/* One wave, n_experts <= 64, one token: the selection topk_block makes,
 * with the same formulas, but no barrier: reductions in registers (DPP
 * moves and readlanes), the rank against the wave's 64 keys in LDS, the
 * selection placed by an LDS scatter. Weights and scores agree with
 * topk_block's to rounding (sums run in another order). lg: the token's
 * raw logits (LDS or global); s_key: 64 u64 of LDS (16-byte aligned);
 * s_sel: top_k ints of LDS. Writes scores_out[e]; lane q < top_k returns the
 * q-th selection in sel_e (-1 past the candidates) and its renormalised
 * weight in sel_w. */
__device__ __forceinline__ void topk_wave_small(const float* lg, const uint16_t* __restrict__ bias,
                                                float* scores_out, uint64_t* s_key, int* s_sel,
                                                int n_experts, int top_k, int kind, int& sel_e,
                                                float& sel_w) {
    const bool sig = kind == WISP_ROUTER_SIGMOID;
    const int lane = threadIdx.x & 63;
    const bool act = lane < n_experts;
    const float l = act ? lg[lane] : -INFINITY;
    /* sigmoid: select on the score itself (it saturates to 1 in fp32, and
     * saturated experts tie, lowest index first, as in the oracle) */
    float key = l;
    if (act && sig)
        key = 1.0f / (1.0f + __expf(-l)) + (bias ? half_bits_to_float(bias[lane]) : 0.0f);
    const uint64_t ce = act ? route_composite(key, lane) : 0ull;
    s_key[lane] = ce;
    const float mx = wave_max_dpp(l);
    const float v = act ? (sig ? 1.0f / (1.0f + __expf(-l)) : __expf(l - mx)) : 0.0f;
    const float denom = wave_sum_dpp(v);
    const float inv = 1.0f / (denom > 0.0f ? denom : 1.0f);
    const float score = sig ? v : v * inv;
    if (act) scores_out[lane] = score;
    /* keys past n_experts are 0 and never outrank: walk only the used pairs */
    const int rank = n_experts <= 8    ? lds_rank<4>(s_key, ce)
                     : n_experts <= 16 ? lds_rank<8>(s_key, ce)
                     : n_experts <= 32 ? lds_rank<16>(s_key, ce)
                                       : lds_rank<32>(s_key, ce);
    const bool picked = act && (ce >> 32) != 0 && rank < top_k;
    /* lane q takes the expert of rank q */
    if (lane < top_k) s_sel[lane] = -1;
    if (picked) s_sel[rank] = lane;
    sel_e = lane < top_k ? s_sel[lane] : -1;
    sel_w = 0.0f;
    if (sel_e >= 0) {
        const float ls = lg[sel_e];
        const float vs = sig ? 1.0f / (1.0f + __expf(-ls)) : __expf(ls - mx);
        sel_w = sig ? vs : vs * inv;
    }
    const float wsum = wave_sum_dpp(sel_w);
    if (wsum > 0.0f) sel_w /= wsum;
}

/* One token's selection by a group of four waves (wl = this wave's index in
 * the group, or -1 for a wave outside every active group), n_experts <=
 * 256, top_k <= 16. Waves wl = 0-3 rank the keys of experts 64 wl + lane
 * against their own wave's 64 keys; a key in the global top_k is in its
 * wave's top_k, so the keys of local rank < top_k are the candidates. After
 * one barrier (every wave of the workgroup must call this together) wave
 * wl = 0 ranks the 4 top_k candidates and calls emit(e, w) with lane q <
 * top_k holding the q-th selection (-1 and 0 past the candidates); then the
 * group writes the scores of its experts, so no global store precedes the
 * barrier or the emit. The selection is topk_block's; weights and scores use
 * the same formulas, with the softmax denominator summed per wave (rescaled
 * to the global maximum), so they agree to rounding. Group LDS: s_key 256
 * u64, s_cand 64 u64 (both 16-byte aligned), s_sel 16 ints, s_red 8
 * floats. bias_e: the fp16 selection bias of expert 64 wl + lane as a
 * float, loaded by the caller ahead of the logits (used when has_bias,
 * for SIGMOID). */
template <typename Emit>
__device__ __forceinline__ void topk_one_token(const float* lg, bool has_bias, float bias_e,
                                               float* scores_out, uint64_t* s_key,
                                               uint64_t* s_cand, int* s_sel, float* s_red,
                                               int n_experts, int top_k, int kind, int wl,
                                               Emit emit) {
    const bool sig = kind == WISP_ROUTER_SIGMOID;
    const int lane = threadIdx.x & 63;
    const bool grp = wl >= 0 && wl < 4;
    const int e = (grp ? wl : 0) * 64 + lane;
    const bool act = grp && e < n_experts;
    const float l = act ? lg[e] : -INFINITY;
    const float sg = sig ? 1.0f / (1.0f + __expf(-l)) : 0.0f;
    const float key = (sig && has_bias && act) ? sg + bias_e : (sig ? sg : l);
    const uint64_t ce = act ? route_composite(key, e) : 0ull;
    if (grp) {
        s_key[e] = ce;
        const int rank = lds_rank<32>(s_key + wl * 64, ce);
        if (lane < top_k) s_cand[wl * top_k + lane] = 0ull;
        if (act && (ce >> 32) != 0 && rank < top_k) s_cand[wl * top_k + rank] = ce;
        if (!sig) {
            const float wmax = wave_max_dpp(l);
            const float wsum = wave_sum_dpp(act ? __expf(l - wmax) : 0.0f);
            if (lane == 0) {
                s_red[wl] = wmax;
                s_red[4 + wl] = wsum;
            }
        }
    }
    __syncthreads();
    if (!grp) return;
    float mx = 0.0f, inv = 1.0f;
    if (!sig) {
        mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
        float den = 0.0f;
        for (int q = 0; q < 4; q++)
            if (s_red[4 + q] != 0.0f) den += s_red[4 + q] * __expf(s_red[q] - mx);
        inv = 1.0f / (den > 0.0f ? den : 1.0f);
    }
    if (wl == 0) {
        const int nc = 4 * top_k;
        const uint64_t cc = lane < nc ? s_cand[lane] : 0ull;
        /* rank among the candidates: 4 top_k <= 64 keys, read in pairs */
        const u64x2* c2 = (const u64x2*)s_cand;
        int rank = 0;
#pragma unroll 8
        for (int q = 0; q < nc / 2; q++) {
            const u64x2 v = c2[q];
            rank += (v.x > cc) + (v.y > cc);
        }
        if (lane < top_k) s_sel[lane] = -1;
        if (lane < nc && (cc >> 32) != 0 && rank < top_k) s_sel[rank] = (int)~(uint32_t)cc;
        const int sel_e = lane < top_k ? s_sel[lane] : -1;
        float v = 0.0f;
        if (sel_e >= 0) {
            const float ls = lg[sel_e];
            v = sig ? 1.0f / (1.0f + __expf(-ls)) : __expf(ls - mx) * inv;
        }
        const float wsum = wave_sum_dpp(v);
        emit(sel_e, wsum > 0.0f ? v / wsum : v);
    }
    if (act) scores_out[e] = sig ? sg : __expf(l - mx) * inv;
}

/* topk_one_token for NT tokens at once per group of four waves: the same
 * steps and formulas for each token, with one barrier for all of them, so
 * the tokens' dependent chains (rank reads, exponentials, reductions) run
 * side by side. Token k uses lg[k], scores_out[k] and its own scratch
 * s_key[k], s_cand[k], s_sel[k], s_red[k] (as topk_one_token's); a token
 * with live[k] false does nothing but still takes part in the barrier.
 * emit(k, e, w) as topk_one_token's emit(e, w), for wave wl = 0. */
template <int NT, typename Emit>
__device__ __forceinline__ void topk_tokens(const float* const (&lg)[NT], const bool (&live)[NT],
                                            bool has_bias, float bias_e,
                                            float* const (&scores_out)[NT],
                                            uint64_t* const (&s_key)[NT],
                                            uint64_t* const (&s_cand)[NT],
                                            int* const (&s_sel)[NT], float* const (&s_red)[NT],
                                            int n_experts, int top_k, int kind, int wl,
                                            Emit emit) {
    const bool sig = kind == WISP_ROUTER_SIGMOID;
    const int lane = threadIdx.x & 63;
    const bool grp = wl >= 0 && wl < 4;
    const int e = (grp ? wl : 0) * 64 + lane;
    float l[NT], sg[NT];
#pragma unroll
    for (int k = 0; k < NT; k++) {
        const bool act = grp && live[k] && e < n_experts;
        l[k] = act ? lg[k][e] : -INFINITY;
        sg[k] = sig ? 1.0f / (1.0f + __expf(-l[k])) : 0.0f;
        const float key = (sig && has_bias && act) ? sg[k] + bias_e : (sig ? sg[k] : l[k]);
        const uint64_t ce = act ? route_composite(key, e) : 0ull;
        if (grp && live[k]) {
            s_key[k][e] = ce;
            const int rank = lds_rank<32>(s_key[k] + wl * 64, ce);
            if (lane < top_k) s_cand[k][wl * top_k + lane] = 0ull;
            if (act && (ce >> 32) != 0 && rank < top_k) s_cand[k][wl * top_k + rank] = ce;
            if (!sig) {
                const float wmax = wave_max_dpp(l[k]);
                const float wsum = wave_sum_dpp(act ? __expf(l[k] - wmax) : 0.0f);
                if (lane == 0) {
                    s_red[k][wl] = wmax;
                    s_red[k][4 + wl] = wsum;
                }
            }
        }
    }
    __syncthreads();
    if (!grp) return;
#pragma unroll
    for (int k = 0; k < NT; k++) {
        if (!live[k]) continue;
        float mx = 0.0f, inv = 1.0f;
        if (!sig) {
            mx = fmaxf(fmaxf(s_red[k][0], s_red[k][1]), fmaxf(s_red[k][2], s_red[k][3]));
            float den = 0.0f;
            for (int q = 0; q < 4; q++)
                if (s_red[k][4 + q] != 0.0f) den += s_red[k][4 + q] * __expf(s_red[k][q] - mx);
            inv = 1.0f / (den > 0.0f ? den : 1.0f);
        }
        if (wl == 0) {
            const int nc = 4 * top_k;
            const uint64_t cc = lane < nc ? s_cand[k][lane] : 0ull;
            const u64x2* c2 = (const u64x2*)s_cand[k];
            int rank = 0;
#pragma unroll 8
            for (int q = 0; q < nc / 2; q++) {
                const u64x2 v = c2[q];
                rank += (v.x > cc) + (v.y > cc);
            }
            if (lane < top_k) s_sel[k][lane] = -1;
            if (lane < nc && (cc >> 32) != 0 && rank < top_k) s_sel[k][rank] = (int)~(uint32_t)cc;
            const int sel_e = lane < top_k ? s_sel[k][lane] : -1;
            float v = 0.0f;
            if (sel_e >= 0) {
                const float ls = lg[k][sel_e];
                v = sig ? 1.0f / (1.0f + __expf(-ls)) : __expf(ls - mx) * inv;
            }
            const float wsum = wave_sum_dpp(v);
            emit(k, sel_e, wsum > 0.0f ? v / wsum : v);
        }
        if (e < n_experts) scores_out[k][e] = sig ? sg[k] : __expf(l[k] - mx) * inv;
    }
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
        if (sig) k = 1.0f / (1.0f + __expf(-l)) + (bias ? half_bits_to_float(bias[e]) : 0.0f);
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
