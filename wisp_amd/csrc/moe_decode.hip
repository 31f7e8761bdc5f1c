/*
 * moe_decode.hip — fused int4 MoE decode for M = 1..4 tokens on gfx950.
 *
 * Replaces the reference's per-expert chain (csrc/core/wisp_engine.c:
 * 1507-1531 and 1563-1674: a router launch and a host round trip, then per
 * expert 3 full-matrix dequants into fp16 scratch, a fused gate/up GEMV, a
 * down GEMV and a scale-accumulate) with three launches per MoE layer:
 *
 *   prep    : optionally the router (logits in router workgroups of this
 *             launch, or in router_logits_kernel just before for rows over
 *             8192; softmax or sigmoid top-k in the prep workgroup), then the
 *             unique-expert list of the M tokens (shared expert first, then
 *             first appearance in flat (token, slot) order) with per-(expert,
 *             token) routing weights, and the reset of the down kernel's
 *             row-tile counters.
 *   gate/up : grid (inter/16 row tiles) x (unique experts). Each wave owns a
 *             K range; per 128-element block it loads 16 B of packed nibbles
 *             per lane for one gate and one up row tile (a lane's 16 B are 32
 *             consecutive elements of one row), unpacks them with 5 integer
 *             ops per 8 values and feeds v_mfma_f32_16x16x32_f16 with the
 *             activations as the A operand (M of its 16 rows used) and the
 *             weights as B. One extra MFMA per block against a constant
 *             operand yields the magic-number excess (a second one sum(x)
 *             when zero points are present); the group scale and zero are
 *             applied per block in fp32. The activations are permuted into
 *             the operand order while they are staged in LDS. The K split is
 *             reduced through LDS in a fixed order; the epilogue writes
 *             h' = w_route * silu(g) * u in fp16, already permuted for the
 *             down kernel.
 *   down    : the K axes of the unique experts' down matrices, concatenated
 *             in unique-list order, form one axis cut into wave units of 8
 *             blocks of 128 (units never straddle experts); grid (hidden/16
 *             row tiles) x (chunks of 4 units). Each wave stages its own
 *             unit's h' and scales in its own LDS region, so nothing waits
 *             for another wave before the dot products; each workgroup writes
 *             its partial sums (routing weights are already folded into h');
 *             the last workgroup of a row tile to arrive adds the tile's
 *             partials in chunk order and writes the output, so the result
 *             is deterministic. The hand-off uses device-coherent stores and
 *             loads of the partials plus an arrival counter, not a fence: a
 *             device-scope fence writes back the whole L2 on this part, far
 *             more costly than the few partials involved.
 *
 * For one token and hidden <= 4096 the gate/up and down workgroups share one
 * launch (expert_kernel): down waves wait on per-unit counters of the gate/up
 * workgroups earlier in the grid.
 *
 * Weights are read once, in place, from the reference blob layout
 * (csrc/core/wisp_engine.h:214-238); nothing is dequantised to memory.
 */
#include "route_common.h"

#include <mutex>

#define DEC_MAX_TOKENS 4
#define DEC_MAX_TOPK 64
#define DEC_MAX_WAVES 8
#define DEC_UNIT_BLOCKS 8     /* down projection: 128-wide K blocks per wave unit */
#define DN_WAVES 4            /* down projection: wave units per workgroup */
#define DEC_HCNT_STRIDE 64    /* ints between wave-unit counters (own memory line each) */
#define DEC_POLL_SLEEP 8      /* s_sleep units (64 cycles) between polls of a counter (8: measured
                                 0.2-0.5 us faster per layer than 16, 4 no better) */
#define DEC_ROUTE_MAX_EXPERTS 1024
#define DEC_PREP_THREADS 512

struct DecodeParams {
    uint64_t p_off[3], s_off[3], z_off[3];
    int hidden, inter, gs, has_zeros;
    int gshift;           /* log2(gs * NG / 128): block -> group index */
    int upe;              /* down projection: wave units per expert, ceil(inter / 1024) */
    int n_q_max;          /* down projection: workgroups per row tile at max_u experts */
    uint32_t m_lo, m_hi, one024;  /* unpack masks 0x000F000F, 0x00F000F0, 0x64006400 */
    int max_u;
    int M;
    int* n_unique;
    const uint8_t** ublob;
    float* uw;            /* [max_u][4] routing weight of each token     */
    const uint16_t* xh;   /* [M][hidden] fp16 activations (caller's or a converted copy) */
    uint16_t* xconv;      /* workspace copy used when the caller's x is fp32 or unaligned */
    uint16_t* hperm;      /* [M][max_u * inter] permuted fp16 h'          */
    float* part;          /* [n_q_max][M][hidden] down partials           */
    int* tile_cnt;        /* [hidden / 16] down workgroups arrived per row tile */
    int* hcnt;            /* [max_u * upe] gate/up workgroups done per wave unit (fused launch) */
    int gsplit;           /* workgroups sharing the K range of one gate/up row tile */
    int gfinish;          /* separate gate/up launch: K splits added by gateup_finish_kernel */
    int* gcnt;            /* [max_u * inter / 16] split workgroups arrived per gate/up row tile */
    float* gpart;         /* [max_u * inter / 16][gsplit][2][16][M] gate/up K-split partials */
    float* out32;         /* [M][hidden] layer output (either may be null) */
    uint16_t* out16;
    int accumulate;
    uint32_t* status;     /* DEC_STATUS_* bits of this call's bounded waits that gave up */
    int poll_limit;       /* polls of one hand-off word or counter before giving up */
    int poll_extra;       /* added to every wait target: nonzero only to force a give-up */
    int keep_status;      /* 1: keep the status bits of the calls before (one MoE block) */
};

/* Routing inputs of the prep kernel. mode 0: idx/w are given; mode 1: raw
 * logits [M][n_experts] were written to `logits` by router_logits_kernel;
 * mode 3: the prep launch is n_rwg router workgroups followed by the prep
 * workgroup (see decode_prep_kernel). In modes 1 and 3 `logits` receives
 * the post-activation scores and idx/w the selection. */
struct RouteArgs {
    const uint16_t* W;
    const uint16_t* bias;
    int kind, mode;
    float* logits;
    int* idx;
    float* w;
    int n_rwg;            /* mode 3: router workgroups of rpw rows each        */
    int rpw;
    uint32_t* epoch;      /* mode 3: calls completed on this workspace         */
    uint64_t* words;      /* mode 3: [M][n_experts] (call token << 32 | logit) */
};

/* ======================================================================= */
/* prep                                                                     */
/* ======================================================================= */

__host__ __device__ constexpr int align_up_dev(int v, int a) { return (v + a - 1) / a * a; }

/* Slots of one key array: at least 256 (the grouped selection gives each of
 * its four waves 64) and n_experts for the workgroup selection. */
__host__ __device__ constexpr int prep_key_slots(int n_experts) {
    return n_experts > 256 ? align_up_dev(n_experts, 64) : 256;
}

/* LDS of the 64-bit selection keys: four arrays, one per token of the
 * grouped selection (two groups of four waves, two tokens each). */
__host__ __device__ constexpr int prep_key_bytes(int n_experts) {
    return DEC_MAX_TOKENS * prep_key_slots(n_experts) * 8;
}

/* Dynamic LDS of the prep kernel in routing modes 1 and 3: selection keys
 * and M rows of scores. */
static inline size_t prep_lds_bytes(int mode, int n_experts, int M) {
    if (mode == 0) return 0;
    return (size_t)prep_key_bytes(n_experts) + align_up_dev(M * n_experts * 4, 16);
}

/* Polls of one hand-off word or counter before a wait gives up: 65,536
 * polls of 512 cycles each, about 14 ms at 2.4 GHz, so every wait ends even
 * if the workgroup it waits for never ran. A wait that gives up sets its
 * bit in the workspace's status word (cleared by the prep workgroup at the
 * start of every call; wisp_moe_decode_status reads it) and poisons what it
 * feeds with NaN, so a broken hand-off never passes for a result. */
#define DEC_POLL_LIMIT (1 << 16)
#define DEC_STATUS_ROUTER_WAIT 1u   /* prep: router logits never arrived  */
#define DEC_STATUS_DOWN_WAIT 2u     /* down wave: h' of its unit never completed */
/* Byte offset of the status word in every decode workspace. */
#define DEC_STATUS_OFFSET 128

__device__ __forceinline__ void dec_report(uint32_t* status, uint32_t bit) {
    __hip_atomic_fetch_or(status, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* The prep workgroup has DEC_PREP_THREADS threads.
 *
 * Mode 3 launches n_rwg + 1 workgroups. Router workgroup g computes the raw
 * logits of rows
 * [rpw g, rpw g + rpw) (rpw = 1 up to 256 experts, so the matrix is read by
 * as many CUs as there are rows: one CU streams only a few tens of GB/s),
 * its threads splitting the row into 16-byte pieces with the matching x
 * elements loaded straight into registers, and publishes each logit as one
 * 64-bit word (call token << 32 | float bits) with a device-coherent store.
 * The last
 * workgroup, the prep proper, polls those words until each carries this
 * call's token, then selects as in mode 1. The token is epoch + 1, epoch a
 * workspace word that the prep workgroup advances once it has seen every
 * word (so every router workgroup has read epoch by then); a word is never
 * reset, so no call needs the workspace zeroed. The prep workgroup is
 * dispatched after the router workgroups, which wait on nothing, so its wait
 * always ends; the poll bound is a second guarantee. */
template <typename XT>
__global__ __launch_bounds__(DEC_PREP_THREADS) void decode_prep_kernel(
    DecodeParams P, RouteArgs R, const void* const* __restrict__ table, const void* shared_blob,
    const XT* __restrict__ x, int top_k, int n_experts) {
    constexpr int NWV = DEC_PREP_THREADS / 64;
    __shared__ __attribute__((aligned(16))) int s_e[DEC_MAX_TOKENS * DEC_MAX_TOPK];
    __shared__ __attribute__((aligned(16))) float s_w[DEC_MAX_TOKENS * DEC_MAX_TOPK];
    __shared__ int s_wcount[NWV];
    __shared__ const uint8_t* s_tab[DEC_ROUTE_MAX_EXPERTS];
    __shared__ float s_red[32];
    __shared__ __attribute__((aligned(16))) uint64_t s_cand[DEC_MAX_TOKENS][64];
    __shared__ int s_sel[DEC_MAX_TOKENS][DEC_MAX_TOPK];
    const int M = P.M;
    const int n_pairs = M * top_k;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;

    if (R.mode == 3 && (int)blockIdx.x < R.n_rwg) {
        /* router workgroup: rows [rpw g, rpw g + rpw), one after another;
         * thread i takes the 16-byte weight pieces i and i + DEC_PREP_THREADS
         * of a row and keeps the matching x elements as raw 16-byte pieces */
        constexpr int RMAX = 4, PIECES = 2, XU = sizeof(XT) / 2;
        __shared__ float s_part[NWV][RMAX * DEC_MAX_TOKENS];
        const uint32_t tok =
            __hip_atomic_load(R.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
        const int n8 = P.hidden / 8;
        const int e0 = blockIdx.x * R.rpw;
        const int nr = min(R.rpw, n_experts - e0);
        u4 xr[DEC_MAX_TOKENS][PIECES][XU];
        u4 wpc[PIECES];
#pragma unroll
        for (int j = 0; j < PIECES; j++) {
            const int pc = min((int)threadIdx.x + j * DEC_PREP_THREADS, n8 - 1);
            wpc[j] = ((const u4*)(R.W + (size_t)e0 * P.hidden))[pc];
#pragma unroll
            for (int t = 0; t < DEC_MAX_TOKENS; t++)
#pragma unroll
                for (int c = 0; c < XU; c++)
                    if (t < M) xr[t][j][c] = ((const u4*)(x + (size_t)t * P.hidden + (size_t)pc * 8))[c];
        }
        for (int r = 0; r < nr; r++) {
            if (r > 0) {
#pragma unroll
                for (int j = 0; j < PIECES; j++) {
                    const int pc = min((int)threadIdx.x + j * DEC_PREP_THREADS, n8 - 1);
                    wpc[j] = ((const u4*)(R.W + (size_t)(e0 + r) * P.hidden))[pc];
                }
            }
#pragma unroll
            for (int t = 0; t < DEC_MAX_TOKENS; t++) {
                if (t >= M) break;
                float a = 0.0f;
#pragma unroll
                for (int j = 0; j < PIECES; j++) {
                    const bool in = (int)threadIdx.x + j * DEC_PREP_THREADS < n8;
                    const h8 wh = __builtin_bit_cast(h8, wpc[j]);
                    float xv[8];
                    if (XU == 1) {
                        const h8 xh = __builtin_bit_cast(h8, xr[t][j][0]);
#pragma unroll
                        for (int q = 0; q < 8; q++) xv[q] = (float)xh[q];
                    } else {
                        const f4 lo = __builtin_bit_cast(f4, xr[t][j][0]);
                        const f4 hi = __builtin_bit_cast(f4, xr[t][j][XU - 1]);
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            xv[q] = lo[q];
                            xv[4 + q] = hi[q];
                        }
                    }
#pragma unroll
                    for (int q = 0; q < 8; q++)
                        a = __builtin_fmaf((float)wh[q], in ? xv[q] : 0.0f, a);
                }
                a = wave_sum_dpp(a);
                if (lane == 0) s_part[wv][r * DEC_MAX_TOKENS + t] = a;
            }
        }
        __syncthreads();
        if ((int)threadIdx.x < nr * DEC_MAX_TOKENS) {
            const int r = threadIdx.x / DEC_MAX_TOKENS, t = threadIdx.x % DEC_MAX_TOKENS;
            if (t < M) {
                float a = 0.0f;
                for (int w = 0; w < NWV; w++) a += s_part[w][threadIdx.x];
                const int e = e0 + r;
                if (R.kind == WISP_ROUTER_SOFTMAX && R.bias) a += half_bits_to_float(R.bias[e]);
                __hip_atomic_store(R.words + (size_t)t * n_experts + e,
                                   ((uint64_t)tok << 32) | __float_as_uint(a), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        /* fp32 x, after its logits: this workgroup's slice of the fp16 copy
         * of x that the next launch's gate/up reads, so the prep workgroup
         * converts nothing (the fp16 instantiation, whose copy is only
         * needed for an unaligned x, leaves it to the prep workgroup) */
        if constexpr (sizeof(XT) == 4) if (P.xconv) {
            const int n = M * P.hidden;
            const int chunk = (n + R.n_rwg - 1) / R.n_rwg;
            const int i1 = min(n, ((int)blockIdx.x + 1) * chunk);
            for (int i = (int)blockIdx.x * chunk + (int)threadIdx.x; i < i1; i += DEC_PREP_THREADS)
                P.xconv[i] = __builtin_bit_cast(uint16_t, (f16)xval<XT>(x, i));
        }
        return;
    }

    /* this call's status starts clear (the down waits of the next launch
     * and the routing wait below set bits), unless it continues the calls
     * of one MoE block */
    if (threadIdx.x == 0 && !P.keep_status)
        __hip_atomic_store(P.status, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int e = threadIdx.x; e < n_experts; e += blockDim.x) s_tab[e] = (const uint8_t*)table[e];
    for (int i = threadIdx.x; i < P.hidden / 16; i += blockDim.x) P.tile_cnt[i] = 0;
    for (int i = threadIdx.x; i < P.max_u * P.upe; i += blockDim.x) P.hcnt[i * DEC_HCNT_STRIDE] = 0;
    if (P.gsplit > 1 && !P.gfinish)   /* arrival counters of the K splits */
        for (int i = threadIdx.x; i < P.max_u * (P.inter / 16); i += blockDim.x) P.gcnt[i] = 0;
    /* x -> fp16 copy when the gate/up kernel cannot read the caller's x
     * (for fp32 x with router workgroups in this launch, they make it) */
    if (P.xconv && (R.mode != 3 || sizeof(XT) == 2)) {
        for (int i = threadIdx.x; i < M * P.hidden; i += blockDim.x)
            P.xconv[i] = __builtin_bit_cast(uint16_t, (f16)xval<XT>(x, i));
    }

    /* NaN when the routing wait gave up (multiplies every routing weight:
     * x * 1 is exact, so it changes nothing otherwise) */
    float poison = 1.0f;
    /* the selection bias of the expert this thread ranks in topk_one_token
     * (64 (wave % 4) + lane), loaded before the wait for the logits */
    const bool has_bias = R.mode != 0 && R.kind == WISP_ROUTER_SIGMOID && R.bias != nullptr;
    const int bias_row = (wv & 3) * 64 + lane;
    const float bias_e =
        has_bias && bias_row < n_experts ? half_bits_to_float(R.bias[bias_row]) : 0.0f;
    if (R.mode != 0) {
        /* dynamic LDS: 64-bit selection keys (scratch of the top-k), then
         * scores [M][n_experts] (the raw logits first) */
        extern __shared__ __attribute__((aligned(16))) uint8_t lds_raw[];
        uint64_t* s_ck = (uint64_t*)lds_raw;
        float* s_sc = (float*)(lds_raw + prep_key_bytes(n_experts));
        if (R.mode == 1) {
            /* raw logits from router_logits_kernel, loaded with everything else */
            for (int i = threadIdx.x; i < M * n_experts; i += blockDim.x) s_sc[i] = R.logits[i];
            __syncthreads();
        } else if (R.mode == 3) {
            /* raw logits published by this launch's router workgroups */
            const uint32_t tok =
                __hip_atomic_load(R.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
            const uint32_t want = tok + (uint32_t)P.poll_extra;
            /* all of this thread's words in one round trip, then only the
             * ones not yet tagged with this call again */
            constexpr int WPT = DEC_MAX_TOKENS * DEC_ROUTE_MAX_EXPERTS / DEC_PREP_THREADS;
            const int n_words = M * n_experts;
            uint64_t v[WPT];
#pragma unroll
            for (int k = 0; k < WPT; k++) {
                const int i = threadIdx.x + k * DEC_PREP_THREADS;
                v[k] = i < n_words ? __hip_atomic_load(R.words + i, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT)
                                   : (uint64_t)want << 32;
            }
            auto all_tagged = [&]() {
                bool ok = true;
#pragma unroll
                for (int k = 0; k < WPT; k++) ok &= (uint32_t)(v[k] >> 32) == want;
                return ok;
            };
            int polls = 0;
            while (!all_tagged() && polls < P.poll_limit) {
                __builtin_amdgcn_s_sleep(8);
                polls++;
#pragma unroll
                for (int k = 0; k < WPT; k++) {
                    const int i = threadIdx.x + k * DEC_PREP_THREADS;
                    if ((uint32_t)(v[k] >> 32) != want)
                        v[k] = __hip_atomic_load(R.words + i, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            const bool gave_up = !all_tagged();
#pragma unroll
            for (int k = 0; k < WPT; k++) {
                const int i = threadIdx.x + k * DEC_PREP_THREADS;
                if (i < n_words) s_sc[i] = __uint_as_float((uint32_t)v[k]);
            }
            if (__syncthreads_or(gave_up)) {
                poison = __builtin_nanf("");
                if (threadIdx.x == 0) dec_report(P.status, DEC_STATUS_ROUTER_WAIT);
            }
            if (threadIdx.x == 0)
                __hip_atomic_store(R.epoch, tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        /* One token: the selection is distinct, so wave 0 writes it and the
         * unique list directly (shared expert first, then rank order). */
        auto one_token_list = [&](int e, float w) {
            const int base = shared_blob ? 1 : 0;
            const bool valid = lane < top_k && e >= 0;
            const uint64_t m = __ballot(valid);
            w *= poison;
            if (lane < top_k) {
                R.idx[lane] = e;
                R.w[lane] = w;
            }
            if (valid) {
                const int slot = base + __popcll(m & ((1ull << lane) - 1ull));
                P.ublob[slot] = s_tab[e];
                for (int v = 0; v < DEC_MAX_TOKENS; v++) P.uw[slot * 4 + v] = v == 0 ? w : 0.0f;
            }
            if (lane == 0) {
                *P.n_unique = base + __popcll(m);
                if (shared_blob) {
                    P.ublob[0] = (const uint8_t*)shared_blob;
                    for (int v = 0; v < DEC_MAX_TOKENS; v++) P.uw[v] = v == 0 ? poison : 0.0f;
                }
            }
        };
        if (M == 1 && n_experts <= 64) {
            /* few experts: wave 0 selects alone, no further barrier */
            if (wv != 0) return;
            int e;
            float w;
            topk_wave_small(s_sc, R.kind == WISP_ROUTER_SIGMOID ? R.bias : nullptr, R.logits,
                            s_ck, s_sel[0], n_experts, top_k, R.kind, e, w);
            one_token_list(e, w);
            return;
        }
        if (n_experts <= 64) {
            /* few experts, 2-4 tokens: wave t selects token t alone, no
             * barrier (the four-wave grouped selection ranks 64-key blocks
             * that would be mostly empty) */
            if (wv < M) {
                int e;
                float w;
                topk_wave_small(s_sc + wv * n_experts,
                                R.kind == WISP_ROUTER_SIGMOID ? R.bias : nullptr,
                                R.logits + (size_t)wv * n_experts, s_ck + wv * 64, s_sel[wv],
                                n_experts, top_k, R.kind, e, w);
                if (lane < top_k) {
                    s_e[wv * top_k + lane] = e;
                    s_w[wv * top_k + lane] = w;
                }
            }
        } else if (n_experts <= 256 && top_k <= 16) {
            /* up to 256 experts: two-level selection by groups of four
             * waves, two tokens per group, one barrier */
            const int grp = wv >> 2;
            const int ka = prep_key_slots(n_experts);
            if (M == 1) {
                topk_one_token(s_sc, has_bias, bias_e, R.logits, s_ck, s_cand[0], s_sel[0], s_red,
                               n_experts, top_k, R.kind, grp == 0 ? (wv & 3) : -1,
                               one_token_list);
                return;
            }
            /* group g selects tokens g and g + 2 in one pass */
            static_assert(DEC_MAX_TOKENS == 2 * (NWV / 4), "two tokens per group");
            const int ta = grp, tb = grp + 2;
            const bool live[2] = {ta < M, tb < M};
            const int ca = live[0] ? ta : 0, cb = live[1] ? tb : 0;
            const float* lg[2] = {s_sc + ca * n_experts, s_sc + cb * n_experts};
            float* so[2] = {R.logits + (size_t)ca * n_experts, R.logits + (size_t)cb * n_experts};
            uint64_t* sk[2] = {s_ck + ta * ka, s_ck + tb * ka};
            uint64_t* sc2[2] = {s_cand[ta], s_cand[tb]};
            int* ss2[2] = {s_sel[ta], s_sel[tb]};
            float* sr[2] = {s_red + 8 * ta, s_red + 8 * tb};
            auto to_lds = [&](int k, int e, float w) {
                const int t = k == 0 ? ta : tb;
                if (lane < top_k) {
                    s_e[t * top_k + lane] = e;
                    s_w[t * top_k + lane] = w;
                }
            };
            topk_tokens<2>(lg, live, has_bias, bias_e, so, sk, sc2, ss2, sr, n_experts, top_k,
                           R.kind, wv & 3, to_lds);
        } else {
            for (int t = 0; t < M; t++)
                topk_block(s_sc + t * n_experts, R.kind == WISP_ROUTER_SIGMOID ? R.bias : nullptr,
                           s_ck, s_sc + t * n_experts, s_red, R.logits + (size_t)t * n_experts,
                           n_experts, top_k, R.kind, s_e + t * top_k, s_w + t * top_k);
            if (M == 1) {
                if (wv != 0) return;
                one_token_list(lane < top_k ? s_e[lane] : -1, lane < top_k ? s_w[lane] : 0.0f);
                return;
            }
        }
    } else {
        for (int p = threadIdx.x; p < n_pairs; p += blockDim.x) {
            s_e[p] = R.idx[p];
            s_w[p] = R.w[p];
        }
    }
    __syncthreads();
    if (R.mode != 0) {
        for (int p = threadIdx.x; p < n_pairs; p += blockDim.x) {
            R.idx[p] = s_e[p];
            R.w[p] = s_w[p] * poison;
        }
    }

    /* unique list: one thread per (token, slot) pair, <= 256 pairs */
    const int base = shared_blob ? 1 : 0;
    const int p = threadIdx.x;
    int e = -1;
    if (p < n_pairs) {
        e = s_e[p];
        if (e < 0 || e >= n_experts) e = -1;
    }
    /* Every pair against every pair, lane-parallel: every lane reads the
     * same pair (an LDS broadcast), token by token so each token's sum has
     * a fixed register. A pair is its expert's first when no earlier pair
     * names the same expert; the first one also sums every token's weight
     * for the expert, in flat pair order. Up to 8 slots per token: fully
     * unrolled with the reads unconditional (in the arrays' bounds) and
     * integer masks instead of conditions, so the reads are all in flight
     * together and nothing branches; a masked weight adds +0, which
     * changes no sum (each starts at +0). Waves past the pairs skip the
     * scan (the trip count is uniform within a wave). */
    float acc[DEC_MAX_TOKENS] = {0.f, 0.f, 0.f, 0.f};
    int seen_before = 0;
    if (wv * 64 < n_pairs) {
        if (top_k <= 8) {
#pragma unroll
            for (int t = 0; t < DEC_MAX_TOKENS; t++)
#pragma unroll
                for (int c = 0; c < 8; c++) {
                    const int q = t * top_k + c;
                    const int eq = s_e[q];
                    const float wq = s_w[q];
                    const int hit = -(int)((t < M) & (c < top_k) & (eq == e));
                    const int before = -(int)(q < p);
                    seen_before |= hit & before;
                    acc[t] += __int_as_float(__float_as_int(wq) & hit & ~before);
                }
        } else {
            for (int q = 0; q < n_pairs; q++) {
                const int t = q / top_k;
                const bool hit = s_e[q] == e;
                if (hit && q < p) seen_before = 1;
                if (hit && q >= p) {
                    for (int v = 0; v < DEC_MAX_TOKENS; v++)
                        if (v == t) acc[v] += s_w[q];
                }
            }
        }
    }
    const bool is_first = e >= 0 && seen_before == 0;
    const uint64_t m = __ballot(is_first);
    if (lane == 0) s_wcount[wv] = __popcll(m);
    __syncthreads();
    int before = base;
    for (int q = 0; q < wv; q++) before += s_wcount[q];
    if (is_first) {
        const int slot = before + __popcll(m & ((1ull << lane) - 1ull));
        P.ublob[slot] = s_tab[e];
        for (int v = 0; v < DEC_MAX_TOKENS; v++) P.uw[slot * 4 + v] = acc[v] * poison;
    }
    if (p == 0) {
        int total = base;
        for (int q = 0; q < NWV; q++) total += s_wcount[q];
        *P.n_unique = total;
        if (shared_blob) {
            P.ublob[0] = (const uint8_t*)shared_blob;
            for (int v = 0; v < DEC_MAX_TOKENS; v++) P.uw[v] = v < M ? poison : 0.0f;
        }
    }
}

/* ======================================================================= */
/* shared streaming machinery                                               */
/* ======================================================================= */

/* One 128-element block for NT row tiles: xa[4] are this lane's activation
 * operands (token `col`, k-slice j), wv[s] the 16 B of nibbles of tile s.
 * Adds scale*(sum - excess) + zero*sum(x) into tot[s][v]. The excess and
 * sum(x) come from MFMAs against constant operands that are equal in every
 * column, so lane `col` holds them for its own tokens. A block with
 * live == false (a padding slot of the unrolled loop) adds nothing. */
template <int M, int NG, int NT, bool HZ>
__device__ __forceinline__ void block_step(const h8 (&xa)[4], const u4 (&wv)[NT], int gamma,
                                           const float (&sc)[NT][NG], const float (&zc)[NT][NG],
                                           bool live, uint32_t m_lo, uint32_t m_hi,
                                           uint32_t one024, float (&tot)[NT][M]) {
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
        if (HZ) {
#pragma unroll
            for (int t = 0; t < 4; t++) xs = mfma16x16x32(xg[t], bsum, xs);
        }
        f4 acc[NT];
#pragma unroll
        for (int s = 0; s < NT; s++) {
            acc[s] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; t++)
                acc[s] = mfma16x16x32(xg[t], unpack8_magic(wv[s][t], m_lo, m_hi, one024), acc[s]);
        }
#pragma unroll
        for (int s = 0; s < NT; s++) {
            const float scl = live ? sc[s][g] : 0.0f;
            const float zcl = live ? zc[s][g] : 0.0f;
#pragma unroll
            for (int v = 0; v < M; v++) {
                float t = __builtin_fmaf(scl, acc[s][v] - ex[v], tot[s][v]);
                if (HZ) t = __builtin_fmaf(zcl, xs[v], t);
                tot[s][v] = t;
            }
        }
    }
}

/* LDS image of one workgroup's operands:
 *   x    [M][XR] fp16  permuted activations of the staged K range, rows
 *                      padded by 32 halves so tokens fall in different banks
 *   sc   [NT][16][GS]  raw fp16 scale bits of the tile rows for the staged
 *   zc   [NT][16][GS]  groups (zeros only when present)
 *   red  [waves][NT][16][M] fp32 K-split partials                        */
struct LdsMap {
    int XR, GS;
    int x_off, sc_off, zc_off, red_off, bytes;
};

__host__ __device__ inline LdsMap lds_map(int M, int NT, int xk, int gs_count, bool hz, int waves) {
    LdsMap L;
    L.XR = xk + 32;
    L.GS = gs_count;
    int off = 0;
    L.x_off = off;
    off += M * L.XR * 2;
    off = (off + 15) & ~15;
    L.sc_off = off;
    off += NT * 16 * gs_count * 2;
    off = (off + 15) & ~15;
    L.zc_off = off;
    if (hz) off += NT * 16 * gs_count * 2;
    off = (off + 15) & ~15;
    L.red_off = off;
    off += waves * NT * 16 * M * 4;
    L.bytes = (off + 15) & ~15;
    return L;
}

/* Copies the raw scale (or zero) bits of 16 consecutive rows starting at
 * row r0 of a [rows][G] fp16 table, groups [g0, g0 + gn), into dst[16][gn]. */
__device__ __forceinline__ void stage_groups(uint16_t* dst, const uint16_t* tab, int G, int r0,
                                             int g0, int gn) {
    for (int i = threadIdx.x; i < 16 * gn; i += blockDim.x) {
        const int r = i / gn, g = i - r * gn;
        dst[i] = gptr(tab)[(size_t)(r0 + r) * G + g0 + g];
    }
}

/* A cooperative global -> LDS copy in two phases, so that its loads can be
 * issued before a wave's weight loads: loads return in order, so anything
 * issued after the weights would wait for all of them. The copy is `rows`
 * rows of `w16` 16-byte pieces; piece q of row r comes from
 * src + r * src_stride + 16 q and goes to dst + r * dst_stride + 16 q. Each
 * thread handles at most CNT pieces (ok() tells whether the copy fits);
 * out-of-range slots load a clamped in-range piece and store nothing. */
/* One 16-byte global -> LDS load per lane: lane l's 16 bytes from src land
 * at dst + 16 l (dst is the same for the whole wave). The load counts on
 * vmcnt like any other; the LDS bytes are there once it has returned. */
__device__ __forceinline__ void lds_load16(const void* src, void* dst) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
}

template <int CNT>
struct Stage16 {
    u4 v[CNT];
    int rows, w16;

    __device__ static bool ok(int rows_, int w16_) {
        return rows_ * w16_ <= CNT * (int)blockDim.x;
    }
    __device__ __forceinline__ void issue(const uint8_t* src, size_t src_stride, int rows_,
                                          int w16_) {
        rows = rows_;
        w16 = w16_;
        const int total = rows * w16;
#pragma unroll
        for (int c = 0; c < CNT; c++) {
            const int i = min((int)threadIdx.x + c * (int)blockDim.x, total - 1);
            const int r = i / w16, q = i - r * w16;
            v[c] = *gptr((const u4*)(src + r * src_stride + 16 * q));
        }
    }
    /* perm: permute each piece (8 fp16) into unpack8_magic slot order with
     * odd elements divided by 16 (a power-of-two scale: exact for
     * |x| >= 2^-10; below that x / 16 is an fp16 subnormal and keeps fewer
     * bits, an error below 2^-24 absolute). */
    template <bool PERM>
    __device__ __forceinline__ void commit(uint8_t* dst, int dst_stride) const {
        const int total = rows * w16;
        const f16 sixteenth = (f16)0.0625f;
#pragma unroll
        for (int c = 0; c < CNT; c++) {
            const int i = (int)threadIdx.x + c * (int)blockDim.x;
            if (i < total) {
                const int r = i / w16, q = i - r * w16;
                u4 o = v[c];
                if (PERM) {
                    const h8 in = __builtin_bit_cast(h8, v[c]);
                    h8 pv;
#pragma unroll
                    for (int e = 0; e < 8; e++) pv[perm_slot(e)] = (e & 1) ? in[e] * sixteenth : in[e];
                    o = __builtin_bit_cast(u4, pv);
                }
                *(u4*)(dst + r * dst_stride + 16 * q) = o;
            }
        }
    }
};

/* Issues the weight loads of the NB blocks b_first .. b_first + NB - 1 of NT
 * row tiles (absolute block indices, each clamped to b_clamp so that every
 * address is in the matrix). A wave issues all of them before anything
 * else: fully unrolled, so no load result is carried across a loop and the
 * compiler never has to copy (and therefore wait on) an in-flight
 * register. */
template <int NT, int NB>
__device__ __forceinline__ void load_blocks(const uint8_t* const (&wp)[NT], int b_first,
                                            int b_clamp, u4 (&w)[NB][NT]) {
#pragma unroll
    for (int p = 0; p < NB; p++) {
        const int bb = min(b_first + p, b_clamp);
#pragma unroll
        for (int s = 0; s < NT; s++) w[p][s] = *gptr((const u4*)(wp[s] + (size_t)bb * 64));
    }
}

/* Computes the preloaded blocks b_first .. b_first + NB - 1 into tot; the
 * ones at or past b_end are padding (zero scale). Activations and scales
 * come from the LDS image, whose K range starts at block xb0 and whose
 * groups start at g_lo. */
template <int M, int NG, int NT, int NB, bool HZ>
__device__ __forceinline__ void compute_blocks(const u4 (&w)[NB][NT], const uint8_t* smem,
                                               const LdsMap& L, int b_first, int b_end, int xb0,
                                               int g_lo, int gshift, int col, int j,
                                               uint32_t m_lo, uint32_t m_hi, uint32_t one024,
                                               float (&tot)[NT][M]) {
    /* A VALU op reads at most one scalar operand on this target: with the
     * masks in SGPRs every bitfield insert of the unpack splits into an and
     * plus an or. Pinning them to VGPRs (an empty asm emits no instruction)
     * lets each output dword be one v_and_or_b32. */
    asm volatile("" : "+v"(m_lo));
    asm volatile("" : "+v"(m_hi));
    asm volatile("" : "+v"(one024));
    const uint16_t* xs = (const uint16_t*)(smem + L.x_off) + (col < M ? col : 0) * L.XR + 32 * j;
    const uint16_t* scs = (const uint16_t*)(smem + L.sc_off) + col * L.GS;
    const uint16_t* zcs = (const uint16_t*)(smem + L.zc_off) + col * L.GS;
    const int gamma = (j * NG) / 4;
#pragma unroll
    for (int p = 0; p < NB; p++) {
        const int b = b_first + p;
        const bool live = b < b_end;
        const int bc = live ? b : xb0;
        h8 xa[4];
#pragma unroll
        for (int t = 0; t < 4; t++) xa[t] = *(const h8*)(xs + (bc - xb0) * 128 + 8 * t);
        float sc[NT][NG], zc[NT][NG];
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const int gi = ((bc * NG + g) >> gshift) - g_lo;
#pragma unroll
            for (int s = 0; s < NT; s++) {
                sc[s][g] = half_bits_to_float(scs[s * 16 * L.GS + gi]);
                zc[s][g] = HZ ? half_bits_to_float(zcs[s * 16 * L.GS + gi]) : 0.0f;
            }
        }
        block_step<M, NG, NT, HZ>(xa, w[p], gamma, sc, zc, live, m_lo, m_hi, one024, tot);
    }
}

/* Copies the first `len` elements of M activation rows (fp16, row stride
 * K) into the LDS x image, permuting each 8-element block into
 * unpack8_magic slot order with odd elements divided by 16 (exact for
 * |x| >= 2^-10, see Stage16::commit). 16-byte accesses. */
template <int M>
__device__ __forceinline__ void stage_x_perm(uint8_t* smem, const LdsMap& L,
                                             const uint16_t* __restrict__ src, int K, int len) {
    uint16_t* xs = (uint16_t*)(smem + L.x_off);
    const int per_row = len / 8;
    const f16 sixteenth = (f16)0.0625f;
    for (int i = threadIdx.x; i < M * per_row; i += blockDim.x) {
        const int v = i / per_row, c = i - v * per_row;
        const h8 in = __builtin_bit_cast(h8, *(const u4*)(src + (size_t)v * K + c * 8));
        h8 o;
#pragma unroll
        for (int e = 0; e < 8; e++) o[perm_slot(e)] = (e & 1) ? in[e] * sixteenth : in[e];
        *(h8*)(xs + v * L.XR + c * 8) = o;
    }
}

/* ======================================================================= */
/* gate/up + SiLU                                                           */
/* ======================================================================= */

/* One gate/up workgroup: TILES gate + TILES up row tiles starting at row
 * 16 TILES rt of unique expert u, over K blocks [nw NB split, nw NB (split
 * + 1)) of the hidden axis (split 0 of 1: the full K), waves split that
 * range. In the fused launch (FUSED) h' is written with device-coherent
 * stores and, once they are acknowledged, the workgroup counts itself on
 * its wave unit's counter (the down waves of the same launch poll it).
 * With P.gsplit > 1 workgroups sharing a row tile (TILES = 1), each stores
 * its gate and up partial sums with device-coherent stores and counts
 * itself on the tile's counter; the last to arrive adds the partials in
 * split order and finishes the tile. */
template <int M, int NG, int TILES, int NB, bool HZ, bool FUSED>
__device__ __forceinline__ void gateup_tile(const DecodeParams& P, int u, int rt, int split,
                                            uint8_t* smem) {
    constexpr int NT = 2 * TILES;
    /* both loads in one round trip (slot u < max_u always exists) */
    const int n_u = *P.n_unique;
    const uint8_t* blob = P.ublob[u];
    if (u >= n_u) return;
    const int K = P.hidden;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int col = lane & 15, j = lane >> 4;
    const int r0 = rt * 16 * TILES;
    const int nblk = K >> 7;
    const int G = K / P.gs;
    /* wave w owns blocks [xb0 + NB w, xb0 + NB w + NB); the host launches
     * min(4, ceil(nblk / NB)) waves and gsplit = ceil(nblk / (waves NB)) */
    const int xb0 = split * nw * NB;
    const int xlen = min(nw * NB, nblk - xb0);      /* blocks of this split */
    if (xlen <= 0) return;   /* the launchers never make an empty split */
    const int b0 = xb0 + wave * NB, b1 = min(b0 + NB, nblk);
    const LdsMap L = lds_map(M, NT, min(K, nw * NB * 128), G, HZ, nw);

    const uint8_t* wp[NT];
#pragma unroll
    for (int s = 0; s < NT; s++) {
        const int mat = s < TILES ? 0 : 1;
        wp[s] = blob + P.p_off[mat] + (size_t)(r0 + 16 * (s % TILES) + col) * (K / 2) + 16 * j;
    }
    /* Order of issue: activations and the tile's scales (small, read by
     * the whole workgroup), then all of this wave's weights; the LDS writes
     * then wait only for the former. The scales (and zeros) of 16
     * consecutive rows are one contiguous run of 32 G bytes. */
    constexpr int XCNT = (M * NB + 3) / 4;
    constexpr int SCNT = NB * NG / 16 > 0 ? NB * NG / 16 : 1;
    Stage16<XCNT> sx;
    Stage16<SCNT> ssc[NT], szc[NT];
    const bool fast = Stage16<XCNT>::ok(M, xlen * 16) && Stage16<SCNT>::ok(1, 2 * G);
    if (fast) {
        sx.issue((const uint8_t*)(P.xh + xb0 * 128), (size_t)K * 2, M, xlen * 16);
#pragma unroll
        for (int s = 0; s < NT; s++) {
            const int mat = s < TILES ? 0 : 1;
            const size_t roff = (size_t)(r0 + 16 * (s % TILES)) * G * 2;
            ssc[s].issue(blob + P.s_off[mat] + roff, 0, 1, 2 * G);
            if (HZ) szc[s].issue(blob + P.z_off[mat] + roff, 0, 1, 2 * G);
        }
    }
    u4 w[NB][NT];
    load_blocks<NT, NB>(wp, b0, nblk - 1, w);
    if (fast) {
        sx.template commit<true>(smem + L.x_off, L.XR * 2);
#pragma unroll
        for (int s = 0; s < NT; s++) {
            ssc[s].template commit<false>(smem + L.sc_off + s * 32 * G, 0);
            if (HZ) szc[s].template commit<false>(smem + L.zc_off + s * 32 * G, 0);
        }
    } else {
        stage_x_perm<M>(smem, L, P.xh + xb0 * 128, K, xlen * 128);
#pragma unroll
        for (int s = 0; s < NT; s++) {
            const int mat = s < TILES ? 0 : 1;
            const int rt = r0 + 16 * (s % TILES);
            stage_groups((uint16_t*)(smem + L.sc_off) + s * 16 * G,
                         (const uint16_t*)(blob + P.s_off[mat]), G, rt, 0, G);
            if (HZ)
                stage_groups((uint16_t*)(smem + L.zc_off) + s * 16 * G,
                             (const uint16_t*)(blob + P.z_off[mat]), G, rt, 0, G);
        }
    }
    __syncthreads();

    float tot[NT][M];
#pragma unroll
    for (int s = 0; s < NT; s++)
#pragma unroll
        for (int v = 0; v < M; v++) tot[s][v] = 0.0f;
    compute_blocks<M, NG, NT, NB, HZ>(w, smem, L, b0, b1, xb0, 0, P.gshift, col, j, P.m_lo,
                                      P.m_hi, P.one024, tot);

    float* red = (float*)(smem + L.red_off);
    if (lane < 16) {
#pragma unroll
        for (int s = 0; s < NT; s++)
#pragma unroll
            for (int v = 0; v < M; v++) red[((wave * NT + s) * 16 + col) * M + v] = tot[s][v];
    }
    __syncthreads();
    /* Wave 0 finishes the tile (at most 64 outputs, one per lane); the
     * other waves end here, so their registers take new workgroups while
     * wave 0's hand-off round trips run. No barrier follows. */
    static_assert(TILES * 16 * M <= 64, "one wave finishes the tile");
    if (wave != 0) return;
    const int n_split = TILES == 1 ? P.gsplit : 1;
    const int tile_id = u * (P.inter / (16 * TILES)) + rt;
    if (n_split > 1) {
        /* K-split: publish this split's sums (lane = 16-row index * M +
         * token); the last arrival finishes */
        if (lane < 16 * M) {
            const int o = lane, v = o % M, c = o / M;
            float g = 0.0f, up = 0.0f;
            for (int ww = 0; ww < nw; ww++) {
                g += red[((ww * NT) * 16 + c) * M + v];
                up += red[((ww * NT + 1) * 16 + c) * M + v];
            }
            float* dst = P.gpart + ((size_t)tile_id * n_split + split) * 32 * M;
            if (FUSED || !P.gfinish) {
                __hip_atomic_store(dst + o, g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(dst + 16 * M + o, up, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            } else {
                dst[o] = g;
                dst[16 * M + o] = up;
            }
        }
        /* With P.gfinish (separate gate/up launch), gateup_finish_kernel,
         * launched next, adds the splits, so the workgroup ends with its
         * stores: the hand-off round trips below hold the workgroup's
         * slot for microseconds. */
        if (!FUSED && P.gfinish) return;
        __builtin_amdgcn_s_waitcnt(0);   /* the wave's partial stores are acknowledged */
        int last = 0;
        if (lane == 0)
            last = __hip_atomic_fetch_add(P.gcnt + tile_id, 1, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT) == n_split - 1;
        if (!__builtin_amdgcn_readfirstlane(last)) return;
    }
    if (lane < TILES * 16 * M) {
        const int o = lane;
        const int v = o % M, rc = o / M, q = rc / 16, c = rc % 16;
        float g = 0.0f, up = 0.0f;
        if (n_split > 1) {
            const float* src = P.gpart + (size_t)tile_id * n_split * 32 * M;
            for (int sp = 0; sp < n_split; sp++) {
                g += __hip_atomic_load(src + sp * 32 * M + o, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                up += __hip_atomic_load(src + sp * 32 * M + 16 * M + o, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
            }
        } else {
            for (int ww = 0; ww < nw; ww++) {
                g += red[((ww * NT + q) * 16 + c) * M + v];
                up += red[((ww * NT + TILES + q) * 16 + c) * M + v];
            }
        }
        const float h = silu_f(g) * up * P.uw[u * 4 + v];
        const int r = r0 + 16 * q + c;
        const int e = r & 7;
        f16 hv = (f16)((e & 1) ? h * 0.0625f : h);
        uint16_t* dst = P.hperm + ((size_t)v * P.max_u + u) * P.inter + (r & ~7) + perm_slot(e);
        if (FUSED)
            __hip_atomic_store(dst, __builtin_bit_cast(uint16_t, hv), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        else
            *dst = __builtin_bit_cast(uint16_t, hv);
    }
    if (FUSED) {
        __builtin_amdgcn_s_waitcnt(0);   /* the wave's h' stores are acknowledged */
        if (lane == 0)
            __hip_atomic_fetch_add(P.hcnt + (u * P.upe + r0 / (DEC_UNIT_BLOCKS * 128)) *
                                                DEC_HCNT_STRIDE, 1,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

/* After a K-split gate/up launch: h' of every (unique expert, row, token)
 * from the splits' partial sums, added in split order from zero as the
 * fused launch's last arrival adds them (so both give identical h'). One
 * thread per output; grid (max_u * inter * M / 256). */
template <int M>
__global__ __launch_bounds__(256) void gateup_finish_kernel(const DecodeParams P) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int n_rt = P.inter / 16;
    const int tile_id = i / (16 * M), o = i - tile_id * 16 * M;
    const int u = tile_id / n_rt;
    if (u >= *P.n_unique) return;
    const int rt = tile_id - u * n_rt;
    const int v = o % M, c = o / M;
    const int n_split = P.gsplit;
    const float* src = P.gpart + (size_t)tile_id * n_split * 32 * M;
    float g = 0.0f, up = 0.0f;
    for (int sp = 0; sp < n_split; sp++) {
        g += src[sp * 32 * M + o];
        up += src[sp * 32 * M + 16 * M + o];
    }
    const float h = silu_f(g) * up * P.uw[u * 4 + v];
    const int r = rt * 16 + c;
    const int e = r & 7;
    const f16 hv = (f16)((e & 1) ? h * 0.0625f : h);
    P.hperm[((size_t)v * P.max_u + u) * P.inter + (r & ~7) + perm_slot(e)] =
        __builtin_bit_cast(uint16_t, hv);
}

/* grid (inter / (16 TILES) * gsplit, max_u): gate/up of unique expert
 * blockIdx.y, row tile blockIdx.x / gsplit, K split blockIdx.x % gsplit. */
template <int M, int NG, int TILES, int NB, bool HZ>
__global__ __launch_bounds__(64 * DEC_MAX_WAVES) void gateup_kernel(const DecodeParams P) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    gateup_tile<M, NG, TILES, NB, HZ, false>(P, blockIdx.y, blockIdx.x / P.gsplit,
                                             blockIdx.x % P.gsplit, smem);
}

/* ======================================================================= */
/* down (per expert and K chunk) + combine                                  */
/* ======================================================================= */

/* out[v][r] (+)= y in fp32 and/or fp16. */
__device__ __forceinline__ void store_out(const DecodeParams& P, size_t i, float y) {
    if (P.out32) {
        if (P.accumulate) y += P.out32[i];
        P.out32[i] = y;
    }
    if (P.out16) P.out16[i] = __builtin_bit_cast(uint16_t, (f16)y);
}

/* LDS image of one down wave: x [M][1024 + 32] (its unit's h', rows padded
 * so tokens fall in different banks), sc [16][GMAX] and zc [16][GMAX] raw
 * fp16 scale and zero bits of the tile's rows for the unit's groups. */
__host__ __device__ inline LdsMap down_wave_map(int M, int gmax, bool hz, int wave, int nw) {
    LdsMap L;
    L.XR = DEC_UNIT_BLOCKS * 128 + 32;
    L.GS = gmax;
    int bytes = M * L.XR * 2;
    bytes = (bytes + 15) & ~15;
    const int sc = bytes;
    bytes += 16 * gmax * 2;
    bytes = (bytes + 15) & ~15;
    const int zc = bytes;
    if (hz) bytes += 16 * gmax * 2;
    bytes = (bytes + 15) & ~15;
    L.x_off = wave * bytes;
    L.sc_off = L.x_off + sc;
    L.zc_off = L.x_off + zc;
    L.red_off = nw * bytes;
    L.bytes = L.red_off + nw * 16 * M * 4;
    return L;
}

/* Down part of the fused launch. Workgroup (row tile rt, chunk q) of nw
 * waves covers wave units [nw q, nw q + nw) of the concatenated K axis and
 * computes part[q][v][row] = sum over its units of down_u[row, unit] .
 * h'_u[v][unit] (routing weight already folded into h'). The last of the row
 * tile's n_q workgroups to arrive adds all of the tile's partials in chunk
 * order and writes the output, so the result is deterministic. The hand-off
 * needs no cache write-back: partials are stored and loaded with
 * device-coherent accesses, every store is acknowledged before the arrival
 * is counted, and the counters are zeroed by the prep kernel of the same
 * call. Each wave first waits until every gate/up workgroup of its unit has
 * counted itself (a bounded poll: those workgroups come earlier in the grid
 * and wait on nothing), then reads h' with device-coherent loads. */
template <int M, int NG, bool HZ>
__device__ __forceinline__ void down_tile(const DecodeParams& P, int q, int rt, uint8_t* smem) {
    constexpr int NB = DEC_UNIT_BLOCKS;
    constexpr int GMAX = NB * NG;
    const int r0 = rt * 16;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int col = lane & 15, j = lane >> 4;
    const int K = P.inter, H = P.hidden;
    const int nblk = K >> 7;
    const int gu = q * nw + wave;
    const int u = min(gu / P.upe, P.max_u - 1);
    /* both loads in one round trip */
    const int n_u = *P.n_unique;
    const uint8_t* blob = P.ublob[u];
    const int n_units = n_u * P.upe;
    const int n_q = (n_units + nw - 1) / nw;
    if (q >= n_q) {
        /* nothing routed: one workgroup per row tile writes the empty sum */
        if (n_u == 0 && q == 0)
            for (int o = threadIdx.x; o < 16 * M; o += blockDim.x)
                store_out(P, (size_t)(o / 16) * H + r0 + o % 16, 0.0f);
        return;
    }
    /* a wave past the last unit (its slot u may hold no blob) loads nothing */
    const bool live = gu < n_units;
    const int lb0 = live ? (gu - u * P.upe) * NB : 0;
    const int lb1 = live ? min(lb0 + NB, nblk) : 0;
    const int nb = lb1 - lb0;
    const int G = K / P.gs;
    const int g_lo = (lb0 * NG) >> P.gshift;
    const int gn = nb > 0 ? ((((lb1 * NG) - 1) >> P.gshift) + 1 - g_lo) : 0;
    const LdsMap L = down_wave_map(M, GMAX, HZ, wave, nw);

    float tot[1][M];
#pragma unroll
    for (int v = 0; v < M; v++) tot[0][v] = 0.0f;
    if (live) {
    /* Order of issue (loads return in order): the first poll of the unit's
     * counter, the scales and the weights, then the wait for the counter
     * (its load returns first), then h' (after the poll, so it sees every
     * gate/up store): the poll's round trip overlaps the weight stream
     * instead of preceding it. */
    int hc = __hip_atomic_load(P.hcnt + gu * DEC_HCNT_STRIDE, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    constexpr int XC = NB / 4;   /* 16-byte pieces of the unit's h' per lane and token */
    u4 xv[M][XC];
    const uint16_t* hsrc = P.hperm + (size_t)u * K + lb0 * 128;
    auto load_h = [&]() {
#pragma unroll
        for (int v = 0; v < M; v++)
#pragma unroll
            for (int c = 0; c < XC; c++) {
                const int i = min(lane + 64 * c, nb * 16 - 1);
                const uint16_t* src = hsrc + (size_t)v * P.max_u * K + i * 8;
                const uint64_t a = __hip_atomic_load((const uint64_t*)src, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
                const uint64_t b = __hip_atomic_load((const uint64_t*)src + 1, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
                xv[v][c] = (u4){(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b,
                                (uint32_t)(b >> 32)};
            }
    };
    uint16_t* xs = (uint16_t*)(smem + L.x_off);
    constexpr int SCNT = (16 * GMAX + 63) / 64;
    uint16_t sv[SCNT], zv[SCNT];
    const uint16_t* stab = (const uint16_t*)(blob + P.s_off[2]);
    const uint16_t* ztab = (const uint16_t*)(blob + P.z_off[2]);
#pragma unroll
    for (int c = 0; c < SCNT; c++) {
        const int i = lane + 64 * c;
        const int ii = min(i, 16 * gn - 1);
        const int rr = ii / gn, gg = ii - rr * gn;
        const size_t at = (size_t)(r0 + rr) * G + g_lo + gg;
        sv[c] = gptr(stab)[at];
        zv[c] = HZ ? gptr(ztab)[at] : (uint16_t)0;
    }
    const uint8_t* wp[1] = {blob + P.p_off[2] + (size_t)(r0 + col) * (K / 2) + 16 * j};
    u4 w[NB][1];
    load_blocks<1, NB>(wp, lb0, lb1 - 1, w);
    /* h' of this unit: written by nb * 8 gate/up workgroups */
    const int want = nb * 8 + P.poll_extra;
    int polls = 0;
    while (hc < want && polls < P.poll_limit) {
        __builtin_amdgcn_s_sleep(DEC_POLL_SLEEP);
        polls++;
        hc = __hip_atomic_load(P.hcnt + gu * DEC_HCNT_STRIDE, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    const bool gave_up = hc < want;
    load_h();

#pragma unroll
    for (int v = 0; v < M; v++)
#pragma unroll
        for (int c = 0; c < XC; c++) {
            const int i = lane + 64 * c;
            if (i < nb * 16) *(u4*)(xs + v * L.XR + i * 8) = xv[v][c];
        }
    uint16_t* ss = (uint16_t*)(smem + L.sc_off);
    uint16_t* zs = (uint16_t*)(smem + L.zc_off);
#pragma unroll
    for (int c = 0; c < SCNT; c++) {
        const int i = lane + 64 * c;
        if (i < 16 * gn) {
            const int rr = i / gn, gg = i - rr * gn;
            ss[rr * GMAX + gg] = sv[c];
            if (HZ) zs[rr * GMAX + gg] = zv[c];
        }
    }
    /* the wave reads only its own region: LDS operations of one wave run in
     * order, so no barrier; keep the compiler from hoisting the reads */
    __builtin_amdgcn_wave_barrier();
    compute_blocks<M, NG, 1, NB, HZ>(w, smem, L, lb0, lb1, lb0, g_lo, P.gshift, col, j,
                                     P.m_lo, P.m_hi, P.one024, tot);
    if (gave_up) {
        /* the unit's h' may be stale: poison the row tile's sums */
#pragma unroll
        for (int v = 0; v < M; v++) tot[0][v] = __builtin_nanf("");
        if (lane == 0) dec_report(P.status, DEC_STATUS_DOWN_WAIT);
    }
    }

    float* red = (float*)(smem + L.red_off);
    if (lane < 16) {
#pragma unroll
        for (int v = 0; v < M; v++) red[(wave * 16 + col) * M + v] = tot[0][v];
    }
    __syncthreads();
    /* Wave 0 finishes (16 M <= 64 outputs); the other waves end here and
     * free their registers for new workgroups. No barrier follows. */
    if (wave != 0) return;
    if (lane < 16 * M) {
        const int o = lane;
        const int v = o % M, cc = o / M;
        float y = 0.0f;
        for (int ww = 0; ww < nw; ww++) y += red[(ww * 16 + cc) * M + v];
        __hip_atomic_store(P.part + ((size_t)q * M + v) * H + r0 + cc, y, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);   /* the wave's partial stores are acknowledged */
    int last = 0;
    if (lane == 0)
        last = __hip_atomic_fetch_add(P.tile_cnt + rt, 1, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == n_q - 1;
    if (!__builtin_amdgcn_readfirstlane(last)) return;
    constexpr int MAXQ = 16;
    if (lane < 16 * M) {
        const int o = lane;
        const int v = o / 16, r = r0 + o % 16;
        const float* src = P.part + (size_t)v * H + r;
        const size_t stride = (size_t)M * H;
        float y = 0.0f;
        for (int q0 = 0; q0 < n_q; q0 += MAXQ) {
            float t[MAXQ];
#pragma unroll
            for (int qq = 0; qq < MAXQ; qq++)
                t[qq] = q0 + qq < n_q ? __hip_atomic_load(src + (size_t)(q0 + qq) * stride,
                                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                      : 0.0f;
#pragma unroll
            for (int qq = 0; qq < MAXQ; qq++) y += t[qq];
        }
        store_out(P, (size_t)v * H + r, y);
    }
}

/* LDS image of a workgroup of the separate down launch: x [M][1024 + 32]
 * (the unit's h', shared by the waves), then per wave sc [16][GMAX] and
 * zc [16][GMAX] (its row tile's raw scale and zero bits). */
__host__ __device__ inline LdsMap down_rows_map(int M, int gmax, bool hz, int wave) {
    LdsMap L;
    L.XR = DEC_UNIT_BLOCKS * 128 + 32;
    L.GS = gmax;
    L.x_off = 0;
    const int xb = (M * L.XR * 2 + 15) & ~15;
    const int tb = (16 * gmax * 2 + 15) & ~15;
    const int pw = hz ? 2 * tb : tb;
    L.sc_off = xb + wave * pw;
    L.zc_off = L.sc_off + tb;
    L.red_off = 0;
    L.bytes = xb + DN_WAVES * pw;
    return L;
}

/* The down projection alone (two launches): workgroup (row group
 * blockIdx.x, wave unit blockIdx.y) stages the unit's h' once in LDS for
 * its DN_WAVES waves, and wave w computes rows r = 16 (DN_WAVES blockIdx.x
 * + w) + [0, 16) of part[unit][v][r] = down_u[r, unit's K range] .
 * h'_u[v][unit's K range] (routing weight folded into h'). It stores them
 * and ends: no workgroup waits on another, and down_combine_kernel adds the
 * units in unit order. Sharing h' across the row tiles of a unit keeps the
 * workgroup's LDS small (10 KB for 4 tokens), so LDS no longer caps the
 * workgroups per CU below what the registers allow. */
template <int M, int NG, bool HZ>
__global__ __launch_bounds__(64 * DN_WAVES)
__attribute__((amdgpu_waves_per_eu(NG == 1 ? (HZ ? 4 : 5) : (NG == 2 && !HZ ? 2 : 1))))
void down_kernel(const DecodeParams P) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int NB = DEC_UNIT_BLOCKS;
    constexpr int GMAX = NB * NG;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, j = lane >> 4;
    const int K = P.inter, H = P.hidden;
    const int nblk = K >> 7;
    const int gu = blockIdx.y;
    const int u = min(gu / P.upe, P.max_u - 1);
    /* both loads in one round trip (slot u < max_u always exists) */
    const int n_u = *P.n_unique;
    const uint8_t* blob = P.ublob[u];
    if (gu >= n_u * P.upe) return;
    const int r0 = (blockIdx.x * DN_WAVES + wave) * 16;
    const int lb0 = (gu - u * P.upe) * NB;
    const int lb1 = min(lb0 + NB, nblk);
    const int nb = lb1 - lb0;
    const int G = K / P.gs;
    const int g_lo = (lb0 * NG) >> P.gshift;
    const int gn = (((lb1 * NG) - 1) >> P.gshift) + 1 - g_lo;
    const LdsMap L = down_rows_map(M, GMAX, HZ, wave);

    /* Order of issue (loads return in order): the unit's h' straight into
     * LDS (2 M pieces of 1 KB spread over the waves; pieces past a short
     * last unit repeat its last 16 bytes, read only by padding blocks of
     * zero scale), the row tile's scales, then its weights. */
    uint16_t* xs = (uint16_t*)(smem + L.x_off);
    const uint16_t* hsrc = P.hperm + (size_t)u * K + lb0 * 128;
    static_assert(DEC_UNIT_BLOCKS * 128 * 2 == 2 * 1024,
                  "a unit's h' per token is staged as two 1 KB pieces");
    constexpr int PCS = (2 * M + DN_WAVES - 1) / DN_WAVES;
#pragma unroll
    for (int k = 0; k < PCS; k++) {
        const int pc = wave + k * DN_WAVES;
        if (pc < 2 * M) {
            const int v = pc >> 1, c = pc & 1;
            const int i = min(lane + 64 * c, nb * 16 - 1);
            lds_load16(hsrc + (size_t)v * P.max_u * K + i * 8,
                       (uint8_t*)(xs + v * L.XR) + 1024 * c);
        }
    }
    constexpr int SCNT = (16 * GMAX + 63) / 64;
    uint16_t sv[SCNT], zv[SCNT];
    const uint16_t* stab = (const uint16_t*)(blob + P.s_off[2]);
    const uint16_t* ztab = (const uint16_t*)(blob + P.z_off[2]);
#pragma unroll
    for (int c = 0; c < SCNT; c++) {
        const int i = min(lane + 64 * c, 16 * gn - 1);
        const int rr = i / gn, gg = i - rr * gn;
        const size_t at = (size_t)(r0 + rr) * G + g_lo + gg;
        sv[c] = gptr(stab)[at];
        zv[c] = HZ ? gptr(ztab)[at] : (uint16_t)0;
    }
    __builtin_amdgcn_sched_barrier(0);   /* the scale loads stay ahead of the weights */
    const uint8_t* wp[1] = {blob + P.p_off[2] + (size_t)(r0 + col) * (K / 2) + 16 * j};
    u4 w[NB][1];
    load_blocks<1, NB>(wp, lb0, lb1 - 1, w);

    /* the scales return after h' (in order), so once they are written
     * every wave's h' pieces are in LDS */
    uint16_t* ss = (uint16_t*)(smem + L.sc_off);
    uint16_t* zs = (uint16_t*)(smem + L.zc_off);
#pragma unroll
    for (int c = 0; c < SCNT; c++) {
        const int i = lane + 64 * c;
        if (i < 16 * gn) {
            const int rr = i / gn, gg = i - rr * gn;
            ss[rr * GMAX + gg] = sv[c];
            if (HZ) zs[rr * GMAX + gg] = zv[c];
        }
    }
    __syncthreads();

    float tot[1][M];
#pragma unroll
    for (int v = 0; v < M; v++) tot[0][v] = 0.0f;
    compute_blocks<M, NG, 1, NB, HZ>(w, smem, L, lb0, lb1, lb0, g_lo, P.gshift, col, j,
                                     P.m_lo, P.m_hi, P.one024, tot);
    if (lane < 16) {
#pragma unroll
        for (int v = 0; v < M; v++) P.part[((size_t)gu * M + v) * H + r0 + col] = tot[0][v];
    }
}

/* After the separate down launch: out[v][r] = the sum of part[unit][v][r]
 * over the call's wave units. Four lanes per output: lane k adds the units
 * [k Q, k Q + Q) in unit order (Q = ceil(units / 4)), all its loads in
 * flight at once for up to 4 DEC_COMBINE_BATCH units, then the first lane
 * adds the four partial sums in lane order, so every call sums in the same
 * order. */
#define DEC_COMBINE_LANES 4
#define DEC_COMBINE_BATCH 32
template <int M>
__global__ __launch_bounds__(256) void down_combine_kernel(const DecodeParams P) {
    const int g = blockIdx.x * 256 + threadIdx.x;
    const int i = g / DEC_COMBINE_LANES, k = g % DEC_COMBINE_LANES;
    const bool live = i < M * P.hidden;
    const int n_units = *P.n_unique * P.upe;
    const int qn = (n_units + DEC_COMBINE_LANES - 1) / DEC_COMBINE_LANES;
    const int q_lo = k * qn, q_hi = min(q_lo + qn, n_units);
    const float* src = P.part + (live ? i : 0);
    const size_t stride = (size_t)M * P.hidden;
    float y = 0.0f;
    for (int q0 = q_lo; q0 < q_hi; q0 += DEC_COMBINE_BATCH) {
        float t[DEC_COMBINE_BATCH];
#pragma unroll
        for (int qq = 0; qq < DEC_COMBINE_BATCH; qq++)
            t[qq] = q0 + qq < q_hi ? src[(size_t)(q0 + qq) * stride] : 0.0f;
#pragma unroll
        for (int qq = 0; qq < DEC_COMBINE_BATCH; qq++) y += t[qq];
    }
    /* every lane takes part in the shuffles (no return before them) */
    float tot = __shfl(y, 0, DEC_COMBINE_LANES);
#pragma unroll
    for (int q = 1; q < DEC_COMBINE_LANES; q++) tot += __shfl(y, q, DEC_COMBINE_LANES);
    if (live && k == 0) store_out(P, i, tot);
}

/* One launch for gate/up and down: the first max_u * inter / 16 * gsplit
 * workgroups are gate/up workgroups (expert-major, then row tile, then K
 * split, so an expert's h' completes early and the splits of a row tile
 * arrive together),
 * the rest down workgroups (chunk-major); a workgroup has as many waves as
 * gate/up needs, which is also the down chunk's unit count. Down waves wait
 * only on workgroups earlier in the grid, which wait on nothing, so every
 * wait ends. */
template <int M, int NG, int NB, bool HZ>
__global__ __launch_bounds__(64 * DEC_MAX_WAVES) void expert_kernel(const DecodeParams P) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int n_rt = P.inter / 16;
    const int per_u = n_rt * P.gsplit;
    const int n_gu = P.max_u * per_u;
    const int b = blockIdx.x;
    if (b < n_gu) {
        const int u = b / per_u, r = b - u * per_u;
        gateup_tile<M, NG, 1, NB, HZ, true>(P, u, r / P.gsplit, r % P.gsplit, smem);
    } else {
        const int d = b - n_gu, n_ro = P.hidden / 16;
        down_tile<M, NG, HZ>(P, d / n_ro, d % n_ro, smem);
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
    if (hidden / 128 > 16 * DEC_MAX_WAVES) return hipErrorInvalidValue;   /* gate/up waves */
    const uint64_t gs = L->group_size;
    const bool gs_ok = gs >= 32 && (gs & (gs - 1)) == 0;
    if (!gs_ok || hidden % gs || inter % gs) return hipErrorInvalidValue;
    for (int m = 0; m < 3; m++) {
        const uint64_t n = (uint64_t)L->rows[m] * L->cols[m];
        /* blobs sit at 8 mod 16 (the reference's 120-byte header then
         * contiguous sections): every section starts 16-byte aligned */
        if ((L->packed_off[m] + 8) % 16 || (L->scales_off[m] + 8) % 16) return hipErrorInvalidValue;
        if (L->has_zeros && (L->zeros_off[m] + 8) % 16) return hipErrorInvalidValue;
        if (L->scales_off[m] < L->packed_off[m] + n / 2) return hipErrorInvalidValue;
        if (L->scales_off[m] % 2 || L->zeros_off[m] % 2) return hipErrorInvalidValue;
        if (L->has_zeros && L->zeros_off[m] < L->scales_off[m] + n / gs * 2)
            return hipErrorInvalidValue;
    }
    return hipSuccess;
}

struct WsLayout {
    size_t nu, epoch, tile_cnt, hcnt, ublob, uw, xconv, hperm, part, rwords, gcnt, gpart, total;
    int max_u, n_q_max;
};

/* Shape of the gate/up workgroups: 4 waves (fewer when the hidden axis has
 * fewer than 32 blocks); a row tile whose K axis needs more than 4 waves of
 * 8 blocks is split over gsplit workgroups of 4 waves x nb blocks
 * (DeepSeek-V3, 56 blocks: 2 x 4 x 7). Measured against one workgroup of 7
 * waves per row tile: DeepSeek-V3 one token 55.2 -> 51.5 us per layer. */
struct FusedShape {
    int waves, nb, gsplit;
};
static FusedShape fused_shape(int nblk) {
    FusedShape f;
    if (nblk <= 32) {
        f.nb = 8;
        f.waves = (nblk + 7) / 8;
        f.gsplit = 1;
        return f;
    }
    f.waves = 4;
    f.gsplit = (nblk + 31) / 32;
    f.nb = (nblk + 4 * f.gsplit - 1) / (4 * f.gsplit);
    if (f.nb != 7) f.nb = 8;   /* compiled: 7 or 8 blocks per wave */
    f.gsplit = (nblk + 4 * f.nb - 1) / (4 * f.nb);
    return f;
}

/* From this many tokens on, the separate gate/up launch hands its K-split
 * partials to gateup_finish_kernel instead of a last-arrival round trip
 * (measured, DeepSeek-V3 per layer: 4 tokens 187.3 -> 177.3 us; 3 tokens
 * 131.9 -> 132.1 and 2 tokens 93.1 -> 94.1, where the extra launch costs
 * what the round trips cost). */
#ifndef DEC_FINISH_MIN_TOKENS
#define DEC_FINISH_MIN_TOKENS 4
#endif
/* The first three regions sit at the same offsets for every layer shape,
 * so one workspace can serve calls of different shapes: the unique count
 * (offset 0) and the status word (DEC_STATUS_OFFSET), the routing epoch,
 * and the routing words, which every call of any shape only ever tags with
 * tokens up to the epoch. */
static WsLayout ws_layout(const WispExpertLayout* L, int M, int top_k, int has_shared) {
    WsLayout w;
    w.max_u = (has_shared ? 1 : 0) + M * top_k;
    size_t off = 0;
    w.nu = off; off += 256;
    w.epoch = off; off += 256;
    w.rwords = off; off += (size_t)DEC_MAX_TOKENS * DEC_ROUTE_MAX_EXPERTS * 8;
    w.tile_cnt = off; off = align_up(off + (size_t)(L->cols[0] / 16) * sizeof(int), 256);
    w.ublob = off; off = align_up(off + (size_t)w.max_u * sizeof(void*), 256);
    w.uw = off; off = align_up(off + (size_t)w.max_u * 4 * sizeof(float), 256);
    w.xconv = off; off = align_up(off + (size_t)M * L->cols[0] * 2, 256);
    w.hperm = off; off = align_up(off + (size_t)w.max_u * M * L->rows[0] * 2, 256);
    const int upe = (int)((L->rows[0] / 128 + DEC_UNIT_BLOCKS - 1) / DEC_UNIT_BLOCKS);
    /* partials: at most one chunk per wave unit (a one-wave workgroup) */
    w.n_q_max = w.max_u * upe;
    w.part = off; off = align_up(off + (size_t)w.n_q_max * M * L->cols[0] * 4, 256);
    w.hcnt = off; off = align_up(off + (size_t)w.max_u * upe * DEC_HCNT_STRIDE * sizeof(int), 256);
    const size_t gtiles = (size_t)w.max_u * (L->rows[0] / 16);
    const int gsplit = fused_shape((int)(L->cols[0] / 128)).gsplit;
    w.gcnt = off; off = align_up(off + (gsplit > 1 ? gtiles * sizeof(int) : 0), 256);
    w.gpart = off;
    off = align_up(off + (gsplit > 1 ? gtiles * gsplit * 32 * M * sizeof(float) : 0), 256);
    w.total = off;
    return w;
}

extern "C" size_t wisp_moe_decode_workspace_bytes(const WispExpertLayout* L, int n_tokens,
                                                  int top_k, int has_shared) {
    if (!L || n_tokens < 1 || n_tokens > DEC_MAX_TOKENS || top_k < 1 || top_k > DEC_MAX_TOPK)
        return 0;
    return ws_layout(L, n_tokens, top_k, has_shared).total;
}

template <int M, int NG, int TILES, int NB, bool HZ>
static hipError_t launch_gateup(const DecodeParams& P, int waves, hipStream_t s) {
    /* every K split of a row tile covers at least one block */
    const int nblk = P.hidden / 128, per = waves * NB;
    if (P.gsplit < 1 || (P.gsplit - 1) * per >= nblk || P.gsplit * per < nblk)
        return hipErrorInvalidValue;
    const int xk = P.hidden < waves * NB * 128 ? P.hidden : waves * NB * 128;
    const LdsMap L = lds_map(M, 2 * TILES, xk, P.hidden / P.gs, HZ, waves);
    auto k = gateup_kernel<M, NG, TILES, NB, HZ>;
    if (L.bytes > 65536)
        (void)hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  L.bytes);
    hipLaunchKernelGGL(k, dim3(P.inter / (16 * TILES) * P.gsplit, P.max_u), dim3(64 * waves),
                       L.bytes, s, P);
    return hipSuccess;
}

template <int M, int NG, bool HZ>
static hipError_t launch_down(const DecodeParams& P, hipStream_t s) {
    if (P.hidden % (16 * DN_WAVES) != 0) return hipErrorInvalidValue;
    const LdsMap L = down_rows_map(M, DEC_UNIT_BLOCKS * NG, HZ, 0);
    auto k = down_kernel<M, NG, HZ>;
    hipLaunchKernelGGL(k, dim3(P.hidden / (16 * DN_WAVES), P.max_u * P.upe), dim3(64 * DN_WAVES),
                       L.bytes, s, P);
    hipLaunchKernelGGL(down_combine_kernel<M>,
                       dim3((M * P.hidden * DEC_COMBINE_LANES + 255) / 256), dim3(256), 0, s, P);
    return hipSuccess;
}

/* gate/up and down in one launch (expert_kernel) */
template <int M, int NG, int NB, bool HZ>
static void launch_fused(DecodeParams P, int waves, hipStream_t s) {
    P.n_q_max = (P.max_u * P.upe + waves - 1) / waves;
    const int xk = P.hidden < waves * NB * 128 ? P.hidden : waves * NB * 128;
    const LdsMap Lg = lds_map(M, 2, xk, P.hidden / P.gs, HZ, waves);
    const LdsMap Ld = down_wave_map(M, DEC_UNIT_BLOCKS * NG, HZ, 0, waves);
    const int lds = Lg.bytes > Ld.bytes ? Lg.bytes : Ld.bytes;
    auto k = expert_kernel<M, NG, NB, HZ>;
    if (lds > 65536)
        (void)hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    const int grid = P.max_u * (P.inter / 16) * P.gsplit + P.n_q_max * (P.hidden / 16);
    hipLaunchKernelGGL(k, dim3(grid), dim3(64 * waves), lds, s, P);
}

/* One launch for gate/up and down for one token, in 4-wave workgroups
 * (fused_shape; P.gsplit was set from it). The fused kernel takes the
 * larger register budget of the two roles; with more tokens (more
 * registers) its down waves ran at half the occupancy of the down kernel
 * alone and the layer got slower (DeepSeek-V3 M=4: 281.6 against
 * 224.7 us), so M > 1 keeps two launches. */
template <int M, int NG, bool HZ>
static hipError_t launch_compute(const DecodeParams& P, hipStream_t s) {
    const FusedShape f = fused_shape(P.hidden / 128);
    if constexpr (M == 1) {
        ev_before(EV_GATEUP, s);
        if (f.nb == 7) launch_fused<M, NG, 7, HZ>(P, f.waves, s);
        else launch_fused<M, NG, 8, HZ>(P, f.waves, s);
        ev_after(EV_GATEUP, s);
        return hipSuccess;
    }
    ev_before(EV_GATEUP, s);
    const hipError_t e = f.nb == 7 ? launch_gateup<M, NG, 1, 7, HZ>(P, f.waves, s)
                                   : launch_gateup<M, NG, 1, 8, HZ>(P, f.waves, s);
    if (e != hipSuccess) return e;
    if (P.gfinish) {
        const int n = P.max_u * P.inter * M;   /* a multiple of 256: inter % 128 == 0 */
        hipLaunchKernelGGL(gateup_finish_kernel<M>, dim3(n / 256), dim3(256), 0, s, P);
    }
    ev_after(EV_GATEUP, s);
    ev_before(EV_DOWN, s);
    const hipError_t ed = launch_down<M, NG, HZ>(P, s);
    if (ed != hipSuccess) return ed;
    ev_after(EV_DOWN, s);
    return hipSuccess;
}

template <int M>
static hipError_t launch_ng(int ng, bool hz, const DecodeParams& P, hipStream_t s) {
    if (ng == 1) return hz ? launch_compute<M, 1, true>(P, s) : launch_compute<M, 1, false>(P, s);
    if (ng == 2) return hz ? launch_compute<M, 2, true>(P, s) : launch_compute<M, 2, false>(P, s);
    return hz ? launch_compute<M, 4, true>(P, s) : launch_compute<M, 4, false>(P, s);
}

/* Bounded-wait settings of every launch: the poll limit, and an amount
 * added to every wait target. Only wisp_amd__test_decode_wait changes them,
 * to make waits give up on purpose (every kernel still exits normally). */
static int g_poll_limit = DEC_POLL_LIMIT;
static int g_poll_extra = 0;

extern "C" void wisp_amd__test_decode_wait(int poll_limit, int extra) {
    g_poll_limit = poll_limit > 0 ? poll_limit : DEC_POLL_LIMIT;
    g_poll_extra = extra;
}

/* Shared body of the decode entry points: R.mode selects where the
 * routing comes from (see RouteArgs). x16: an fp16 copy of an fp32 x
 * (16-byte aligned, [M][hidden], each element the fp16 rounding of x's),
 * made by the caller; the experts read it and the prep kernel converts
 * nothing. */
static hipError_t decode_run(const void* const* d_expert_table, const void* d_shared_blob,
                             const WispExpertLayout* L, const void* d_x, int x_dtype, int M,
                             RouteArgs R, int top_k, int n_experts, void* d_workspace,
                             size_t workspace_bytes, int accumulate, float* d_out_f32,
                             wisp_half* d_out_f16, hipStream_t s,
                             const uint16_t* x16 = nullptr, bool keep_status = false) {
    if (wisp_expert_layout_check(L) != hipSuccess) return hipErrorInvalidValue;
    const WsLayout w = ws_layout(L, M, top_k, d_shared_blob != nullptr);
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
    {
        const int ngs = P.gs >= 128 ? P.gs : 128;   /* gs * NG */
        int sh = 0;
        while ((128 << sh) < ngs) sh++;
        P.gshift = sh;
    }
    P.upe = (P.inter / 128 + DEC_UNIT_BLOCKS - 1) / DEC_UNIT_BLOCKS;
    P.n_q_max = w.n_q_max;   /* set per launch shape in launch_compute */
    P.m_lo = 0x000F000Fu;
    P.m_hi = 0x00F000F0u;
    P.one024 = 0x64006400u;
    P.max_u = w.max_u;
    P.M = M;
    char* ws = (char*)d_workspace;
    P.n_unique = (int*)(ws + w.nu);
    P.tile_cnt = (int*)(ws + w.tile_cnt);
    P.hcnt = (int*)(ws + w.hcnt);
    P.ublob = (const uint8_t**)(ws + w.ublob);
    P.uw = (float*)(ws + w.uw);
    const bool x_direct = x_dtype == WISP_DTYPE_F16 && ((uintptr_t)d_x % 16) == 0;
    P.xconv = x_direct || x16 ? nullptr : (uint16_t*)(ws + w.xconv);
    P.xh = x_direct ? (const uint16_t*)d_x : (x16 ? x16 : P.xconv);
    P.hperm = (uint16_t*)(ws + w.hperm);
    P.part = (float*)(ws + w.part);
    P.gsplit = fused_shape(P.hidden / 128).gsplit;
    P.gfinish = M >= DEC_FINISH_MIN_TOKENS && P.gsplit > 1;
    P.gcnt = (int*)(ws + w.gcnt);
    P.gpart = (float*)(ws + w.gpart);
    P.out32 = d_out_f32;
    P.out16 = (uint16_t*)d_out_f16;
    P.accumulate = accumulate ? 1 : 0;
    P.status = (uint32_t*)(ws + DEC_STATUS_OFFSET);
    P.poll_limit = g_poll_limit;
    P.poll_extra = g_poll_extra;
    P.keep_status = keep_status ? 1 : 0;

    const size_t lds = prep_lds_bytes(R.mode, n_experts, M);
    int grid = 1;
    if (R.mode == 3) {
        R.rpw = (n_experts + 255) / 256;
        R.n_rwg = (n_experts + R.rpw - 1) / R.rpw;
        R.epoch = (uint32_t*)(ws + w.epoch);
        R.words = (uint64_t*)(ws + w.rwords);
        grid = R.n_rwg + 1;
    }
    ev_before(EV_PREP, s);
    /* dynamic LDS <= 8 KiB keys + 16 KiB scores (1024 experts, 4 tokens) */
    if (x_dtype == WISP_DTYPE_F16)
        hipLaunchKernelGGL(decode_prep_kernel<uint16_t>, dim3(grid), dim3(DEC_PREP_THREADS), lds, s,
                           P, R, d_expert_table, d_shared_blob, (const uint16_t*)d_x, top_k,
                           n_experts);
    else
        hipLaunchKernelGGL(decode_prep_kernel<float>, dim3(grid), dim3(DEC_PREP_THREADS), lds, s,
                           P, R, d_expert_table, d_shared_blob, (const float*)d_x, top_k,
                           n_experts);
    ev_after(EV_PREP, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;

    const int ng = P.gs >= 128 ? 1 : 128 / P.gs;
    const bool hz = P.has_zeros != 0;
    switch (M) {
        case 1: e = launch_ng<1>(ng, hz, P, s); break;
        case 2: e = launch_ng<2>(ng, hz, P, s); break;
        case 3: e = launch_ng<3>(ng, hz, P, s); break;
        default: e = launch_ng<4>(ng, hz, P, s); break;
    }
    if (e != hipSuccess) return e;
    return hipGetLastError();
}

/* n_experts is bounded by the prep workgroup's LDS copy of the expert
 * table (DEC_ROUTE_MAX_EXPERTS entries). */
static bool decode_args_ok(const void* table, const void* x, int x_dtype, int M, int top_k,
                           int n_experts, const void* ws, const float* o32, const wisp_half* o16) {
    return M >= 1 && M <= DEC_MAX_TOKENS && top_k >= 1 && top_k <= DEC_MAX_TOPK &&
           n_experts >= 1 && n_experts <= DEC_ROUTE_MAX_EXPERTS && table && x && ws &&
           (o32 || o16) && (x_dtype == WISP_DTYPE_F16 || x_dtype == WISP_DTYPE_F32);
}

extern "C" hipError_t wisp_gpu_moe_decode_int4(const void* const* d_expert_table,
                                               const void* d_shared_blob,
                                               const WispExpertLayout* L, const void* d_x,
                                               int x_dtype, int n_tokens, const int* d_topk_idx,
                                               const float* d_topk_w, int top_k, int n_experts,
                                               void* d_workspace, size_t workspace_bytes,
                                               int accumulate, float* d_out_f32,
                                               wisp_half* d_out_f16, hipStream_t s) {
    if (!decode_args_ok(d_expert_table, d_x, x_dtype, n_tokens, top_k, n_experts, d_workspace,
                        d_out_f32, d_out_f16) || !d_topk_idx || !d_topk_w)
        return hipErrorInvalidValue;
    RouteArgs R = {nullptr, nullptr, 0, 0, nullptr, (int*)d_topk_idx, (float*)d_topk_w,
                   0, 0, nullptr, nullptr};
    return decode_run(d_expert_table, d_shared_blob, L, d_x, x_dtype, n_tokens, R, top_k,
                      n_experts, d_workspace, workspace_bytes, accumulate, d_out_f32, d_out_f16, s);
}

/* Raw router logits for the prep kernel when the router matrix is too large
 * to run inside it (defined in moe_route.hip). */
hipError_t wisp_amd__router_logits(const wisp_half* W, const wisp_half* bias, const void* x,
                                   int x_dtype, int n_tokens, int hidden, int n_experts,
                                   int add_bias, float* logits, hipStream_t s);

static bool layer_args_ok(const wisp_half* d_router_w, int router_kind, const float* d_scores,
                          const int* d_topk_idx, const float* d_topk_w, int top_k, int n_experts,
                          const WispExpertLayout* L) {
    return d_router_w && d_scores && d_topk_idx && d_topk_w && top_k <= n_experts &&
           (router_kind == WISP_ROUTER_SOFTMAX || router_kind == WISP_ROUTER_SIGMOID) &&
           wisp_expert_layout_check(L) == hipSuccess;
}

/* Body of the two layer entry points, arguments already checked. */
static hipError_t layer_run(const wisp_half* d_router_w, const wisp_half* d_router_bias,
                            int router_kind, float* d_scores, int* d_topk_idx, float* d_topk_w,
                            const void* const* d_expert_table, const void* d_shared_blob,
                            const WispExpertLayout* L, const void* d_x, int x_dtype, int n_tokens,
                            int top_k, int n_experts, void* d_workspace, size_t workspace_bytes,
                            int accumulate, float* d_out_f32, wisp_half* d_out_f16,
                            hipStream_t s, const uint16_t* x16 = nullptr,
                            bool keep_status = false) {
    const int hidden = (int)L->cols[0];
    /* the router GEMV runs in router workgroups of the prep launch (mode 3):
     * each thread takes at most 2 16-byte pieces of a row, so rows up to
     * 8192, and 16-byte aligned W and x; otherwise it gets a launch of its
     * own (mode 1) */
    const int mode = hidden <= 2 * DEC_PREP_THREADS * 8 && (uintptr_t)d_router_w % 16 == 0 &&
                             (uintptr_t)d_x % 16 == 0
                         ? 3
                         : 1;
    RouteArgs R = {(const uint16_t*)d_router_w, (const uint16_t*)d_router_bias, router_kind,
                   mode, d_scores, d_topk_idx, d_topk_w, 0, 0, nullptr, nullptr};
    if (mode == 1) {
        ev_before(EV_ROUTE, s);
        hipError_t e = wisp_amd__router_logits(d_router_w, d_router_bias, d_x, x_dtype, n_tokens,
                                               hidden, n_experts,
                                               router_kind == WISP_ROUTER_SOFTMAX, d_scores, s);
        ev_after(EV_ROUTE, s);
        if (e != hipSuccess) return e;
    }
    return decode_run(d_expert_table, d_shared_blob, L, d_x, x_dtype, n_tokens, R, top_k,
                      n_experts, d_workspace, workspace_bytes, accumulate, d_out_f32, d_out_f16, s,
                      x16, keep_status);
}

extern "C" hipError_t wisp_gpu_moe_layer_decode_int4(
    const wisp_half* d_router_w, const wisp_half* d_router_bias, int router_kind,
    float* d_scores, int* d_topk_idx, float* d_topk_w, const void* const* d_expert_table,
    const void* d_shared_blob, const WispExpertLayout* L, const void* d_x, int x_dtype,
    int n_tokens, int top_k, int n_experts, void* d_workspace, size_t workspace_bytes,
    int accumulate, float* d_out_f32, wisp_half* d_out_f16, hipStream_t s) {
    if (!decode_args_ok(d_expert_table, d_x, x_dtype, n_tokens, top_k, n_experts, d_workspace,
                        d_out_f32, d_out_f16) ||
        !layer_args_ok(d_router_w, router_kind, d_scores, d_topk_idx, d_topk_w, top_k, n_experts,
                       L))
        return hipErrorInvalidValue;
    return layer_run(d_router_w, d_router_bias, router_kind, d_scores, d_topk_idx, d_topk_w,
                     d_expert_table, d_shared_blob, L, d_x, x_dtype, n_tokens, top_k, n_experts,
                     d_workspace, workspace_bytes, accumulate, d_out_f32, d_out_f16, s);
}

/* ---- the layer entry point that allocates nothing -----------------------
 * Its workspace is this file-scope device array: one copy per device, held
 * until the process ends. In host code `scratch` only names the symbol;
 * its device address comes from hipGetSymbolAddress, once per device, with
 * that device current, and only that address is handed to kernels and
 * copies. Every call on a device shares the array and leaves its contents
 * behind: the prep kernel zeroes the counters each call needs, and the
 * routing epoch and words are built to persist (a zero-filled array is a
 * valid start). Calls that overlap on one device race. */
#define WISP_NOALLOC_MAX_DEVICES 64
static __device__ __align__(256) uint8_t scratch[WISP_NOALLOC_SCRATCH_BYTES];
static void* g_scratch_ptr[WISP_NOALLOC_MAX_DEVICES];
static std::mutex g_scratch_mu;

/* Device address of `scratch` on the device of stream s (the current device
 * for the null stream). */
static hipError_t noalloc_scratch(hipStream_t s, void** out) {
    int dev = 0;
    hipError_t e = hipSuccess;
    if (s) {
        dev = hipGetStreamDeviceId(s);
        if (dev < 0) return hipErrorInvalidResourceHandle;
    } else {
        e = hipGetDevice(&dev);
        if (e != hipSuccess) return e;
    }
    if (dev >= WISP_NOALLOC_MAX_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        int cur = 0;
        e = hipGetDevice(&cur);
        if (e != hipSuccess) return e;
        if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) (void)hipSetDevice(cur);
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

extern "C" hipError_t wisp_gpu_moe_layer_decode_int4_noalloc(
    const wisp_half* d_router_w, const wisp_half* d_router_bias, int router_kind,
    float* d_scores, int* d_topk_idx, float* d_topk_w, const void* const* d_expert_table,
    const void* d_shared_blob, const WispExpertLayout* L, const void* d_x, int x_dtype,
    int n_tokens, int top_k, int n_experts, int accumulate, float* d_out_f32,
    wisp_half* d_out_f16, hipStream_t s) {
    const void* any = (const void*)1;   /* the workspace is checked below */
    if (!decode_args_ok(d_expert_table, d_x, x_dtype, n_tokens, top_k, n_experts, any, d_out_f32,
                        d_out_f16) ||
        !layer_args_ok(d_router_w, router_kind, d_scores, d_topk_idx, d_topk_w, top_k, n_experts,
                       L))
        return hipErrorInvalidValue;
    const size_t need = ws_layout(L, n_tokens, top_k, d_shared_blob != nullptr).total;
    if (need > WISP_NOALLOC_SCRATCH_BYTES) return hipErrorInvalidValue;
    void* ws = nullptr;
    hipError_t e = noalloc_scratch(s, &ws);
    if (e != hipSuccess) return e;
    return layer_run(d_router_w, d_router_bias, router_kind, d_scores, d_topk_idx, d_topk_w,
                     d_expert_table, d_shared_blob, L, d_x, x_dtype, n_tokens, top_k, n_experts, ws,
                     WISP_NOALLOC_SCRATCH_BYTES, accumulate, d_out_f32, d_out_f16, s);
}

/* ---- the FFN half of a decode step (RMSNorm, MoE layer, residual) ------- */

/* The fixed leading regions of every decode workspace (unique count and
 * status, routing epoch, routing words): the block's prefill path starts
 * after them, so a workspace shared by both paths keeps its routing state. */
#define DEC_WS_HEADER ((size_t)512 + (size_t)DEC_MAX_TOKENS * DEC_ROUTE_MAX_EXPERTS * 8)

hipError_t wisp_amd__rmsnorm_rows(const float* x, const wisp_half* w, float* y32, wisp_half* y16,
                                  int rows, int n, float eps, hipStream_t s);

/* Rows up to which the MoE block runs the fused decode (fp32 routing), in
 * calls of up to DEC_MAX_TOKENS rows; more rows take the grouped GEMM. */
#ifndef BLOCK_DECODE_MAX_ROWS
#define BLOCK_DECODE_MAX_ROWS WISP_BLOCK_DECODE_MAX_ROWS
#endif
struct BlockWs {
    size_t pf, xn, xn16, total;
    bool decode;
};

static BlockWs block_ws(const WispExpertLayout* L, int M, int top_k, int n_experts,
                        int has_shared) {
    BlockWs b = {0, 0, 0, 0, M <= BLOCK_DECODE_MAX_ROWS};
    const size_t hidden = L->cols[0];
    if (b.decode) {
        const int mc = M < DEC_MAX_TOKENS ? M : DEC_MAX_TOKENS;   /* rows per decode call */
        b.xn = align_up(ws_layout(L, mc, top_k, has_shared).total, 256);
        b.xn16 = b.xn + align_up((size_t)M * hidden * 4, 256);
        b.total = b.xn16 + align_up((size_t)M * hidden * 2, 256);
    } else {
        b.pf = wisp_moe_prefill_workspace_bytes(L, M, top_k, n_experts, has_shared);
        if (b.pf == 0) return b;
        b.xn = align_up(DEC_WS_HEADER + b.pf, 256);
        b.total = b.xn + align_up((size_t)M * hidden * 2, 256);
    }
    return b;
}

extern "C" size_t wisp_moe_block_workspace_bytes(const WispExpertLayout* L, int n_tokens,
                                                 int top_k, int n_experts, int has_shared) {
    if (!L || n_tokens < 1 || top_k < 1 || top_k > DEC_MAX_TOPK || n_experts < 1 ||
        n_experts > DEC_ROUTE_MAX_EXPERTS || wisp_expert_layout_check(L) != hipSuccess)
        return 0;
    return block_ws(L, n_tokens, top_k, n_experts, has_shared).total;
}

extern "C" hipError_t wisp_gpu_moe_block_int4(
    float* d_x, const wisp_half* d_post_norm_w, float eps, const wisp_half* d_router_w,
    const wisp_half* d_router_bias, int router_kind, float* d_scores, int* d_topk_idx,
    float* d_topk_w, const void* const* d_expert_table, const void* d_shared_blob,
    const WispExpertLayout* L, int n_tokens, int top_k, int n_experts, void* d_workspace,
    size_t workspace_bytes, hipStream_t s) {
    const int M = n_tokens;
    if (!d_x || !d_post_norm_w || !d_workspace || M < 1 || top_k < 1 || top_k > DEC_MAX_TOPK ||
        n_experts < 1 || n_experts > DEC_ROUTE_MAX_EXPERTS || !d_expert_table ||
        !layer_args_ok(d_router_w, router_kind, d_scores, d_topk_idx, d_topk_w, top_k, n_experts,
                       L))
        return hipErrorInvalidValue;
    const BlockWs b = block_ws(L, M, top_k, n_experts, d_shared_blob != nullptr);
    if (b.total == 0 || workspace_bytes < b.total) return hipErrorInvalidValue;
    const int hidden = (int)L->cols[0];
    char* ws = (char*)d_workspace;
    hipError_t e;
    if (b.decode) {
        /* fp32 normalised rows for the router, and their fp16 rounding for
         * the experts, both written by the RMSNorm launch (the prep
         * workgroup then converts nothing: 4 rows, DeepSeek-V3 shape,
         * 172.3 -> 163.1 us per call) */
        float* xn = (float*)(ws + b.xn);
        wisp_half* xn16 = (wisp_half*)(ws + b.xn16);
        e = wisp_amd__rmsnorm_rows(d_x, d_post_norm_w, xn, xn16, M, hidden, eps, s);
        if (e != hipSuccess) return e;
        /* up to DEC_MAX_TOKENS rows per decode call, in row order on s */
        for (int r0 = 0; r0 < M; r0 += DEC_MAX_TOKENS) {
            const int mc = M - r0 < DEC_MAX_TOKENS ? M - r0 : DEC_MAX_TOKENS;
            e = layer_run(d_router_w, d_router_bias, router_kind,
                          d_scores + (size_t)r0 * n_experts, d_topk_idx + (size_t)r0 * top_k,
                          d_topk_w + (size_t)r0 * top_k, d_expert_table, d_shared_blob, L,
                          xn + (size_t)r0 * hidden, WISP_DTYPE_F32, mc, top_k, n_experts,
                          d_workspace, b.xn, /*accumulate=*/1, d_x + (size_t)r0 * hidden,
                          nullptr, s, (const uint16_t*)(xn16 + (size_t)r0 * hidden),
                          /*keep_status=*/r0 > 0);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    if ((uintptr_t)d_x % 16) return hipErrorInvalidValue;   /* the prefill's fp32 output */
    wisp_half* xn = (wisp_half*)(ws + b.xn);
    e = wisp_amd__rmsnorm_rows(d_x, d_post_norm_w, nullptr, xn, M, hidden, eps, s);
    if (e != hipSuccess) return e;
    e = wisp_gpu_moe_route(d_router_w, d_router_bias, xn, M, hidden, n_experts, top_k,
                           router_kind, d_scores, d_topk_idx, d_topk_w, s);
    if (e != hipSuccess) return e;
    return wisp_gpu_moe_prefill_int4(d_expert_table, d_shared_blob, L, xn, M, d_topk_idx,
                                     d_topk_w, top_k, n_experts, ws + DEC_WS_HEADER, b.pf,
                                     /*accumulate=*/1, d_x, nullptr, s);
}

extern "C" hipError_t wisp_moe_decode_status(void* d_workspace, hipStream_t s, uint32_t* flags,
                                             int clear) {
    if (!flags) return hipErrorInvalidValue;
    *flags = 0;
    char* ws = (char*)d_workspace;
    if (!ws) {
        /* the static workspace of wisp_gpu_moe_layer_decode_int4_noalloc */
        void* p = nullptr;
        hipError_t e = noalloc_scratch(s, &p);
        if (e != hipSuccess) return e;
        ws = (char*)p;
    }
    hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) return e;
    uint32_t v = 0;
    e = hipMemcpy(&v, ws + DEC_STATUS_OFFSET, sizeof(v), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return e;
    if (clear && v) {
        const uint32_t zero = 0;
        e = hipMemcpy(ws + DEC_STATUS_OFFSET, &zero, sizeof(zero), hipMemcpyHostToDevice);
        if (e != hipSuccess) return e;
    }
    *flags = v;
    return hipSuccess;
}
