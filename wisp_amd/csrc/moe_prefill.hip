/*
 * moe_prefill.hip — int4 MoE prefill as a grouped GEMM over routed token
 * tiles on gfx950 (MFMA fp16, fp32 accumulate).
 *
 * The reference has no batched MoE: prefill and speculative verify call the
 * single-token decode once per token (csrc/core/wisp_engine.c:2292-2307,
 * 2317-2330), so every selected expert's weights are read once per token.
 * Here every expert's weights are read once per tile of up to 128 of its
 * tokens:
 *
 *   prep    : (token, slot) pairs with the shared expert as slot 0 (expert
 *             id n_experts, weight 1), so the combine order is the
 *             reference's: shared, then routed experts in rank order
 *             (csrc/core/wisp_engine.c:1594-1602, 1653-1670).
 *   offsets : wisp_gpu_expert_offsets (counting sort of the pairs by
 *             expert, stable in flat pair order).
 *   tiles   : one workgroup turns the expert counts into the tile list
 *             (expert, first pair, rows <= 128).
 *   gate/up : grid (tiles, inter/128). A wave owns 2 gate + 2 up row tiles
 *             (16 rows each) of one expert; per 128-wide K block each lane
 *             loads 16 B of packed nibbles per row tile (32 consecutive K
 *             of one row), dequantises them in registers to fp16
 *             fp16((q - 8) * s + z) (the reference dequant,
 *             csrc/cuda/expert_loader.cu:42) and feeds them as the B operand
 *             of v_mfma_f32_16x16x32_f16 against up to 8 16-token A tiles
 *             gathered from x into double-buffered LDS. Sub-tiles past the
 *             tile's token count are skipped. Epilogue:
 *             h = w_route * silu(g) * u, fp16, in sorted pair order.
 *   down    : same kernel shape over h (rows contiguous per expert), 4 row
 *             tiles per wave; writes y' = down . h' (fp16) per pair.
 *   combine : out[t] (+)= sum over the token's slots in order of y'.
 *
 * Weights are read in place from the reference blob layout
 * (csrc/core/wisp_engine.h:214-238); nothing is dequantised to memory.
 */
#include "hip_common.h"

#include <mutex>

#define PF_BM 128                 /* tokens per tile                         */
#define PF_WAVES 8                /* waves per workgroup (NT = 2 row tiles each) */
#define PF_RING 4                 /* weight blocks in the register ring (3 in flight) */
#define PF_NT 2                   /* row tiles of 16 weight rows per wave        */
#define PF_XCDS 8                 /* accelerator dies: workgroups are dealt to them round-robin */
#define PF_AROW 136               /* LDS A row stride in halves (128 + 8)    */
#define PF_MAX_EXPERTS 4096      /* capacity of the tile-list kernel */
#define PF_MAX_EXPERTS1 1024      /* routed + shared experts: wisp_gpu_expert_offsets' limit */
#define PF_CLASSES 3              /* tiles of <= 32, <= 64, <= 128 tokens    */
#define PF_SCALE_LDS_MAX 40960    /* byte budget of the LDS scale (and zero) image */
#define PF_SCALE_LDS_WIDE 65536   /* the same for the wide full-tile kernel      */
#define PF_SCALE_PIECES 4         /* 16-byte scale pieces per lane and row tile when staged */
#define PF_WIDE_RING 2         /* weight blocks in the ring of the wide full-tile kernel */
#define PF_SMALL_CHUNK_DN 16      /* down K chunk of the <= 64-token tiles (all 16 blocks of inter 2048) */
#define PF_CHUNK 8                /* K blocks per straight-line pipeline chunk (when they divide K) */
#define PF_COMBINE_SLOTS 16       /* slots per token the combine loads at once (top_k + shared) */
#define PF_WIDE_CHUNK_DN 16       /* down K chunk of the wide full-tile kernel (all 16 blocks of inter 2048) */

struct PfParams {
    uint64_t p_off[3], s_off[3], z_off[3];
    int hidden, inter, gs, has_zeros;
    int n_tokens, top_k1, n_experts1, max_tiles;
    const uint8_t** table1;   /* [n_experts1] blob pointers, shared last     */
    int* idx1;                /* [n_tokens][top_k1] expert id per pair       */
    float* w1;                /* [n_tokens][top_k1] routing weight per pair  */
    int* counts;              /* [n_experts1]                                */
    int* offsets;             /* [n_experts1 + 1]                            */
    int* order;               /* [n_pairs] flat pair index, sorted by expert */
    int* inv;                 /* [n_pairs] position of each pair in order    */
    int* n_tiles;             /* [PF_CLASSES]                                */
    int4* tiles;              /* [PF_CLASSES][max_tiles] (expert, first position, rows) */
    uint16_t* H;              /* [n_pairs][inter] fp16 h', sorted order      */
    uint16_t* Y;              /* [n_pairs][hidden] fp16 y', sorted order     */
    const uint16_t* x;        /* [n_tokens][hidden] fp16                      */
    float* out32;
    uint16_t* out16;
    int accumulate;
};

/* ======================================================================= */
/* prep and tile list                                                       */
/* ======================================================================= */

/* idx1/w1: slot 0 = shared expert (id n_experts1 - 1, weight 1) when
 * present, then the routed slots; table1 = table plus the shared blob. */
__global__ __launch_bounds__(256) void pf_prep_kernel(PfParams P, const void* const* table,
                                                      const void* shared_blob, const int* idx,
                                                      const float* w, int top_k,
                                                      int n_experts) {
    const int sh = shared_blob ? 1 : 0;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n_experts) P.table1[i] = (const uint8_t*)table[i];
    if (i == 0 && sh) P.table1[n_experts] = (const uint8_t*)shared_blob;
    if (i < P.n_tokens * P.top_k1) {
        const int t = i / P.top_k1, k = i - t * P.top_k1;
        int e;
        float wv;
        if (sh && k == 0) {
            e = n_experts;
            wv = 1.0f;
        } else {
            e = idx[t * top_k + k - sh];
            wv = w[t * top_k + k - sh];
            if (e < 0 || e >= n_experts) e = -1;
        }
        P.idx1[i] = e;
        P.w1[i] = wv;
    }
}

/* Tile class of a tile with `rows` tokens: its compile-time count of
 * 16-token sub-tiles is 2, 4 or 8. */
__host__ __device__ inline int pf_class(int rows) { return rows <= 32 ? 0 : (rows <= 64 ? 1 : 2); }

#define PF_TILE_THREADS 1024
#define PF_TILE_EPT (PF_MAX_EXPERTS / PF_TILE_THREADS)   /* experts per thread */

/* One workgroup: tiles of up to PF_BM pairs per expert, experts in order,
 * appended to the list of their class (tiles[c * max_tiles + i]). An
 * expert of c pairs gives c / PF_BM full tiles (the last class), then one
 * tile of the remainder. Thread t takes experts [PF_TILE_EPT t, +PF_TILE_EPT),
 * counts its tiles per class, and an exclusive scan over the threads per
 * class gives its first slots, so the lists come out in expert order. */
__global__ __launch_bounds__(PF_TILE_THREADS) void pf_tiles_kernel(PfParams P) {
    __shared__ int s_wsum[PF_CLASSES][PF_TILE_THREADS / 64];
    const int E = P.n_experts1;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    int cnt[PF_TILE_EPT], off[PF_TILE_EPT];
    int nk[PF_CLASSES] = {0, 0, 0};
#pragma unroll
    for (int j = 0; j < PF_TILE_EPT; j++) {
        const int e = PF_TILE_EPT * tid + j;
        cnt[j] = e < E ? P.counts[e] : 0;
        off[j] = e < E ? P.offsets[e] : 0;
    }
#pragma unroll
    for (int j = 0; j < PF_TILE_EPT; j++) {
        nk[PF_CLASSES - 1] += cnt[j] / PF_BM;
        if (cnt[j] % PF_BM) nk[pf_class(cnt[j] % PF_BM)]++;
    }
    int pos[PF_CLASSES], incl[PF_CLASSES];
#pragma unroll
    for (int k = 0; k < PF_CLASSES; k++) {
        int v = nk[k];
        for (int d = 1; d < 64; d <<= 1) {
            const int y = __shfl_up(v, d, 64);
            if (lane >= d) v += y;
        }
        incl[k] = v;
        if (lane == 63) s_wsum[k][wv] = v;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < PF_CLASSES; k++) {
        for (int w = 0; w < wv; w++) incl[k] += s_wsum[k][w];
        pos[k] = incl[k] - nk[k];
    }
#pragma unroll
    for (int j = 0; j < PF_TILE_EPT; j++) {
        const int e = PF_TILE_EPT * tid + j;
        const int full = cnt[j] / PF_BM, rem = cnt[j] % PF_BM;
        for (int q = 0; q < full; q++) {
            const int k = PF_CLASSES - 1;
            if (pos[k] < P.max_tiles)
                P.tiles[k * P.max_tiles + pos[k]] = make_int4(e, off[j] + q * PF_BM, PF_BM, 0);
            pos[k]++;
        }
        if (rem) {
            const int k = pf_class(rem);
            if (pos[k] < P.max_tiles)
                P.tiles[k * P.max_tiles + pos[k]] = make_int4(e, off[j] + full * PF_BM, rem, 0);
            pos[k]++;
        }
    }
    if (tid == PF_TILE_THREADS - 1)
        for (int k = 0; k < PF_CLASSES; k++) P.n_tiles[k] = min(incl[k], P.max_tiles);
}

/* ======================================================================= */
/* grouped GEMM                                                             */
/* ======================================================================= */

/* 8 fp16 values e0..e7 (natural order) -> slot order e0 e4 e1 e5 e2 e6 e3 e7
 * (the order dequant8 produces). */
__device__ __forceinline__ u4 perm8_halves(u4 v) {
    u4 o;
    o.x = (v.x & 0xFFFFu) | (v.z << 16);
    o.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
    o.z = (v.y & 0xFFFFu) | (v.w << 16);
    o.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
    return o;
}

/* Two nibbles already OR-ed into fp16 1024.0 -> fp16((q - 8) * s + z):
 * subtracting 1032 gives q - 8 exactly; one packed multiply (or fma with
 * the zero) rounds once to fp16. */
template <bool HZ>
__device__ __forceinline__ uint32_t dequant2(uint32_t d, h2 s2, h2 z2) {
    const h2 off = {(f16)1032.0f, (f16)1032.0f};
    const h2 q = __builtin_bit_cast(h2, d) - off;
    return __builtin_bit_cast(uint32_t, HZ ? q * s2 + z2 : q * s2);
}

/* 8 nibbles of one dword -> fp16((q - 8) * s + z) in slot order
 * e0 e4 e1 e5 e2 e6 e3 e7. OR-ing a nibble into the mantissa of 1024.0
 * (0x6400) gives exactly 1024 + q. Written with one scalar per dword: an
 * element of a vector value subscripted by an unrolled loop index inside
 * __builtin_bit_cast was folded to element 0 by this compiler. m =
 * 0x000F000F and one024 = 0x64006400 come in VGPRs (see pf_gemm_kernel), so
 * each and-or is one v_and_or_b32 (two literal operands would split it). */
template <bool HZ>
__device__ __forceinline__ h8 dequant8(uint32_t w, h2 s2, h2 z2, uint32_t m, uint32_t one024) {
    u4 o;
    o.x = dequant2<HZ>((w & m) | one024, s2, z2);
    o.y = dequant2<HZ>(((w >> 4) & m) | one024, s2, z2);
    o.z = dequant2<HZ>(((w >> 8) & m) | one024, s2, z2);
    o.w = dequant2<HZ>(((w >> 12) & m) | one024, s2, z2);
    return __builtin_bit_cast(h8, o);
}

/* grid (tiles of class CLS, n-blocks); WV waves, each owning NT row tiles
 * of 16 weight rows. GATEUP: the workgroup covers FEAT = 8 NT WV h features
 * [FEAT by, FEAT by + FEAT): wave w owns gate rows f0 .. f0 + 8 NT - 1 and
 * the same up rows, f0 = FEAT by + 8 NT w (row tiles s < NT/2 gate, the
 * rest up). DOWN: output rows [DROWS by, +DROWS), DROWS = 16 NT WV: wave w
 * owns NT row tiles from DROWS by + 16 NT w. K = hidden (GATEUP) or inter
 * (DOWN) in 128-wide
 * blocks. TV: 16-token sub-tiles of the class (rows past the tile's count
 * are zeros); R: weight blocks held in the register ring (R - 1 in flight
 * while one is computed). Eight waves with half the rows each halve the
 * accumulator and ring registers, so two waves fit on a SIMD and one
 * wave's dequant overlaps another's MFMAs.
 *
 * Pipeline of step b: commit the A tile of block b + 1 (loaded during step
 * b - 1) to the other LDS buffer, issue the A loads of block b + 2, issue
 * the weights of block b + R - 1, compute block b, barrier.
 *
 * SS: each wave first copies the scales (and zeros) of its row tiles for
 * the whole K axis into dynamic LDS, [WV][NT][16][G] (16 consecutive rows
 * are one contiguous run, copied with 16-byte loads), and the K loop reads
 * them from there. Otherwise every step loads one 2-byte scale per lane and
 * row tile, 16 rows and so 16 memory transactions per instruction: 18 % of
 * the DeepSeek-V3 prefill layer on MI355X. */
template <bool GATEUP, bool HZ, int TV, int R, int WV, bool SS, int NT, int CH = 0>
__global__ __launch_bounds__(64 * WV) void pf_gemm_kernel(const PfParams P, int cls) {
    constexpr int THREADS = 64 * WV;
    constexpr int FEAT = 8 * NT * WV;            /* gate/up: h features per workgroup */
    constexpr int DROWS = 16 * NT * WV;          /* down: output rows per workgroup */
    constexpr int BM = 16 * TV;
    constexpr int APT = BM * 16 / THREADS;       /* A pieces (16 B) per thread per block */
    static_assert(APT >= 1 && APT * THREADS == BM * 16, "A staging must divide evenly");
    __shared__ __attribute__((aligned(16))) uint16_t s_a[2][BM * PF_AROW];
    __shared__ int s_row[BM];      /* source row of each tile row (-1: none) */
    __shared__ float s_wr[BM];     /* routing weight of each tile row        */
    extern __shared__ __attribute__((aligned(16))) uint16_t s_scl[];   /* SS image */
    /* XCD-aware order: the hardware deals workgroups to the PF_XCDS dies
     * round-robin by linear id (x fastest), and each die has its own L2.
     * Die d's k-th workgroup takes tile 8 (k / ny) + d, n-block k % ny, so
     * all n-blocks of a tile run together on one die and its gathered
     * token rows come from that die's L2 after the first read (gridDim.x
     * is a multiple of PF_XCDS). The map is a bijection for any PF_XCDS;
     * the die count only decides the locality. */
    const int ny = gridDim.y;
    const int lin = blockIdx.x + gridDim.x * blockIdx.y;
    const int slot = lin / PF_XCDS;
    const int tile = (slot / ny) * PF_XCDS + lin % PF_XCDS;
    const int by = slot % ny;
    const int n_tiles = P.n_tiles[cls];
    if (tile >= n_tiles) return;
    const int4 td = P.tiles[cls * P.max_tiles + tile];
    const int e = td.x, p0 = td.y, nv = td.z;
    const uint8_t* blob = P.table1[e];
    const int K = GATEUP ? P.hidden : P.inter;
    const int nblk = K / 128;
    const int G = K / P.gs;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, j = lane >> 4;

    for (int r = threadIdx.x; r < BM; r += THREADS) {
        if (r < nv) {
            const int pair = P.order[p0 + r];
            s_row[r] = GATEUP ? pair / P.top_k1 : p0 + r;
            s_wr[r] = P.w1[pair];
        } else {
            s_row[r] = -1;
            s_wr[r] = 0.0f;
        }
    }

    /* weight row tiles of this wave */
    const uint8_t* wp[NT];
    const uint16_t* sp[NT];
    const uint16_t* zp[NT];
#pragma unroll
    for (int s = 0; s < NT; s++) {
        int mat, row;
        if (GATEUP) {
            mat = s < NT / 2 ? 0 : 1;
            row = by * FEAT + wave * (FEAT / WV) + 16 * (s % (NT / 2)) + col;
        } else {
            mat = 2;
            row = by * DROWS + wave * (DROWS / WV) + 16 * s + col;
        }
        wp[s] = blob + P.p_off[mat] + (size_t)row * (K / 2) + 16 * j;
        sp[s] = (const uint16_t*)(blob + P.s_off[mat]) + (size_t)row * G;
        zp[s] = (const uint16_t*)(blob + P.z_off[mat]) + (size_t)row * G;
    }
    /* group of this lane's 32 K values in block b: (128 b + 32 j) / gs */
    const int gshift = 31 - __builtin_clz(P.gs);
    /* this wave's scale (zero) image: row tile s, row col at
     * s_sc[(s * 16 + col) * G] (s_zc likewise) */
    uint16_t* const s_sc = s_scl + (size_t)wave * NT * 16 * G;
    uint16_t* const s_zc = s_scl + (size_t)(WV + wave) * NT * 16 * G;
    if (SS) {
        /* 16 rows x G fp16 = 2 G pieces of 16 B per row tile; all loads
         * first, then the LDS writes (the weights come after) */
        u4 sv[NT][PF_SCALE_PIECES], zv[NT][PF_SCALE_PIECES];
#pragma unroll
        for (int s = 0; s < NT; s++) {
            const uint16_t* sb = sp[s] - (size_t)col * G;   /* the tile's first row */
            const uint16_t* zb = zp[s] - (size_t)col * G;
#pragma unroll
            for (int c = 0; c < PF_SCALE_PIECES; c++) {
                const int q = min(lane + 64 * c, 2 * G - 1);
                sv[s][c] = *(const u4*)(sb + 8 * q);
                if (HZ) zv[s][c] = *(const u4*)(zb + 8 * q);
            }
        }
#pragma unroll
        for (int s = 0; s < NT; s++)
#pragma unroll
            for (int c = 0; c < PF_SCALE_PIECES; c++) {
                const int q = lane + 64 * c;
                if (q < 2 * G) {
                    *(u4*)(s_sc + s * 16 * G + 8 * q) = sv[s][c];
                    if (HZ) *(u4*)(s_zc + s * 16 * G + 8 * q) = zv[s][c];
                }
            }
    }

    f4 acc[TV][NT];
#pragma unroll
    for (int t = 0; t < TV; t++)
#pragma unroll
        for (int s = 0; s < NT; s++) acc[t][s] = (f4){0.0f, 0.0f, 0.0f, 0.0f};

    __syncthreads();   /* s_row visible */

    /* A staging: BM rows x 128 K of a block, 16 B pieces. In the chunked
     * loop (CH > 0) every load is unconditional: a padding row reads the
     * tile's first row and is zeroed when committed, so no load sits under
     * an exec mask (whose zero default the compiler keeps in a copied
     * register, and every copy of an in-flight register is a wait). */
    const uint16_t* asrc = GATEUP ? P.x : P.H;
    u4 areg[APT];
    int aoff[APT];     /* element offset of each piece's source row (-1: zero) */
    bool alive[APT];
#pragma unroll
    for (int c = 0; c < APT; c++) {
        const int i = threadIdx.x + c * THREADS;
        const int src = s_row[i >> 4];
        alive[c] = src >= 0;
        if (CH > 0) aoff[c] = (src >= 0 ? src : s_row[0]) * K + 8 * (i & 15);
        else aoff[c] = src >= 0 ? src * K + 8 * (i & 15) : -1;
    }
    auto a_issue = [&](int b) {
#pragma unroll
        for (int c = 0; c < APT; c++) {
            if (CH > 0) areg[c] = *(const u4*)(asrc + (size_t)aoff[c] + b * 128);
            else
                areg[c] = aoff[c] >= 0 ? *(const u4*)(asrc + (size_t)aoff[c] + b * 128)
                                       : (u4){0u, 0u, 0u, 0u};
        }
    };
    auto a_commit = [&](int buf) {
#pragma unroll
        for (int c = 0; c < APT; c++) {
            const int i = threadIdx.x + c * THREADS;
            u4 v = perm8_halves(areg[c]);
            if (CH > 0 && !alive[c]) v = (u4){0u, 0u, 0u, 0u};
            *(u4*)(&s_a[buf][(i >> 4) * PF_AROW + 8 * (i & 15)]) = v;
        }
    };

    /* weight ring: block b lives in slot b % R */
    u4 wr[R][NT];
    uint16_t sr[R][NT], zr[R][NT];
    auto w_issue = [&](int slot, int b) {
        const int bb = min(b, nblk - 1);
        const int g = (bb * 128 + 32 * j) >> gshift;
#pragma unroll
        for (int s = 0; s < NT; s++) {
            wr[slot][s] = *(const u4*)(wp[s] + (size_t)bb * 64);
            if (!SS) {
                sr[slot][s] = sp[s][g];
                if (HZ) zr[slot][s] = zp[s][g];
            }
        }
    };

    /* unpack constants pinned to VGPRs (an empty asm emits nothing): a VALU
     * op takes at most one literal, so with literal masks every and-or of
     * the dequant became a v_and_b32 plus a v_or_b32 */
    uint32_t nib_mask = 0x000F000Fu, nib_one = 0x64006400u;
    asm volatile("" : "+v"(nib_mask));
    asm volatile("" : "+v"(nib_one));

    /* computes block b from ring slot r and the A buffer of b */
    auto compute_block = [&](int b, int r) {
        const uint16_t* abuf = &s_a[b & 1][0];
        if (SS) {
            const int g = (b * 128 + 32 * j) >> gshift;
#pragma unroll
            for (int s = 0; s < NT; s++) {
                sr[r][s] = s_sc[(s * 16 + col) * G + g];
                if (HZ) zr[r][s] = s_zc[(s * 16 + col) * G + g];
            }
        }
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            if constexpr (NT > 2 && R == 2) {
                /* wide waves with a ring of two (the registers it frees):
                 * every activation fragment of the k step, then the NT
                 * weight fragments, then the TV x NT MFMAs */
                h8 af[TV];
#pragma unroll
                for (int t = 0; t < TV; t++)
                    af[t] = *(const h8*)(abuf + (16 * t + col) * PF_AROW + 32 * j + 8 * kk);
                h8 bf[NT];
#pragma unroll
                for (int s = 0; s < NT; s++) {
                    const f16 sc = __builtin_bit_cast(f16, sr[r][s]);
                    const f16 zc = HZ ? __builtin_bit_cast(f16, zr[r][s]) : (f16)0.0f;
                    bf[s] = dequant8<HZ>(wr[r][s][kk], (h2){sc, sc}, (h2){zc, zc},
                                         nib_mask, nib_one);
                }
#pragma unroll
                for (int t = 0; t < TV; t++)
#pragma unroll
                    for (int s = 0; s < NT; s++)
                        acc[t][s] = mfma16x16x32(af[t], bf[s], acc[t][s]);
                __builtin_amdgcn_sched_barrier(0);
            } else if constexpr (NT > 2) {
                /* wide waves: the NT weight fragments first, then one
                 * activation fragment at a time (registers) */
                h8 bf[NT];
#pragma unroll
                for (int s = 0; s < NT; s++) {
                    const f16 sc = __builtin_bit_cast(f16, sr[r][s]);
                    const f16 zc = HZ ? __builtin_bit_cast(f16, zr[r][s]) : (f16)0.0f;
                    bf[s] = dequant8<HZ>(wr[r][s][kk], (h2){sc, sc}, (h2){zc, zc},
                                         nib_mask, nib_one);
                }
#pragma unroll
                for (int t = 0; t < TV; t++) {
                    const h8 af =
                        *(const h8*)(abuf + (16 * t + col) * PF_AROW + 32 * j + 8 * kk);
#pragma unroll
                    for (int s = 0; s < NT; s++)
                        acc[t][s] = mfma16x16x32(af, bf[s], acc[t][s]);
                }
                __builtin_amdgcn_sched_barrier(0);
            } else {
                h8 af[TV];
#pragma unroll
                for (int t = 0; t < TV; t++)
                    af[t] = *(const h8*)(abuf + (16 * t + col) * PF_AROW + 32 * j + 8 * kk);
#pragma unroll
                for (int s = 0; s < NT; s++) {
                    const f16 sc = __builtin_bit_cast(f16, sr[r][s]);
                    const f16 zc = HZ ? __builtin_bit_cast(f16, zr[r][s]) : (f16)0.0f;
                    const h8 bf = dequant8<HZ>(wr[r][s][kk], (h2){sc, sc}, (h2){zc, zc},
                                               nib_mask, nib_one);
#pragma unroll
                    for (int t = 0; t < TV; t++)
                        acc[t][s] = mfma16x16x32(af[t], bf, acc[t][s]);
                }
            }
        }
    };

    if (CH > 0) {
        /* K in chunks of CH blocks (nblk % CH == 0, checked by the
         * launcher), each chunk one straight-line pipeline: A of block b + 2
         * and the weights of block b + R - 1 are issued during block b, but
         * nothing in flight crosses the loop's back edge, so the compiler
         * waits for exactly the loads each step needs instead of draining
         * the ring; the pipeline refills once per chunk. */
        for (int c0 = 0; c0 < nblk; c0 += CH) {
            a_issue(c0);
            a_commit(c0 & 1);
            if (CH > 1) a_issue(c0 + 1);
#pragma unroll
            for (int r = 0; r < R - 1; r++) w_issue(r, c0 + r);
            __syncthreads();
#pragma unroll
            for (int r = 0; r < CH; r++) {
                const int b = c0 + r;
                if (r + 1 < CH) a_commit((b + 1) & 1);
                if (r + 2 < CH) a_issue(b + 2);
                if (r + R - 1 < CH) w_issue((r + R - 1) % R, b + R - 1);
                compute_block(b, r % R);
                __syncthreads();
            }
        }
    } else {
        a_issue(0);
        a_commit(0);
        if (nblk > 1) a_issue(1);
    #pragma unroll
        for (int r = 0; r < R - 1; r++) w_issue(r, r);
        __syncthreads();

        for (int b0 = 0; b0 < nblk; b0 += R) {
    #pragma unroll
            for (int r = 0; r < R; r++) {
                const int b = b0 + r;
                if (b < nblk) {
                    if (b + 1 < nblk) a_commit((b + 1) & 1);
                    if (b + 2 < nblk) a_issue(b + 2);
                    w_issue((r + R - 1) % R, b + R - 1);
                    const uint16_t* abuf = &s_a[b & 1][0];
                    if (SS) {
                        const int g = (b * 128 + 32 * j) >> gshift;
    #pragma unroll
                        for (int s = 0; s < NT; s++) {
                            sr[r][s] = s_sc[(s * 16 + col) * G + g];
                            if (HZ) zr[r][s] = s_zc[(s * 16 + col) * G + g];
                        }
                    }
    #pragma unroll
                    for (int kk = 0; kk < 4; kk++) {
                        if constexpr (NT > 2) {
                            /* wide waves: the NT weight fragments first, then one
                             * activation fragment at a time (registers) */
                            h8 bf[NT];
    #pragma unroll
                            for (int s = 0; s < NT; s++) {
                                const f16 sc = __builtin_bit_cast(f16, sr[r][s]);
                                const f16 zc = HZ ? __builtin_bit_cast(f16, zr[r][s]) : (f16)0.0f;
                                bf[s] = dequant8<HZ>(wr[r][s][kk], (h2){sc, sc}, (h2){zc, zc},
                                                     nib_mask, nib_one);
                            }
    #pragma unroll
                            for (int t = 0; t < TV; t++) {
                                const h8 af =
                                    *(const h8*)(abuf + (16 * t + col) * PF_AROW + 32 * j + 8 * kk);
    #pragma unroll
                                for (int s = 0; s < NT; s++)
                                    acc[t][s] = mfma16x16x32(af, bf[s], acc[t][s]);
                            }
                            __builtin_amdgcn_sched_barrier(0);
                        } else {
                            h8 af[TV];
    #pragma unroll
                            for (int t = 0; t < TV; t++)
                                af[t] = *(const h8*)(abuf + (16 * t + col) * PF_AROW + 32 * j + 8 * kk);
    #pragma unroll
                            for (int s = 0; s < NT; s++) {
                                const f16 sc = __builtin_bit_cast(f16, sr[r][s]);
                                const f16 zc = HZ ? __builtin_bit_cast(f16, zr[r][s]) : (f16)0.0f;
                                const h8 bf = dequant8<HZ>(wr[r][s][kk], (h2){sc, sc}, (h2){zc, zc},
                                                           nib_mask, nib_one);
    #pragma unroll
                                for (int t = 0; t < TV; t++)
                                    acc[t][s] = mfma16x16x32(af[t], bf, acc[t][s]);
                            }
                        }
                    }
                    __syncthreads();
                }
            }
        }
    }

    /* epilogue: lane holds D[4 (l/16) + v][l % 16] of each 16 x 16 tile */
#pragma unroll
    for (int t = 0; t < TV; t++) {
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int r = 16 * t + 4 * j + v;
            if (r < nv) {
                if (GATEUP) {
                    const float wrt = s_wr[r];
#pragma unroll
                    for (int s = 0; s < NT / 2; s++) {
                        const float g = acc[t][s][v], u = acc[t][NT / 2 + s][v];
                        const float h = silu_f(g) * u * wrt;
                        const int c = by * FEAT + wave * (FEAT / WV) + 16 * s + col;
                        P.H[(size_t)(p0 + r) * P.inter + c] = __builtin_bit_cast(uint16_t, (f16)h);
                    }
                } else {
#pragma unroll
                    for (int s = 0; s < NT; s++) {
                        const int c = by * DROWS + wave * (DROWS / WV) + 16 * s + col;
                        P.Y[(size_t)(p0 + r) * P.hidden + c] =
                            __builtin_bit_cast(uint16_t, (f16)acc[t][s][v]);
                    }
                }
            }
        }
    }
}

/* out[t][c] (+)= sum over slots k (in order) of y'[inv[t * top_k1 + k]][c];
 * 8 columns per thread with 16-byte loads (hidden % 256 == 0). */
__global__ __launch_bounds__(256) void pf_combine_kernel(const PfParams P) {
    const int c8 = P.hidden / 8;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)P.n_tokens * c8) return;
    const int t = (int)(i / c8), c = 8 * (int)(i - (size_t)t * c8);
    float y[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (P.top_k1 <= PF_COMBINE_SLOTS) {
        /* every slot's position, then every row, then the sum in slot
         * order: two round trips instead of two per slot */
        int pv[PF_COMBINE_SLOTS];
#pragma unroll
        for (int k = 0; k < PF_COMBINE_SLOTS; k++)
            pv[k] = k < P.top_k1 ? P.inv[t * P.top_k1 + k] : -1;
        h8 v[PF_COMBINE_SLOTS];
#pragma unroll
        for (int k = 0; k < PF_COMBINE_SLOTS; k++)
            v[k] = pv[k] >= 0 ? *(const h8*)(P.Y + (size_t)pv[k] * P.hidden + c) : (h8){};
#pragma unroll
        for (int k = 0; k < PF_COMBINE_SLOTS; k++)
            if (pv[k] >= 0) {
#pragma unroll
                for (int q = 0; q < 8; q++) y[q] += (float)v[k][q];
            }
    } else {
        for (int k = 0; k < P.top_k1; k++) {
            const int p = P.inv[t * P.top_k1 + k];
            if (p >= 0) {
                const h8 v = *(const h8*)(P.Y + (size_t)p * P.hidden + c);
#pragma unroll
                for (int q = 0; q < 8; q++) y[q] += (float)v[q];
            }
        }
    }
    const size_t o = (size_t)t * P.hidden + c;
    if (P.out32) {
        if (P.accumulate) {
            const f4 a = *(const f4*)(P.out32 + o), b = *(const f4*)(P.out32 + o + 4);
#pragma unroll
            for (int q = 0; q < 4; q++) { y[q] += a[q]; y[4 + q] += b[q]; }
        }
        *(f4*)(P.out32 + o) = (f4){y[0], y[1], y[2], y[3]};
        *(f4*)(P.out32 + o + 4) = (f4){y[4], y[5], y[6], y[7]};
    }
    if (P.out16) {
        h8 h;
#pragma unroll
        for (int q = 0; q < 8; q++) h[q] = (f16)y[q];
        *(h8*)(P.out16 + o) = h;
    }
}

/* ======================================================================= */
/* host side                                                                */
/* ======================================================================= */

struct PfWs {
    size_t table1, idx1, w1, counts, offsets, order, inv, ntiles, tiles, H, Y, total;
    int max_tiles;
};

static PfWs pf_ws_layout(const WispExpertLayout* L, int n_tokens, int top_k, int n_experts,
                         int has_shared) {
    PfWs w;
    const size_t k1 = (size_t)top_k + (has_shared ? 1 : 0);
    const size_t e1 = (size_t)n_experts + (has_shared ? 1 : 0);
    const size_t np = (size_t)n_tokens * k1;
    w.max_tiles = (int)((np + PF_BM - 1) / PF_BM + e1);
    size_t off = 0;
    w.table1 = off; off = align_up(off + e1 * sizeof(void*), 256);
    w.idx1 = off; off = align_up(off + np * 4, 256);
    w.w1 = off; off = align_up(off + np * 4, 256);
    w.counts = off; off = align_up(off + e1 * 4, 256);
    w.offsets = off; off = align_up(off + (e1 + 1) * 4, 256);
    w.order = off; off = align_up(off + np * 4, 256);
    w.inv = off; off = align_up(off + np * 4, 256);
    w.ntiles = off; off = align_up(off + PF_CLASSES * 4, 256);
    w.tiles = off; off = align_up(off + (size_t)PF_CLASSES * w.max_tiles * 16, 256);
    w.H = off; off = align_up(off + np * L->rows[0] * 2, 256);
    w.Y = off; off = align_up(off + np * L->cols[0] * 2, 256);
    w.total = off;
    return w;
}

static bool pf_shape_ok(const WispExpertLayout* L) {
    if (wisp_expert_layout_check(L) != hipSuccess) return false;
    const uint32_t inter = L->rows[0], hidden = L->cols[0];
    /* gate/up n-blocks of 128 h features, down n-blocks of 256 rows, group
     * size a power of two >= 32 (one scale per lane's 32 K values) */
    return inter % 128 == 0 && hidden % 256 == 0 && L->group_size >= 32;
}

extern "C" size_t wisp_moe_prefill_workspace_bytes(const WispExpertLayout* L, int n_tokens,
                                                   int top_k, int n_experts, int has_shared) {
    if (!L || n_tokens < 1 || top_k < 1 || n_experts < 1 || n_experts + 1 > PF_MAX_EXPERTS1)
        return 0;
    return pf_ws_layout(L, n_tokens, top_k, n_experts, has_shared).total;
}

/* One launch per tile class (sub-tiles per tile 2 / 4 / 8), each with its
 * own register budget; eight waves and a ring of four weight blocks measured
 * best for every class on MI355X (deeper rings cost occupancy). */
/* One class: scales (and zeros) staged in LDS when the image fits `budget`
 * and PF_SCALE_PIECES pieces per lane, else loaded per step. */
template <bool GATEUP, bool HZ, int TV, int R, int WV, int NT>
static void pf_launch_one(const PfParams& P, int gx, int cls, size_t budget, hipStream_t s) {
    const int K = GATEUP ? P.hidden : P.inter;
    const int G = K / P.gs;
    const size_t lds = (size_t)WV * NT * 16 * G * 2 * (HZ ? 2 : 1);
    const int ny = GATEUP ? P.inter / (8 * NT * WV) : P.hidden / (16 * NT * WV);
    if (lds <= budget && 2 * G <= 64 * PF_SCALE_PIECES) {
        /* the small tiles' down K loop in one straight-line chunk when it
         * divides (no pipeline refill at chunk edges: 2.75 -> 2.74 ms;
         * their gate/up loop in 28- or 56-block chunks needed more
         * registers and was no faster or slower) */
        constexpr int CS = TV <= 4 && !GATEUP ? PF_SMALL_CHUNK_DN : PF_CHUNK;
        auto k = (K / 128) % CS == 0 ? pf_gemm_kernel<GATEUP, HZ, TV, R, WV, true, NT, CS>
                 : (K / 128) % PF_CHUNK == 0 ? pf_gemm_kernel<GATEUP, HZ, TV, R, WV, true, NT, PF_CHUNK>
                                            : pf_gemm_kernel<GATEUP, HZ, TV, R, WV, true, NT>;
        if (lds > 65536)
            (void)hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)lds);
        hipLaunchKernelGGL(k, dim3(gx, ny), dim3(64 * WV), lds, s, P, cls);
    } else {
        hipLaunchKernelGGL((pf_gemm_kernel<GATEUP, HZ, TV, R, WV, false, NT>), dim3(gx, ny),
                           dim3(64 * WV), 0, s, P, cls);
    }
}

/* The full 128-token tiles without zero points: 4 row tiles per wave
 * (256 h features or 512 output rows per workgroup, ring of 2: measured
 * 1 % faster on the DeepSeek-V3 2048-token layer than a ring of 3), so each
 * activation fragment read from LDS feeds 4 MFMAs instead of 2; it fits
 * 256 VGPRs only with the scales in LDS and no zeros. Returns false when
 * the shape or the scale image does not allow it. */
template <bool GATEUP, bool HZ>
static bool pf_launch_wide(const PfParams& P, int gx, hipStream_t s) {
    if constexpr (HZ) {
        return false;
    } else {
        constexpr int NTW = 4;
        const int K = GATEUP ? P.hidden : P.inter;
        const int G = K / P.gs;
        const size_t lds = (size_t)PF_WAVES * NTW * 16 * G * 2;
        if (P.inter % (8 * NTW * PF_WAVES) || P.hidden % (16 * NTW * PF_WAVES) ||
            lds > PF_SCALE_LDS_WIDE || 2 * G > 64 * PF_SCALE_PIECES)
            return false;
        /* down in one chunk when it divides (2.672 -> 2.666 ms; the gate/up
         * loop in chunks of 14 or 28 blocks spilled and was slower) */
        constexpr int WC = GATEUP ? PF_CHUNK : PF_WIDE_CHUNK_DN;
        auto k = (K / 128) % WC == 0
                     ? pf_gemm_kernel<GATEUP, false, 8, PF_WIDE_RING, PF_WAVES, true, NTW, WC>
                     : pf_gemm_kernel<GATEUP, false, 8, PF_WIDE_RING, PF_WAVES, true, NTW>;
        if (lds > 65536)
            (void)hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)lds);
        const int ny = GATEUP ? P.inter / (8 * NTW * PF_WAVES) : P.hidden / (16 * NTW * PF_WAVES);
        hipLaunchKernelGGL(k, dim3(gx, ny), dim3(64 * PF_WAVES), lds, s, P, 2);
        return true;
    }
}

/* Eight waves of 2 row tiles and a ring of four weight blocks for the other
 * tiles (measured on MI355X: 4 row tiles per wave for the small classes cost
 * a workgroup per CU and were slower, as were 4-wave workgroups with
 * accumulators in AGPRs for the full tiles). */
template <bool GATEUP, bool HZ>
static void pf_launch_full(const PfParams& P, const int* gx, hipStream_t s) {
    if (!pf_launch_wide<GATEUP, HZ>(P, gx[2], s))
        pf_launch_one<GATEUP, HZ, 8, PF_RING, PF_WAVES, PF_NT>(P, gx[2], 2, PF_SCALE_LDS_MAX, s);
}
template <bool GATEUP, bool HZ>
static void pf_launch_small(const PfParams& P, const int* gx, hipStream_t s) {
    pf_launch_one<GATEUP, HZ, 4, PF_RING, PF_WAVES, PF_NT>(P, gx[1], 1, PF_SCALE_LDS_MAX, s);
    /* ring of 3 for the <= 32-token tiles: 79 VGPRs, 6 waves per SIMD (3
     * workgroups per CU instead of 2), 1.5 % faster layer */
    pf_launch_one<GATEUP, HZ, 2, 3, PF_WAVES, PF_NT>(P, gx[0], 0, PF_SCALE_LDS_MAX, s);
}

/* The library's second stream (declared in hip_common.h). Prefill runs
 * its small tiles there: the tiles of 65-128 tokens are bound by the matrix
 * cores and run one workgroup per CU (DeepSeek-V3, 2048 tokens: 928 gate/up
 * workgroups, so the fourth round of 256 has 160 and leaves CUs idle); the
 * small tiles are bound by memory and fill the CUs the others leave free. */
#define SIDE_MAX_DEVICES 64
std::mutex wisp_amd__side_mu;
static SideStream g_side[SIDE_MAX_DEVICES];

hipError_t wisp_amd__side(hipStream_t s, SideStream* out) {
    *out = SideStream{nullptr, nullptr, nullptr};
    int dev = 0, cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    dev = s ? hipGetStreamDeviceId(s) : cur;
    if (dev < 0) return hipErrorInvalidResourceHandle;
    if (dev >= SIDE_MAX_DEVICES) return hipErrorInvalidDevice;
    if (!g_side[dev].s2) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if ((e = hipStreamIsCapturing(s, &cs)) != hipSuccess) return e;
        if (cs != hipStreamCaptureStatusNone) return hipSuccess;
        if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
        SideStream n{nullptr, nullptr, nullptr};
        e = hipStreamCreateWithFlags(&n.s2, hipStreamNonBlocking);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&n.fork, hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&n.join, hipEventDisableTiming);
        if (cur != dev) (void)hipSetDevice(cur);
        if (e != hipSuccess) return e;
        g_side[dev] = n;
    }
    *out = g_side[dev];
    return hipSuccess;
}

extern "C" hipError_t wisp_gpu_expert_offsets(const int* d_topk_idx, int n_tokens, int top_k,
                                              int n_experts, int* d_counts, int* d_offsets,
                                              int* d_order, int* d_inv, hipStream_t s);

extern "C" hipError_t wisp_gpu_moe_prefill_int4(const void* const* d_expert_table,
                                                const void* d_shared_blob,
                                                const WispExpertLayout* L, const wisp_half* d_x,
                                                int n_tokens, const int* d_topk_idx,
                                                const float* d_topk_w, int top_k, int n_experts,
                                                void* d_workspace, size_t workspace_bytes,
                                                int accumulate, float* d_out_f32,
                                                wisp_half* d_out_f16, hipStream_t s) {
    if (!L || n_tokens < 1 || top_k < 1 || n_experts < 1 || n_experts + 1 > PF_MAX_EXPERTS1 ||
        !d_expert_table || !d_x || !d_topk_idx || !d_topk_w || !d_workspace ||
        (!d_out_f32 && !d_out_f16) || ((uintptr_t)d_x % 16) || ((uintptr_t)d_out_f32 % 16) ||
        ((uintptr_t)d_out_f16 % 16))
        return hipErrorInvalidValue;
    if (!pf_shape_ok(L)) return hipErrorInvalidValue;
    const int sh = d_shared_blob ? 1 : 0;
    const PfWs w = pf_ws_layout(L, n_tokens, top_k, n_experts, sh);
    if (workspace_bytes < w.total) return hipErrorInvalidValue;
    if ((long)n_tokens * (top_k + sh) > (1L << 30)) return hipErrorInvalidValue;

    PfParams P;
    for (int m = 0; m < 3; m++) {
        P.p_off[m] = L->packed_off[m];
        P.s_off[m] = L->scales_off[m];
        P.z_off[m] = L->zeros_off[m];
    }
    P.hidden = (int)L->cols[0];
    P.inter = (int)L->rows[0];
    P.gs = (int)L->group_size;
    P.has_zeros = L->has_zeros ? 1 : 0;
    P.n_tokens = n_tokens;
    P.top_k1 = top_k + sh;
    P.n_experts1 = n_experts + sh;
    P.max_tiles = w.max_tiles;
    char* ws = (char*)d_workspace;
    P.table1 = (const uint8_t**)(ws + w.table1);
    P.idx1 = (int*)(ws + w.idx1);
    P.w1 = (float*)(ws + w.w1);
    P.counts = (int*)(ws + w.counts);
    P.offsets = (int*)(ws + w.offsets);
    P.order = (int*)(ws + w.order);
    P.inv = (int*)(ws + w.inv);
    P.n_tiles = (int*)(ws + w.ntiles);
    P.tiles = (int4*)(ws + w.tiles);
    P.H = (uint16_t*)(ws + w.H);
    P.Y = (uint16_t*)(ws + w.Y);
    P.x = (const uint16_t*)d_x;
    P.out32 = d_out_f32;
    P.out16 = (uint16_t*)d_out_f16;
    P.accumulate = accumulate ? 1 : 0;

    const int n_pairs = n_tokens * P.top_k1;
    const int prep_n = n_pairs > n_experts ? n_pairs : n_experts;
    hipLaunchKernelGGL(pf_prep_kernel, dim3((prep_n + 255) / 256), dim3(256), 0, s, P,
                       d_expert_table, d_shared_blob, d_topk_idx, d_topk_w, top_k, n_experts);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    e = wisp_gpu_expert_offsets(P.idx1, n_tokens, P.top_k1, P.n_experts1, P.counts, P.offsets,
                                P.order, P.inv, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(pf_tiles_kernel, dim3(1), dim3(PF_TILE_THREADS), 0, s, P);
    const bool hz = P.has_zeros != 0;
    /* grid.x per class: an upper bound on its tile count */
    const int np = n_tokens * P.top_k1;
    int gx[PF_CLASSES] = {P.n_experts1, np / 33 + P.n_experts1, np / 65 + P.n_experts1};
    for (int k = 0; k < PF_CLASSES; k++) {
        gx[k] = gx[k] < P.max_tiles ? gx[k] : P.max_tiles;
        gx[k] = (gx[k] + PF_XCDS - 1) / PF_XCDS * PF_XCDS;   /* whole dies (XCD-aware order) */
    }
    /* small tiles (gate/up, then their down) on the side stream, full
     * tiles on the caller's; the caller's stream waits for both before the
     * combine. EV_PF_GATEUP / EV_PF_DOWN time the full tiles' launches. */
    SideStream side;
    std::lock_guard<std::mutex> lk(wisp_amd__side_mu);
    if ((e = wisp_amd__side(s, &side)) != hipSuccess) return e;
    /* no second stream yet and the caller's stream is being captured:
     * every class runs on the caller's stream (the next call made outside
     * a capture creates it) */
    hipStream_t s2 = side.s2 ? side.s2 : s;
    const hipEvent_t fork = side.fork, join = side.join;
    if (fork) {
        if ((e = hipEventRecord(fork, s)) != hipSuccess) return e;
        if ((e = hipStreamWaitEvent(s2, fork, 0)) != hipSuccess) return e;
    }
    if (hz) {
        pf_launch_small<true, true>(P, gx, s2);
        pf_launch_small<false, true>(P, gx, s2);
    } else {
        pf_launch_small<true, false>(P, gx, s2);
        pf_launch_small<false, false>(P, gx, s2);
    }
    if (join && (e = hipEventRecord(join, s2)) != hipSuccess) return e;
    ev_before(EV_PF_GATEUP, s);
    if (hz) pf_launch_full<true, true>(P, gx, s);
    else pf_launch_full<true, false>(P, gx, s);
    ev_after(EV_PF_GATEUP, s);
    ev_before(EV_PF_DOWN, s);
    if (hz) pf_launch_full<false, true>(P, gx, s);
    else pf_launch_full<false, false>(P, gx, s);
    ev_after(EV_PF_DOWN, s);
    if (join && (e = hipStreamWaitEvent(s, join, 0)) != hipSuccess) return e;
    const size_t n_out = (size_t)n_tokens * (P.hidden / 8);
    hipLaunchKernelGGL(pf_combine_kernel, dim3((unsigned)((n_out + 255) / 256)), dim3(256), 0, s,
                       P);
    return hipGetLastError();
}
