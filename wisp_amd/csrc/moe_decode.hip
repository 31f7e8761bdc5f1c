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
#define DEC_MAX_WAVES 8
#define DEC_CHUNK_BLOCKS 32   /* down-projection K chunk per workgroup: 4096 elements */

struct DecodeParams {
    uint64_t p_off[3], s_off[3], z_off[3];
    int hidden, inter, gs, has_zeros;
    int gshift;           /* log2(gs * NG / 128): block -> group index */
    int n_chunks;         /* down-projection K chunks: ceil(inter/128 / DEC_CHUNK_BLOCKS) */
    uint32_t m_lo, m_hi, one024;  /* unpack masks 0x000F000F, 0x00F000F0, 0x64006400 */
    int max_u;
    int* n_unique;
    const uint8_t** ublob;
    float* uw;            /* [max_u][4] routing weight of each token     */
    uint16_t* xperm;      /* [M][hidden] permuted fp16 activations        */
    uint16_t* hperm;      /* [max_u][M][inter] permuted fp16 h'           */
    float* part;          /* [max_u][n_chunks][M][hidden] down partials   */
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

/* Copies M activation rows (K range [k0, k0 + xk) of rows of length K) into
 * the LDS x image with 16-byte accesses. */
template <int M>
__device__ __forceinline__ void stage_x(uint8_t* smem, const LdsMap& L, const uint16_t* src, int K,
                                        int k0, int xk) {
    uint16_t* xs = (uint16_t*)(smem + L.x_off);
    const int per_row = xk / 8;
    for (int i = threadIdx.x; i < M * per_row; i += blockDim.x) {
        const int v = i / per_row, c = i - v * per_row;
        *(u4*)(xs + v * L.XR + c * 8) = *(const u4*)(src + (size_t)v * K + k0 + c * 8);
    }
}

/* Copies the raw scale (or zero) bits of 16 consecutive rows starting at
 * row r0 of a [rows][G] fp16 table, groups [g0, g0 + gn), into dst[16][gn]. */
__device__ __forceinline__ void stage_groups(uint16_t* dst, const uint16_t* tab, int G, int r0,
                                             int g0, int gn) {
    for (int i = threadIdx.x; i < 16 * gn; i += blockDim.x) {
        const int r = i / gn, g = i - r * gn;
        dst[i] = tab[(size_t)(r0 + r) * G + g0 + g];
    }
}

/* Streams blocks [b0, b1) (absolute block indices of the weight rows) of NT
 * row tiles into tot, in batches of PF blocks: the weight loads of a whole
 * batch are issued first, then the batch is computed. No load result is
 * carried across loop iterations, so the compiler never has to copy (and
 * therefore wait on) an in-flight register; latency is covered by the other
 * resident waves. Activations and scales come from the LDS image, whose K
 * range starts at block xb0 and whose groups start at g_lo. The last batch
 * clamps its loads to the last block (the repeats hit in cache) and
 * computes its padding slots with zero scale. */
template <int M, int NG, int NT, int PF, bool HZ>
__device__ __forceinline__ void stream_blocks(const uint8_t* const (&wp)[NT], const uint8_t* smem,
                                              const LdsMap& L, int b0, int b1, int xb0, int g_lo,
                                              int gshift, int col, int j, uint32_t m_lo,
                                              uint32_t m_hi, uint32_t one024,
                                              float (&tot)[NT][M]) {
    constexpr int B = PF;
    if (b0 >= b1) return;
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
    for (int base = b0; base < b1; base += B) {
        u4 w[B][NT];
#pragma unroll
        for (int p = 0; p < B; p++) {
            const int bb = min(base + p, b1 - 1);
#pragma unroll
            for (int s = 0; s < NT; s++) w[p][s] = *(const u4*)(wp[s] + (size_t)bb * 64);
        }
#pragma unroll
        for (int p = 0; p < B; p++) {
            const int b = base + p;
            const int bc = min(b, b1 - 1);
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
            block_step<M, NG, NT, HZ>(xa, w[p], gamma, sc, zc, b < b1, m_lo, m_hi, one024, tot);
        }
    }
}

/* ======================================================================= */
/* gate/up + SiLU                                                           */
/* ======================================================================= */

/* grid (inter / (16 TILES), max_u); workgroup = TILES gate + TILES up row
 * tiles of unique expert blockIdx.y over the full hidden K, waves split K. */
template <int M, int NG, int TILES, int PF, bool HZ>
__global__ __launch_bounds__(64 * DEC_MAX_WAVES) void gateup_kernel(const DecodeParams P) {
    constexpr int NT = 2 * TILES;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int u = blockIdx.y;
    if (u >= *P.n_unique) return;
    const uint8_t* blob = P.ublob[u];
    const int K = P.hidden;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int col = lane & 15, j = lane >> 4;
    const int r0 = blockIdx.x * 16 * TILES;
    const int nblk = K >> 7;
    const int G = K / P.gs;
    const int b0 = wave * nblk / nw, b1 = (wave + 1) * nblk / nw;
    const LdsMap L = lds_map(M, NT, K, G, HZ, nw);

    const uint8_t* wp[NT];
#pragma unroll
    for (int s = 0; s < NT; s++) {
        const int mat = s < TILES ? 0 : 1;
        wp[s] = blob + P.p_off[mat] + (size_t)(r0 + 16 * (s % TILES) + col) * (K / 2) + 16 * j;
    }
    stage_x<M>(smem, L, P.xperm, K, 0, K);
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
    __syncthreads();

    float tot[NT][M];
#pragma unroll
    for (int s = 0; s < NT; s++)
#pragma unroll
        for (int v = 0; v < M; v++) tot[s][v] = 0.0f;
    stream_blocks<M, NG, NT, PF, HZ>(wp, smem, L, b0, b1, 0, 0, P.gshift, col, j, P.m_lo, P.m_hi,
                                     P.one024, tot);

    float* red = (float*)(smem + L.red_off);
    if (lane < 16) {
#pragma unroll
        for (int s = 0; s < NT; s++)
#pragma unroll
            for (int v = 0; v < M; v++) red[((wave * NT + s) * 16 + col) * M + v] = tot[s][v];
    }
    __syncthreads();
    for (int o = threadIdx.x; o < TILES * 16 * M; o += blockDim.x) {
        const int v = o % M, rc = o / M, q = rc / 16, c = rc % 16;
        float g = 0.0f, up = 0.0f;
        for (int ww = 0; ww < nw; ww++) {
            g += red[((ww * NT + q) * 16 + c) * M + v];
            up += red[((ww * NT + TILES + q) * 16 + c) * M + v];
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
/* down (per expert and K chunk) + combine                                  */
/* ======================================================================= */

/* grid (hidden / (16 TILES), max_u * n_chunks): workgroup (row tile,
 * unique expert u, K chunk c of DEC_CHUNK_BLOCKS blocks) writes
 * part[u][c][v][row] = down_u[row, chunk] . h'_u[v][chunk] (routing weight
 * already folded into h'). */
template <int M, int NG, int TILES, int PF, bool HZ>
__global__ __launch_bounds__(64 * DEC_MAX_WAVES) void down_kernel(const DecodeParams P) {
    constexpr int NT = TILES;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int nch = P.n_chunks;
    const int u = blockIdx.y / nch, c = blockIdx.y - u * nch;
    if (u >= *P.n_unique) return;
    const uint8_t* blob = P.ublob[u];
    const int K = P.inter, H = P.hidden;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int col = lane & 15, j = lane >> 4;
    const int r0 = blockIdx.x * 16 * TILES;
    const int nblk = K >> 7;
    const int G = K / P.gs;
    const int cb0 = c * DEC_CHUNK_BLOCKS, cb1 = min(cb0 + DEC_CHUNK_BLOCKS, nblk);
    const int g_lo = (cb0 * NG) >> P.gshift, g_hi = (((cb1 * NG) - 1) >> P.gshift) + 1;
    const int nb = cb1 - cb0;
    const int b0 = cb0 + wave * nb / nw, b1 = cb0 + (wave + 1) * nb / nw;
    const LdsMap L = lds_map(M, NT, DEC_CHUNK_BLOCKS * 128, g_hi - g_lo, HZ, nw);

    const uint8_t* wp[NT];
#pragma unroll
    for (int s = 0; s < NT; s++)
        wp[s] = blob + P.p_off[2] + (size_t)(r0 + 16 * s + col) * (K / 2) + 16 * j;
    stage_x<M>(smem, L, P.hperm + (size_t)u * M * K, K, cb0 * 128, nb * 128);
#pragma unroll
    for (int s = 0; s < NT; s++) {
        stage_groups((uint16_t*)(smem + L.sc_off) + s * 16 * L.GS,
                     (const uint16_t*)(blob + P.s_off[2]), G, r0 + 16 * s, g_lo, L.GS);
        if (HZ)
            stage_groups((uint16_t*)(smem + L.zc_off) + s * 16 * L.GS,
                         (const uint16_t*)(blob + P.z_off[2]), G, r0 + 16 * s, g_lo, L.GS);
    }
    __syncthreads();

    float tot[NT][M];
#pragma unroll
    for (int s = 0; s < NT; s++)
#pragma unroll
        for (int v = 0; v < M; v++) tot[s][v] = 0.0f;
    stream_blocks<M, NG, NT, PF, HZ>(wp, smem, L, b0, b1, cb0, g_lo, P.gshift, col, j, P.m_lo,
                                     P.m_hi, P.one024, tot);

    float* red = (float*)(smem + L.red_off);
    if (lane < 16) {
#pragma unroll
        for (int s = 0; s < NT; s++)
#pragma unroll
            for (int v = 0; v < M; v++) red[((wave * NT + s) * 16 + col) * M + v] = tot[s][v];
    }
    __syncthreads();
    for (int o = threadIdx.x; o < TILES * 16 * M; o += blockDim.x) {
        const int v = o % M, rc = o / M, q = rc / 16, cc = rc % 16;
        float y = 0.0f;
        for (int ww = 0; ww < nw; ww++) y += red[((ww * NT + q) * 16 + cc) * M + v];
        P.part[(((size_t)u * nch + c) * M + v) * H + r0 + 16 * q + cc] = y;
    }
}

/* out[v][r] (+)= sum over unique experts u (list order) and K chunks c of
 * part[u][c][v][r]. */
__global__ __launch_bounds__(256) void combine_kernel(const DecodeParams P, int M, float* out32,
                                                      uint16_t* out16, int accumulate) {
    const int n_u = *P.n_unique;
    const int H = P.hidden, nch = P.n_chunks;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= M * H) return;
    const int v = i / H, r = i - v * H;
    float y = 0.0f;
    for (int u = 0; u < n_u; u++)
        for (int c = 0; c < nch; c++) y += P.part[(((size_t)u * nch + c) * M + v) * H + r];
    if (out32) {
        if (accumulate) y += out32[i];
        out32[i] = y;
    }
    if (out16) out16[i] = __builtin_bit_cast(uint16_t, (f16)y);
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
    const bool gs_ok = gs >= 32 && (gs & (gs - 1)) == 0;
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
    size_t nu, ublob, uw, xperm, hperm, part, total;
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
    const size_t nch = ((L->rows[0] / 128) + DEC_CHUNK_BLOCKS - 1) / DEC_CHUNK_BLOCKS;
    w.part = off; off = align_up(off + (size_t)w.max_u * nch * M * L->cols[0] * 4, 256);
    w.total = off;
    return w;
}

extern "C" size_t wisp_moe_decode_workspace_bytes(const WispExpertLayout* L, int n_tokens,
                                                  int top_k, int has_shared) {
    if (!L || n_tokens < 1 || n_tokens > DEC_MAX_TOKENS || top_k < 1 || top_k > DEC_MAX_TOPK)
        return 0;
    return ws_layout(L, n_tokens, top_k, has_shared).total;
}

/* Launch shape of the two expert kernels. Values <= 0 select the built-in
 * heuristic. Set only through wisp_amd__decode_config (tuning sweeps). */
struct DecodeCfg {
    int gu_tiles, gu_waves, gu_pf, dn_tiles, dn_waves, dn_pf;
};
static DecodeCfg g_dec_cfg = {0, 0, 0, 0, 0, 0};

extern "C" void wisp_amd__decode_config(int gu_tiles, int gu_waves, int gu_pf, int dn_tiles,
                                        int dn_waves, int dn_pf) {
    g_dec_cfg = {gu_tiles, gu_waves, gu_pf, dn_tiles, dn_waves, dn_pf};
}

/* Waves per workgroup so that each wave streams about `per_wave` blocks. */
static int waves_for(int blocks_total, int per_wave, int max_waves) {
    int w = blocks_total / per_wave;
    if (w < 1) w = 1;
    if (w > max_waves) w = max_waves;
    return w;
}

template <int M, int NG, int TILES, int PF, bool HZ>
static void launch_gateup(const DecodeParams& P, int waves, hipStream_t s) {
    const LdsMap L = lds_map(M, 2 * TILES, P.hidden, P.hidden / P.gs, HZ, waves);
    auto k = gateup_kernel<M, NG, TILES, PF, HZ>;
    if (L.bytes > 65536)
        (void)hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, L.bytes);
    hipLaunchKernelGGL(k, dim3(P.inter / (16 * TILES), P.max_u), dim3(64 * waves), L.bytes, s, P);
}

template <int M, int NG, int TILES, int PF, bool HZ>
static void launch_down(const DecodeParams& P, int waves, hipStream_t s) {
    /* LDS sized for the largest chunk: full DEC_CHUNK_BLOCKS and its groups */
    const int ng_hi = (((DEC_CHUNK_BLOCKS * NG) - 1) >> P.gshift) + 2;
    const LdsMap L = lds_map(M, TILES, DEC_CHUNK_BLOCKS * 128, ng_hi, HZ, waves);
    auto k = down_kernel<M, NG, TILES, PF, HZ>;
    if (L.bytes > 65536)
        (void)hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, L.bytes);
    hipLaunchKernelGGL(k, dim3(P.hidden / (16 * TILES), P.max_u * P.n_chunks), dim3(64 * waves),
                       L.bytes, s, P);
}

template <int M, int NG, bool HZ>
static void launch_compute(const DecodeParams& P, float* out32, uint16_t* out16, int accumulate,
                           hipStream_t s) {
    const DecodeCfg c = g_dec_cfg;
    const int gu_waves = c.gu_waves > 0 ? (c.gu_waves > DEC_MAX_WAVES ? DEC_MAX_WAVES : c.gu_waves)
                                        : waves_for(P.hidden / 128, 8, 4);
    const int chunk = (P.inter / 128) < DEC_CHUNK_BLOCKS ? (P.inter / 128) : DEC_CHUNK_BLOCKS;
    const int dn_waves = c.dn_waves > 0 ? (c.dn_waves > DEC_MAX_WAVES ? DEC_MAX_WAVES : c.dn_waves)
                                        : waves_for(chunk, 8, 4);
    /* Defaults (measured on MI355X at the Mixtral and DeepSeek-V3 decode
     * shapes): one row tile per matrix, batches of 2 blocks, about 8 blocks
     * per wave and at most 4 waves. Other tile / batch variants are built
     * for the common case only (group size >= 128, no zero points). */
    auto variant = [](int tiles, int pf) { return 10 * (tiles == 2 ? 2 : 1) + (pf == 8 ? 8 : (pf == 4 ? 4 : 2)); };
    const int gv = (NG == 1 && !HZ) ? variant(c.gu_tiles, c.gu_pf) : 0;
    const int dv = (NG == 1 && !HZ) ? variant(c.dn_tiles, c.dn_pf) : 0;
    ev_before(EV_GATEUP, s);
    switch (gv) {
        case 12: launch_gateup<M, 1, 1, 2, false>(P, gu_waves, s); break;
        case 14: launch_gateup<M, 1, 1, 4, false>(P, gu_waves, s); break;
        case 18: launch_gateup<M, 1, 1, 8, false>(P, gu_waves, s); break;
        case 22: launch_gateup<M, 1, 2, 2, false>(P, gu_waves, s); break;
        case 24: launch_gateup<M, 1, 2, 4, false>(P, gu_waves, s); break;
        default: launch_gateup<M, NG, 1, 2, HZ>(P, gu_waves, s); break;
    }
    ev_after(EV_GATEUP, s);
    ev_before(EV_DOWN, s);
    switch (dv) {
        case 12: launch_down<M, 1, 1, 2, false>(P, dn_waves, s); break;
        case 14: launch_down<M, 1, 1, 4, false>(P, dn_waves, s); break;
        case 18: launch_down<M, 1, 1, 8, false>(P, dn_waves, s); break;
        case 22: launch_down<M, 1, 2, 2, false>(P, dn_waves, s); break;
        case 24: launch_down<M, 1, 2, 4, false>(P, dn_waves, s); break;
        default: launch_down<M, NG, 1, 2, HZ>(P, dn_waves, s); break;
    }
    ev_after(EV_DOWN, s);
    ev_before(EV_COMBINE, s);
    const int n = M * P.hidden;
    hipLaunchKernelGGL(combine_kernel, dim3((n + 255) / 256), dim3(256), 0, s, P, M, out32, out16,
                       accumulate);
    ev_after(EV_COMBINE, s);
}

template <int M>
static void launch_ng(int ng, bool hz, const DecodeParams& P, float* o32, uint16_t* o16, int acc,
                      hipStream_t s) {
    if (ng == 1) {
        if (hz) launch_compute<M, 1, true>(P, o32, o16, acc, s);
        else launch_compute<M, 1, false>(P, o32, o16, acc, s);
    } else if (ng == 2) {
        if (hz) launch_compute<M, 2, true>(P, o32, o16, acc, s);
        else launch_compute<M, 2, false>(P, o32, o16, acc, s);
    } else {
        if (hz) launch_compute<M, 4, true>(P, o32, o16, acc, s);
        else launch_compute<M, 4, false>(P, o32, o16, acc, s);
    }
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
    {
        const int ngs = P.gs >= 128 ? P.gs : 128;   /* gs * NG */
        int sh = 0;
        while ((128 << sh) < ngs) sh++;
        P.gshift = sh;
    }
    P.n_chunks = ((P.inter / 128) + DEC_CHUNK_BLOCKS - 1) / DEC_CHUNK_BLOCKS;
    P.m_lo = 0x000F000Fu;
    P.m_hi = 0x00F000F0u;
    P.one024 = 0x64006400u;
    P.max_u = w.max_u;
    char* ws = (char*)d_workspace;
    P.n_unique = (int*)(ws + w.nu);
    P.ublob = (const uint8_t**)(ws + w.ublob);
    P.uw = (float*)(ws + w.uw);
    P.xperm = (uint16_t*)(ws + w.xperm);
    P.hperm = (uint16_t*)(ws + w.hperm);
    P.part = (float*)(ws + w.part);

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
    const bool hz = P.has_zeros != 0;
    switch (n_tokens) {
        case 1: launch_ng<1>(ng, hz, P, d_out_f32, d_out_f16, accumulate, s); break;
        case 2: launch_ng<2>(ng, hz, P, d_out_f32, d_out_f16, accumulate, s); break;
        case 3: launch_ng<3>(ng, hz, P, d_out_f32, d_out_f16, accumulate, s); break;
        default: launch_ng<4>(ng, hz, P, d_out_f32, d_out_f16, accumulate, s); break;
    }
    return hipGetLastError();
}
