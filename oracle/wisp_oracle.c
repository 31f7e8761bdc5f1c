/*
 * wisp_oracle.c — CPU oracle for the int4 routed-expert MoE path.
 *
 * TEST INFRASTRUCTURE ONLY (see wisp_oracle.h). Restates the reference's
 * scalar CPU semantics; the citations are to the reference tree.
 *
 * Parity status of each function (the checks live in tests/):
 *   orc_half_to_float / orc_float_to_half  pinned: exhaustive over all 2^16
 *       inputs against numpy's IEEE fp16, and against the reference helper.
 *   orc_unpack_int4 / orc_pack_int4 / orc_dequant_*  pinned: the reference's
 *       0x88 known answer (tests/test_adapters.py:262-267), the golden
 *       dequant fixture, and the compiled reference probe.
 *   orc_blob_*  pinned: the reference layout constants
 *       (tests/test_adapters.py:281-308) and the compiled reference parser.
 *   orc_gemv_int4 / orc_expert_ffn / orc_swiglu / orc_router_softmax_topk /
 *       orc_moe_combine  pinned against the reference's own scalar C compiled
 *       from its sources (oracle/_ref), plus a float64 brute force.
 *   orc_router_sigmoid_topk, orc_expert_offsets  build-defined (the reference
 *       has no counterpart); pinned by closed forms and brute force.
 */
#include "wisp_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#if defined(__x86_64__)
#include <immintrin.h>
#endif

/* ======================================================================= */
/* fp16 <-> fp32                                                            */
/* ======================================================================= */

float orc_half_to_float(uint16_t h) {
    /* Decode by value: sign * mantissa * 2^(exp-25) covers normals and
     * subnormals alike; exp 31 is inf/nan. Exact in fp32. */
    uint32_t sign = (uint32_t)(h >> 15);
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    float v;
    if (e == 31u) {
        uint32_t bits = (sign << 31) | 0x7F800000u | (m << 13);
        memcpy(&v, &bits, 4);
        return v;
    }
    if (e == 0u) v = ldexpf((float)m, -24);
    else v = ldexpf((float)(m | 0x400u), (int)e - 25);
    return sign ? -v : v;
}

uint16_t orc_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {                       /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    }
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);   /* overflow */
    if (ax < 0x38800000u) {
        /* Result is subnormal (or zero): quantise to multiples of 2^-24
         * with round-half-even, done on the exact integer mantissa. */
        if (ax < 0x33000000u) return sign;          /* < 2^-25 rounds to 0 */
        uint32_t e = ax >> 23;                      /* 102..112 */
        uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;                  /* value = mant*2^(e-150) */
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    /* Normal: rebias exponent, round 13 dropped bits half-even. */
    uint32_t r = ax - 0x38000000u;                  /* exponent 127 -> 15 */
    uint32_t q = r >> 13;
    uint32_t rem = r & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

uint16_t orc_float_to_half_trunc(float f) {
    /* Restates csrc/core/wisp_engine.c:77-91: truncating conversion with
     * flush-to-zero below 2^-25 and saturation to inf at exponent >= 31. */
    uint32_t bits;
    memcpy(&bits, &f, 4);
    uint32_t sign = (bits >> 16) & 0x8000u;
    int32_t e = (int32_t)((bits >> 23) & 0xFFu) - 112;
    uint32_t mant = bits & 0x7FFFFFu;
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        mant |= 0x800000u;
        return (uint16_t)(sign | (mant >> (uint32_t)(14 - e)));
    }
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)e << 10) | (mant >> 13));
}

/* ======================================================================= */
/* int4 format                                                              */
/* ======================================================================= */

static inline int nib_at(const uint8_t* packed, size_t i) {
    uint8_t b = packed[i >> 1];
    return (i & 1u) ? (b >> 4) : (b & 0x0F);
}

void orc_unpack_int4(const uint8_t* packed, size_t n, uint8_t* nib) {
    for (size_t i = 0; i < n; i++) nib[i] = (uint8_t)nib_at(packed, i);
}

void orc_pack_int4(const uint8_t* nib, size_t n, uint8_t* packed) {
    size_t nb = (n + 1) / 2;
    for (size_t b = 0; b < nb; b++) {
        uint8_t lo = nib[2 * b] & 0x0F;
        uint8_t hi = (2 * b + 1 < n) ? (nib[2 * b + 1] & 0x0F) : 0;
        packed[b] = (uint8_t)(lo | (hi << 4));
    }
}

void orc_dequant_f32(const uint8_t* packed, const uint16_t* scales,
                     const uint16_t* zeros, size_t n, int gs, float* out) {
    for (size_t i = 0; i < n; i++) {
        size_t g = i / (size_t)gs;
        float s = orc_half_to_float(scales[g]);
        float z = orc_half_to_float(zeros[g]);
        out[i] = (float)(nib_at(packed, i) - 8) * s + z;
    }
}

void orc_dequant_fp16(const uint8_t* packed, const uint16_t* scales,
                      const uint16_t* zeros, size_t n, int gs, uint16_t* out) {
    for (size_t i = 0; i < n; i++) {
        size_t g = i / (size_t)gs;
        float s = orc_half_to_float(scales[g]);
        float z = orc_half_to_float(zeros[g]);
        /* product first, then the add: two fp32 roundings, then fp16 RNE */
        float p = (float)(nib_at(packed, i) - 8) * s;
        out[i] = orc_float_to_half(p + z);
    }
}

/* ======================================================================= */
/* expert blob                                                              */
/* ======================================================================= */

static uint32_t rd32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
           ((uint32_t)p[3] << 24);
}
static uint64_t rd64(const uint8_t* p) {
    return (uint64_t)rd32(p) | ((uint64_t)rd32(p + 4) << 32);
}
static void wr32(uint8_t* p, uint32_t v) {
    for (int i = 0; i < 4; i++) p[i] = (uint8_t)(v >> (8 * i));
}
static void wr64(uint8_t* p, uint64_t v) {
    wr32(p, (uint32_t)v);
    wr32(p + 4, (uint32_t)(v >> 32));
}

int orc_blob_parse(const void* blob, size_t size, OrcBlobMeta* meta) {
    const uint8_t* b = (const uint8_t*)blob;
    if (!b || size < ORC_BLOB_HEADER) return -1;
    if (rd32(b) != ORC_BLOB_MAGIC || rd32(b + 4) != ORC_BLOB_VERSION ||
        rd32(b + 20) != 3u)
        return -2;
    memset(meta, 0, sizeof(*meta));
    meta->layer_id = rd32(b + 8);
    meta->expert_id = rd32(b + 12);
    meta->group_size = rd32(b + 16);
    uint64_t off = ORC_BLOB_HEADER;
    for (int m = 0; m < 3; m++) {
        const uint8_t* mh = b + 24 + 32 * m;
        meta->rows[m] = rd32(mh);
        meta->cols[m] = rd32(mh + 4);
        meta->packed_off[m] = off; off += rd64(mh + 8);
        meta->scales_off[m] = off; off += rd64(mh + 16);
        meta->zeros_off[m] = off;  off += rd64(mh + 24);
    }
    meta->total_bytes = off;
    return off > size ? -3 : 0;
}

static void mat_sizes(uint32_t rows, uint32_t cols, uint32_t gs,
                      uint64_t* pb, uint64_t* sb) {
    uint64_t n = (uint64_t)rows * cols;
    *pb = (n + 1) / 2;
    *sb = ((n + gs - 1) / gs) * 2;
}

size_t orc_blob_size(uint32_t inter, uint32_t hidden, uint32_t gs) {
    uint32_t r[3] = {inter, inter, hidden}, c[3] = {hidden, hidden, inter};
    size_t total = ORC_BLOB_HEADER;
    for (int m = 0; m < 3; m++) {
        uint64_t pb, sb;
        mat_sizes(r[m], c[m], gs, &pb, &sb);
        total += pb + 2 * sb;
    }
    return total;
}

size_t orc_blob_write(void* dst, uint32_t layer, uint32_t expert, uint32_t gs,
                      uint32_t inter, uint32_t hidden,
                      const uint8_t* const packed[3],
                      const uint16_t* const scales[3],
                      const uint16_t* const zeros[3]) {
    uint8_t* b = (uint8_t*)dst;
    uint32_t r[3] = {inter, inter, hidden}, c[3] = {hidden, hidden, inter};
    wr32(b, ORC_BLOB_MAGIC);
    wr32(b + 4, ORC_BLOB_VERSION);
    wr32(b + 8, layer);
    wr32(b + 12, expert);
    wr32(b + 16, gs);
    wr32(b + 20, 3u);
    uint64_t off = ORC_BLOB_HEADER;
    for (int m = 0; m < 3; m++) {
        uint64_t pb, sb;
        mat_sizes(r[m], c[m], gs, &pb, &sb);
        uint8_t* mh = b + 24 + 32 * m;
        wr32(mh, r[m]);
        wr32(mh + 4, c[m]);
        wr64(mh + 8, pb);
        wr64(mh + 16, sb);
        wr64(mh + 24, sb);
        memcpy(b + off, packed[m], pb); off += pb;
        memcpy(b + off, scales[m], sb); off += sb;
        memcpy(b + off, zeros[m], sb);  off += sb;
    }
    return (size_t)off;
}

/* ======================================================================= */
/* expert math                                                              */
/* ======================================================================= */

void orc_gemv_int4(const uint8_t* packed, const uint16_t* scales,
                   const uint16_t* zeros, const float* x, float* y,
                   int rows, int cols, int gs) {
    int r;
    #pragma omp parallel for schedule(static)
    for (r = 0; r < rows; r++) {
        size_t base = (size_t)r * (size_t)cols;
        float acc = 0.0f;
        for (int c = 0; c < cols; c++) {
            size_t i = base + (size_t)c;
            size_t g = i / (size_t)gs;
            float w = (float)(nib_at(packed, i) - 8) * orc_half_to_float(scales[g]);
            w = w + orc_half_to_float(zeros[g]);
            acc = acc + w * x[c];
        }
        y[r] = acc;
    }
}

void orc_gemv_int4_f64(const uint8_t* packed, const uint16_t* scales,
                       const uint16_t* zeros, const double* x, double* y,
                       int rows, int cols, int gs) {
    int r;
    #pragma omp parallel for schedule(static)
    for (r = 0; r < rows; r++) {
        size_t base = (size_t)r * (size_t)cols;
        double acc = 0.0;
        for (int c = 0; c < cols; c++) {
            size_t i = base + (size_t)c;
            size_t g = i / (size_t)gs;
            double w = (double)(nib_at(packed, i) - 8) *
                       (double)orc_half_to_float(scales[g]) +
                       (double)orc_half_to_float(zeros[g]);
            acc += w * x[c];
        }
        y[r] = acc;
    }
}

void orc_gemv_f16(const uint16_t* W, const float* x, float* y,
                  int rows, int cols) {
    int r;
    #pragma omp parallel for schedule(static)
    for (r = 0; r < rows; r++) {
        const uint16_t* row = W + (size_t)r * (size_t)cols;
        float acc = 0.0f;
        for (int c = 0; c < cols; c++) acc = acc + orc_half_to_float(row[c]) * x[c];
        y[r] = acc;
    }
}

/* y[c] = sum_r fp32(W[r,c]) * x[r], rows in order
 * (csrc/core/wisp_engine.c:647-658). */
void orc_gemv_t_f16(const uint16_t* W, const float* x, float* y,
                    int rows, int cols) {
    int c;
    #pragma omp parallel for schedule(static)
    for (c = 0; c < cols; c++) {
        float acc = 0.0f;
        for (int r = 0; r < rows; r++)
            acc = acc + orc_half_to_float(W[(size_t)r * (size_t)cols + c]) * x[r];
        y[c] = acc;
    }
}

/* y = x * (float)(1 / sqrt(ss / n + eps)) * fp32(w), the sum of squares ss
 * accumulated in double (csrc/core/wisp_engine.c:660-671, scalar branch);
 * y may alias x. */
void orc_rmsnorm(const float* x, const uint16_t* w, float* y, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    float scale = (float)(1.0 / sqrt(ss / n + eps));
    for (int i = 0; i < n; i++) y[i] = x[i] * scale * orc_half_to_float(w[i]);
}

/* x += d (csrc/core/wisp_engine.c:673-675). */
void orc_residual_add(float* x, const float* d, int n) {
    for (int i = 0; i < n; i++) x[i] = x[i] + d[i];
}

void orc_swiglu(const float* g, const float* u, float* o, int n) {
    for (int i = 0; i < n; i++) {
        float s = g[i] / (1.0f + expf(-g[i]));
        o[i] = s * u[i];
    }
}

void orc_scale_accum(float* acc, const float* x, float w, int n) {
    for (int i = 0; i < n; i++) acc[i] = acc[i] + w * x[i];
}

typedef void (*gemv_fn)(const uint8_t*, const uint16_t*, const uint16_t*,
                        const float*, float*, int, int, int);

static void expert_ffn_with(gemv_fn gemv, const void* blob,
                            const OrcBlobMeta* m, const float* x, float* acc,
                            float w, float* scratch) {
    const uint8_t* b = (const uint8_t*)blob;
    int inter = (int)m->rows[0];
    int hidden = (int)m->rows[2];
    int gs = (int)m->group_size;
    float* gate = scratch;
    float* up = scratch + inter;
    float* h = scratch + 2 * (size_t)inter;
    float* y = scratch + 3 * (size_t)inter;
    for (int k = 0; k < 2; k++) {
        gemv(b + m->packed_off[k], (const uint16_t*)(b + m->scales_off[k]),
             (const uint16_t*)(b + m->zeros_off[k]), x, k ? up : gate,
             (int)m->rows[k], (int)m->cols[k], gs);
    }
    orc_swiglu(gate, up, h, inter);
    gemv(b + m->packed_off[2], (const uint16_t*)(b + m->scales_off[2]),
         (const uint16_t*)(b + m->zeros_off[2]), h, y, hidden,
         (int)m->cols[2], gs);
    orc_scale_accum(acc, y, w, hidden);
}

void orc_expert_ffn(const void* blob, const OrcBlobMeta* m, const float* x,
                    float* acc, float w, float* scratch) {
    expert_ffn_with(orc_gemv_int4, blob, m, x, acc, w, scratch);
}

/* ======================================================================= */
/* routing                                                                  */
/* ======================================================================= */

void orc_topk_select(const float* scores, int n, int k, int* idx, float* val) {
    for (int j = 0; j < k; j++) {
        int best = -1;
        float bv = -1.0f;
        for (int e = 0; e < n; e++) {
            int taken = 0;
            for (int t = 0; t < j; t++) taken |= (idx[t] == e);
            if (!taken && scores[e] > bv) { bv = scores[e]; best = e; }
        }
        idx[j] = best;
        val[j] = bv;
    }
}

static void router_logits(const uint16_t* W, const uint16_t* bias,
                          const float* x, float* logits, int n_experts,
                          int hidden) {
    orc_gemv_f16(W, x, logits, n_experts, hidden);
    if (bias)
        for (int e = 0; e < n_experts; e++)
            logits[e] = logits[e] + orc_half_to_float(bias[e]);
}

void orc_router_softmax_topk(const uint16_t* W, const uint16_t* bias,
                             const float* x, float* logits, int n_experts,
                             int hidden, int top_k, int* idx, float* w) {
    router_logits(W, bias, x, logits, n_experts, hidden);
    float mx = -1e30f;
    for (int e = 0; e < n_experts; e++) mx = logits[e] > mx ? logits[e] : mx;
    float denom = 0.0f;
    for (int e = 0; e < n_experts; e++) {
        logits[e] = expf(logits[e] - mx);
        denom = denom + logits[e];
    }
    for (int e = 0; e < n_experts; e++) logits[e] = logits[e] / denom;
    orc_topk_select(logits, n_experts, top_k, idx, w);
    float wsum = 0.0f;
    for (int j = 0; j < top_k; j++) wsum = wsum + w[j];
    if (wsum > 0.0f)
        for (int j = 0; j < top_k; j++) w[j] = w[j] / wsum;
}

void orc_router_sigmoid_topk(const uint16_t* W, const uint16_t* bias,
                             const float* x, float* logits, int n_experts,
                             int hidden, int top_k, int* idx, float* w) {
    orc_gemv_f16(W, x, logits, n_experts, hidden);
    float* sel = (float*)malloc(sizeof(float) * (size_t)n_experts);
    for (int e = 0; e < n_experts; e++) {
        logits[e] = 1.0f / (1.0f + expf(-logits[e]));
        sel[e] = logits[e] + (bias ? orc_half_to_float(bias[e]) : 0.0f);
    }
    orc_topk_select(sel, n_experts, top_k, idx, w);
    float wsum = 0.0f;
    for (int j = 0; j < top_k; j++) {
        w[j] = idx[j] >= 0 ? logits[idx[j]] : 0.0f;
        wsum = wsum + w[j];
    }
    if (wsum > 0.0f)
        for (int j = 0; j < top_k; j++) w[j] = w[j] / wsum;
    free(sel);
}

/* ======================================================================= */
/* MoE layer                                                                */
/* ======================================================================= */

void orc_moe_combine(const void* const* blobs, const OrcBlobMeta* m,
                     const void* shared_blob, const float* x,
                     const int* idx, const float* w, int top_k,
                     float* out, float* scratch) {
    int hidden = (int)m->rows[2];
    memset(out, 0, sizeof(float) * (size_t)hidden);
    if (shared_blob) orc_expert_ffn(shared_blob, m, x, out, 1.0f, scratch);
    for (int k = 0; k < top_k; k++) {
        if (idx[k] < 0) continue;
        orc_expert_ffn(blobs[idx[k]], m, x, out, w[k], scratch);
    }
}

void orc_expert_offsets(const int* topk_idx, int n_tokens, int top_k,
                        int n_experts, int* counts, int* offsets, int* order) {
    int n_pairs = n_tokens * top_k;
    for (int e = 0; e < n_experts; e++) counts[e] = 0;
    for (int p = 0; p < n_pairs; p++) {
        int e = topk_idx[p];
        if (e >= 0 && e < n_experts) counts[e]++;
    }
    offsets[0] = 0;
    for (int e = 0; e < n_experts; e++) offsets[e + 1] = offsets[e] + counts[e];
    int* fill = (int*)calloc((size_t)n_experts + 1, sizeof(int));
    for (int p = 0; p < n_pairs; p++) {
        int e = topk_idx[p];
        if (e < 0 || e >= n_experts) continue;
        order[offsets[e] + fill[e]++] = p;
    }
    free(fill);
}

/* ======================================================================= */
/* timed CPU baseline                                                       */
/* ======================================================================= */

#if defined(__x86_64__)
__attribute__((target("avx512f,avx512bw,avx512vl,fma,f16c")))
static void gemv_int4_avx512(const uint8_t* packed, const uint16_t* scales,
                             const uint16_t* zeros, const float* x, float* y,
                             int rows, int cols, int gs) {
    int r;
    const int gpr = cols / gs;
    #pragma omp parallel for schedule(static)
    for (r = 0; r < rows; r++) {
        const uint8_t* prow = packed + (size_t)r * (size_t)cols / 2;
        const uint16_t* srow = scales + (size_t)r * gpr;
        const uint16_t* zrow = zeros + (size_t)r * gpr;
        __m512 acc = _mm512_setzero_ps();
        const __m128i lomask = _mm_set1_epi8(0x0F);
        const __m128i eight = _mm_set1_epi8(8);
        for (int g = 0; g < gpr; g++) {
            __m512 s = _mm512_set1_ps(_cvtsh_ss(srow[g]));
            __m512 z = _mm512_set1_ps(_cvtsh_ss(zrow[g]));
            const uint8_t* pg = prow + (size_t)g * gs / 2;
            const float* xg = x + (size_t)g * gs;
            for (int c = 0; c < gs; c += 16) {
                __m128i b = _mm_loadl_epi64((const __m128i*)(pg + c / 2));
                __m128i lo = _mm_and_si128(b, lomask);
                __m128i hi = _mm_and_si128(_mm_srli_epi16(b, 4), lomask);
                __m128i q = _mm_sub_epi8(_mm_unpacklo_epi8(lo, hi), eight);
                __m512 qf = _mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(q));
                __m512 w = _mm512_fmadd_ps(qf, s, z);
                acc = _mm512_fmadd_ps(w, _mm512_loadu_ps(xg + c), acc);
            }
        }
        y[r] = _mm512_reduce_add_ps(acc);
    }
}

__attribute__((target("avx2,fma,f16c")))
static void gemv_int4_avx2(const uint8_t* packed, const uint16_t* scales,
                           const uint16_t* zeros, const float* x, float* y,
                           int rows, int cols, int gs) {
    int r;
    const int gpr = cols / gs;
    #pragma omp parallel for schedule(static)
    for (r = 0; r < rows; r++) {
        const uint8_t* prow = packed + (size_t)r * (size_t)cols / 2;
        const uint16_t* srow = scales + (size_t)r * gpr;
        const uint16_t* zrow = zeros + (size_t)r * gpr;
        __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
        const __m128i lomask = _mm_set1_epi8(0x0F);
        const __m128i eight = _mm_set1_epi8(8);
        for (int g = 0; g < gpr; g++) {
            __m256 s = _mm256_set1_ps(_cvtsh_ss(srow[g]));
            __m256 z = _mm256_set1_ps(_cvtsh_ss(zrow[g]));
            const uint8_t* pg = prow + (size_t)g * gs / 2;
            const float* xg = x + (size_t)g * gs;
            for (int c = 0; c < gs; c += 16) {
                __m128i b = _mm_loadl_epi64((const __m128i*)(pg + c / 2));
                __m128i lo = _mm_and_si128(b, lomask);
                __m128i hi = _mm_and_si128(_mm_srli_epi16(b, 4), lomask);
                __m128i q = _mm_sub_epi8(_mm_unpacklo_epi8(lo, hi), eight);
                __m256 q0 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(q));
                __m256 q1 = _mm256_cvtepi32_ps(
                    _mm256_cvtepi8_epi32(_mm_srli_si128(q, 8)));
                acc0 = _mm256_fmadd_ps(_mm256_fmadd_ps(q0, s, z),
                                       _mm256_loadu_ps(xg + c), acc0);
                acc1 = _mm256_fmadd_ps(_mm256_fmadd_ps(q1, s, z),
                                       _mm256_loadu_ps(xg + c + 8), acc1);
            }
        }
        __m256 a = _mm256_add_ps(acc0, acc1);
        __m128 h = _mm_add_ps(_mm256_castps256_ps128(a), _mm256_extractf128_ps(a, 1));
        h = _mm_add_ps(h, _mm_movehl_ps(h, h));
        h = _mm_add_ss(h, _mm_shuffle_ps(h, h, 1));
        y[r] = _mm_cvtss_f32(h);
    }
}
#endif

int orc_fast_isa(void) {
#if defined(__x86_64__)
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
        __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("f16c"))
        return 2;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") &&
        __builtin_cpu_supports("f16c"))
        return 1;
#endif
    return 0;
}

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void orc_gemv_int4_fast(const uint8_t* packed, const uint16_t* scales,
                        const uint16_t* zeros, const float* x, float* y,
                        int rows, int cols, int gs) {
    int vec_ok = gs >= 16 && gs % 16 == 0 && cols % gs == 0;
#if defined(__x86_64__)
    static int isa = -1;
    if (isa < 0) isa = orc_fast_isa();
    if (vec_ok && isa == 2) {
        gemv_int4_avx512(packed, scales, zeros, x, y, rows, cols, gs);
        return;
    }
    if (vec_ok && isa == 1) {
        gemv_int4_avx2(packed, scales, zeros, x, y, rows, cols, gs);
        return;
    }
#else
    (void)vec_ok;
#endif
    orc_gemv_int4(packed, scales, zeros, x, y, rows, cols, gs);
}

void orc_expert_ffn_fast(const void* blob, const OrcBlobMeta* m,
                         const float* x, float* acc, float w, float* scratch) {
    expert_ffn_with(orc_gemv_int4_fast, blob, m, x, acc, w, scratch);
}

/* ======================================================================= */
/* synthetic data                                                           */
/* ======================================================================= */

static inline uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void orc_fill_random_bytes(uint8_t* dst, size_t n, uint64_t seed) {
    size_t nblk = n / 8;
    uint64_t key = splitmix64(seed ^ 0x5EEDC0DE5EEDC0DEull);
    long long i;
    #pragma omp parallel for schedule(static)
    for (i = 0; i < (long long)nblk; i++) {
        uint64_t v = splitmix64(key + (uint64_t)i * 0x9E3779B97F4A7C15ull);
        memcpy(dst + (size_t)i * 8, &v, 8);
    }
    if (n % 8) {
        uint64_t v = splitmix64(key + (uint64_t)nblk * 0x9E3779B97F4A7C15ull);
        memcpy(dst + nblk * 8, &v, n % 8);
    }
}
