/*
 * wisp_oracle.h — CPU oracle for the int4 routed-expert MoE path.
 *
 * TEST INFRASTRUCTURE ONLY. This library restates, in plain C, the scalar
 * CPU semantics of the reference engine's expert path so that the HIP
 * implementation can be checked against it. Only tests/, the smoke check
 * in __graft_entry__.py and the cpu_baseline leg of bench.py may load it.
 * The product library (wisp_amd/) never links, loads or falls back to it.
 *
 * Every function cites the reference file:line it restates. Functions
 * whose behaviour the reference does not define (sigmoid router, expert
 * offset builder, the fast AVX-512 baseline) say "build-defined" and are
 * pinned by closed forms in tests/test_oracle.py.
 */
#ifndef WISP_ORACLE_H
#define WISP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 <-> fp32 ---------------------------------------------------- */

/* Exact fp16 -> fp32 (restates csrc/core/wisp_engine.c:53-75). */
float orc_half_to_float(uint16_t h);
/* fp32 -> fp16, round to nearest even: what the reference GPU dequant
 * kernel's __float2half does (csrc/cuda/expert_loader.cu:42). */
uint16_t orc_float_to_half(float f);
/* The reference's own host helper (csrc/core/wisp_engine.c:77-91), which
 * truncates the mantissa. Kept for parity tests of that helper only. */
uint16_t orc_float_to_half_trunc(float f);

/* ---- int4 format ------------------------------------------------------ */

/* nib[i] = low nibble of packed[i/2] for even i, high nibble for odd i
 * (csrc/cuda/expert_loader.cu:35-36; wisp/converter/quantizer.py:74-79). */
void orc_unpack_int4(const uint8_t* packed, size_t n, uint8_t* nib);
/* Inverse of orc_unpack_int4; an odd tail pads the last high nibble with 0
 * (wisp/converter/quantizer.py:75-79). */
void orc_pack_int4(const uint8_t* nib, size_t n, uint8_t* packed);
/* out[i] = fp16_rn((nib_i - 8) * fp32(s[i/gs]) + fp32(z[i/gs]))
 * (csrc/cuda/expert_loader.cu:23-43). */
void orc_dequant_fp16(const uint8_t* packed, const uint16_t* scales,
                      const uint16_t* zeros, size_t n, int gs, uint16_t* out);
/* Same, kept in fp32 (csrc/core/wisp_engine.c:338-344 probe). */
void orc_dequant_f32(const uint8_t* packed, const uint16_t* scales,
                     const uint16_t* zeros, size_t n, int gs, float* out);

/* ---- expert blob (csrc/core/wisp_engine.h:214-251) --------------------- */

#define ORC_BLOB_MAGIC   0x57455850u
#define ORC_BLOB_VERSION 1u
#define ORC_BLOB_HEADER  120u

typedef struct {
    uint64_t packed_off[3], scales_off[3], zeros_off[3];
    uint32_t rows[3], cols[3];
    uint32_t group_size, layer_id, expert_id;
    uint64_t total_bytes;
} OrcBlobMeta;

/* 0 on success; -1 too small, -2 bad magic/version/n_mats, -3 truncated
 * (csrc/core/wisp_engine.c:268-303). */
int orc_blob_parse(const void* blob, size_t size, OrcBlobMeta* meta);
/* Writes header + [packed|scales|zeros] x {gate, up, down} into dst (which
 * must hold orc_blob_size(...) bytes); returns bytes written
 * (wisp/converter/partitioner.py:56-89). */
size_t orc_blob_size(uint32_t inter, uint32_t hidden, uint32_t gs);
size_t orc_blob_write(void* dst, uint32_t layer, uint32_t expert, uint32_t gs,
                      uint32_t inter, uint32_t hidden,
                      const uint8_t* const packed[3],
                      const uint16_t* const scales[3],
                      const uint16_t* const zeros[3]);

/* ---- expert math (scalar reference semantics, fp32) --------------------- */

/* y[r] = sum_c ((nib-8)*s + z) * x[c], fp32 accumulate in column order
 * (csrc/core/wisp_engine.c:822-845, the #else branch). */
void orc_gemv_int4(const uint8_t* packed, const uint16_t* scales,
                   const uint16_t* zeros, const float* x, float* y,
                   int rows, int cols, int gs);
/* float64 truth of the same contraction (not a reference function). */
void orc_gemv_int4_f64(const uint8_t* packed, const uint16_t* scales,
                       const uint16_t* zeros, const double* x, double* y,
                       int rows, int cols, int gs);
/* y[r] = sum_c fp32(W[r,c]) * x[c] (csrc/core/wisp_engine.c:630-645). */
void orc_gemv_f16(const uint16_t* W, const float* x, float* y,
                  int rows, int cols);
/* y[c] = sum_r fp32(W[r,c]) * x[r] (csrc/core/wisp_engine.c:647-658). */
void orc_gemv_t_f16(const uint16_t* W, const float* x, float* y,
                    int rows, int cols);
/* RMSNorm, double sum of squares (csrc/core/wisp_engine.c:660-671, scalar
 * branch); y may alias x. */
void orc_rmsnorm(const float* x, const uint16_t* w, float* y, int n, float eps);
/* x += d (csrc/core/wisp_engine.c:673-675). */
void orc_residual_add(float* x, const float* d, int n);
/* o = g / (1 + expf(-g)) * u (csrc/core/wisp_engine.c:677-686). */
void orc_swiglu(const float* g, const float* u, float* o, int n);
/* acc += w * x (csrc/core/wisp_engine.c:688-690). */
void orc_scale_accum(float* acc, const float* x, float w, int n);

/* One expert's FFN from a blob, accumulated into acc with weight w:
 * gate, up, swiglu, down, scale_accum (csrc/core/wisp_engine.c:1534-1561).
 * scratch must hold 3*inter + hidden floats. */
void orc_expert_ffn(const void* blob, const OrcBlobMeta* m, const float* x,
                    float* acc, float w, float* scratch);

/* ---- routing ------------------------------------------------------------ */

/* k passes of argmax over untaken entries, strict '>' in ascending index,
 * so ties go to the lowest index; bestv starts at -1 so negative scores are
 * never chosen (csrc/core/wisp_engine.c:803-815; csrc/cuda/router.cu:118-130).
 * Writes idx[k] and the selected raw scores. */
void orc_topk_select(const float* scores, int n, int k, int* idx, float* val);
/* Router: logits = W x (+bias), softmax, top-k, renormalise
 * (csrc/core/wisp_engine.c:782-818). logits is scratch [n_experts]. */
void orc_router_softmax_topk(const uint16_t* W, const uint16_t* bias,
                             const float* x, float* logits, int n_experts,
                             int hidden, int top_k, int* idx, float* w);
/* Build-defined sigmoid router (no reference counterpart): s = 1/(1+e^-l);
 * selection on s (+ bias if given), ties to the lowest index; weights are
 * the selected unbiased s renormalised to sum 1. */
void orc_router_sigmoid_topk(const uint16_t* W, const uint16_t* bias,
                             const float* x, float* logits, int n_experts,
                             int hidden, int top_k, int* idx, float* w);

/* ---- MoE layer ----------------------------------------------------------- */

/* CPU run_moe semantics for one token (csrc/core/wisp_engine.c:1563-1674):
 * out = 0; out += 1.0 * shared(x) (if shared_blob); then for k in rank order
 * out += w[k] * expert_{idx[k]}(x). Experts with idx < 0 are skipped.
 * blobs[e] is expert e's blob; scratch as orc_expert_ffn. */
void orc_moe_combine(const void* const* blobs, const OrcBlobMeta* m,
                     const void* shared_blob, const float* x,
                     const int* idx, const float* w, int top_k,
                     float* out, float* scratch);

/* Build-defined expert-offset builder for M tokens x top_k slots:
 * counts[e] = #pairs routed to e; offsets = exclusive scan (n_experts+1);
 * pairs are placed stably in flat (token*top_k + slot) order within each
 * expert: order[offsets[e] + j] = flat index of e's j-th pair. */
void orc_expert_offsets(const int* topk_idx, int n_tokens, int top_k,
                        int n_experts, int* counts, int* offsets, int* order);

/* ---- timed CPU baseline (build-defined vectorisation) -------------------- */

/* Same contraction as orc_gemv_int4, OpenMP static over rows; uses AVX-512
 * (F16C converts, FMA) when the CPU has it, else AVX2+FMA+F16C, else the
 * scalar loop. Summation order differs from orc_gemv_int4 (lane-parallel). */
void orc_gemv_int4_fast(const uint8_t* packed, const uint16_t* scales,
                        const uint16_t* zeros, const float* x, float* y,
                        int rows, int cols, int gs);
/* orc_expert_ffn with orc_gemv_int4_fast. */
void orc_expert_ffn_fast(const void* blob, const OrcBlobMeta* m,
                         const float* x, float* acc, float w, float* scratch);
/* Which path orc_gemv_int4_fast takes here: 2 = AVX-512, 1 = AVX2, 0 = scalar. */
int orc_fast_isa(void);
/* Threads the OpenMP region will use. */
int orc_num_threads(void);

/* ---- synthetic data (deterministic, thread-parallel) -------------------- */

/* Fills dst[0..n) with uniform random bytes from a counter-based generator
 * (splitmix64 of seed and the 8-byte block index); same bytes for the same
 * (seed, n) on every machine and thread count. */
void orc_fill_random_bytes(uint8_t* dst, size_t n, uint64_t seed);

#ifdef __cplusplus
}
#endif
#endif /* WISP_ORACLE_H */
