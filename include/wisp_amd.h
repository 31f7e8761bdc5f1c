/*
 * wisp_amd.h — C-ABI of the MI355X (gfx950) int4 routed-expert MoE path.
 *
 * Plain extern "C" functions over device pointers, sizes and HIP streams;
 * all device buffers are caller-owned unless stated. Every launcher is
 * stream-ordered and host-non-blocking unless stated.
 *
 * Section 1 keeps the reference engine's kernel-launcher names, argument
 * order and error behaviour (csrc/core/wisp_engine.h:496-583, the expert
 * path subset) with HIP types in place of the CUDA ones, so the reference's
 * gpu_expert_ffn call shape (csrc/core/wisp_engine.c:1507-1531) links
 * unchanged. The later sections are new launchers for what the reference
 * does not have: device-side routing, the expert-offset builder,
 * gather/scatter, a fused int4 decode for M = 1..4 tokens and the prefill
 * grouped GEMM.
 *
 * Quant format (csrc/cuda/expert_loader.cu:8-13): two int4 values per byte,
 * low nibble = even flat index; groups of group_size consecutive elements of
 * the row-major matrix share one fp16 scale and one fp16 zero;
 * value = (nibble - 8) * scale + zero.
 */
#ifndef WISP_AMD_H
#define WISP_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifndef __HIP_PLATFORM_AMD__
#define __HIP_PLATFORM_AMD__ 1
#endif
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Raw fp16 bits; same size/layout as the reference's wisp_half
 * (csrc/core/wisp_engine.h:32-40). */
typedef uint16_t wisp_half;

/* ======================================================================= *
 * 1. Reference launcher interface (hot-path subset)
 * ======================================================================= */

/* out[i] = fp16((nib_i - 8) * s[i/gs] + z[i/gs]) for i < n_elements.
 * Returns hipErrorInvalidValue for n_elements <= 0 or group_size <= 0,
 * else the launch status. Replaces csrc/cuda/expert_loader.cu:46-63
 * (declared at csrc/core/wisp_engine.h:545-550). */
hipError_t launch_dequant_expert(const uint8_t* d_packed,
                                 const wisp_half* d_scales,
                                 const wisp_half* d_zeros,
                                 wisp_half* d_output,
                                 int n_elements, int group_size,
                                 hipStream_t stream);

/* Three H2D copies (packed, scales, zeros) into the tmp buffers on `stream`,
 * then launch_dequant_expert into d_output. Replaces
 * csrc/cuda/expert_loader.cu:67-97 (csrc/core/wisp_engine.h:551-559). */
hipError_t async_load_expert(const uint8_t* h_packed,
                             const wisp_half* h_scales,
                             const wisp_half* h_zeros,
                             uint8_t* d_packed_tmp,
                             wisp_half* d_scales_tmp,
                             wisp_half* d_zeros_tmp,
                             wisp_half* d_output,
                             int n_elements, int group_size,
                             hipStream_t stream);

/* y[r] = sum_c W[r,c] * x[c]; fp16 W, fp32 x/y/accumulate. Early-returns
 * on rows <= 0 or cols <= 0. Replaces csrc/cuda/matmul.cu:43-65
 * (csrc/core/wisp_engine.h:499-500). */
void wisp_gpu_gemv_f16(const wisp_half* W, const float* x, float* y,
                       int rows, int cols, hipStream_t s);

/* h[r] = silu(Wg[r].x) * (Wu[r].x); fp16 W, fp32 x/h. Early-returns on
 * inter <= 0 or cols <= 0. Replaces csrc/cuda/matmul.cu:163-205
 * (csrc/core/wisp_engine.h:509-511). */
void wisp_gpu_swiglu_ffn(const wisp_half* Wg, const wisp_half* Wu,
                         const float* x, float* h, int inter, int cols,
                         hipStream_t s);

/* acc[i] += w * x[i]. Early-returns on n <= 0. Replaces
 * csrc/cuda/matmul.cu:150-161 (csrc/core/wisp_engine.h:512-513). */
void wisp_gpu_scale_accum(float* acc, const float* x, float w, int n,
                          hipStream_t s);

/* y = W^T x; fp16 W [rows, cols], fp32 x [rows], y [cols]. Early-returns on
 * rows <= 0 or cols <= 0. Replaces csrc/cuda/matmul.cu:67-89
 * (csrc/core/wisp_engine.h:501-502). */
void wisp_gpu_gemv_t_f16(const wisp_half* W, const float* x, float* y,
                         int rows, int cols, hipStream_t s);

/* y = x / sqrt(mean(x^2) + eps) * w over n elements (fp32 x/y, fp16 w;
 * y may alias x). Early-returns on n <= 0. Replaces
 * csrc/cuda/matmul.cu:92-121 (csrc/core/wisp_engine.h:503-504). */
void wisp_gpu_rmsnorm(const float* x, const wisp_half* w, float* y,
                      int n, float eps, hipStream_t s);

/* x[i] += delta[i]. Early-returns on n <= 0. Replaces
 * csrc/cuda/matmul.cu:124-134 (csrc/core/wisp_engine.h:505-506). */
void wisp_gpu_residual_add(float* x, const float* delta, int n,
                           hipStream_t s);

/* out[i] = silu(gate[i]) * up[i]. Early-returns on n <= 0. Replaces
 * csrc/cuda/matmul.cu:136-148 (csrc/core/wisp_engine.h:507-508). */
void wisp_gpu_swiglu(const float* gate, const float* up, float* out, int n,
                     hipStream_t s);

/* logits = W x + bias (fp16 W/bias, fp32 x), softmax, top-k (ties to the
 * lowest index), renormalised weights. out_idx/out_w are HOST pointers
 * (pinned for true asynchrony) filled by async D2H on `s`; the caller
 * synchronises `s` before reading them. top_k is clamped to 64; returns
 * early on n_experts <= 0 or top_k <= 0. The selection is staged in a
 * file-scope device array per device (no allocation). Replaces
 * csrc/cuda/router.cu:140-171 (csrc/core/wisp_engine.h:534-537). */
void wisp_gpu_router_topk(const wisp_half* W, const wisp_half* bias,
                          const float* x, float* logits_scratch,
                          int n_experts, int hidden, int top_k,
                          int* out_idx, float* out_w, hipStream_t s);

/* ======================================================================= *
 * 2. Expert blob layout
 *    Blob = 120 B header (csrc/core/wisp_engine.h:214-238) then, for gate,
 *    up, down in order, [packed][scales][zeros].
 * ======================================================================= */

typedef struct {
    uint64_t packed_off[3];   /* byte offsets from the blob base            */
    uint64_t scales_off[3];
    uint64_t zeros_off[3];
    uint32_t rows[3];         /* gate [inter,hidden], up [inter,hidden],    */
    uint32_t cols[3];         /* down [hidden,inter]                        */
    uint32_t group_size;
    uint32_t has_zeros;       /* 0: zeros are all +0 and are not read       */
    uint64_t total_bytes;     /* header + all sections                      */
} WispExpertLayout;

/* Parse a blob header held in HOST memory (same checks as
 * csrc/core/wisp_engine.c:268-303). Sets has_zeros = 1. Returns 0, or
 * -1 too small / -2 bad magic, version or n_mats / -3 truncated. */
int wisp_expert_layout_from_blob(const void* host_blob, size_t blob_size,
                                 WispExpertLayout* out);

/* 0 if the fused int4 kernels accept this layout with blobs at the given
 * device address alignment: all sections 16-byte aligned for blob bases at
 * 8 mod 16 (the tier's slot placement), gate/up [inter, hidden], down
 * [hidden, inter], hidden and inter multiples of 128, group_size in
 * a power of two >= 32 dividing both. Else hipErrorInvalidValue. */
hipError_t wisp_expert_layout_check(const WispExpertLayout* L);

/* ======================================================================= *
 * 3. Routing (device-resident) and the expert-offset builder
 * ======================================================================= */

enum { WISP_ROUTER_SOFTMAX = 0, WISP_ROUTER_SIGMOID = 1 };

/* For each of n_tokens rows of x (fp16 [n_tokens, hidden]):
 *   logits = W x (+ bias for softmax, fp32 accumulate), then
 *   SOFTMAX: p = softmax(logits); top-k of p; w = p_k / sum p_k
 *            (csrc/core/wisp_engine.c:782-818)
 *   SIGMOID: s = sigmoid(logits); top-k of s (+ bias if given);
 *            w = s_k / sum s_k (no reference counterpart)
 * Ties go to the lowest expert index. Writes d_logits [n_tokens, n_experts]
 * (the post-activation scores), d_topk_idx / d_topk_w [n_tokens, top_k].
 * n_experts <= 1024, top_k <= 64, hidden % 8 == 0. */
hipError_t wisp_gpu_moe_route(const wisp_half* d_router_w,
                              const wisp_half* d_bias, const wisp_half* d_x,
                              int n_tokens, int hidden, int n_experts,
                              int top_k, int kind, float* d_logits,
                              int* d_topk_idx, float* d_topk_w,
                              hipStream_t s);

/* Top-k selection and weights only, from given raw logits
 * [n_tokens, n_experts] (fp32), with the same rules as wisp_gpu_moe_route.
 * d_scores receives the post-activation scores. */
hipError_t wisp_gpu_topk_from_logits(const float* d_logits,
                                     const wisp_half* d_bias, int n_tokens,
                                     int n_experts, int top_k, int kind,
                                     float* d_scores, int* d_topk_idx,
                                     float* d_topk_w, hipStream_t s);

/* Expert-offset builder over the n_tokens*top_k (token, slot) pairs:
 * counts[e]; offsets = exclusive scan, n_experts+1 entries; order[] lists
 * flat pair indices (token*top_k + slot) grouped by expert, stable in flat
 * order within an expert; inv[flat] = position of that pair in order[]
 * (-1 for pairs with an out-of-range expert id). One workgroup;
 * n_experts <= 1024 (a histogram row per wave in LDS). */
hipError_t wisp_gpu_expert_offsets(const int* d_topk_idx, int n_tokens,
                                   int top_k, int n_experts, int* d_counts,
                                   int* d_offsets, int* d_order, int* d_inv,
                                   hipStream_t s);

/* Gather: xg[p, :] = x[order[p] / top_k, :] for p < n_pairs (fp16). The
 * first n_pairs entries of order must be valid pair indices of x's tokens
 * (offsets[n_experts] of wisp_gpu_expert_offsets); negative entries are
 * skipped. */
hipError_t wisp_gpu_moe_gather(const wisp_half* d_x, const int* d_order,
                               int n_pairs, int top_k, int hidden,
                               wisp_half* d_xg, hipStream_t s);

/* Weighted combine ("scatter-add" done as a per-token gather so it is
 * deterministic): out[t, :] (+)= sum over slots k in order of
 * w[t, k] * y[inv[t*top_k + k], :]; pairs with inv < 0 are skipped.
 * y fp32 [n_pairs, hidden]; out fp32 [n_tokens, hidden]; accumulate != 0
 * adds to out instead of overwriting. */
hipError_t wisp_gpu_moe_scatter(const float* d_y, const int* d_inv,
                                const float* d_topk_w, int n_tokens,
                                int top_k, int hidden, int accumulate,
                                float* d_out, hipStream_t s);

/* ======================================================================= *
 * 4. Fused int4 MoE decode, M = 1..4 tokens
 *
 *    out[t] = shared(x_t) + sum_k w[t,k] * expert_{idx[t,k]}(x_t)
 *    expert(x) = down . (silu(gate . x) * (up . x))
 *
 *    A prep launch (unique-expert list, routing weights; with routing, the
 *    router GEMV in workgroups of the same launch), then (a) gate+up+SiLU
 *    over every unique expert touched by the M tokens, (b) the down
 *    projections of all of them, whose last workgroup per output row tile
 *    adds the partials in a fixed order (routing weights are folded in
 *    before the down projection), so repeated calls give identical bits.
 *    (a) and (b) are one launch for one token, two otherwise. Weights stream from the blobs in place; nothing is
 *    dequantised to memory. Routing stays on the device.
 * ======================================================================= */

enum { WISP_DTYPE_F16 = 0, WISP_DTYPE_F32 = 1 };

/* Workspace bytes for wisp_gpu_moe_decode_int4. A decode workspace is
 * dedicated to the decode entry points (it may be shared by calls of
 * different shapes, one at a time): it carries a routing epoch and tagged
 * routing words from call to call, so it must not be reused for anything
 * else between them. It needs no zeroing, not even before its first use. */
size_t wisp_moe_decode_workspace_bytes(const WispExpertLayout* L,
                                       int n_tokens, int top_k,
                                       int has_shared);

/* Bits of the decode status word. The decode kernels hand work from one
 * workgroup to another through bounded waits (about 14 ms); a wait that
 * gives up sets its bit and poisons the outputs it feeds with NaN. */
enum {
    WISP_DECODE_ROUTER_WAIT = 1,   /* router logits never reached the prep  */
    WISP_DECODE_DOWN_WAIT = 2      /* a down projection never saw its h'    */
};

/* Waits for stream s, then returns in *flags the status bits of the most
 * recent decode call on d_workspace (0: every wait of that call completed;
 * each call starts from 0, so check after every call that matters), and
 * clears them when clear != 0. Undefined before the first call. d_workspace
 * NULL: the static workspace of wisp_gpu_moe_layer_decode_int4_noalloc on
 * the device of s. Synchronous. */
hipError_t wisp_moe_decode_status(void* d_workspace, hipStream_t s,
                                  uint32_t* flags, int clear);

/* n_experts: 1..1024; top_k: 1..64.
 * d_expert_table: device array [n_experts] of device blob base pointers
 *   (each blob base at 8 mod 16, see wisp_expert_layout_check).
 * d_shared_blob: device blob of the always-on shared expert, or NULL.
 * d_x: [n_tokens, hidden], fp16 or fp32 per x_dtype.
 * d_topk_idx / d_topk_w: [n_tokens, top_k] (device); idx < 0 is skipped.
 * d_out_f32 / d_out_f16: [n_tokens, hidden]; either may be NULL. With
 *   accumulate != 0, d_out_f32 is added to instead of overwritten.
 * Returns hipErrorInvalidValue for n_tokens outside 1..4, n_experts or
 * top_k outside the ranges above, a layout that wisp_expert_layout_check
 * rejects, or a workspace that is too small. */
hipError_t wisp_gpu_moe_decode_int4(const void* const* d_expert_table,
                                    const void* d_shared_blob,
                                    const WispExpertLayout* L,
                                    const void* d_x, int x_dtype,
                                    int n_tokens, const int* d_topk_idx,
                                    const float* d_topk_w, int top_k,
                                    int n_experts, void* d_workspace,
                                    size_t workspace_bytes, int accumulate,
                                    float* d_out_f32, wisp_half* d_out_f16,
                                    hipStream_t s);

/* One MoE layer for M = 1..4 tokens, routing included, with no host round
 * trip: router logits = W x (+ bias), softmax or sigmoid top-k with the
 * rules of wisp_gpu_moe_route, then everything wisp_gpu_moe_decode_int4
 * does. The router GEMV runs in router workgroups of the prep launch
 * (3 launches per layer, 2 for one token, where gate/up and down share
 * one launch) when hidden <= 8192 and W and x are 16-byte
 * aligned, else in one launch before it. Writes the
 * post-activation scores [n_tokens, n_experts] to d_scores and the
 * selection [n_tokens, top_k] to d_topk_idx / d_topk_w (device), as
 * wisp_gpu_moe_route does. Workspace: wisp_moe_decode_workspace_bytes.
 * Replaces the routed-expert part of run_moe for VRAM-resident experts
 * (csrc/core/wisp_engine.c:1563-1674: router launch, host sync at :1576,
 * then the per-expert gpu_expert_ffn loop at :1653-1670). */
hipError_t wisp_gpu_moe_layer_decode_int4(const wisp_half* d_router_w,
                                          const wisp_half* d_router_bias,
                                          int router_kind, float* d_scores,
                                          int* d_topk_idx, float* d_topk_w,
                                          const void* const* d_expert_table,
                                          const void* d_shared_blob,
                                          const WispExpertLayout* L,
                                          const void* d_x, int x_dtype,
                                          int n_tokens, int top_k,
                                          int n_experts, void* d_workspace,
                                          size_t workspace_bytes,
                                          int accumulate, float* d_out_f32,
                                          wisp_half* d_out_f16, hipStream_t s);

/* Bytes of the static workspace of wisp_gpu_moe_layer_decode_int4_noalloc
 * (one per device, held until the process ends). */
#define WISP_NOALLOC_SCRATCH_BYTES (16u << 20)

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): wisp_gpu_moe_layer_decode_int4 without the workspace
 * arguments. Its workspace is a library-owned static device array of
 * WISP_NOALLOC_SCRATCH_BYTES per device; the call allocates nothing.
 * Returns hipErrorInvalidValue, before any launch, when the layer's
 * workspace (wisp_moe_decode_workspace_bytes) would exceed that size: it
 * fits DeepSeek-V3 (hidden 7168, inter 2048, top-8 + shared) and
 * Mixtral-8x7B (hidden 4096, inter 14336, top-2) layers for 1..4 tokens.
 * Every call on a device shares the one array, so calls that overlap on a
 * device (two streams, two host threads) race: issue them in one stream
 * order. The status word of wisp_moe_decode_status is that array's
 * (d_workspace = NULL). */
hipError_t wisp_gpu_moe_layer_decode_int4_noalloc(
    const wisp_half* d_router_w, const wisp_half* d_router_bias,
    int router_kind, float* d_scores, int* d_topk_idx, float* d_topk_w,
    const void* const* d_expert_table, const void* d_shared_blob,
    const WispExpertLayout* L, const void* d_x, int x_dtype, int n_tokens,
    int top_k, int n_experts, int accumulate, float* d_out_f32,
    wisp_half* d_out_f16, hipStream_t s);

/* ---- the FFN half of a decode step ---------------------------------------
 *
 * For a MoE layer, decode_step runs (csrc/core/wisp_engine.c:1718-1722)
 *     norm = RMSNorm(x) * post_norm;  ffn = MoE(norm);  x += ffn
 * wisp_gpu_moe_block_int4 does all three for n_tokens rows of the fp32
 * residual stream x [n_tokens][hidden] (updated in place), so the engine's
 * op_rmsnorm / run_moe / op_residual sequence becomes one call per layer.
 * Any n_tokens: up to WISP_BLOCK_DECODE_MAX_ROWS rows (decode,
 * speculative verify of the drafted tokens) use the fused decode (the
 * router in fp32 on the normalised rows, then
 * wisp_gpu_moe_layer_decode_int4 accumulating into x, in calls of up to 4
 * rows); more rows (prefill) route on fp16 normalised rows
 * (wisp_gpu_moe_route) and run the grouped GEMM
 * (wisp_gpu_moe_prefill_int4) accumulating into x, one pass over the
 * experts for all rows instead of the reference's per-token decode_step
 * loop (csrc/core/wisp_engine.c:2292-2307, 2317-2330). The routing of every
 * row lands in d_scores / d_topk_idx / d_topk_w as in the layer call.
 * Needs hidden % 256 == 0 and a 16-byte aligned x for more than 4 rows.
 * The workspace (wisp_moe_block_workspace_bytes for the largest n_tokens
 * used) is dedicated to this call and may be shared by calls of different
 * n_tokens, one at a time; it needs no zeroing. Up to
 * WISP_BLOCK_DECODE_MAX_ROWS rows, wisp_moe_decode_status on it reports the
 * bounded waits of every decode call the block made. */
/* DeepSeek-V3 shape, per call: 8 rows 325 us in two decode calls against
 * 367 us in the grouped GEMM; 12 rows 481 against 470 us. */
#define WISP_BLOCK_DECODE_MAX_ROWS 8
size_t wisp_moe_block_workspace_bytes(const WispExpertLayout* L, int n_tokens,
                                      int top_k, int n_experts, int has_shared);
hipError_t wisp_gpu_moe_block_int4(float* d_x, const wisp_half* d_post_norm_w,
                                   float eps, const wisp_half* d_router_w,
                                   const wisp_half* d_router_bias,
                                   int router_kind, float* d_scores,
                                   int* d_topk_idx, float* d_topk_w,
                                   const void* const* d_expert_table,
                                   const void* d_shared_blob,
                                   const WispExpertLayout* L, int n_tokens,
                                   int top_k, int n_experts, void* d_workspace,
                                   size_t workspace_bytes, hipStream_t s);

/* ======================================================================= *
 * 5. Fused int4 MoE prefill (grouped GEMM over routed token tiles)
 *
 *    out[t] = shared(x_t) + sum_k w[t,k] * expert_{idx[t,k]}(x_t) for any
 *    number of tokens. The (token, slot) pairs are sorted by expert
 *    (wisp_gpu_expert_offsets), cut into tiles of up to 128 tokens of one
 *    expert, and each tile runs gate+up+SiLU and down as GEMMs on the
 *    matrix cores: int4 weights are dequantised in registers to fp16
 *    (the reference dequant, csrc/cuda/expert_loader.cu:42) and multiplied
 *    with fp16 activations, fp32 accumulate. h and the per-pair down
 *    outputs are fp16 in the workspace; the combine adds each token's slots
 *    in order (shared first, then rank order), so results are
 *    deterministic. Replaces the reference's per-token loop over
 *    decode_step (csrc/core/wisp_engine.c:2292-2307), which re-reads every
 *    selected expert's weights for every token.
 * ======================================================================= */

/* Workspace bytes for wisp_gpu_moe_prefill_int4 (0 for invalid sizes). */
size_t wisp_moe_prefill_workspace_bytes(const WispExpertLayout* L,
                                        int n_tokens, int top_k,
                                        int n_experts, int has_shared);

/* Arguments as wisp_gpu_moe_decode_int4, with any n_tokens >= 1, fp16 x
 * and 16-byte aligned x and outputs. Also needs hidden % 256 == 0 and
 * n_experts + 1 <= 1024. Returns hipErrorInvalidValue on bad arguments or a small
 * workspace. */
hipError_t wisp_gpu_moe_prefill_int4(const void* const* d_expert_table,
                                     const void* d_shared_blob,
                                     const WispExpertLayout* L,
                                     const wisp_half* d_x, int n_tokens,
                                     const int* d_topk_idx,
                                     const float* d_topk_w, int top_k,
                                     int n_experts, void* d_workspace,
                                     size_t workspace_bytes, int accumulate,
                                     float* d_out_f32, wisp_half* d_out_f16,
                                     hipStream_t s);

/* ======================================================================= *
 * 6. VRAM tier of the expert cache
 *
 *    Every expert blob of every layer sits in pinned host memory (the RAM
 *    tier); a fixed number of VRAM slots caches the hot ones with the
 *    reference's policy (csrc/core/wisp_engine.c:1138-1296): a first touch
 *    takes a free slot or rides the scratch ring; a later RAM hit is served
 *    through the scratch ring until the expert has been hit promote_hits
 *    times (the reference's WISP_PROMOTE_HITS = 3), then it is promoted
 *    into a slot, evicting the least recently used resident expert that
 *    the current layer has not resolved. Copies are hipMemcpyAsync on the
 *    tier's own stream, ordered by events. One owner thread; not
 *    thread-safe.
 * ======================================================================= */

/* Lookup paths (same numbering as the reference trace harness). */
enum {
    WISP_TIER_VRAM_HIT = 0,       /* resident in a VRAM slot                   */
    WISP_TIER_RAM_SCRATCH = 1,    /* RAM hit below the promotion count          */
    WISP_TIER_RAM_PROMOTE = 2,    /* RAM hit that earned a VRAM slot            */
    WISP_TIER_COLD_VRAM = 3,      /* first touch, free slot available           */
    WISP_TIER_COLD_SCRATCH = 4    /* first touch, no free slot                  */
};
/* Indices of the statistics array. The VRAM hit rate is
 * VRAM_HITS / LOOKUPS; the reference reports (vram + ram) / total
 * (csrc/core/wisp_engine.c:2343-2344), which is always 1 here. */
enum {
    WISP_TIER_LOOKUPS = 0, WISP_TIER_VRAM_HITS, WISP_TIER_RAM_HITS,
    WISP_TIER_FIRST_TOUCH,       /* SSD misses: first touches, and experts back after a RAM eviction */
    WISP_TIER_PROMOTIONS, WISP_TIER_EVICTIONS, WISP_TIER_SCRATCH_SERVES, WISP_TIER_H2D_BYTES,
    WISP_TIER_RAM_EVICTIONS,     /* bounded RAM tier: experts dropped from RAM  */
    WISP_TIER_SSD_BYTES,         /* bounded RAM tier: bytes read from expert files */
    WISP_TIER_D2H_BYTES,         /* bounded RAM tier: evicted experts copied back */
    WISP_TIER_N_STATS
};

/* The policy alone, on the host (no device calls): for tests and for
 * engines that move the bytes themselves. */
typedef struct WispTierPolicy WispTierPolicy;
WispTierPolicy* wisp_tier_policy_create(int n_layers, int n_experts,
                                        int n_slots, int scratch_slots,
                                        int promote_hits);
/* The same policy with a RAM tier of n_ram_slots blobs over the expert
 * files (the reference's RAM LRU with its byte budget, :1053-1068; an
 * expert dropped from RAM loses its hit count and comes back as an SSD
 * miss; a VRAM victim is copied back into RAM). n_ram_slots must exceed
 * scratch_slots. */
WispTierPolicy* wisp_tier_policy_create_ram(int n_layers, int n_experts,
                                            int n_ram_slots, int n_slots,
                                            int scratch_slots, int promote_hits);
void wisp_tier_policy_destroy(WispTierPolicy* t);
/* Starts the lookups of one layer: experts resolved from here on are not
 * evicted until the next call. */
void wisp_tier_policy_begin_layer(WispTierPolicy* t);
/* One lookup; returns the path (WISP_TIER_*), or -1 for bad arguments.
 * *slot = VRAM slot or scratch-ring index; *victim_layer / *victim_expert =
 * the expert evicted by a promotion, else -1. */
int wisp_tier_policy_lookup(WispTierPolicy* t, int layer, int expert,
                            int* slot, int* victim_layer, int* victim_expert);
/* out[WISP_TIER_N_STATS] (H2D_BYTES stays 0). */
void wisp_tier_policy_stats(const WispTierPolicy* t, uint64_t* out);

/* The tier with its device memory. host_blobs: [n_layers * n_experts]
 * pinned host pointers (hipHostMalloc), blob of expert e of layer l at
 * index l * n_experts + e, each blob_bytes long. Allocates n_slots +
 * scratch_slots device slots (blob at slot + 8, so that every section is
 * 16-byte aligned) and a device table [n_layers][n_experts] of blob
 * pointers. n_experts: 1..1024 (the decode kernels' limit). Returns NULL
 * and sets *err on failure. */
typedef struct WispExpertTier WispExpertTier;
WispExpertTier* wisp_tier_create(int n_layers, int n_experts,
                                 size_t blob_bytes,
                                 const void* const* host_blobs, int n_slots,
                                 int scratch_slots, int promote_hits,
                                 hipError_t* err);
/* The three-tier cache: VRAM slots, a RAM tier of n_ram_slots pinned blob
 * slots (> scratch_slots), and the expert files under model_path
 * (<model_path>/experts/L%03u_E%05u.bin, each blob_bytes long) as the SSD
 * tier. An SSD miss reads its file into a RAM slot (the LRU RAM entry is
 * dropped when the tier is full; experts of the layer being fetched are
 * kept), in parallel threads for the misses of one layer, then copies as
 * a RAM hit would; a VRAM victim of a promotion is copied back into RAM
 * (device to host on the tier's stream). Replaces the SSD path of
 * wisp_expert_fetch (csrc/core/wisp_engine.c:1205-1296) and its pinned
 * staging pool (csrc/core/mem_pool.c:27-122). A missing or short file
 * makes wisp_tier_fetch_layer return hipErrorFileNotFound. */
WispExpertTier* wisp_tier_create_ssd(int n_layers, int n_experts,
                                     size_t blob_bytes, const char* model_path,
                                     int n_ram_slots, int n_slots,
                                     int scratch_slots, int promote_hits,
                                     hipError_t* err);
void wisp_tier_destroy(WispExpertTier* t);
/* Device table row of a layer: [n_experts] blob pointers, valid for the
 * experts of the last wisp_tier_fetch_layer of that layer. */
void** wisp_tier_device_table(WispExpertTier* t, int layer);
/* Resolves n expert ids of one layer (host array; ids < 0 are skipped):
 * policy lookups, hipMemcpyAsync from the pinned blobs on the tier's
 * stream for everything not already resident (each copy first waits for
 * the kernels that last read its slot), then the layer's table row is
 * copied to the device on `compute`. out_path[i] (may be NULL) receives
 * each id's path. Kernels reading experts whose path is not
 * WISP_TIER_VRAM_HIT must be launched after wisp_tier_wait_copies; VRAM
 * hits can be used at once. The distinct valid ids must not outnumber
 * the scratch slots (hipErrorInvalidValue), so that the ring never wraps
 * within a layer (the reference sizes it top_k + 2 for one token).
 * Replaces the per-expert wisp_expert_fetch calls of run_moe
 * (csrc/core/wisp_engine.c:1653-1665). */
hipError_t wisp_tier_fetch_layer(WispExpertTier* t, int layer,
                                 const int* expert_ids, int n, int* out_path,
                                 hipStream_t compute);
/* Makes `compute` wait for the copies of the last fetch. */
hipError_t wisp_tier_wait_copies(WispExpertTier* t, hipStream_t compute);
/* Call after the last launch that reads the layer's experts on `compute`:
 * a later copy into one of their slots waits for it. */
hipError_t wisp_tier_release_layer(WispExpertTier* t, hipStream_t compute);
/* out[WISP_TIER_N_STATS]. */
void wisp_tier_stats(const WispExpertTier* t, uint64_t* out);

/* One MoE decode layer (n_tokens * top_k <= 256) whose routing is known on
 * the host (h_topk_idx / h_topk_w [n_tokens][top_k], as run_moe has it
 * after its routing sync, csrc/core/wisp_engine.c:1576): fetch, then the
 * fused decode of the experts already resident plus the shared expert on
 * `compute` while the missing ones are copied on the tier's stream, then
 * the copied experts as an accumulating second pass, then release. The
 * fp32 output d_out_f32 is required (the second pass accumulates into
 * it); d_out_f16 may be NULL. Workspace as wisp_gpu_moe_decode_int4. */
hipError_t wisp_tier_moe_decode_layer(WispExpertTier* t, int layer,
                                      const void* d_shared_blob,
                                      const WispExpertLayout* L,
                                      const void* d_x, int x_dtype,
                                      int n_tokens, const int* h_topk_idx,
                                      const float* h_topk_w, int top_k,
                                      void* d_workspace, size_t workspace_bytes,
                                      float* d_out_f32, wisp_half* d_out_f16,
                                      hipStream_t compute);

/* ======================================================================= *
 * 7. Real-weight ingestion (host only)
 *
 *    The converter's group-wise int4 quantizer and the expert file format,
 *    so real checkpoints become the blobs the kernels read, and the reader
 *    that brings a blob file into (pinned) host memory for the tiers.
 * ======================================================================= */

enum { WISP_WEIGHT_F32 = 0, WISP_WEIGHT_F16 = 1, WISP_WEIGHT_BF16 = 2 };

/* Group-wise asymmetric int4 quantization of a row-major [rows, cols]
 * matrix, byte-identical to the reference converter's quantize_int4
 * (wisp/converter/quantizer.py:46-86): per group of group_size consecutive
 * elements (the last one padded with the last element), zero = (max + min)
 * / 2, scale = max((max - min) / 15, 1e-8) in fp32, q = clamp(round half to
 * even((x - zero) / scale) + 8, 0, 15), packed two per byte (low nibble =
 * even element; an odd count leaves the last high nibble 0); scale and zero
 * stored as fp16 (round to nearest even). w is fp32, fp16 or bf16 per dtype
 * (WISP_WEIGHT_*). packed holds ceil(n/2) bytes, scales and zeros
 * ceil(n/group_size) entries each. Returns 0, -1 for bad arguments, -2 for
 * a non-finite weight (the reference would write meaningless nibbles). */
int wisp_quantize_int4(const void* w, int dtype, uint32_t rows, uint32_t cols,
                       uint32_t group_size, uint8_t* packed, wisp_half* scales,
                       wisp_half* zeros);

/* Bytes of an expert blob with matrices rows[m] x cols[m] (gate, up, down):
 * the 120-byte header plus [packed][scales][zeros] per matrix. 0 for bad
 * arguments. */
size_t wisp_expert_blob_bytes(const uint32_t rows[3], const uint32_t cols[3],
                              uint32_t group_size);

/* Writes an expert blob (the reference file format, wisp/converter/
 * partitioner.py:56-89) into dst. Returns the bytes written, or 0 when
 * capacity is too small or an argument is bad. */
size_t wisp_expert_blob_write(void* dst, size_t capacity, uint32_t layer,
                              uint32_t expert, uint32_t group_size,
                              const uint32_t rows[3], const uint32_t cols[3],
                              const uint8_t* const packed[3],
                              const wisp_half* const scales[3],
                              const wisp_half* const zeros[3]);

/* Quantizes one expert (gate and up [inter, hidden], down [hidden, inter],
 * each row-major in dtype) and writes its blob into dst: the converter's
 * per-expert path (wisp/converter/partitioner.py:160-180 quantizes each
 * projection, :56-89 writes the file). Returns the blob bytes, 0 on error. */
size_t wisp_expert_quantize_blob(const void* gate, const void* up,
                                 const void* down, int dtype, uint32_t inter,
                                 uint32_t hidden, uint32_t group_size,
                                 uint32_t layer, uint32_t expert, void* dst,
                                 size_t capacity);

/* Error codes of the expert file functions. */
enum {
    WISP_IO_BAD_ARGUMENT = -1,
    WISP_IO_MISSING = -2,       /* cannot open the file                     */
    WISP_IO_TOO_LARGE = -3,     /* empty, or larger than the destination     */
    WISP_IO_SHORT_READ = -4     /* read or write ended early                 */
};

/* out = "<model_path>/experts/L%03u_E%05u.bin" (wisp/converter/manifest.py
 * expert_filename). Returns 0, or -1 when it does not fit. */
int wisp_expert_file_path(char* out, size_t capacity, const char* model_path,
                          uint32_t layer, uint32_t expert);

/* Reads a whole expert file into dst (max_bytes), as read_expert_ssd does
 * (csrc/core/wisp_engine.c:351-380). Returns the bytes read (> 0) or a
 * WISP_IO_* code. */
int64_t wisp_expert_file_read(const char* model_path, uint32_t layer,
                              uint32_t expert, void* dst, size_t max_bytes);

/* Writes a blob to its expert file through a temporary file and a rename
 * (wisp/converter/partitioner.py:79-89). The experts/ directory must exist.
 * Returns 0 or a WISP_IO_* code. */
int wisp_expert_file_write(const char* model_path, uint32_t layer,
                           uint32_t expert, const void* blob, size_t bytes);

/* ======================================================================= *
 * 9. Profiling hook
 * ======================================================================= */

/* When events != NULL, the fused launchers record events[2*k] before and
 * events[2*k+1] after each kernel of kind k < n_pairs on the launch stream:
 * k = 0 router (wisp_gpu_moe_route, or the router GEMV launch of
 * wisp_gpu_moe_layer_decode_int4), 1 decode prep, 2 decode gate/up (with
 * the down projection when both share one launch), 3 decode down (it also
 * writes the layer output; not recorded when it shares the gate/up
 * launch), 4 unused, 5 prefill gate/up, 6 prefill down. Process-wide; for timing runs only; not
 * thread-safe. */
void wisp_amd_set_kernel_events(hipEvent_t* events, int n_pairs);

/* Library version string. */
const char* wisp_amd_version(void);

#ifdef __cplusplus
}
#endif
#endif /* WISP_AMD_H */
