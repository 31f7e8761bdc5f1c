/*
 * engine_call_shape.c — a C11 caller of libwisp_amd.so written the way the
 * reference engine calls its GPU launchers (TEST CODE).
 *
 * The reference's C engine includes csrc/core/wisp_engine.h, whose section 7
 * declares the launchers with CUDA types (csrc/core/wisp_engine.h:496-559).
 * This file includes include/wisp_amd.h, maps the two CUDA type names to
 * their HIP counterparts once, and then repeats the reference's
 * declarations as they are written there: C accepts a repeated declaration
 * only when it is compatible with the first, so this file compiles only
 * while the library keeps the reference's names, argument types and order.
 *
 * It then runs, from C, the reference's per-expert call sequence
 * gpu_expert_ffn (csrc/core/wisp_engine.c:1507-1531: three dequants into
 * fp16 scratch, the fused gate/up/SiLU, the down GEMV, the weighted
 * accumulate, each dequant checked like WISP_CHECK_CUDA) and one
 * wisp_gpu_moe_layer_decode_int4 call, on buffers it allocates itself.
 * tests/test_gpu_c_boundary.py loads it with ctypes and checks the results
 * against the golden fixtures and the oracle.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "wisp_amd.h"

typedef hipStream_t cudaStream_t;
typedef hipError_t cudaError_t;
#define cudaSuccess hipSuccess

/* csrc/core/wisp_engine.h:499-500, 509-513, 534-537, 545-559, as written */
void wisp_gpu_gemv_f16(const wisp_half* W, const float* x, float* y,
                       int rows, int cols, cudaStream_t s);
void wisp_gpu_swiglu_ffn(const wisp_half* Wg, const wisp_half* Wu,
                         const float* x, float* h, int inter, int cols,
                         cudaStream_t s);   /* fused gate+up+silu*up */
void wisp_gpu_scale_accum(float* acc, const float* x, float w, int n,
                          cudaStream_t s);
void wisp_gpu_router_topk(const wisp_half* W, const wisp_half* bias,
                          const float* x, float* logits_scratch,
                          int n_experts, int hidden, int top_k,
                          int* out_idx, float* out_w, cudaStream_t s);
cudaError_t launch_dequant_expert(const uint8_t* d_packed,
                                  const wisp_half* d_scales,
                                  const wisp_half* d_zeros,
                                  wisp_half* d_output,
                                  int n_elements, int group_size,
                                  cudaStream_t stream);
cudaError_t async_load_expert(const uint8_t* h_packed,
                              const wisp_half* h_scales,
                              const wisp_half* h_zeros,
                              uint8_t* d_packed_tmp,
                              wisp_half* d_scales_tmp,
                              wisp_half* d_zeros_tmp,
                              wisp_half* d_output,
                              int n_elements, int group_size,
                              cudaStream_t stream);

#define TRY(call)                          \
    do {                                   \
        cudaError_t e_ = (call);           \
        if (e_ != cudaSuccess) {           \
            rc = (int)e_;                  \
            goto done;                     \
        }                                  \
    } while (0)

/* The engine's per-expert FFN: acc (host, [hidden], in/out) += weight *
 * down . (silu(gate . x) * (up . x)) for the expert blob at host_blob.
 * Returns 0 or a HIP error code (negative: a bad blob header). */
int c_gpu_expert_ffn(const void* host_blob, size_t blob_bytes, const float* host_x,
                     float weight, float* host_acc) {
    WispExpertLayout m;
    if (wisp_expert_layout_from_blob(host_blob, blob_bytes, &m) != 0) return -1;
    int rc = 0;
    const int inter = (int)m.rows[0], hidden = (int)m.cols[0];
    uint8_t* blob = NULL;
    wisp_half* dq[3] = {NULL, NULL, NULL};
    float *x = NULL, *h = NULL, *y = NULL, *acc = NULL;
    cudaStream_t s = NULL;
    TRY(hipStreamCreate(&s));
    TRY(hipMalloc((void**)&blob, blob_bytes));
    for (int i = 0; i < 3; i++)
        TRY(hipMalloc((void**)&dq[i], (size_t)m.rows[i] * m.cols[i] * sizeof(wisp_half)));
    TRY(hipMalloc((void**)&x, (size_t)hidden * sizeof(float)));
    TRY(hipMalloc((void**)&h, (size_t)inter * sizeof(float)));
    TRY(hipMalloc((void**)&y, (size_t)hidden * sizeof(float)));
    TRY(hipMalloc((void**)&acc, (size_t)hidden * sizeof(float)));
    TRY(hipMemcpy(blob, host_blob, blob_bytes, hipMemcpyHostToDevice));
    TRY(hipMemcpy(x, host_x, (size_t)hidden * sizeof(float), hipMemcpyHostToDevice));
    TRY(hipMemcpy(acc, host_acc, (size_t)hidden * sizeof(float), hipMemcpyHostToDevice));

    /* csrc/core/wisp_engine.c:1510-1530 */
    for (int i = 0; i < 3; i++)
        TRY(launch_dequant_expert(blob + m.packed_off[i],
                                  (const wisp_half*)(blob + m.scales_off[i]),
                                  (const wisp_half*)(blob + m.zeros_off[i]), dq[i],
                                  (int)(m.rows[i] * m.cols[i]), (int)m.group_size, s));
    wisp_gpu_swiglu_ffn(dq[0], dq[1], x, h, inter, (int)m.cols[0], s);
    wisp_gpu_gemv_f16(dq[2], h, y, (int)m.rows[2], (int)m.cols[2], s);
    wisp_gpu_scale_accum(acc, y, weight, (int)m.rows[2], s);

    TRY(hipStreamSynchronize(s));
    TRY(hipGetLastError());
    TRY(hipMemcpy(host_acc, acc, (size_t)hidden * sizeof(float), hipMemcpyDeviceToHost));
done:
    if (s) (void)hipStreamSynchronize(s);
    (void)hipFree(blob);
    for (int i = 0; i < 3; i++) (void)hipFree(dq[i]);
    (void)hipFree(x);
    (void)hipFree(h);
    (void)hipFree(y);
    (void)hipFree(acc);
    if (s) (void)hipStreamDestroy(s);
    return rc;
}

/* One MoE decode layer from C: n_experts blobs of blob_bytes each,
 * contiguous in host memory, a softmax or sigmoid router (fp16 W
 * [n_experts][hidden], optional fp16 bias), n_tokens fp32 tokens; writes
 * the selection (host idx/w [n_tokens][top_k]) and the fp32 layer output
 * (host out [n_tokens][hidden]). Returns 0 or a HIP error code. */
int c_moe_layer_decode(const void* host_blobs, size_t blob_bytes, int n_experts,
                       int has_zeros, const wisp_half* host_router_w,
                       const wisp_half* host_bias, int router_kind, const float* host_x,
                       int n_tokens, int top_k, int* host_idx, float* host_w,
                       float* host_out) {
    WispExpertLayout L;
    if (wisp_expert_layout_from_blob(host_blobs, blob_bytes, &L) != 0) return -1;
    L.has_zeros = has_zeros ? 1u : 0u;
    const int hidden = (int)L.cols[0];
    /* each blob at 8 mod 16 in a 4 KiB-rounded slot, as the tier places it */
    const size_t stride = (blob_bytes + 8 + 4095) / 4096 * 4096;
    int rc = 0;
    uint8_t* arena = NULL;
    void** table = NULL;
    wisp_half *W = NULL, *bias = NULL;
    float *x = NULL, *scores = NULL, *w = NULL, *out = NULL;
    int* idx = NULL;
    void* ws = NULL;
    void** h_table = (void**)malloc((size_t)n_experts * sizeof(void*));
    if (!h_table) return (int)hipErrorOutOfMemory;
    const size_t ws_bytes = wisp_moe_decode_workspace_bytes(&L, n_tokens, top_k, 0);
    if (ws_bytes == 0) {
        free(h_table);
        return (int)hipErrorInvalidValue;
    }
    TRY(hipMalloc((void**)&arena, stride * (size_t)n_experts));
    TRY(hipMalloc((void**)&table, (size_t)n_experts * sizeof(void*)));
    TRY(hipMalloc((void**)&W, (size_t)n_experts * hidden * sizeof(wisp_half)));
    if (host_bias) TRY(hipMalloc((void**)&bias, (size_t)n_experts * sizeof(wisp_half)));
    TRY(hipMalloc((void**)&x, (size_t)n_tokens * hidden * sizeof(float)));
    TRY(hipMalloc((void**)&scores, (size_t)n_tokens * n_experts * sizeof(float)));
    TRY(hipMalloc((void**)&idx, (size_t)n_tokens * top_k * sizeof(int)));
    TRY(hipMalloc((void**)&w, (size_t)n_tokens * top_k * sizeof(float)));
    TRY(hipMalloc((void**)&out, (size_t)n_tokens * hidden * sizeof(float)));
    TRY(hipMalloc(&ws, ws_bytes));
    for (int e = 0; e < n_experts; e++) {
        uint8_t* dst = arena + (size_t)e * stride + 8;
        h_table[e] = dst;
        TRY(hipMemcpy(dst, (const uint8_t*)host_blobs + (size_t)e * blob_bytes, blob_bytes,
                      hipMemcpyHostToDevice));
    }
    TRY(hipMemcpy(table, h_table, (size_t)n_experts * sizeof(void*), hipMemcpyHostToDevice));
    TRY(hipMemcpy(W, host_router_w, (size_t)n_experts * hidden * sizeof(wisp_half),
                  hipMemcpyHostToDevice));
    if (host_bias)
        TRY(hipMemcpy(bias, host_bias, (size_t)n_experts * sizeof(wisp_half),
                      hipMemcpyHostToDevice));
    TRY(hipMemcpy(x, host_x, (size_t)n_tokens * hidden * sizeof(float), hipMemcpyHostToDevice));
    TRY(wisp_gpu_moe_layer_decode_int4(W, bias, router_kind, scores, idx, w,
                                       (const void* const*)table, NULL, &L, x,
                                       WISP_DTYPE_F32, n_tokens, top_k, n_experts, ws, ws_bytes,
                                       0, out, NULL, NULL));
    TRY(hipDeviceSynchronize());
    {
        uint32_t flags = 0;
        TRY(wisp_moe_decode_status(ws, NULL, &flags, 1));
        if (flags) {
            rc = -2;
            goto done;
        }
    }
    TRY(hipMemcpy(host_idx, idx, (size_t)n_tokens * top_k * sizeof(int), hipMemcpyDeviceToHost));
    TRY(hipMemcpy(host_w, w, (size_t)n_tokens * top_k * sizeof(float), hipMemcpyDeviceToHost));
    TRY(hipMemcpy(host_out, out, (size_t)n_tokens * hidden * sizeof(float),
                  hipMemcpyDeviceToHost));
done:
    (void)hipDeviceSynchronize();
    (void)hipFree(arena);
    (void)hipFree(table);
    (void)hipFree(W);
    (void)hipFree(bias);
    (void)hipFree(x);
    (void)hipFree(scores);
    (void)hipFree(idx);
    (void)hipFree(w);
    (void)hipFree(out);
    (void)hipFree(ws);
    free(h_table);
    return rc;
}
