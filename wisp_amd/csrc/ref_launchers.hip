/*
 * ref_launchers.hip — the reference engine's expert-path launchers
 * (csrc/core/wisp_engine.h:496-583 subset) rebuilt for gfx950.
 *
 * These keep the reference's names, argument order, element formulas and
 * early-return/error behaviour so the reference's gpu_expert_ffn call shape
 * (csrc/core/wisp_engine.c:1507-1531) runs on them unchanged. The data
 * paths are new: 8 nibbles per thread with one 32-bit load and a 16-byte
 * store for the dequant; one wave per output row with 16-byte weight loads
 * and a shuffle reduction for the fp16 GEMVs (the reference uses one
 * 256-thread block per row with scalar __half loads).
 */
#include "hip_common.h"

/* ======================================================================= */
/* int4 -> fp16 dequant (csrc/cuda/expert_loader.cu:23-43)                  */
/* ======================================================================= */

/* value = fp16_rn(fma(nib - 8, s, z)); (nib-8)*s is exact in fp32, so the
 * fma equals the reference's mul-then-add. */
__device__ __forceinline__ uint16_t dq_one(int nib, float s, float z) {
    f16 h = (f16)__builtin_fmaf((float)(nib - 8), s, z);
    return __builtin_bit_cast(uint16_t, h);
}

/* 8 consecutive elements per thread; requires gs % 8 == 0, n % 8 == 0,
 * packed 4-byte aligned and out 16-byte aligned (checked by the host). */
__global__ void dequant8_kernel(const uint32_t* __restrict__ packed,
                                const uint16_t* __restrict__ scales,
                                const uint16_t* __restrict__ zeros,
                                u4* __restrict__ out, long n8, int gs) {
    long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n8) return;
    uint32_t w = packed[t];
    long g = (t * 8) / gs;
    float s = half_bits_to_float(scales[g]);
    float z = half_bits_to_float(zeros[g]);
    uint16_t v[8];
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = dq_one((w >> (4 * e)) & 0xF, s, z);
    u4 o;
    o.x = v[0] | ((uint32_t)v[1] << 16);
    o.y = v[2] | ((uint32_t)v[3] << 16);
    o.z = v[4] | ((uint32_t)v[5] << 16);
    o.w = v[6] | ((uint32_t)v[7] << 16);
    out[t] = o;
}

/* Any alignment / group size: one element per thread, as the format is
 * defined (csrc/cuda/expert_loader.cu:31-42). */
__global__ void dequant1_kernel(const uint8_t* __restrict__ packed,
                                const uint16_t* __restrict__ scales,
                                const uint16_t* __restrict__ zeros,
                                uint16_t* __restrict__ out, long n, int gs) {
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint8_t b = packed[i >> 1];
    int nib = (i & 1) ? (b >> 4) : (b & 0x0F);
    long g = i / gs;
    out[i] = dq_one(nib, half_bits_to_float(scales[g]), half_bits_to_float(zeros[g]));
}

extern "C" hipError_t launch_dequant_expert(const uint8_t* d_packed,
                                            const wisp_half* d_scales,
                                            const wisp_half* d_zeros,
                                            wisp_half* d_output,
                                            int n_elements, int group_size,
                                            hipStream_t stream) {
    if (n_elements <= 0 || group_size <= 0) return hipErrorInvalidValue;
    const int T = 256;
    bool vec = (group_size % 8 == 0) && (n_elements % 8 == 0) &&
               ((uintptr_t)d_packed % 4 == 0) && ((uintptr_t)d_output % 16 == 0);
    if (vec) {
        long n8 = n_elements / 8;
        unsigned blocks = (unsigned)((n8 + T - 1) / T);
        hipLaunchKernelGGL(dequant8_kernel, dim3(blocks), dim3(T), 0, stream,
                           (const uint32_t*)d_packed, d_scales, d_zeros,
                           (u4*)d_output, n8, group_size);
    } else {
        unsigned blocks = (unsigned)(((long)n_elements + T - 1) / T);
        hipLaunchKernelGGL(dequant1_kernel, dim3(blocks), dim3(T), 0, stream,
                           d_packed, d_scales, d_zeros, d_output,
                           (long)n_elements, group_size);
    }
    return hipGetLastError();
}

extern "C" hipError_t async_load_expert(const uint8_t* h_packed,
                                        const wisp_half* h_scales,
                                        const wisp_half* h_zeros,
                                        uint8_t* d_packed_tmp,
                                        wisp_half* d_scales_tmp,
                                        wisp_half* d_zeros_tmp,
                                        wisp_half* d_output,
                                        int n_elements, int group_size,
                                        hipStream_t stream) {
    if (n_elements <= 0 || group_size <= 0) return hipErrorInvalidValue;
    size_t n_groups = ((size_t)n_elements + group_size - 1) / group_size;
    size_t packed_bytes = ((size_t)n_elements + 1) / 2;
    size_t scale_bytes = n_groups * sizeof(wisp_half);
    hipError_t e;
    e = hipMemcpyAsync(d_packed_tmp, h_packed, packed_bytes, hipMemcpyHostToDevice, stream);
    if (e != hipSuccess) return e;
    e = hipMemcpyAsync(d_scales_tmp, h_scales, scale_bytes, hipMemcpyHostToDevice, stream);
    if (e != hipSuccess) return e;
    e = hipMemcpyAsync(d_zeros_tmp, h_zeros, scale_bytes, hipMemcpyHostToDevice, stream);
    if (e != hipSuccess) return e;
    return launch_dequant_expert(d_packed_tmp, d_scales_tmp, d_zeros_tmp, d_output,
                                 n_elements, group_size, stream);
}

/* ======================================================================= */
/* fp16-weight GEMVs (csrc/cuda/matmul.cu:43-65, 150-205)                   */
/* ======================================================================= */

/* Partial dot of one row with fp32 x for this lane; a wave covers the row.
 * Vector path: 8 halves (16 B) per lane per step. */
template <bool VEC>
__device__ __forceinline__ float row_dot_f16_part(const uint16_t* __restrict__ row,
                                                  const float* __restrict__ x,
                                                  int cols, int lane) {
    float acc = 0.0f;
    if (VEC) {
        const u4* r8 = (const u4*)row;
        const f4* x4 = (const f4*)x;
        int n8 = cols / 8;
        for (int c = lane; c < n8; c += WAVE) {
            u4 w = r8[c];
            f4 xa = x4[2 * c], xb = x4[2 * c + 1];
            h8 wh = __builtin_bit_cast(h8, w);
            acc = __builtin_fmaf((float)wh[0], xa.x, acc);
            acc = __builtin_fmaf((float)wh[1], xa.y, acc);
            acc = __builtin_fmaf((float)wh[2], xa.z, acc);
            acc = __builtin_fmaf((float)wh[3], xa.w, acc);
            acc = __builtin_fmaf((float)wh[4], xb.x, acc);
            acc = __builtin_fmaf((float)wh[5], xb.y, acc);
            acc = __builtin_fmaf((float)wh[6], xb.z, acc);
            acc = __builtin_fmaf((float)wh[7], xb.w, acc);
        }
    } else {
        for (int c = lane; c < cols; c += WAVE)
            acc = __builtin_fmaf(half_bits_to_float(row[c]), x[c], acc);
    }
    return acc;
}

template <bool VEC>
__global__ __launch_bounds__(256) void gemv_f16_kernel(const uint16_t* __restrict__ W,
                                                       const float* __restrict__ x,
                                                       float* __restrict__ y,
                                                       int rows, int cols) {
    int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    int lane = threadIdx.x & 63;
    if (r >= rows) return;
    float acc = row_dot_f16_part<VEC>(W + (size_t)r * cols, x, cols, lane);
    acc = wave_sum(acc);
    if (lane == 0) y[r] = acc;
}

template <bool VEC>
__global__ __launch_bounds__(256) void swiglu_ffn_kernel(const uint16_t* __restrict__ Wg,
                                                         const uint16_t* __restrict__ Wu,
                                                         const float* __restrict__ x,
                                                         float* __restrict__ h,
                                                         int inter, int cols) {
    int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    int lane = threadIdx.x & 63;
    if (r >= inter) return;
    float g = row_dot_f16_part<VEC>(Wg + (size_t)r * cols, x, cols, lane);
    float u = row_dot_f16_part<VEC>(Wu + (size_t)r * cols, x, cols, lane);
    g = wave_sum(g);
    u = wave_sum(u);
    if (lane == 0) h[r] = silu_f(g) * u;
}

static bool f16_vec_ok(const void* W, const void* x, int cols) {
    return cols % 8 == 0 && (uintptr_t)W % 16 == 0 && (uintptr_t)x % 16 == 0;
}

extern "C" void wisp_gpu_gemv_f16(const wisp_half* W, const float* x, float* y,
                                  int rows, int cols, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return;
    dim3 grid((rows + 3) / 4), block(256);
    if (f16_vec_ok(W, x, cols))
        hipLaunchKernelGGL(gemv_f16_kernel<true>, grid, block, 0, s, W, x, y, rows, cols);
    else
        hipLaunchKernelGGL(gemv_f16_kernel<false>, grid, block, 0, s, W, x, y, rows, cols);
}

extern "C" void wisp_gpu_swiglu_ffn(const wisp_half* Wg, const wisp_half* Wu,
                                    const float* x, float* h, int inter,
                                    int cols, hipStream_t s) {
    if (inter <= 0 || cols <= 0) return;
    dim3 grid((inter + 3) / 4), block(256);
    if (f16_vec_ok(Wg, x, cols) && (uintptr_t)Wu % 16 == 0)
        hipLaunchKernelGGL(swiglu_ffn_kernel<true>, grid, block, 0, s, Wg, Wu, x, h, inter, cols);
    else
        hipLaunchKernelGGL(swiglu_ffn_kernel<false>, grid, block, 0, s, Wg, Wu, x, h, inter, cols);
}

__global__ void scale_accum_kernel(float* __restrict__ acc, const float* __restrict__ x,
                                   float w, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) acc[i] = __builtin_fmaf(w, x[i], acc[i]);
}

extern "C" void wisp_gpu_scale_accum(float* acc, const float* x, float w, int n,
                                     hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(scale_accum_kernel, dim3((n + 255) / 256), dim3(256), 0, s,
                       acc, x, w, n);
}

/* Plain 16-byte-per-lane copy of a known byte count. Not part of the
 * reference interface: hardware byte counters (FETCH_SIZE / WRITE_SIZE)
 * read over this kernel give the factor that turns their units into bytes
 * moved. Requires 16-byte aligned pointers and bytes % 16 == 0. */
__global__ void copy_calibration_kernel(uint4* __restrict__ dst, const uint4* __restrict__ src,
                                        size_t n16) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16; i += stride)
        dst[i] = src[i];
}

extern "C" hipError_t wisp_amd__copy_calibration(void* dst, const void* src, size_t bytes,
                                                 hipStream_t s) {
    if (bytes == 0 || bytes % 16 || (uintptr_t)dst % 16 || (uintptr_t)src % 16)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(copy_calibration_kernel, dim3(4096), dim3(256), 0, s, (uint4*)dst,
                       (const uint4*)src, bytes / 16);
    return hipGetLastError();
}
