/*
 * layer_ops.hip — the decode step's operations on either side of the MoE
 * layer (csrc/core/wisp_engine.c:1709-1722: post-attention RMSNorm, the
 * residual add, the dense fp16 GEMVs and SwiGLU), for gfx950.
 *
 * The reference launchers keep their names, argument order and
 * early-return behaviour (csrc/core/wisp_engine.h:499-508;
 * csrc/cuda/matmul.cu:67-148). The MI355X kernels differ in shape:
 *   RMSNorm   one workgroup of 512 threads per row, 16-byte loads, each
 *             thread keeping its slice of x in registers between the sum of
 *             squares and the scaling (one read of x), fp32 sum reduced with
 *             DPP row moves and LDS;
 *   gemv_t    y = W^T x: a workgroup owns 32 output columns; its 256
 *             threads read 64-byte row segments (4 threads per row, 64 rows
 *             at a time, 16 B each) and reduce over the row lanes in LDS in
 *             a fixed order;
 *   elementwise ops: 16-byte loads and stores, 4 floats per thread.
 * wisp_amd__rmsnorm_rows normalises M rows at once into fp32 and/or fp16
 * for the fused MoE block (moe_decode.hip).
 */
#include "route_common.h"

#define RN_THREADS 512
#define RN_REG_F4 8   /* float4 pieces per thread kept in registers: rows <= 16384 */

/* ---- RMSNorm ------------------------------------------------------------ */

/* y = x * (1 / sqrt(mean(x^2) + eps)) * w for row blockIdx.x of x [rows][n]
 * (row stride n); writes y32 and/or y16 (either may be null). Safe in place
 * (y32 == x): every element is read before the barrier that precedes the
 * writes, by the thread that later writes it. */
__global__ __launch_bounds__(RN_THREADS) void rmsnorm_rows_kernel(
    const float* x, const uint16_t* __restrict__ w, float* y32, uint16_t* y16, int n, float eps) {
    __shared__ float s_part[RN_THREADS / 64];
    const int row = blockIdx.x;
    const float* xr = x + (size_t)row * n;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const bool vec = (n % 4) == 0 && n / 4 <= RN_REG_F4 * RN_THREADS && ((uintptr_t)x % 16) == 0 &&
                     ((uintptr_t)w % 8) == 0 && ((uintptr_t)y32 % 16) == 0 &&
                     ((uintptr_t)y16 % 8) == 0;
    float ss = 0.0f;
    f4 v[RN_REG_F4];
    if (vec) {
#pragma unroll
        for (int c = 0; c < RN_REG_F4; c++) {
            const int i = tid + c * RN_THREADS;
            v[c] = i < n / 4 ? ((const f4*)xr)[i] : (f4){0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int c = 0; c < RN_REG_F4; c++)
#pragma unroll
            for (int q = 0; q < 4; q++) ss = __builtin_fmaf(v[c][q], v[c][q], ss);
    } else {
        for (int i = tid; i < n; i += RN_THREADS) ss = __builtin_fmaf(xr[i], xr[i], ss);
    }
    ss = wave_sum_dpp(ss);
    if (lane == 0) s_part[wv] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < RN_THREADS / 64; i++) tot += s_part[i];
    const float scale = 1.0f / sqrtf(tot / (float)n + eps);
    float* yr32 = y32 ? y32 + (size_t)row * n : nullptr;
    uint16_t* yr16 = y16 ? y16 + (size_t)row * n : nullptr;
    if (vec) {
#pragma unroll
        for (int c = 0; c < RN_REG_F4; c++) {
            const int i = tid + c * RN_THREADS;
            if (i < n / 4) {
                const uint2 wb = ((const uint2*)w)[i];
                const h2 w01 = __builtin_bit_cast(h2, wb.x), w23 = __builtin_bit_cast(h2, wb.y);
                const f4 o = {v[c][0] * scale * (float)w01[0], v[c][1] * scale * (float)w01[1],
                              v[c][2] * scale * (float)w23[0], v[c][3] * scale * (float)w23[1]};
                if (yr32) ((f4*)yr32)[i] = o;
                if (yr16) {
                    const h2 a = {(f16)o[0], (f16)o[1]}, b = {(f16)o[2], (f16)o[3]};
                    ((uint2*)yr16)[i] = (uint2){__builtin_bit_cast(uint32_t, a),
                                                __builtin_bit_cast(uint32_t, b)};
                }
            }
        }
    } else {
        for (int i = tid; i < n; i += RN_THREADS) {
            const float o = xr[i] * scale * half_bits_to_float(w[i]);
            if (yr32) yr32[i] = o;
            if (yr16) yr16[i] = __builtin_bit_cast(uint16_t, (f16)o);
        }
    }
}

/* M rows of x [rows][n] fp32 -> y32 (fp32) and/or y16 (fp16); internal,
 * for the fused MoE block. */
hipError_t wisp_amd__rmsnorm_rows(const float* x, const wisp_half* w, float* y32, wisp_half* y16,
                                  int rows, int n, float eps, hipStream_t s) {
    if (rows <= 0 || n <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(rows), dim3(RN_THREADS), 0, s, x,
                       (const uint16_t*)w, y32, (uint16_t*)y16, n, eps);
    return hipGetLastError();
}

/* y = x * rsqrt(mean(x^2) + eps) * w over n elements; early-returns on
 * n <= 0 (csrc/cuda/matmul.cu:92-121). */
extern "C" void wisp_gpu_rmsnorm(const float* x, const wisp_half* w, float* y, int n, float eps,
                                 hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(1), dim3(RN_THREADS), 0, s, x,
                       (const uint16_t*)w, y, (uint16_t*)nullptr, n, eps);
}

/* ---- elementwise ---------------------------------------------------------- */

#define EW_THREADS 256

__global__ __launch_bounds__(EW_THREADS) void residual_add_kernel(float* x, const float* d, int n) {
    const int i4 = blockIdx.x * EW_THREADS + threadIdx.x;
    const int base = i4 * 4;
    if (base + 3 < n && ((uintptr_t)x % 16) == 0 && ((uintptr_t)d % 16) == 0) {
        f4 a = ((f4*)x)[i4];
        const f4 b = ((const f4*)d)[i4];
#pragma unroll
        for (int q = 0; q < 4; q++) a[q] += b[q];
        ((f4*)x)[i4] = a;
    } else {
        for (int i = base; i < n && i < base + 4; i++) x[i] += d[i];
    }
}

/* x += d; early-returns on n <= 0 (csrc/cuda/matmul.cu:124-134). */
extern "C" void wisp_gpu_residual_add(float* x, const float* delta, int n, hipStream_t s) {
    if (n <= 0) return;
    const int blocks = ((n + 3) / 4 + EW_THREADS - 1) / EW_THREADS;
    hipLaunchKernelGGL(residual_add_kernel, dim3(blocks), dim3(EW_THREADS), 0, s, x, delta, n);
}

__global__ __launch_bounds__(EW_THREADS) void swiglu_kernel(const float* g, const float* u,
                                                            float* o, int n) {
    const int i4 = blockIdx.x * EW_THREADS + threadIdx.x;
    const int base = i4 * 4;
    if (base + 3 < n && ((uintptr_t)g % 16) == 0 && ((uintptr_t)u % 16) == 0 &&
        ((uintptr_t)o % 16) == 0) {
        const f4 gv = ((const f4*)g)[i4], uv = ((const f4*)u)[i4];
        f4 r;
#pragma unroll
        for (int q = 0; q < 4; q++) r[q] = silu_f(gv[q]) * uv[q];
        ((f4*)o)[i4] = r;
    } else {
        for (int i = base; i < n && i < base + 4; i++) o[i] = silu_f(g[i]) * u[i];
    }
}

/* o = silu(g) * u; early-returns on n <= 0 (csrc/cuda/matmul.cu:136-148). */
extern "C" void wisp_gpu_swiglu(const float* gate, const float* up, float* out, int n,
                                hipStream_t s) {
    if (n <= 0) return;
    const int blocks = ((n + 3) / 4 + EW_THREADS - 1) / EW_THREADS;
    hipLaunchKernelGGL(swiglu_kernel, dim3(blocks), dim3(EW_THREADS), 0, s, gate, up, out, n);
}

/* ---- y = W^T x ---------------------------------------------------------------- */

#define GT_THREADS 256
#define GT_COLS 32            /* output columns per workgroup                  */
#define GT_CPT 8              /* columns per thread (one 16-byte piece)        */
#define GT_RLANES (GT_THREADS / (GT_COLS / GT_CPT))   /* row lanes: 64             */

/* Workgroup b owns columns [32 b, 32 b + 32); thread t reads columns
 * 32 b + 8 (t % 4) .. + 8 of rows t / 4, t / 4 + 64, ... (16-byte loads when
 * the row segment is aligned and whole), then the 64 row lanes of each
 * column are added in row-lane order. */
__global__ __launch_bounds__(GT_THREADS) void gemv_t_f16_kernel(const uint16_t* __restrict__ W,
                                                                const float* __restrict__ x,
                                                                float* __restrict__ y, int rows,
                                                                int cols) {
    __shared__ float s_acc[GT_RLANES][GT_COLS + 1];
    const int c0 = blockIdx.x * GT_COLS + (threadIdx.x % (GT_COLS / GT_CPT)) * GT_CPT;
    const int rl = threadIdx.x / (GT_COLS / GT_CPT);
    float acc[GT_CPT];
#pragma unroll
    for (int q = 0; q < GT_CPT; q++) acc[q] = 0.0f;
    const bool vec = (cols % 8) == 0 && ((uintptr_t)W % 16) == 0 && c0 + GT_CPT <= cols;
    for (int r = rl; r < rows; r += GT_RLANES) {
        const float xr = x[r];
        const uint16_t* row = W + (size_t)r * cols;
        if (vec) {
            const h8 wv = *(const h8*)(row + c0);
#pragma unroll
            for (int q = 0; q < GT_CPT; q++) acc[q] = __builtin_fmaf((float)wv[q], xr, acc[q]);
        } else {
#pragma unroll
            for (int q = 0; q < GT_CPT; q++)
                if (c0 + q < cols) acc[q] = __builtin_fmaf(half_bits_to_float(row[c0 + q]), xr, acc[q]);
        }
    }
    const int cl = (threadIdx.x % (GT_COLS / GT_CPT)) * GT_CPT;
#pragma unroll
    for (int q = 0; q < GT_CPT; q++) s_acc[rl][cl + q] = acc[q];
    __syncthreads();
    if (threadIdx.x < GT_COLS) {
        const int c = blockIdx.x * GT_COLS + threadIdx.x;
        float sum = 0.0f;
        for (int i = 0; i < GT_RLANES; i++) sum += s_acc[i][threadIdx.x];
        if (c < cols) y[c] = sum;
    }
}

/* y = W^T x, fp16 W [rows, cols], fp32 x [rows] / y [cols]; early-returns
 * on rows <= 0 or cols <= 0 (csrc/cuda/matmul.cu:67-89). */
extern "C" void wisp_gpu_gemv_t_f16(const wisp_half* W, const float* x, float* y, int rows,
                                    int cols, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return;
    hipLaunchKernelGGL(gemv_t_f16_kernel, dim3((cols + GT_COLS - 1) / GT_COLS), dim3(GT_THREADS),
                       0, s, (const uint16_t*)W, x, y, rows, cols);
}
