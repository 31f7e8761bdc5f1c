/*
 * hip_common.h — device helpers shared by the gfx950 kernels (internal).
 */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "../../include/wisp_amd.h"

typedef _Float16 f16;
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

#define WAVE 64

/* ---- int4 unpack without conversions ----------------------------------
 * One dword holds 8 nibbles n0..n7 (n0 in bits 0-3: low nibble = even
 * element). OR-ing a nibble into the mantissa of fp16 1024.0 (0x6400)
 * yields the exact fp16 value 1024 + n; a high nibble (bits 4-7 of its
 * half) yields 1024 + 16 n. Four and-or ops and one shift give 8 fp16
 * values in the k-slot order
 *     slot: 0   1   2   3   4   5   6   7
 *     elem: e0  e4  e1  e5  e2  e6  e3  e7
 *     val : 1024+n (even elements)   1024+16n (odd elements)
 * The activation operand is permuted to the same slot order with odd
 * elements pre-divided by 16, so each product is (1024 + n) x for even and
 * (64 x + n x) for odd elements; the constant excess
 *     1032 * sum(x_even) + 1152 * sum(x_odd / 16)
 * over a block turns the sum into sum((n - 8) x) exactly in real
 * arithmetic. The excess itself is produced by one more MFMA against a
 * constant operand (see mfma_excess_operand).                              */
/* Written in bitfield-insert form, (w & m) | (o & ~m), which equals
 * (w & m) | o for these masks, with m and o taken from kernel arguments:
 * the compiler then emits one v_bfi_b32 per output dword (with literal
 * masks it emits v_and_b32 + v_or_b32). */
__device__ __forceinline__ h8 unpack8_magic(uint32_t w, uint32_t m_lo, uint32_t m_hi,
                                            uint32_t one024) {
    const uint32_t t = w >> 8;
    u4 v;
    v.x = (w & m_lo) | (one024 & ~m_lo);
    v.y = (w & m_hi) | (one024 & ~m_hi);
    v.z = (t & m_lo) | (one024 & ~m_lo);
    v.w = (t & m_hi) | (one024 & ~m_hi);
    return __builtin_bit_cast(h8, v);
}

/* Slot of element e (0..7) of an 8-element block in the order above. */
__device__ __host__ __forceinline__ int perm_slot(int e) {
    return ((e & 3) << 1) | (e >> 2);
}

/* Constant B operands for the correction MFMAs, the same in every column so
 * that each lane receives its own token's value (no cross-lane read):
 *   excess pattern: 1032 on even-element slots, 1152 on odd-element slots
 *   sum pattern   : 1 / 16, giving sum(x) for the zero-point term.      */
__device__ __forceinline__ h8 mfma_excess_operand() {
    h8 c;
    c[0] = (f16)1032.0f; c[1] = (f16)1032.0f; c[2] = (f16)1152.0f; c[3] = (f16)1152.0f;
    c[4] = (f16)1032.0f; c[5] = (f16)1032.0f; c[6] = (f16)1152.0f; c[7] = (f16)1152.0f;
    return c;
}
__device__ __forceinline__ h8 mfma_sum_operand() {
    h8 c;
    c[0] = (f16)1.0f; c[1] = (f16)1.0f; c[2] = (f16)16.0f; c[3] = (f16)16.0f;
    c[4] = (f16)1.0f; c[5] = (f16)1.0f; c[6] = (f16)16.0f; c[7] = (f16)16.0f;
    return c;
}

/* D(16x16, fp32) += A(16x32, fp16) B(32x16, fp16). Lane l supplies A row
 * l%16 and B column l%16 for k-slice l/16 (8 values each); it receives
 * D[4*(l/16) + v][l%16] for v = 0..3. */
__device__ __forceinline__ f4 mfma16x16x32(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

/* The global-address-space view of a pointer. Pointers read from memory
 * (an expert table, a blob's sections) are generic to the compiler, so loads
 * through them become FLAT loads, which also count in lgkmcnt: every wait
 * for a scalar load or LDS access then waits for all of them too. Loads
 * through this view are global loads, counted in vmcnt only. */
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gptr(const T* p) {
    return (const __attribute__((address_space(1))) T*)p;
}

__device__ __forceinline__ float silu_f(float g) {
    return g / (1.0f + __expf(-g));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, WAVE);
    return v;
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    return (float)__builtin_bit_cast(f16, h);
}

/* ---- profiling hook (wisp_amd_set_kernel_events) -----------------------
 * Fixed event-pair slot per kernel kind. */
enum { EV_ROUTE = 0, EV_PREP = 1, EV_GATEUP = 2, EV_DOWN = 3, EV_COMBINE = 4, EV_PF_GATEUP = 5,
       EV_PF_DOWN = 6, EV_KINDS = 7 };
extern "C" hipEvent_t* wisp_amd__events;
extern "C" int wisp_amd__event_pairs;

static inline void ev_before(int i, hipStream_t s) {
    if (wisp_amd__events && i < wisp_amd__event_pairs)
        (void)hipEventRecord(wisp_amd__events[2 * i], s);
}
static inline void ev_after(int i, hipStream_t s) {
    if (wisp_amd__events && i < wisp_amd__event_pairs)
        (void)hipEventRecord(wisp_amd__events[2 * i + 1], s);
}

/* ---- the library's second stream ---------------------------------------
 * One per device, with two events (timing off) for a fork from and a join
 * back to the caller's stream; created by the first call that asks for it
 * outside a graph capture and kept until the process ends (the prefill
 * runs its small tiles there). A caller takes wisp_amd__side_mu before
 * wisp_amd__side() and keeps it until its join is enqueued, so calls from
 * several host threads cannot interleave their records on the shared
 * events. */
struct SideStream {
    hipStream_t s2;
    hipEvent_t fork, join;
};
extern std::mutex wisp_amd__side_mu;
/* With wisp_amd__side_mu held: the second stream of the device of `s` in
 * *out, or out->s2 == nullptr when it does not exist yet and `s` is being
 * captured (no stream is created inside a capture). */
hipError_t wisp_amd__side(hipStream_t s, SideStream* out);

static inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
