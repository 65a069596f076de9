// Shared device/host helpers for the gfx950 MoE + DSA library.
//
// Everything here is CDNA4 (gfx950) specific: 64-lane wavefronts, MFMA
// builtins, the OCP fp8 conversion instruction.  There is no other target.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include <type_traits>
#include <utility>

#include "../../include/amdmoe.h"

namespace amdmoe {

constexpr int kWave = 64;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------------ status
// Records a message for amdmoe_last_error() and returns the status code.
int set_error(int code, const char* fmt, ...);

#define AMDMOE_HIP_TRY(expr)                                                           \
    do {                                                                               \
        hipError_t e_ = (expr);                                                        \
        if (e_ != hipSuccess)                                                          \
            return ::amdmoe::set_error(AMDMOE_ERR_HIP, "%s:%d: %s: %s", __FILE__,       \
                                       __LINE__, #expr, hipGetErrorString(e_));        \
    } while (0)

#define AMDMOE_CHECK_ARG(cond, ...)                                                    \
    do {                                                                               \
        if (!(cond)) return ::amdmoe::set_error(AMDMOE_ERR_INVALID, __VA_ARGS__);      \
    } while (0)

// Launch check: a launch failure surfaces through hipGetLastError.
#define AMDMOE_LAUNCH_CHECK()                                                          \
    do {                                                                               \
        hipError_t e_ = hipGetLastError();                                             \
        if (e_ != hipSuccess)                                                          \
            return ::amdmoe::set_error(AMDMOE_ERR_HIP, "%s:%d: kernel launch: %s",      \
                                       __FILE__, __LINE__, hipGetErrorString(e_));     \
    } while (0)

// ------------------------------------------------------------------ formats
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(((uint32_t)h) << 16);
}

// Round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Two floats -> two bf16 (a in the low half), round to nearest even: the
// gfx950 v_cvt_pk_bf16_f32 (same results as f32_to_bf16 for every non-NaN
// input; NaNs stay NaNs).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}

// v / s rounded to nearest, for values that share the divisor s (a block
// scale): one correctly rounded reciprocal r = RN(1/s) per block, then per
// value q0 = RN(v r) and one FMA correction, RN(q0 + RN(v - s q0) r).  By
// Markstein's theorem (r within half an ulp of 1/s, q0 within one ulp of
// v/s, so v - s q0 is exact under an FMA) the result is the correctly
// rounded quotient, the same value as an IEEE division.  The identity needs
// r, q0 and the residual in the normal range, which holds for s >= 2^-64
// and every quotient that does not round to zero in e4m3; smaller scales
// take the IEEE division.
struct BlockDivisor {
    float s, r;
    bool fast;
};
__device__ __forceinline__ BlockDivisor block_divisor(float s) {
    return {s, __fdiv_rn(1.0f, s), s >= 0x1p-64f};
}
__device__ __forceinline__ float div_rn(const BlockDivisor& d, float v) {
    if (!d.fast) return __fdiv_rn(v, d.s);
    const float q0 = v * d.r;
    return __builtin_fmaf(__builtin_fmaf(-q0, d.s, v), d.r, q0);
}

// Four floats -> four OCP e4m3 bytes (RNE).  Inputs are pre-clamped to
// +-448 so the hardware conversion never sees an out-of-range value; the
// result then equals round-to-nearest-even with saturation.
__device__ __forceinline__ uint32_t f32x4_to_e4m3x4(float a, float b, float c, float d) {
    a = fminf(fmaxf(a, -448.0f), 448.0f);
    b = fminf(fmaxf(b, -448.0f), 448.0f);
    c = fminf(fmaxf(c, -448.0f), 448.0f);
    d = fminf(fmaxf(d, -448.0f), 448.0f);
    int v = 0;
    v = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, v, false);
    v = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, v, true);
    return (uint32_t)v;
}

// The same conversion for inputs known to lie within +-448 up to rounding
// (RNE takes anything below 464 to at most 448).
__device__ __forceinline__ uint32_t f32x4_to_e4m3x4_noclamp(float a, float b, float c, float d) {
    int v = 0;
    v = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, v, false);
    v = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, v, true);
    return (uint32_t)v;
}

// ------------------------------------------------------------------ MFMA
// 16x16 output tiles.  Operand lane layout (A and B alike): lane l supplies
// row/column (l & 15) and the K-slot group (l >> 4).  Output: lane l holds
// C[4*(l>>4) + i][l & 15], i = 0..3.
__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// OCP e4m3 x e4m3, K = 128, unit (E8M0 = 127) hardware scales.
__device__ __forceinline__ f32x4 mfma_fp8(i32x8 a, i32x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// ------------------------------------------------------------------ exact order
// A binary32 product and sum that are never fused into an FMA (hipcc
// contracts a*b+c by default, and __fmul_rn / __fadd_rn are plain * and +):
// kernels that reproduce a reference loop's rounding use these.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}
// acc + a*b, rounded after the product and after the sum
__device__ __forceinline__ float mac_rn(float acc, float a, float b) {
#pragma clang fp contract(off)
    return acc + a * b;
}

// ------------------------------------------------------------------ wave ops
__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Orders this wave's LDS writes before its subsequent LDS reads by other
// lanes of the same wave (waits for the writes, fences the compiler).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// ------------------------------------------------------------------ LDS DMA
// Direct global->LDS loads (buffer_load ... lds): lane l of a wave writes its
// `size` bytes at M0 + l*size, where M0 is the (wave-uniform) LDS pointer.
// A voffset past the descriptor's range reads as zeros.
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(1))) void* gptr_t;  // a global-memory pointer (global_load_lds)
constexpr int kRsrcFlags = 0x00020000;   // raw buffer, 32-bit data format
constexpr uint32_t kOob = 0x80000000u;   // voffset that fails the range check

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, long bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, kRsrcFlags);
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14, expcnt/lgkmcnt maxed).
template <int N> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier without the memory fence of __syncthreads (which would
// wait for every outstanding load, draining a DMA ring); the empty asm
// statements keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void bare_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// This wave's LDS operations have completed (lgkmcnt(0) only).
__device__ __forceinline__ void lds_wait() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xF | (7 << 4) | (0 << 8) | (3 << 14));
    asm volatile("" ::: "memory");
}

// LDS writes issued before it are visible to every wave after it: waits for
// this wave's LDS operations only (lgkmcnt(0); vector-memory and export
// counters unconstrained, so direct-to-LDS loads keep flowing), then
// s_barrier.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xF | (7 << 4) | (0 << 8) | (3 << 14));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>), in order
// (compile-time indices, e.g. for instruction immediates)
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>()), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>());
}

// ------------------------------------------------------------------ host
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
inline long ceil_div(long a, long b) { return (a + b - 1) / b; }

}  // namespace amdmoe
