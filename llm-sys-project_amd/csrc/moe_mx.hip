// OCP Microscaling (MX) formats for the MXFP4 expert layer: the quantisers
// and the weight packer.  No counterpart in the reference (fp32 only); the
// format follows the OCP MX specification v1.0:
//   a block of 32 consecutive elements along K shares one E8M0 scale
//   X = 2^(E - 127); E = floor(log2 max|v|) - emax_elem (E2M1: 2, E4M3: 8),
//   clamped to [0, 254] (an all-zero block gets 0); each element is the
//   round-to-nearest-even of v / X in the element format, saturated.
// Weights: E2M1 (FP4), two per byte, even element in the low nibble;
// activations: E4M3 (FP8).  The grouped GEMM consumes the weights in
// fragment order (pack_mxfp4_kernel) and applies both operands' E8M0 scales
// in the MFMA itself (v_mfma_scale_f32_16x16x128_f8f6f4, A = E2M1,
// B = E4M3), so no scale arithmetic is left for the VALU.
#include "internal.hpp"

namespace amdmoe {

// E8M0 exponent of a block with absolute maximum amax, for an element
// format whose largest binade is 2^emax: floor(log2 amax) - emax + 127 is
// amax's biased exponent - emax (a subnormal amax has biased exponent 0).
__device__ __forceinline__ int mx_e8(float amax, int emax) {
    return min(max((int)((__float_as_uint(amax) >> 23) & 0xff) - emax, 0), 254);
}

// Round to nearest even E2M1, saturating at 6 (NaN too): within a binade
// the values are the multiples of a power-of-two step whose parity is the
// mantissa bit, so RNE is rint(a / step).
__device__ __forceinline__ uint32_t f32_to_e2m1(float v) {
    const uint32_t sign = (__float_as_uint(v) >> 31) << 3;
    const float a = fabsf(v);
    if (!(a < 6.0f)) return sign | 7u;
    const float step = a < 2.0f ? 0.5f : (a < 4.0f ? 1.0f : 2.0f);
    const float r = rintf(a * (1.0f / step)) * step;
    const uint32_t code = r < 2.0f ? (uint32_t)(r * 2.0f)
                                   : (r < 4.0f ? 4u + (uint32_t)(r - 2.0f) : (r < 6.0f ? 6u : 7u));
    return sign | code;
}

// One thread per 32-element block of a fp32 row: E2M1 codes (16 bytes) and
// the block's E8M0 scale.
__global__ __launch_bounds__(256) void quant_weight_mxfp4_kernel(const float* __restrict__ w, long nblk,
                                                                 uint8_t* __restrict__ q,
                                                                 uint8_t* __restrict__ s) {
    const long b = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
    const f32x4* src = (const f32x4*)(w + 32 * b);
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const f32x4 t = src[i];
        v[4 * i] = t[0], v[4 * i + 1] = t[1], v[4 * i + 2] = t[2], v[4 * i + 3] = t[3];
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    const int e8 = mx_e8(amax, 2);
    const float inv = __builtin_amdgcn_ldexpf(1.0f, 127 - e8);
    u32x4 o;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        uint32_t x = 0;
#pragma unroll
        for (int j = 0; j < 8; j++) x |= f32_to_e2m1(v[8 * d + j] * inv) << (4 * j);
        o[d] = x;
    }
    *(u32x4*)(q + 16 * b) = o;
    s[b] = (uint8_t)e8;
}

// One thread per 32-element block of a bf16 row: E4M3 codes and the E8M0
// scale (MXFP8 activations).
__global__ __launch_bounds__(256) void quant_rows_mxfp8_kernel(const uint16_t* __restrict__ x, long nblk,
                                                               uint8_t* __restrict__ q,
                                                               uint8_t* __restrict__ s) {
    const long b = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
    const u32x4* src = (const u32x4*)(x + 32 * b);
    float v[32];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const u32x4 t = src[i];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[8 * i + 2 * j] = __uint_as_float(t[j] << 16);
            v[8 * i + 2 * j + 1] = __uint_as_float(t[j] & 0xffff0000u);
        }
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    const int e8 = mx_e8(amax, 8);
    const float inv = __builtin_amdgcn_ldexpf(1.0f, 127 - e8);
    u32x4 o0, o1;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        o0[k] = f32x4_to_e4m3x4(v[4 * k] * inv, v[4 * k + 1] * inv, v[4 * k + 2] * inv, v[4 * k + 3] * inv);
        o1[k] = f32x4_to_e4m3x4(v[16 + 4 * k] * inv, v[16 + 4 * k + 1] * inv, v[16 + 4 * k + 2] * inv,
                                v[16 + 4 * k + 3] * inv);
    }
    *(u32x4*)(q + 32 * b) = o0;
    *(u32x4*)(q + 32 * b + 16) = o1;
    s[b] = (uint8_t)e8;
}

// Row-major MXFP4 [E][N][K/2] codes + [E][N][K/32] scales -> fragment
// order: per expert, per 16 rows x 128 K (one MFMA operand), 1 KB of codes
// stored [lane l][16 B] with lane l = 16g + r holding row r, bytes
// 64kb + 16g .. +15 (K elements 128kb + 32g .. +31), and 64 scale bytes
// [lane l] = scale of (row r, block 4kb + g); blocks ordered [N/16][K/128].
// One thread per 16-byte chunk of codes (and its scale byte).
__global__ __launch_bounds__(256) void pack_mxfp4_kernel(const uint8_t* __restrict__ q,
                                                         const uint8_t* __restrict__ s, long nchunks,
                                                         int N, int K, uint8_t* __restrict__ qp,
                                                         uint8_t* __restrict__ sp) {
    const long c = (long)blockIdx.x * blockDim.x + threadIdx.x;  // output chunk
    if (c >= nchunks) return;
    const int nk = K / 128;
    const int l = (int)(c & 63);
    long rest = c >> 6;
    const int kb = (int)(rest % nk);
    rest /= nk;
    const long n16 = rest % (N / 16);
    const long e = rest / (N / 16);
    const int r = l & 15, g = l >> 4;
    const long row = e * N + 16 * n16 + r;
    *(u32x4*)(qp + 16 * c) = *(const u32x4*)(q + row * (K / 2) + 64 * kb + 16 * g);
    sp[c] = s[row * (K / 32) + 4 * kb + g];
}

int launch_quant_weight_mxfp4(const float* w, long rows, int cols, uint8_t* q, uint8_t* s,
                              hipStream_t st) {
    AMDMOE_CHECK_ARG(rows >= 0 && cols > 0 && cols % 32 == 0, "quant_weight_mxfp4: cols=%d must be a multiple of 32", cols);
    AMDMOE_CHECK_ARG(w && q && s, "null tensor pointer");
    const long nblk = rows * (cols / 32);
    if (nblk == 0) return AMDMOE_OK;
    hipLaunchKernelGGL(quant_weight_mxfp4_kernel, dim3((unsigned)ceil_div(nblk, 256)), dim3(256), 0, st, w, nblk, q, s);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

int launch_quant_rows_mxfp8(const uint16_t* x, long rows, int cols, uint8_t* q, uint8_t* s,
                            hipStream_t st) {
    AMDMOE_CHECK_ARG(rows >= 0 && cols > 0 && cols % 32 == 0, "quant_rows_mxfp8: cols=%d must be a multiple of 32", cols);
    AMDMOE_CHECK_ARG(x && q && s, "null tensor pointer");
    const long nblk = rows * (cols / 32);
    if (nblk == 0) return AMDMOE_OK;
    hipLaunchKernelGGL(quant_rows_mxfp8_kernel, dim3((unsigned)ceil_div(nblk, 256)), dim3(256), 0, st, x, nblk, q, s);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

int launch_pack_mxfp4(const uint8_t* q, const uint8_t* s, long E, int N, int K, uint8_t* qp,
                      uint8_t* sp, hipStream_t st) {
    AMDMOE_CHECK_ARG(E >= 0 && N > 0 && K > 0 && N % 16 == 0 && K % 128 == 0,
                     "pack_weights_mxfp4: rows=%d must be a multiple of 16, cols=%d of 128", N, K);
    AMDMOE_CHECK_ARG(q && s && qp && sp, "null tensor pointer");
    AMDMOE_CHECK_ARG(qp != q && sp != s, "pack_weights_mxfp4: output aliases input");
    const long nchunks = E * (N / 16) * (K / 128) * 64;
    if (nchunks == 0) return AMDMOE_OK;
    hipLaunchKernelGGL(pack_mxfp4_kernel, dim3((unsigned)ceil_div(nchunks, 256)), dim3(256), 0, st, q, s,
                       nchunks, N, K, qp, sp);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

}  // namespace amdmoe
