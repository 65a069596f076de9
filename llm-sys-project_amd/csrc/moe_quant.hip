// fp8 formats of the BASELINE DeepSeek-V3 config (the reference is fp32
// only, so these have no reference counterpart; the CPU oracle's
// orc_quant_rows_1x128 / orc_quant_weight_128x128 define them):
//   activations: one fp32 scale per row per 128 columns, scale = amax/448,
//                q = e4m3_rne_sat(v / scale)  (scale 1 for an all-zero block)
//   weights:     one fp32 scale per 128x128 block, scale = u*amax/448.
// The divisions are IEEE round-to-nearest (__fdiv_rn; for the activations
// div_rn, whose reciprocal and FMA correction give the same quotients), so
// the codes are bit-identical to the oracle's.
#include "internal.hpp"

namespace amdmoe {

// max over the 16 lanes of a DPP row (xor 1, xor 2, half-row mirror, row
// mirror): every lane of the row ends with the row's maximum
template <int CTRL>
__device__ __forceinline__ float dpp_max(float v) {
    return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v),
                                                                CTRL, 0xF, 0xF, false)));
}

// One wave per row.  A 128-column block is one 16-lane row of the wave
// (8 values = 16 bytes per lane), so a wave step covers 4 blocks and the
// block amax is a DPP reduction within the row; 8 steps (64 KB per CU) are
// loaded before any is converted.
constexpr int kQrBatch = 8;

__global__ __launch_bounds__(256) void quant_rows_kernel(const uint16_t* __restrict__ x, long rows,
                                                         int cols, uint8_t* __restrict__ q,
                                                         float* __restrict__ scale) {
    const long r = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;  // whole wave
    const int lane = threadIdx.x & 63;
    const int nb = cols / 128;
    const int nsteps = (nb + 3) / 4;
    const uint16_t* xr = x + (size_t)r * cols;
    uint8_t* qr = q + (size_t)r * cols;
    for (int s0 = 0; s0 < nsteps; s0 += kQrBatch) {
        u32x4 v[kQrBatch];
#pragma unroll
        for (int i = 0; i < kQrBatch; i++) {
            const int col = (s0 + i) * 512 + 8 * lane;
            v[i] = col < cols ? *(const u32x4*)(xr + col) : (u32x4){0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < kQrBatch; i++) {
            const int col = (s0 + i) * 512 + 8 * lane;
            float f[8];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                f[2 * k] = __uint_as_float(v[i][k] << 16);
                f[2 * k + 1] = __uint_as_float(v[i][k] & 0xffff0000u);
            }
            float am = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; k++) am = fmaxf(am, fabsf(f[k]));
            am = dpp_max<0x140>(dpp_max<0x141>(dpp_max<0x4E>(dpp_max<0xB1>(am))));
            if (col >= cols) continue;  // the whole 16-lane block is past the row
            const float sc = am > 0.0f ? __fdiv_rn(am, 448.0f) : 1.0f;
            const BlockDivisor d = block_divisor(sc);
            u32x2 c;
            c[0] = f32x4_to_e4m3x4(div_rn(d, f[0]), div_rn(d, f[1]), div_rn(d, f[2]), div_rn(d, f[3]));
            c[1] = f32x4_to_e4m3x4(div_rn(d, f[4]), div_rn(d, f[5]), div_rn(d, f[6]), div_rn(d, f[7]));
            *(u32x2*)(qr + col) = c;
            if ((lane & 15) == 0) scale[r * nb + col / 128] = sc;
        }
    }
}

int launch_quant_rows(const uint16_t* x, long rows, int cols, uint8_t* q, float* scale,
                      hipStream_t st) {
    AMDMOE_CHECK_ARG(cols % 128 == 0 && cols > 0, "quant_rows: cols=%d not a multiple of 128", cols);
    if (rows == 0) return AMDMOE_OK;
    AMDMOE_CHECK_ARG(ceil_div(rows, 4) < (1L << 31), "quant_rows: %ld rows", rows);
    hipLaunchKernelGGL(quant_rows_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, st, x,
                       rows, cols, q, scale);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

// One block of 256 threads per 128x128 weight block; each thread owns 64
// values (half a row).
__global__ __launch_bounds__(256) void quant_weight_kernel(const float* __restrict__ w, int cols,
                                                           const float* __restrict__ u,
                                                           uint8_t* __restrict__ q,
                                                           float* __restrict__ scale) {
    __shared__ float s_max[4];
    const int cb = cols / 128;
    const int bi = blockIdx.y, bj = blockIdx.x;
    const int tid = threadIdx.x;
    const int r = bi * 128 + (tid >> 1);
    const int c0 = bj * 128 + (tid & 1) * 64;
    const float* src = w + (size_t)r * cols + c0;
    float v[64];
    float amax = 0.0f;
    for (int j = 0; j < 64; j += 4) {
        float4 t = *(const float4*)(src + j);
        v[j] = t.x; v[j + 1] = t.y; v[j + 2] = t.z; v[j + 3] = t.w;
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(t.x), fabsf(t.y)), fmaxf(fabsf(t.z), fabsf(t.w))));
    }
    amax = wave_max(amax);
    if ((tid & 63) == 0) s_max[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
    float s = amax > 0.0f ? __fdiv_rn(mul_rn(u[bi * cb + bj], amax), 448.0f) : 1.0f;
    uint8_t* dst = q + (size_t)r * cols + c0;
    for (int j = 0; j < 64; j += 16) {
        u32x4 pk;
        for (int k = 0; k < 4; k++)
            pk[k] = f32x4_to_e4m3x4(__fdiv_rn(v[j + 4 * k], s), __fdiv_rn(v[j + 4 * k + 1], s),
                                    __fdiv_rn(v[j + 4 * k + 2], s), __fdiv_rn(v[j + 4 * k + 3], s));
        *(u32x4*)(dst + j) = pk;
    }
    if (tid == 0) scale[bi * cb + bj] = s;
}

int launch_quant_weight(const float* w, long rows, int cols, const float* u, uint8_t* q,
                        float* scale, hipStream_t st) {
    AMDMOE_CHECK_ARG(rows % 128 == 0 && cols % 128 == 0 && rows > 0 && cols > 0,
                     "quant_weight: [%ld, %d] not a multiple of 128x128", rows, cols);
    AMDMOE_CHECK_ARG(rows / 128 <= 65535, "quant_weight: too many row blocks (%ld)", rows / 128);
    hipLaunchKernelGGL(quant_weight_kernel, dim3(cols / 128, (unsigned)(rows / 128)), dim3(256), 0,
                       st, w, cols, u, q, scale);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

}  // namespace amdmoe
