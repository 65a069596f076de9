// fp8 formats of the BASELINE DeepSeek-V3 config (the reference is fp32
// only, so these have no reference counterpart; the CPU oracle's
// orc_quant_rows_1x128 / orc_quant_weight_128x128 define them):
//   activations: one fp32 scale per row per 128 columns, scale = amax/448,
//                q = e4m3_rne_sat(v / scale)  (scale 1 for an all-zero block)
//   weights:     one fp32 scale per 128x128 block, scale = u*amax/448.
// The divisions are IEEE round-to-nearest (__fdiv_rn) so the codes are
// bit-identical to the oracle's.
#include "internal.hpp"

namespace amdmoe {

// One wave per (row, 128-column block); each lane converts 2 values.
__global__ __launch_bounds__(256) void quant_rows_kernel(const uint16_t* __restrict__ x, long rows,
                                                         int cols, uint8_t* __restrict__ q,
                                                         float* __restrict__ scale) {
    const int nb = cols / 128;
    const long job = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (job >= rows * nb) return;
    const int lane = threadIdx.x & 63;
    const long r = job / nb;
    const int b = (int)(job % nb);
    const size_t off = (size_t)r * cols + (size_t)b * 128 + lane * 2;
    uint32_t pair = *(const uint32_t*)(x + off);
    float v0 = bf16_to_f32((uint16_t)(pair & 0xffff)), v1 = bf16_to_f32((uint16_t)(pair >> 16));
    float amax = wave_max(fmaxf(fabsf(v0), fabsf(v1)));
    float s = amax > 0.0f ? __fdiv_rn(amax, 448.0f) : 1.0f;
    uint32_t c = f32x4_to_e4m3x4(__fdiv_rn(v0, s), __fdiv_rn(v1, s), 0.0f, 0.0f);
    *(uint16_t*)(q + off) = (uint16_t)(c & 0xffff);
    if (lane == 0) scale[r * nb + b] = s;
}

int launch_quant_rows(const uint16_t* x, long rows, int cols, uint8_t* q, float* scale,
                      hipStream_t st) {
    AMDMOE_CHECK_ARG(cols % 128 == 0 && cols > 0, "quant_rows: cols=%d not a multiple of 128", cols);
    long jobs = rows * (cols / 128);
    if (jobs == 0) return AMDMOE_OK;
    hipLaunchKernelGGL(quant_rows_kernel, dim3((unsigned)ceil_div(jobs, 4)), dim3(256), 0, st, x,
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
