// Weight packing for the grouped GEMM: an expert weight matrix [N][K] bytes
// (row-major, the layout of W1 [E,2I,D] and W2 [E,D,I] in
// kernels/moe/naive_moe.cuh:66-72, here e4m3 bytes) is rewritten, once at
// load time, into fragment blocks: for every 16 rows x 128 bytes of K
// (one MFMA column tile x one K-step) the 2 KB are stored as
//   [half h][lane l][16 bytes],  l = 16q + r,
// holding row r, bytes 128*kb + 64h + 16q .. +16 -- exactly the 16 bytes
// MFMA operand lane l loads for that half.  Blocks are ordered
// [expert][N/16][K/128].  A wave then reads each half of a K-step as one
// contiguous 1 KB instead of 16 rows x 64 bytes.
#include "internal.hpp"

namespace amdmoe {

// One wave per 16x128-byte block.
__global__ __launch_bounds__(256) void pack_weights_kernel(const uint8_t* __restrict__ w, long nblk,
                                                           long nkb, long K,
                                                           uint8_t* __restrict__ out) {
    const long b = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nblk) return;
    const int l = threadIdx.x & 63, q = l >> 4, r = l & 15;
    const long kb = b % nkb, rb = b / nkb;  // rb = expert * N/16 + n16
    const uint8_t* src = w + (rb * 16 + r) * K + kb * 128 + 16 * q;
    uint8_t* dst = out + b * 2048 + 16 * l;
    *(u32x4*)dst = *(const u32x4*)src;
    *(u32x4*)(dst + 1024) = *(const u32x4*)(src + 64);
}

int launch_pack_weights(const uint8_t* w, long E, long N, long K, uint8_t* out, hipStream_t st) {
    AMDMOE_CHECK_ARG(E >= 1 && N >= 16 && K >= 128 && N % 16 == 0 && K % 128 == 0,
                     "pack_weights: need E >= 1, N %% 16 == 0, K %% 128 == 0 (E=%ld N=%ld K=%ld)", E, N, K);
    AMDMOE_CHECK_ARG(w != out, "pack_weights: in-place packing is not supported");
    const long nkb = K / 128, nblk = E * (N / 16) * nkb;
    AMDMOE_CHECK_ARG((nblk + 3) / 4 < (1L << 31), "pack_weights: too many blocks");
    hipLaunchKernelGGL(pack_weights_kernel, dim3((unsigned)((nblk + 3) / 4)), dim3(256), 0, st, w, nblk,
                       nkb, K, out);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

}  // namespace amdmoe
