// fp32 expert GEMMs for shapes the MFMA path does not tile: hidden_dim or
// intermediate_dim not a multiple of 32 (the reference's moe_forward,
// kernels/moe/naive_moe.cu:400-471, takes any D and I).
//
// Same work decomposition as the MFMA path -- the permutation's M-tiles
// {expert, first sorted row, rows} of up to 256 expert-sorted rows, one
// launch per GEMM over all experts -- but each workgroup computes a 64 x 64
// output tile with 4 x 4 fp32 FMAs per thread from 16-deep K slices staged
// in LDS, with every load bounds-checked, so any K and N work:
//   UP   act[row, n] = silu(x[tok] . W1[e, n]) * (x[tok] . W1[e, I + n]):
//        the 64 tile columns are 32 gate columns n0.. and the 32 matching
//        up columns I + n0.., arranged so that a thread holds the gate and
//        up values of the same two n (SwiGLU in registers, with the
//        reference's expf and IEEE division, naive_moe.cu:297-310);
//   DOWN ypair[slot, n] = w(slot) * (act[row] . W2[e, n]).
// combine_f32_any_kernel then sums each token's rows in ascending expert
// order (the reference's scatter order, tests/test_moe.cu:123-132) for any
// D.  This path serves odd shapes; aligned shapes take the MFMA kernels.
#include "internal.hpp"

namespace amdmoe {

constexpr int kGBM = 64, kGBN = 64, kGBK = 16;

template <int MODE>
__global__ __launch_bounds__(256) void grouped_gemm_f32_any_kernel(
    const float* __restrict__ a, const int* __restrict__ a_map, const float* __restrict__ w,
    long w_expert_elems, int K, int n_out, const int4* __restrict__ tiles,
    const int* __restrict__ num_tiles, int n_tiles_n, float* __restrict__ out,
    const int* __restrict__ sorted_slot, const float* __restrict__ sorted_w) {
    __shared__ float As[kGBK][kGBM + 1];
    __shared__ float Ws[kGBK][kGBN + 1];
    __shared__ long s_arow[kGBM];
    constexpr int kSub = kMTile / kGBM;  // 64-row sub-tiles of an M-tile
    const int item = blockIdx.x;
    const int nt = item % n_tiles_n;
    const int mt_sub = item / n_tiles_n;
    const int mt = mt_sub / kSub, sub = mt_sub % kSub;
    if (mt >= *num_tiles) return;
    const int4 tile = tiles[mt];
    const int e = tile.x, rows = tile.z;
    const int r0 = sub * kGBM;
    if (r0 >= rows) return;
    const int row0 = tile.y + r0;
    const int live = min(kGBM, rows - r0);
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;

    // A row (index into a) of each of the 64 tile rows, -1 past the tile
    if (tid < kGBM)
        s_arow[tid] = tid < live ? (MODE == MODE_UP ? (long)a_map[row0 + tid] : (long)(row0 + tid)) : -1;
    // weight row of tile column c: UP c < 32 -> gate n0 + c, else up I + n0 + c - 32
    const float* we = w + (size_t)e * w_expert_elems;
    auto wrow = [&](int c) -> long {
        if (MODE == MODE_UP) {
            const int n = nt * 32 + (c & 31);
            if (n >= n_out) return -1;
            return c < 32 ? (long)n : (long)n_out + n;
        }
        const int n = nt * kGBN + c;
        return n < n_out ? (long)n : -1;
    };
    __syncthreads();

    float acc[4][4] = {};
    // staging: thread loads A element (row lr, k lk) and W element (col lr, k lk)
    // for 4 (row, k) pairs: idx = tid + 256 j, lr = idx / 16, lk = idx % 16
    for (int k0 = 0; k0 < K; k0 += kGBK) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = tid + 256 * j, lr = i >> 4, lk = i & 15;
            const int k = k0 + lk;
            const long ar = s_arow[lr];
            As[lk][lr] = ar >= 0 && k < K ? a[ar * K + k] : 0.0f;
            const long wr = wrow(lr);
            Ws[lk][lr] = wr >= 0 && k < K ? we[wr * K + k] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kGBK; kk++) {
            float av[4], wv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) av[i] = As[kk][ty + 16 * i];
#pragma unroll
            for (int j = 0; j < 4; j++) wv[j] = Ws[kk][tx + 16 * j];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = fmaf(av[i], wv[j], acc[i][j]);
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = ty + 16 * i;
        if (r >= live) continue;
        const size_t pos = (size_t)row0 + r;
        if (MODE == MODE_UP) {
            // columns j = 0, 1 are gate n = nt*32 + tx + 16j; j = 2, 3 the matching up
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int n = nt * 32 + tx + 16 * j;
                if (n >= n_out) continue;
                const float g = acc[i][j], u = acc[i][j + 2];
                out[pos * n_out + n] = g / (1.0f + expf(-g)) * u;
            }
        } else {
            const size_t slot = (size_t)sorted_slot[pos];
            const float wgt = sorted_w[pos];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int n = nt * kGBN + tx + 16 * j;
                if (n < n_out) out[slot * n_out + n] = acc[i][j] * wgt;
            }
        }
    }
}

// y[t, :] = sum of token t's weighted rows ypair[t*K + k, :] in ascending
// expert order (first occurrence of each valid expert), any D.
__global__ __launch_bounds__(256) void combine_f32_any_kernel(const float* __restrict__ ypair,
                                                              const int* __restrict__ idx, int K,
                                                              int E, int D, float* __restrict__ y) {
    __shared__ int s_ord[64];
    __shared__ int s_n;
    const int t = blockIdx.x;
    if (threadIdx.x == 0) {
        int n = 0;
        int ek[64];
        for (int k = 0; k < K; k++) {
            const int e = idx[(size_t)t * K + k];
            if (e < 0 || e >= E) continue;
            bool dup = false;
            for (int j = 0; j < k; j++) dup |= idx[(size_t)t * K + j] == e;
            if (dup) continue;
            int p = n++;
            while (p > 0 && ek[p - 1] > e) {
                ek[p] = ek[p - 1];
                s_ord[p] = s_ord[p - 1];
                p--;
            }
            ek[p] = e;
            s_ord[p] = k;
        }
        s_n = n;
    }
    __syncthreads();
    const int n = s_n;
    for (int c = threadIdx.x; c < D; c += blockDim.x) {
        float acc = 0.0f;
        for (int j = 0; j < n; j++) acc = add_rn(acc, ypair[((size_t)t * K + s_ord[j]) * D + c]);
        y[(size_t)t * D + c] = acc;
    }
}

int launch_experts_f32_any(const float* x, const float* w1, const float* w2, int T, int E, int K,
                           int D, int I, const int4* tiles, const int* num_tiles, long max_tiles,
                           const int* sorted_token, const int* sorted_slot, const float* sorted_w,
                           const int* idx, float* act, float* ypair, float* y, hipStream_t st) {
    AMDMOE_CHECK_ARG(K <= 64, "moe_forward: top_k=%d > 64", K);
    if (T == 0 || max_tiles == 0) return AMDMOE_OK;
    constexpr int kSub = kMTile / kGBM;
    const int nt_up = (int)ceil_div(I, 32), nt_dn = (int)ceil_div(D, kGBN);
    const long g_up = max_tiles * kSub * nt_up, g_dn = max_tiles * kSub * nt_dn;
    AMDMOE_CHECK_ARG(g_up < (1L << 31) && g_dn < (1L << 31), "moe_forward: grid too large");
    hipLaunchKernelGGL(grouped_gemm_f32_any_kernel<MODE_UP>, dim3((unsigned)g_up), dim3(256), 0, st,
                       x, sorted_token, w1, 2L * I * D, D, I, tiles, num_tiles, nt_up, act,
                       nullptr, nullptr);
    AMDMOE_LAUNCH_CHECK();
    hipLaunchKernelGGL(grouped_gemm_f32_any_kernel<MODE_DOWN>, dim3((unsigned)g_dn), dim3(256), 0, st,
                       act, nullptr, w2, (long)D * I, I, D, tiles, num_tiles, nt_dn, ypair,
                       sorted_slot, sorted_w);
    AMDMOE_LAUNCH_CHECK();
    hipLaunchKernelGGL(combine_f32_any_kernel, dim3(T), dim3(256), 0, st, ypair, idx, K, E, D, y);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

}  // namespace amdmoe
