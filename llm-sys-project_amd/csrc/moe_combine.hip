// Combine and the reference's remaining elementwise / surface stages.
//
// combine_kernel: y[t,:] = sum over token t's routed slots, in ascending
// expert order, of ypair[t*K+k,:] (already weighted by the down-projection
// epilogue).  This is the reference's accumulation order
// (tests/test_moe.cu:123-132: out starts at 0, experts ascending,
// out += w*g2), so the fp32 path reproduces it exactly given the same
// per-expert rows.
//
// naive_gemm / swiglu / moe_scatter keep the reference stage contracts
// (kernels/moe/naive_moe.cuh:44-62) for callers that drive the stages
// themselves; moe_forward does not use them.
#include "internal.hpp"

namespace amdmoe {

template <typename PT> struct Vec8;
template <> struct Vec8<float> {
    static __device__ __forceinline__ void load(const float* p, float* v) {
        f32x4 a = *(const f32x4*)p, b = *(const f32x4*)(p + 4);
        for (int i = 0; i < 4; i++) { v[i] = a[i]; v[4 + i] = b[i]; }
    }
};
template <> struct Vec8<uint16_t> {
    static __device__ __forceinline__ void load(const uint16_t* p, float* v) {
        u32x4 a = *(const u32x4*)p;
        for (int i = 0; i < 4; i++) {
            v[2 * i] = __uint_as_float(a[i] << 16);
            v[2 * i + 1] = __uint_as_float(a[i] & 0xffff0000u);
        }
    }
};

// nsp > 1 (fp32 rows of a down projection whose K was split): a slot's row
// is the sum of its nsp partial rows, sp_stride elements apart, added in
// split order before it joins the expert-order sum.
template <typename PT, bool OUT_BF16>
__global__ __launch_bounds__(256) void combine_kernel(const PT* __restrict__ ypair,
                                                      const int* __restrict__ idx, int T, int K,
                                                      int E, int D, void* __restrict__ y, int nsp,
                                                      size_t sp_stride) {
    __shared__ int s_ord[64];
    __shared__ int s_n;
    const int t = blockIdx.x;
    if (threadIdx.x == 0) {
        // valid first-occurrence slots, insertion-sorted by expert id
        int n = 0;
        int ek[64];
        for (int k = 0; k < K; k++) {
            int e = idx[(size_t)t * K + k];
            if (e < 0 || e >= E) continue;
            bool dup = false;
            for (int j = 0; j < k; j++) dup |= idx[(size_t)t * K + j] == e;
            if (dup) continue;
            int p = n++;
            while (p > 0 && ek[p - 1] > e) { ek[p] = ek[p - 1]; s_ord[p] = s_ord[p - 1]; p--; }
            ek[p] = e;
            s_ord[p] = k;
        }
        s_n = n;
    }
    __syncthreads();
    const int n = s_n;
    for (int c = threadIdx.x; c < D / 8; c += blockDim.x) {
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int j = 0; j < n; j++) {
            float v[8];
            const PT* src = ypair + ((size_t)t * K + s_ord[j]) * D + 8 * c;
            Vec8<PT>::load(src, v);
            for (int sp = 1; sp < nsp; sp++) {
                float u[8];
                Vec8<PT>::load(src + sp * sp_stride, u);
                for (int i = 0; i < 8; i++) v[i] = add_rn(v[i], u[i]);
            }
            for (int i = 0; i < 8; i++) acc[i] = add_rn(acc[i], v[i]);
        }
        if (OUT_BF16) {
            u32x4 o;
            for (int i = 0; i < 4; i++) o[i] = pack_bf16x2(acc[2 * i], acc[2 * i + 1]);
            *(u32x4*)((uint16_t*)y + (size_t)t * D + 8 * c) = o;
        } else {
            float* dst = (float*)y + (size_t)t * D + 8 * c;
            *(f32x4*)dst = (f32x4){acc[0], acc[1], acc[2], acc[3]};
            *(f32x4*)(dst + 4) = (f32x4){acc[4], acc[5], acc[6], acc[7]};
        }
    }
}

// ypair is read once and y written once: both as streaming (non-temporal)
// accesses, which keeps them from displacing cached data (12% faster at
// DSV3 T=4096).
// bf16 form for K <= 64: the slot order is computed in parallel (lane k of
// wave 0: is slot k the first occurrence of a valid expert, and its rank
// among the kept slots by expert id), and each thread loads all of its rows
// (8 at a time, 4 column groups each) before adding them in that order, so
// 32 loads per thread are in flight.
template <int kG>  // 8-column groups per thread; blockIdx.y picks the block's 256 * kG groups
__global__ __launch_bounds__(256) void combine_bf16_kernel(const uint16_t* __restrict__ ypair,
                                                           const int* __restrict__ idx, int T,
                                                           int K, int E, int D,
                                                           uint16_t* __restrict__ y) {
    __shared__ int s_ord[64];
    __shared__ int s_n;
    const int t = blockIdx.x, tid = threadIdx.x;
    if (tid < 64) {
        const int e = tid < K ? idx[(size_t)t * K + tid] : -1;
        const bool valid = e >= 0 && e < E;
        bool dup = false;
        for (int j = 0; j < K; j++) {
            const int ej = __shfl(e, j, kWave);
            dup |= j < tid && ej == e;
        }
        const bool kept = valid && !dup;
        const unsigned long long kb = __ballot(kept);
        int rank = 0;
        for (int j = 0; j < K; j++) {
            const int ej = __shfl(e, j, kWave);
            rank += ((kb >> j) & 1) && ej < e;
        }
        if (kept) s_ord[rank] = tid;
        if (tid == 0) s_n = __popcll(kb);
    }
    __syncthreads();
    const int n = s_n;
    const int ng = D / 8;  // 8-column groups
    constexpr int kR = 8;
    const int g0 = 256 * kG * blockIdx.y;  // this block's first column group
    f32x4 acc[kG][2];
#pragma unroll
    for (int i = 0; i < kG; i++) acc[i][0] = acc[i][1] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int j0 = 0; j0 < n; j0 += kR) {
        u32x4 v[kR][kG];
#pragma unroll
        for (int j = 0; j < kR; j++) {
            const int jj = j0 + j;
            const uint16_t* row = ypair + ((size_t)t * K + s_ord[jj < n ? jj : 0]) * D;
#pragma unroll
            for (int i = 0; i < kG; i++) {
                const int c = g0 + tid + 256 * i;
                v[j][i] = (jj < n && c < ng) ? __builtin_nontemporal_load((const u32x4*)(row + 8 * c))
                                             : (u32x4){0u, 0u, 0u, 0u};
            }
        }
#pragma unroll
        for (int j = 0; j < kR; j++) {
            if (j0 + j >= n) break;  // uniform
#pragma unroll
            for (int i = 0; i < kG; i++)
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    acc[i][m >> 1][2 * (m & 1)] += __uint_as_float(v[j][i][m] << 16);
                    acc[i][m >> 1][2 * (m & 1) + 1] += __uint_as_float(v[j][i][m] & 0xffff0000u);
                }
        }
    }
#pragma unroll
    for (int i = 0; i < kG; i++) {
        const int c = g0 + tid + 256 * i;
        if (c >= ng) break;
        u32x4 o;
        for (int m = 0; m < 4; m++) o[m] = pack_bf16x2(acc[i][m >> 1][2 * (m & 1)], acc[i][m >> 1][2 * (m & 1) + 1]);
        __builtin_nontemporal_store(o, (u32x4*)(y + (size_t)t * D + 8 * c));
    }
}

int launch_combine(int ypair_dt, int out_dt, const void* ypair, const int* idx, int T, int K, int E,
                   int D, void* y, hipStream_t st, int nsplit) {
    AMDMOE_CHECK_ARG(K <= 64 && D % 8 == 0, "combine: K=%d D=%d unsupported", K, D);
    AMDMOE_CHECK_ARG(ypair_dt == DT_F32 || out_dt == DT_BF16, "combine: bf16 rows need a bf16 output");
    AMDMOE_CHECK_ARG(nsplit >= 1 && (nsplit == 1 || ypair_dt == DT_F32), "combine: %d partial row sets need fp32 rows",
                     nsplit);
    const size_t sp_stride = (size_t)T * K * D;
    if (T == 0) return AMDMOE_OK;
    if (ypair_dt == DT_F32 && out_dt == DT_F32)
        hipLaunchKernelGGL((combine_kernel<float, false>), dim3(T), dim3(256), 0, st,
                           (const float*)ypair, idx, T, K, E, D, y, nsplit, sp_stride);
    else if (ypair_dt == DT_F32)
        // fp32 rows, bf16 output (the bf16 layer): the sum is rounded once
        hipLaunchKernelGGL((combine_kernel<float, true>), dim3(T), dim3(256), 0, st,
                           (const float*)ypair, idx, T, K, E, D, y, nsplit, sp_stride);
    else if (D <= 8 * 256 * 4 && T <= 64)
        // few tokens: a token's columns over several workgroups (one 8-column
        // group per thread), so no CU streams a whole token's K rows alone
        hipLaunchKernelGGL(combine_bf16_kernel<1>, dim3(T, (unsigned)ceil_div(D / 8, 256)), dim3(256), 0, st,
                           (const uint16_t*)ypair, idx, T, K, E, D, (uint16_t*)y);
    else if (D <= 8 * 256 * 4)
        hipLaunchKernelGGL(combine_bf16_kernel<4>, dim3(T), dim3(256), 0, st, (const uint16_t*)ypair,
                           idx, T, K, E, D, (uint16_t*)y);
    else
        hipLaunchKernelGGL((combine_kernel<uint16_t, true>), dim3(T), dim3(256), 0, st,
                           (const uint16_t*)ypair, idx, T, K, E, D, y, 1, sp_stride);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

// ---------------------------------------------------------------- naive_gemm
// C[M,N] = A[M,K] * B[K,N] (B row-major, not transposed): 64x64 output tile
// per 256-thread block, 4x4 outputs per thread, K staged through LDS 16 at a
// time.  Surface-only entry (the forward uses the grouped MFMA kernels).
__global__ __launch_bounds__(256) void gemm_nn_f32_kernel(const float* __restrict__ A,
                                                          const float* __restrict__ B,
                                                          float* __restrict__ C, int M, int N,
                                                          int K) {
    __shared__ float As[16][65];
    __shared__ float Bs[16][65];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += 16) {
        for (int j = threadIdx.x; j < 1024; j += 256) {
            int r = j >> 4, c = j & 15;  // A tile 64 rows x 16 k
            int gm = m0 + r, gk = k0 + c;
            As[c][r] = (gm < M && gk < K) ? A[(size_t)gm * K + gk] : 0.f;
            int kr = j >> 6, nc = j & 63;  // B tile 16 k x 64 cols
            int bk = k0 + kr, bn = n0 + nc;
            Bs[kr][nc] = (bk < K && bn < N) ? B[(size_t)bk * N + bn] : 0.f;
        }
        __syncthreads();
        for (int kk = 0; kk < 16; kk++)
            for (int i = 0; i < 4; i++)
                for (int j = 0; j < 4; j++) acc[i][j] += As[kk][ty * 4 + i] * Bs[kk][tx * 4 + j];
        __syncthreads();
    }
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++) {
            int gm = m0 + ty * 4 + i, gn = n0 + tx * 4 + j;
            if (gm < M && gn < N) C[(size_t)gm * N + gn] = acc[i][j];
        }
}

int launch_naive_gemm_f32(const float* A, const float* B, float* C, int M, int N, int K,
                          hipStream_t st) {
    if (M == 0 || N == 0) return AMDMOE_OK;
    AMDMOE_CHECK_ARG((M + 63) / 64 <= 65535, "naive_gemm: M=%d too large", M);
    hipLaunchKernelGGL(gemm_nn_f32_kernel, dim3((N + 63) / 64, (M + 63) / 64), dim3(256), 0, st,
                       A, B, C, M, N, K);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

// ---------------------------------------------------------------- swiglu
__global__ void swiglu_f32_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                  float* __restrict__ out, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        float x = g[i];
        out[i] = x / (1.0f + expf(-x)) * u[i];
    }
}

int launch_swiglu_f32(const float* gate, const float* up, float* out, int n, hipStream_t st) {
    if (n <= 0) return AMDMOE_OK;
    hipLaunchKernelGGL(swiglu_f32_kernel, dim3((n + 255) / 256), dim3(256), 0, st, gate, up, out, n);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

// ---------------------------------------------------------------- scatter
// output[token_map[m], :] += w * expert_out[m, :], w = weight of the first
// slot of that token holding `expert` (naive_moe.cu:315-335).  A token
// appears once per expert, so rows never collide and no atomics are needed.
__global__ void scatter_f32_kernel(const float* __restrict__ eo, const int* __restrict__ tmap,
                                   const float* __restrict__ wts, const int* __restrict__ idx,
                                   int expert, float* __restrict__ out, int K, int D) {
    const int m = blockIdx.y;
    const int d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= D) return;
    const int t = tmap[m];
    float w = 0.0f;
    for (int k = 0; k < K; k++)
        if (idx[(size_t)t * K + k] == expert) { w = wts[(size_t)t * K + k]; break; }
    // the product is rounded before the sum, as in the reference's atomicAdd
    float* o = out + (size_t)t * D + d;
    *o = add_rn(*o, mul_rn(w, eo[(size_t)m * D + d]));
}

int launch_scatter_f32(const float* expert_out, const int* token_map, const float* wts,
                       const int* idx, int expert, float* out, int count, int T, int K, int D,
                       hipStream_t st) {
    if (count <= 0) return AMDMOE_OK;
    AMDMOE_CHECK_ARG(count <= T && count <= 65535, "moe_scatter: count=%d out of range", count);
    hipLaunchKernelGGL(scatter_f32_kernel, dim3((D + 255) / 256, count), dim3(256), 0, st,
                       expert_out, token_map, wts, idx, expert, out, K, D);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

}  // namespace amdmoe
