// The DSA stage functions of the reference's header (kernels/dsa/naive_dsa.cuh:31-68),
// fp32, with the reference's semantics: the gather of the selected K_c/K_p/V
// rows into [Q,S,*] buffers, the score dot products (accumulated into the
// caller's [Q,H,S] scores), the per-(q,h) softmax in place, and the
// attention-weighted sum of the gathered V rows.  dsa_forward's fused path
// (dsa.hip) does not use them; they exist for callers that compose the
// stages themselves, as naive_dsa.cu:435-474 does.
//
// Every value is formed in the reference kernel's order of operations
// (sequential sums over d or s in one fp32 accumulator, product then sum,
// no contraction), so the results are those of its single-thread loops.
#include "internal.hpp"

#include <float.h>

namespace amdmoe {

// ---------------------------------------------------------------- gather
// naive_dsa.cu:13-60 (three kernels, one per output).  One wave per (q,s)
// row copies the selected row of each cache; 16-byte pieces when the row
// length and the pointers allow.  An index outside [0, N) gathers zeros (the
// reference reads out of bounds there).
__device__ __forceinline__ void copy_row(const float* __restrict__ src, float* __restrict__ dst,
                                         int n, bool vec, bool ok, int lane) {
    if (vec) {
        const int n4 = n >> 2;
        for (int i = lane; i < n4; i += kWave)
            ((f32x4*)dst)[i] = ok ? ((const f32x4*)src)[i] : (f32x4){0.f, 0.f, 0.f, 0.f};
    } else {
        for (int i = lane; i < n; i += kWave) dst[i] = ok ? src[i] : 0.0f;
    }
}

__global__ __launch_bounds__(256) void dsa_gather_kernel(const float* __restrict__ kc,
                                                         const float* __restrict__ kp,
                                                         const float* __restrict__ v,
                                                         const int* __restrict__ idx,
                                                         float* __restrict__ gkc,
                                                         float* __restrict__ gkp,
                                                         float* __restrict__ gv, long rows,
                                                         int Dc, int Dp, long N, bool vc,
                                                         bool vp) {
    const int lane = threadIdx.x & 63;
    const long nw = (long)gridDim.x * 4;
    for (long r = (long)blockIdx.x * 4 + (threadIdx.x >> 6); r < rows; r += nw) {
        const long row = idx[r];
        const bool ok = row >= 0 && row < N;
        const long src = ok ? row : 0;
        copy_row(kc + src * Dc, gkc + r * Dc, Dc, vc, ok, lane);
        if (Dp > 0) copy_row(kp + src * Dp, gkp + r * Dp, Dp, vp, ok, lane);
        copy_row(v + src * Dc, gv + r * Dc, Dc, vc, ok, lane);
    }
}

// ---------------------------------------------------------------- dots
// naive_dsa.cu:89-134 (compressed), 157-206 (positional), 208-276 (fused):
// sum = sequential dot over d (fused: over Dc, then Dp, in one
// accumulator), then scores[q,h,s] += sum.
// Workgroup: one query, 64 tokens, 32 heads; 4 waves, lane = token, wave w
// owns heads 8w..8w+7.  The gathered rows are staged through LDS in
// 64-column slabs (row pitch 65 floats: lanes read distinct banks), the
// query slab is read as a broadcast.
constexpr int kDotS = 64, kDotH = 32, kDotD = 64, kDotPitch = kDotD + 1;

enum { DOT_C = 1, DOT_P = 2 };

__global__ __launch_bounds__(256) void dsa_dot_kernel(const float* __restrict__ qn,
                                                      const float* __restrict__ qp,
                                                      const float* __restrict__ kc,
                                                      const float* __restrict__ kp,
                                                      float* __restrict__ scores, int H, int S,
                                                      int Dc, int Dp, int parts) {
    __shared__ float s_k[kDotS * kDotPitch];
    __shared__ float s_q[kDotH * kDotD];
    const int q = blockIdx.z, s0 = blockIdx.x * kDotS, h0 = blockIdx.y * kDotH;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int part = 0; part < 2; part++) {
        if (!(parts & (part == 0 ? DOT_C : DOT_P))) continue;
        const int L = part == 0 ? Dc : Dp;
        const float* kr = part == 0 ? kc : kp;
        const float* qr = part == 0 ? qn : qp;
        for (int d0 = 0; d0 < L; d0 += kDotD) {
            const int ts = min(kDotD, L - d0);
            __syncthreads();  // the previous slab has been consumed
            for (int i = tid; i < kDotS * kDotD; i += 256) {
                const int r = i >> 6, c = i & 63;
                const int s = s0 + r;
                s_k[r * kDotPitch + c] =
                    (s < S && c < ts) ? kr[((size_t)q * S + s) * L + d0 + c] : 0.0f;
            }
            for (int i = tid; i < kDotH * kDotD; i += 256) {
                const int r = i >> 6, c = i & 63;
                const int h = h0 + r;
                s_q[i] = (h < H && c < ts) ? qr[((size_t)q * H + h) * L + d0 + c] : 0.0f;
            }
            __syncthreads();
            const float* kk = s_k + lane * kDotPitch;
            const float* qq = s_q + (8 * wave) * kDotD;
            for (int d = 0; d < ts; d++) {
                const float kv = kk[d];
#pragma unroll
                for (int j = 0; j < 8; j++) acc[j] = mac_rn(acc[j], qq[j * kDotD + d], kv);
            }
        }
    }
    const int s = s0 + lane;
    if (s >= S) return;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int h = h0 + 8 * wave + j;
        if (h < H) {
            float* p = scores + ((size_t)q * H + h) * S + s;
            *p = add_rn(*p, acc[j]);
        }
    }
}

// ---------------------------------------------------------------- softmax
// naive_dsa.cu:278-296: mx = max_s row[s]; row[s] = expf(row[s] - mx) with
// the sum taken in s order; then row[s] *= 1/sum.  One wave per row; the
// exponentials go through LDS in chunks so one lane can sum them in order,
// and are recomputed (identically) for the final scaling.
constexpr int kSmChunk = 4096;

__global__ __launch_bounds__(64) void dsa_softmax_kernel(float* __restrict__ scores, long rows,
                                                         int S) {
    __shared__ float s_e[kSmChunk];
    const int lane = threadIdx.x;
    for (long r = blockIdx.x; r < rows; r += gridDim.x) {
        float* row = scores + r * S;
        float mx = -FLT_MAX;
        for (int s = lane; s < S; s += kWave) mx = fmaxf(mx, row[s]);
        mx = wave_max(mx);
        float sum = 0.0f;
        for (int c0 = 0; c0 < S; c0 += kSmChunk) {
            const int n = min(kSmChunk, S - c0);
            for (int i = lane; i < n; i += kWave) s_e[i] = expf(row[c0 + i] - mx);
            __syncthreads();
            if (lane == 0)
                for (int i = 0; i < n; i++) sum = add_rn(sum, s_e[i]);
            __syncthreads();
        }
        const float inv = __fdiv_rn(1.0f, __shfl(sum, 0, kWave));
        for (int s = lane; s < S; s += kWave) row[s] = mul_rn(expf(row[s] - mx), inv);
    }
}

// ---------------------------------------------------------------- output
// naive_dsa.cu:300-316: out[q,h,d] = sequential sum over s of
// attn[q,h,s] * v[q,s,d] (overwrites out).  Workgroup: one query, 32 heads,
// 256 columns; lane = column, each thread holds the 32 heads' sums; the
// attention weights are staged through LDS 64 tokens at a time and read as
// broadcasts, the V rows are read straight from memory (coalesced).
constexpr int kOpH = 32, kOpS = 64;

__global__ __launch_bounds__(256) void dsa_output_proj_kernel(const float* __restrict__ attn,
                                                              const float* __restrict__ v,
                                                              float* __restrict__ out, int H,
                                                              int S, int Dc) {
    __shared__ float s_a[kOpH * kOpS];
    const int q = blockIdx.z, h0 = blockIdx.y * kOpH;
    const int tid = threadIdx.x, d = blockIdx.x * 256 + tid;
    const int nh = min(kOpH, H - h0);
    float acc[kOpH];
#pragma unroll
    for (int j = 0; j < kOpH; j++) acc[j] = 0.0f;
    for (int t0 = 0; t0 < S; t0 += kOpS) {
        const int ts = min(kOpS, S - t0);
        __syncthreads();
        for (int i = tid; i < kOpH * kOpS; i += 256) {
            const int j = i >> 6, c = i & 63;
            s_a[i] = (j < nh && c < ts) ? attn[((size_t)q * H + h0 + j) * S + t0 + c] : 0.0f;
        }
        __syncthreads();
        if (d < Dc)
            for (int c = 0; c < ts; c++) {
                const float vv = v[((size_t)q * S + t0 + c) * Dc + d];
#pragma unroll
                for (int j = 0; j < kOpH; j++) acc[j] = mac_rn(acc[j], s_a[j * kOpS + c], vv);
            }
    }
    if (d >= Dc) return;
#pragma unroll
    for (int j = 0; j < kOpH; j++)
        if (j < nh) out[((size_t)q * H + h0 + j) * Dc + d] = acc[j];
}

// ---------------------------------------------------------------- launch
static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int launch_dsa_gather(const float* kc, const float* kp, const float* v, const int* idx, float* gkc,
                      float* gkp, float* gv, int Q, int S, int Dc, int Dp, long N, hipStream_t st) {
    const long rows = (long)Q * S;
    if (rows == 0) return AMDMOE_OK;
    const bool vc = Dc % 4 == 0 && aligned16(kc) && aligned16(v) && aligned16(gkc) && aligned16(gv);
    const bool vp = Dp % 4 == 0 && aligned16(kp) && aligned16(gkp);
    const long blocks = std::min(ceil_div(rows, 4), 65536L);
    hipLaunchKernelGGL(dsa_gather_kernel, dim3((unsigned)blocks), dim3(256), 0, st, kc, kp, v, idx,
                       gkc, gkp, gv, rows, Dc, Dp, N, vc, vp);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

int launch_dsa_dot(const float* qn, const float* qp, const float* kc, const float* kp,
                   float* scores, int Q, int H, int S, int Dc, int Dp, int parts, hipStream_t st) {
    if ((long)Q * H * S == 0) return AMDMOE_OK;
    AMDMOE_CHECK_ARG(Q <= 65535 && ceil_div(H, kDotH) <= 65535, "dsa dot: Q=%d or H=%d too large", Q, H);
    const dim3 grid((unsigned)ceil_div(S, kDotS), (unsigned)ceil_div(H, kDotH), (unsigned)Q);
    hipLaunchKernelGGL(dsa_dot_kernel, grid, dim3(256), 0, st, qn, qp, kc, kp, scores, H, S, Dc, Dp,
                       parts);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

int launch_dsa_softmax(float* scores, long rows, int S, hipStream_t st) {
    if (rows == 0 || S == 0) return AMDMOE_OK;
    const long blocks = std::min(rows, 1L << 20);
    hipLaunchKernelGGL(dsa_softmax_kernel, dim3((unsigned)blocks), dim3(64), 0, st, scores, rows, S);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

int launch_dsa_output_proj(const float* attn, const float* v, float* out, int Q, int H, int S,
                           int Dc, hipStream_t st) {
    if ((long)Q * H * Dc == 0) return AMDMOE_OK;
    AMDMOE_CHECK_ARG(Q <= 65535 && ceil_div(H, kOpH) <= 65535, "dsa output_proj: Q=%d or H=%d too large", Q, H);
    const dim3 grid((unsigned)ceil_div(Dc, 256), (unsigned)ceil_div(H, kOpH), (unsigned)Q);
    hipLaunchKernelGGL(dsa_output_proj_kernel, grid, dim3(256), 0, st, attn, v, out, H, S, Dc);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

}  // namespace amdmoe
