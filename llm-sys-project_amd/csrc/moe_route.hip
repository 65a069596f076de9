// R1 -- routing: gate logits, softmax over experts, top-K, renormalisation,
// fused in one kernel per token block (the logits never leave the CU).
//
// Reference semantics (kernels/moe/naive_moe.cu:87-142, the CPU copy in
// tests/test_moe.cu:38-69):
//   logits[t,e] = sum_d x[t,d]*Wg[e,d]                (fp32)
//   p = softmax(logits[t,:]): mx = max, p = expf(l-mx), s = sum (ascending e), p /= s
//   replace-min top-K over e ascending: the victim is the FIRST slot holding
//   the strictly smallest value; a candidate replaces it only if strictly
//   greater.  Output slot order = insertion history.
//   renormalise: s = sum of slot values in slot order; if (s > 0) w /= s.
//
// Two logit producers:
//   route_exact_kernel -- fp32 gate weights.  One lane per (token, expert)
//     runs the reference's sequential fp32 sum (explicit round-to-nearest
//     mul then add, never contracted), so logits are bit-identical to the
//     reference's CPU loop.
//   route_mfma_kernel  -- bf16 x and bf16 gate (DeepSeek-V3 shape, E=256,
//     D=7168): the gate GEMM runs on bf16 MFMA with fp32 accumulation.
// Both then run the same wave routine: softmax with the reference's
// sequential denominator, and a ballot-driven exact simulation of the
// replace-min loop (only insertions cost work: ~K*(1+ln(E/K)) of them).
#include "internal.hpp"

#include <float.h>

namespace amdmoe {

// Routing of one token by one wave.  `p` (LDS) holds E logits and is
// overwritten with probabilities.  K <= 64.
__device__ void wave_route_token(float* p, int E, int K, int* out_idx, float* out_wts) {
    const int lane = lane_id();
    // softmax (tests/test_moe.cu:14-20)
    float mx = -FLT_MAX;
    for (int e = lane; e < E; e += kWave) mx = fmaxf(mx, p[e]);
    mx = wave_max(mx);
    for (int e = lane; e < E; e += kWave) p[e] = expf(p[e] - mx);
    wave_lds_sync();
    // The denominator is summed in ascending expert order, as the reference
    // does, so p matches it to the last bit whenever expf does.
    float s = 0.0f;
    if (lane == 0)
        for (int e = 0; e < E; e++) s = __fadd_rn(s, p[e]);
    s = __shfl(s, 0, kWave);
    for (int e = lane; e < E; e += kWave) p[e] = __fdiv_rn(p[e], s);
    wave_lds_sync();

    // replace-min top-K.  Lane k < K owns slot k.
    float sv = -FLT_MAX;
    int si = -1;
    auto argmin_slot = [&](float& thr) -> int {
        float v = lane < K ? sv : INFINITY;
        int k = lane < K ? lane : kWave;
        for (int o = 32; o > 0; o >>= 1) {
            float ov = __shfl_xor(v, o, kWave);
            int ok = __shfl_xor(k, o, kWave);
            if (ov < v || (ov == v && ok < k)) { v = ov; k = ok; }
        }
        thr = v;
        return k;
    };
    float thr;
    int m = argmin_slot(thr);
    int pos = 0;
    while (pos < E) {
        int found = E;
        for (int c = pos; c < E; c += kWave) {
            int e = c + lane;
            bool hit = (e < E) && (p[e] > thr);
            unsigned long long b = __ballot(hit);
            if (b) { found = c + __ffsll(b) - 1; break; }
        }
        if (found >= E) break;
        if (lane == m) { sv = p[found]; si = found; }
        pos = found + 1;
        m = argmin_slot(thr);
    }
    // renormalise in slot order (tests/test_moe.cu:65-68)
    float tot = 0.0f;
    for (int k = 0; k < K; k++) tot = __fadd_rn(tot, __shfl(sv, k, kWave));
    if (lane < K) {
        float w = tot > 0.0f ? __fdiv_rn(sv, tot) : sv;
        out_idx[lane] = si;
        out_wts[lane] = w;
    }
}

template <typename T> __device__ __forceinline__ float load_f(const T* p);
template <> __device__ __forceinline__ float load_f<float>(const float* p) { return *p; }
template <> __device__ __forceinline__ float load_f<uint16_t>(const uint16_t* p) {
    return bf16_to_f32(*p);
}

// ---------------------------------------------------------------- exact
// Block = 256 threads = 4 waves.  tpb tokens per block (tpb*E <= 256 when
// E <= 256; for E > 256 tpb = 1 and lanes loop over experts).
template <typename XT, typename GT>
__global__ __launch_bounds__(256) void route_exact_kernel(const XT* __restrict__ x,
                                                          const GT* __restrict__ wg,
                                                          const float* __restrict__ bias, int T,
                                                          int E, int K, int D, int tpb,
                                                          int* __restrict__ idx,
                                                          float* __restrict__ wts) {
    extern __shared__ float s_logit[];  // [tpb][E]
    const int tid = threadIdx.x;
    const int t0 = blockIdx.x * tpb;
    const int nslots = tpb * E;
    for (int j = tid; j < nslots; j += blockDim.x) {
        int lt = j / E, e = j % E;
        int t = t0 + lt;
        float sum = 0.0f;
        if (t < T) {
            const XT* xr = x + (size_t)t * D;
            const GT* wr = wg + (size_t)e * D;
            for (int d = 0; d < D; d++) sum = __fadd_rn(sum, __fmul_rn(load_f(xr + d), load_f(wr + d)));
            if (bias) sum = __fadd_rn(sum, bias[e]);
        }
        s_logit[j] = sum;
    }
    __syncthreads();
    const int wave = tid >> 6;
    for (int lt = wave; lt < tpb; lt += blockDim.x >> 6) {
        int t = t0 + lt;
        if (t >= T) break;
        wave_route_token(s_logit + lt * E, E, K, idx + (size_t)t * K, wts + (size_t)t * K);
    }
}

// ---------------------------------------------------------------- MFMA
// bf16 x [T,D] and bf16 Wg [E,D], E <= 256, D % 64 == 0.
// Block = 512 threads = 8 waves, 32 tokens.  Wave w: token row tile (w & 1),
// expert column group (w >> 1) of 64 experts (4 MFMA column tiles).
// K-step = 64 bf16 = 128 bytes per row; LDS rows padded to 144 bytes.
constexpr int kRtTok = 32;
constexpr int kRtPitch = 144;
constexpr int kRtStage = (kRtTok + 256) * kRtPitch;

__global__ __launch_bounds__(512) void route_mfma_kernel(const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ wg, int T,
                                                         int E, int K, int D,
                                                         int* __restrict__ idx,
                                                         float* __restrict__ wts) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = blockIdx.x * kRtTok;
    const int nk = D / 64;
    const size_t row_bytes = (size_t)D * 2;

    // global -> register staging: x 32 rows * 8 chunks = 256 chunks (threads
    // < 256), Wg 256 rows * 8 chunks = 2048 chunks (4 per thread).
    const uint8_t* xsrc = nullptr;
    int xrow = tid >> 3, xch = tid & 7;
    if (tid < 256 && t0 + xrow < T) xsrc = (const uint8_t*)x + (size_t)(t0 + xrow) * row_bytes + xch * 16;
    const uint8_t* wsrc[4];
    int wrow[4], wch[4];
    for (int j = 0; j < 4; j++) {
        int c = tid + 512 * j;
        wrow[j] = c >> 3;
        wch[j] = c & 7;
        wsrc[j] = wrow[j] < E ? (const uint8_t*)wg + (size_t)wrow[j] * row_bytes + wch[j] * 16 : nullptr;
    }
    u32x4 rx, rw[4];
    const u32x4 zero4 = {0u, 0u, 0u, 0u};
    auto gload = [&](int kt) {
        size_t off = (size_t)kt * 128;
        rx = xsrc ? *(const u32x4*)(xsrc + off) : zero4;
        for (int j = 0; j < 4; j++) rw[j] = wsrc[j] ? *(const u32x4*)(wsrc[j] + off) : zero4;
    };
    auto sstore = [&](int st) {
        uint8_t* base = smem + st * kRtStage;
        if (tid < 256) *(u32x4*)(base + xrow * kRtPitch + xch * 16) = rx;
        for (int j = 0; j < 4; j++)
            *(u32x4*)(base + (kRtTok + wrow[j]) * kRtPitch + wch[j] * 16) = rw[j];
    };

    f32x4 acc[4];
    for (int j = 0; j < 4; j++) acc[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    const int rt = wave & 1, cg = wave >> 1;
    const bool active = cg * 64 < E;

    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        if (kt + 1 < nk) gload(kt + 1);
        const uint8_t* base = smem + (kt & 1) * kRtStage;
        if (active) {
            const int q = lane >> 4, r = lane & 15;
            const uint8_t* ap = base + (rt * 16 + r) * kRtPitch + q * 16;
            u32x4 a0 = *(const u32x4*)ap, a1 = *(const u32x4*)(ap + 64);
            for (int ct = 0; ct < 4; ct++) {
                const uint8_t* bp = base + (kRtTok + cg * 64 + ct * 16 + r) * kRtPitch + q * 16;
                u32x4 b0 = *(const u32x4*)bp, b1 = *(const u32x4*)(bp + 64);
                acc[ct] = mfma_bf16(a0, b0, acc[ct]);
                acc[ct] = mfma_bf16(a1, b1, acc[ct]);
            }
        }
        if (kt + 1 < nk) sstore((kt + 1) & 1);
        __syncthreads();
    }
    // logits -> LDS [32][E]
    float* s_logit = (float*)smem;
    if (active) {
        const int q = lane >> 4, c = lane & 15;
        for (int ct = 0; ct < 4; ct++) {
            int e = cg * 64 + ct * 16 + c;
            if (e < E)
                for (int i = 0; i < 4; i++) s_logit[(rt * 16 + q * 4 + i) * E + e] = acc[ct][i];
        }
    }
    __syncthreads();
    for (int lt = wave; lt < kRtTok; lt += 8) {
        int t = t0 + lt;
        if (t >= T) break;
        wave_route_token(s_logit + lt * E, E, K, idx + (size_t)t * K, wts + (size_t)t * K);
    }
}

// ---------------------------------------------------------------- launch
template <typename XT, typename GT>
int launch_route_exact(const XT* x, const GT* wg, const float* bias, int T, int E, int K, int D,
                       int* idx, float* wts, hipStream_t st) {
    int tpb = E <= 256 ? 256 / E : 1;
    if (tpb > 64) tpb = 64;
    size_t lds = sizeof(float) * (size_t)tpb * E;
    AMDMOE_CHECK_ARG(lds <= 64 * 1024, "routing: E=%d too large for the exact gate", E);
    int grid = (int)ceil_div(T, tpb);
    hipLaunchKernelGGL((route_exact_kernel<XT, GT>), dim3(grid), dim3(256), lds, st, x, wg, bias,
                       T, E, K, D, tpb, idx, wts);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

template int launch_route_exact<float, float>(const float*, const float*, const float*, int, int,
                                              int, int, int*, float*, hipStream_t);
template int launch_route_exact<uint16_t, float>(const uint16_t*, const float*, const float*, int,
                                                 int, int, int, int*, float*, hipStream_t);
template int launch_route_exact<uint16_t, uint16_t>(const uint16_t*, const uint16_t*,
                                                    const float*, int, int, int, int, int*,
                                                    float*, hipStream_t);

bool route_mfma_supported(int E, int D) { return E >= 1 && E <= 256 && D % 64 == 0; }

int launch_route_mfma(const uint16_t* x, const uint16_t* wg, int T, int E, int K, int D, int* idx,
                      float* wts, hipStream_t st) {
    size_t lds = 2 * (size_t)kRtStage;
    size_t lds_logit = sizeof(float) * (size_t)kRtTok * E;
    if (lds_logit > lds) lds = lds_logit;
    static bool attr_set = false;
    if (!attr_set) {
        AMDMOE_HIP_TRY(hipFuncSetAttribute((const void*)route_mfma_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        attr_set = true;
    }
    int grid = (int)ceil_div(T, kRtTok);
    hipLaunchKernelGGL(route_mfma_kernel, dim3(grid), dim3(512), lds, st, x, wg, T, E, K, D, idx,
                       wts);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

}  // namespace amdmoe
