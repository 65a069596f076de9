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

// Uniform-index element of a 4-register array (j is wave-uniform).
__device__ __forceinline__ float pick4(const float (&v)[4], int j) {
    return j == 0 ? v[0] : (j == 1 ? v[1] : (j == 2 ? v[2] : v[3]));
}

// Routing of one token by one wave.  `p` (LDS) holds the E logits.
// E <= 256: the probabilities live in registers (expert e = lane + 64j).
__device__ void wave_route_token_reg(const float* p, int E, int K, int* out_idx, float* out_wts) {
    const int lane = lane_id();
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int e = lane + 64 * j;
        v[j] = e < E ? p[e] : -FLT_MAX;
    }
    // softmax (tests/test_moe.cu:14-20)
    float mx = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
    mx = wave_max(mx);
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = lane + 64 * j < E ? expf(v[j] - mx) : 0.0f;
    // The denominator is summed in ascending expert order, exactly as the
    // reference does: lane values are read out one by one (v_readlane).
    float s = 0.0f;
    const int nj = (E + 63) / 64;
    for (int j = 0; j < nj; j++) {
        const float x = pick4(v, j);
        const int n = min(64, E - 64 * j);
        if (n == 64) {
#pragma unroll
            for (int l = 0; l < 64; l++)
                s = __fadd_rn(s, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l)));
        } else {
            for (int l = 0; l < n; l++) s = __fadd_rn(s, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l)));
        }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = __fdiv_rn(v[j], s);

    // replace-min top-K.  Lane k < K owns slot k; the first-minimum slot is
    // found by a reduction over the lowest power of two >= K lanes.
    int width = 1;
    while (width < K) width <<= 1;
    float sv = -FLT_MAX;
    int si = -1;
    auto argmin_slot = [&](float& thr) -> int {
        float mv = lane < K ? sv : INFINITY;
        int mk = lane < K ? lane : kWave;
        for (int o = 1; o < width; o <<= 1) {
            const float ov = __shfl_xor(mv, o, kWave);
            const int ok = __shfl_xor(mk, o, kWave);
            if (ov < mv || (ov == mv && ok < mk)) { mv = ov; mk = ok; }
        }
        thr = __shfl(mv, 0, kWave);
        return __shfl(mk, 0, kWave);
    };
    float thr;
    int m = argmin_slot(thr);
    int pos = 0;
    while (pos < E) {
        // first expert e >= pos with p_e > thr: experts are lane-major per
        // register, so the first register with a hit holds the smallest e
        int found = E;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int e = lane + 64 * j;
            const unsigned long long b = __ballot(e < E && e >= pos && v[j] > thr);
            if (found == E && b) found = 64 * j + __ffsll(b) - 1;
        }
        if (found >= E) break;
        const float val = __int_as_float(
            __builtin_amdgcn_readlane(__float_as_int(pick4(v, found >> 6)), found & 63));
        if (lane == m) { sv = val; si = found; }
        pos = found + 1;
        m = argmin_slot(thr);
    }
    // renormalise in slot order (tests/test_moe.cu:65-68)
    float tot = 0.0f;
    for (int k = 0; k < K; k++) tot = __fadd_rn(tot, __shfl(sv, k, kWave));
    if (lane < K) {
        out_idx[lane] = si;
        out_wts[lane] = tot > 0.0f ? __fdiv_rn(sv, tot) : sv;
    }
}

// Generic form for any E: probabilities in LDS (overwrites `p`).
__device__ void wave_route_token_lds(float* p, int E, int K, int* out_idx, float* out_wts) {
    const int lane = lane_id();
    float mx = -FLT_MAX;
    for (int e = lane; e < E; e += kWave) mx = fmaxf(mx, p[e]);
    mx = wave_max(mx);
    for (int e = lane; e < E; e += kWave) p[e] = expf(p[e] - mx);
    wave_lds_sync();
    float s = 0.0f;
    if (lane == 0)
        for (int e = 0; e < E; e++) s = __fadd_rn(s, p[e]);
    s = __shfl(s, 0, kWave);
    for (int e = lane; e < E; e += kWave) p[e] = __fdiv_rn(p[e], s);
    wave_lds_sync();
    float sv = -FLT_MAX;
    int si = -1;
    auto argmin_slot = [&](float& thr) -> int {
        float v = lane < K ? sv : INFINITY;
        int k = lane < K ? lane : kWave;
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(v, o, kWave);
            const int ok = __shfl_xor(k, o, kWave);
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
            const int e = c + lane;
            const unsigned long long b = __ballot((e < E) && (p[e] > thr));
            if (b) { found = c + __ffsll(b) - 1; break; }
        }
        if (found >= E) break;
        if (lane == m) { sv = p[found]; si = found; }
        pos = found + 1;
        m = argmin_slot(thr);
    }
    float tot = 0.0f;
    for (int k = 0; k < K; k++) tot = __fadd_rn(tot, __shfl(sv, k, kWave));
    if (lane < K) {
        out_idx[lane] = si;
        out_wts[lane] = tot > 0.0f ? __fdiv_rn(sv, tot) : sv;
    }
}

__device__ __forceinline__ void wave_route_token(float* p, int E, int K, int* out_idx, float* out_wts) {
    if (E <= 256) wave_route_token_reg(p, E, K, out_idx, out_wts);
    else wave_route_token_lds(p, E, K, out_idx, out_wts);
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
// Block = 256 threads = 4 waves, 32 tokens; wave w owns experts
// [64w, 64w+64) (4 MFMA column tiles) for both 16-token row tiles.
// Each K-step (64 bf16 = 128 bytes of every row) streams the x tile (4 KB)
// and the whole gate matrix slice (32 KB) global -> LDS through a 3-stage
// direct-load ring (buffer_load ... lds), so two steps are in flight while
// one is consumed; rows past T or E read as zeros.  LDS rows are 128 bytes,
// 16-byte chunks XOR-swizzled by (row & 7).  The gate matrix is re-read by
// every block from L2; the block count (T/32) keeps that traffic at
// E*D*2*T/32 bytes.
constexpr int kRtTok = 32;
constexpr int kRtStage = (kRtTok + 256) * 128;  // 36864
constexpr int kRtNS = 3;
constexpr int kRtLds = kRtNS * kRtStage;        // 110592

__global__ __launch_bounds__(256, 1) void route_mfma_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ wg, int T,
                                                            int E, int K, int D,
                                                            int* __restrict__ idx,
                                                            float* __restrict__ wts) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t0 = blockIdx.x * kRtTok;
    const int nk = D / 64;
    const long row_bytes = (long)D * 2;

    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (long)T * row_bytes);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(wg, (long)E * row_bytes);
    const int lrow = lane >> 3, lchunk = (lane & 7) ^ lrow;
    // x: 4 slabs of 8 rows (one per wave); Wg: 32 slabs (8 per wave)
    const int xr = t0 + 8 * wave + lrow;
    const uint32_t voff_x = xr < T ? (uint32_t)(xr * row_bytes + 16 * lchunk) : kOob;
    uint32_t voff_w[8];
    for (int j = 0; j < 8; j++) {
        const int r = 64 * wave + 8 * j + lrow;
        voff_w[j] = r < E ? (uint32_t)(r * row_bytes + 16 * lchunk) : kOob;
    }
    // rotated K order per block: gate rows are 128-byte slices at a fixed
    // stride, so blocks in lockstep would all hit the same memory channels
    const int kt0 = (int)(((unsigned)blockIdx.x * 13u) % (unsigned)nk);
    auto issue = [&](int st, int kt) {
        uint8_t* base = smem + st * kRtStage;
        kt += kt0;
        if (kt >= nk) kt -= nk;
        const int soff = kt * 128;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr_t)(base + 8 * wave * 128), 16, voff_x, soff, 0, 0);
        for (int j = 0; j < 8; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rw, (lds_ptr_t)(base + (kRtTok + 64 * wave + 8 * j) * 128), 16, voff_w[j], soff, 0, 0);
    };

    const int q = lane >> 4, r16 = lane & 15;
    const int off_lo = 16 * (q ^ (r16 & 7)), off_hi = 16 * ((4 + q) ^ (r16 & 7));
    const bool active = 64 * wave < E;
    f32x4 acc[2][4];
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 4; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    issue(0, 0);
    if (nk > 1) issue(1, 1);
    for (int kt = 0; kt < nk; kt++) {
        if (kt + 1 < nk) wait_vmcnt<9>();
        else wait_vmcnt<0>();
        bare_barrier();
        if (kt + 2 < nk) issue((kt + 2) % kRtNS, kt + 2);
        if (active) {
            const uint8_t* base = smem + (kt % kRtNS) * kRtStage;
            u32x4 alo[2], ahi[2];
            for (int rt = 0; rt < 2; rt++) {
                const uint8_t* p = base + (16 * rt + r16) * 128;
                alo[rt] = *(const u32x4*)(p + off_lo);
                ahi[rt] = *(const u32x4*)(p + off_hi);
            }
            for (int ct = 0; ct < 4; ct++) {
                const uint8_t* p = base + (kRtTok + 64 * wave + 16 * ct + r16) * 128;
                const u32x4 blo = *(const u32x4*)(p + off_lo), bhi = *(const u32x4*)(p + off_hi);
                for (int rt = 0; rt < 2; rt++) {
                    acc[rt][ct] = mfma_bf16(alo[rt], blo, acc[rt][ct]);
                    acc[rt][ct] = mfma_bf16(ahi[rt], bhi, acc[rt][ct]);
                }
            }
        }
    }
    __syncthreads();
    // logits -> LDS [32][E]
    float* s_logit = (float*)smem;
    if (active) {
        for (int rt = 0; rt < 2; rt++)
            for (int ct = 0; ct < 4; ct++) {
                const int e = 64 * wave + 16 * ct + r16;
                if (e < E)
                    for (int i = 0; i < 4; i++) s_logit[(16 * rt + 4 * q + i) * E + e] = acc[rt][ct][i];
            }
    }
    __syncthreads();
    for (int lt = wave; lt < kRtTok; lt += 4) {
        const int t = t0 + lt;
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
    const size_t lds = kRtLds;  // >= the 32 x E fp32 logits of the epilogue
    static bool attr_set = false;
    if (!attr_set) {
        AMDMOE_HIP_TRY(hipFuncSetAttribute((const void*)route_mfma_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        attr_set = true;
    }
    int grid = (int)ceil_div(T, kRtTok);
    hipLaunchKernelGGL(route_mfma_kernel, dim3(grid), dim3(256), lds, st, x, wg, T, E, K, D, idx,
                       wts);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

}  // namespace amdmoe
