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

// min over lanes [0, width) of a row of 16 lanes (width a power of two <= 16),
// by DPP within the row: xor 1, xor 2 (quad permutes), then the half-row and
// full-row mirrors pair every lane of one group with one of the other.
// Lanes outside [0, width) must hold +inf.
template <int CTRL>
__device__ __forceinline__ float dpp_min(float v) {
    return fminf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false)));
}
__device__ __forceinline__ float row_min16(float v, int width) {
    v = dpp_min<0xB1>(v);                  // quad_perm [1,0,3,2]
    if (width > 2) v = dpp_min<0x4E>(v);   // quad_perm [2,3,0,1]
    if (width > 4) v = dpp_min<0x141>(v);  // row_half_mirror
    if (width > 8) v = dpp_min<0x140>(v);  // row_mirror
    return v;
}

// Routing of one token by one wave, E <= 256: `v` holds the logits of
// experts lane + 64j (j < 4; -FLT_MAX past E).
__device__ void wave_route_token_reg(float (&v)[4], int E, int K, int* out_idx, float* out_wts) {
    const int lane = lane_id();
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
                s = add_rn(s, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l)));
        } else {
            for (int l = 0; l < n; l++) s = add_rn(s, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l)));
        }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = __fdiv_rn(v[j], s);

    // replace-min top-K.  Lane k < K owns slot k.  The victim is the first
    // slot holding the smallest value: its value comes from a DPP min over
    // the slot lanes (K <= 16) and its position from a ballot of the lanes
    // equal to it.
    float sv = -FLT_MAX;
    int si = -1;
    auto argmin_slot = [&](float& thr) -> int {
        const float mine = lane < K ? sv : INFINITY;
        float mv;
        if (K <= 16) {
            mv = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(row_min16(mine, K))));
        } else {
            mv = mine;
            for (int o = 1; o < kWave; o <<= 1) mv = fminf(mv, __shfl_xor(mv, o, kWave));
            mv = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(mv)));
        }
        thr = mv;
        return __ffsll(__ballot(lane < K && sv == mv)) - 1;
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
    for (int k = 0; k < K; k++)
        tot = add_rn(tot, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sv), k)));
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
        for (int e = 0; e < E; e++) s = add_rn(s, p[e]);
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
    for (int k = 0; k < K; k++) tot = add_rn(tot, __shfl(sv, k, kWave));
    if (lane < K) {
        out_idx[lane] = si;
        out_wts[lane] = tot > 0.0f ? __fdiv_rn(sv, tot) : sv;
    }
}

__device__ __forceinline__ void wave_route_token(float* p, int E, int K, int* out_idx, float* out_wts) {
    if (E <= 256) {
        const int lane = lane_id();
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = lane + 64 * j < E ? p[lane + 64 * j] : -FLT_MAX;
        wave_route_token_reg(v, E, K, out_idx, out_wts);
    } else {
        wave_route_token_lds(p, E, K, out_idx, out_wts);
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
            for (int d = 0; d < D; d++) sum = mac_rn(sum, load_f(xr + d), load_f(wr + d));
            if (bias) sum = add_rn(sum, bias[e]);
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
// bf16 x [T,D] and bf16 Wg [E,D], E <= 256, D % 64 == 0.  Two launches:
//
// route_logits_kernel: the gate GEMM, logits [T,E] fp32 into a scratch
//   buffer.  Block = 256 threads, a 32-token x 128-expert tile (wave w owns
//   experts [32w, 32w+32): 2 row tiles x 2 column tiles of 16x16 MFMA).
//   Each K-step (64 bf16 = 128 bytes of every row) streams the x rows (4 KB)
//   and the gate rows (16 KB) global -> LDS through a 3-stage direct-load
//   ring, so two steps are in flight while one is consumed; rows past T or E
//   read as zeros.  LDS rows are 128 bytes, 16-byte chunks XOR-swizzled by
//   (row & 7).  With T/32 x E/128 blocks (256 at T=4096, E=256) every CU
//   streams; the gate matrix is re-read per token tile from L2.
// route_topk_kernel: one wave per token (softmax + replace-min top-K +
//   renormalisation, wave_route_token_reg), 4 tokens per block, so a CU
//   interleaves many tokens' latency-bound shuffle chains.
constexpr int kRtTok = 32;
constexpr int kRtExp = 128;
constexpr int kRtStage = (kRtTok + kRtExp) * 128;  // 20480
constexpr int kRtNS = 3;
constexpr int kRtLds = kRtNS * kRtStage;           // 61440

__global__ __launch_bounds__(256) void route_logits_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ wg, int T,
                                                           int E, int D, float* __restrict__ logits) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t0 = blockIdx.x * kRtTok, e0 = blockIdx.y * kRtExp;
    const int nk = D / 64;
    const long row_bytes = (long)D * 2;

    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (long)T * row_bytes);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(wg, (long)E * row_bytes);
    const int lrow = lane >> 3, lchunk = (lane & 7) ^ lrow;
    // x: 4 slabs of 8 rows (one per wave); Wg: 16 slabs (4 per wave)
    const int xr = t0 + 8 * wave + lrow;
    const uint32_t voff_x = xr < T ? (uint32_t)(xr * row_bytes + 16 * lchunk) : kOob;
    uint32_t voff_w[4];
    for (int j = 0; j < 4; j++) {
        const int r = e0 + 32 * wave + 8 * j + lrow;
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
        for (int j = 0; j < 4; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rw, (lds_ptr_t)(base + (kRtTok + 32 * wave + 8 * j) * 128), 16, voff_w[j], soff, 0, 0);
    };

    const int q = lane >> 4, r16 = lane & 15;
    const int off_lo = 16 * (q ^ (r16 & 7)), off_hi = 16 * ((4 + q) ^ (r16 & 7));
    f32x4 acc[2][2];
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 2; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    issue(0, 0);
    if (nk > 1) issue(1, 1);
    for (int kt = 0; kt < nk; kt++) {
        if (kt + 1 < nk) wait_vmcnt<5>();
        else wait_vmcnt<0>();
        bare_barrier();
        if (kt + 2 < nk) issue((kt + 2) % kRtNS, kt + 2);
        const uint8_t* base = smem + (kt % kRtNS) * kRtStage;
        u32x4 alo[2], ahi[2];
        for (int rt = 0; rt < 2; rt++) {
            const uint8_t* p = base + (16 * rt + r16) * 128;
            alo[rt] = *(const u32x4*)(p + off_lo);
            ahi[rt] = *(const u32x4*)(p + off_hi);
        }
        for (int ct = 0; ct < 2; ct++) {
            const uint8_t* p = base + (kRtTok + 32 * wave + 16 * ct + r16) * 128;
            const u32x4 blo = *(const u32x4*)(p + off_lo), bhi = *(const u32x4*)(p + off_hi);
            for (int rt = 0; rt < 2; rt++) {
                acc[rt][ct] = mfma_bf16(alo[rt], blo, acc[rt][ct]);
                acc[rt][ct] = mfma_bf16(ahi[rt], bhi, acc[rt][ct]);
            }
        }
    }
    // lane (q, r16) holds logits of tokens 16rt + 4q + i, expert 16ct + r16
    for (int rt = 0; rt < 2; rt++)
        for (int ct = 0; ct < 2; ct++) {
            const int e = e0 + 32 * wave + 16 * ct + r16;
            for (int i = 0; i < 4; i++) {
                const int t = t0 + 16 * rt + 4 * q + i;
                if (e < E && t < T) logits[(size_t)t * E + e] = acc[rt][ct][i];
            }
        }
}

__global__ __launch_bounds__(256) void route_topk_kernel(const float* __restrict__ logits, int T,
                                                         int E, int K, int* __restrict__ idx,
                                                         float* __restrict__ wts) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;  // whole wave
    const float* row = logits + (size_t)t * E;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = lane + 64 * j < E ? row[lane + 64 * j] : -FLT_MAX;
    wave_route_token_reg(v, E, K, idx + (size_t)t * K, wts + (size_t)t * K);
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

size_t route_mfma_scratch_bytes(int T, int E) { return (size_t)T * E * sizeof(float); }

int launch_route_mfma(const uint16_t* x, const uint16_t* wg, int T, int E, int K, int D, int* idx,
                      float* wts, float* logits, hipStream_t st) {
    AMDMOE_CHECK_ARG(route_mfma_supported(E, D), "routing: MFMA gate needs E <= 256 and D %% 64 == 0");
    dim3 g1((unsigned)ceil_div(T, kRtTok), (unsigned)ceil_div(E, kRtExp));
    hipLaunchKernelGGL(route_logits_kernel, g1, dim3(256), kRtLds, st, x, wg, T, E, D, logits);
    AMDMOE_LAUNCH_CHECK();
    hipLaunchKernelGGL(route_topk_kernel, dim3((unsigned)ceil_div(T, 4)), dim3(256), 0, st, logits,
                       T, E, K, idx, wts);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

}  // namespace amdmoe
