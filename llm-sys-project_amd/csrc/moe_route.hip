// R1 -- routing: gate logits, softmax over experts, top-K, renormalisation.
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
//   route_logits_kernel -- bf16 x and bf16 gate (DeepSeek-V3 shape, E=256,
//     D=7168): the gate GEMM runs on bf16 MFMA with fp32 accumulation, split
//     along D over the CUs; route_topk_kernel / route_topk_block_kernel sum
//     the chunk partials in chunk order.
// Both then run the same wave routine: softmax (with the reference's
// sequential denominator for the fp32 gate, a wave tree sum after the MFMA
// gate), and a ballot-driven exact simulation of the replace-min loop (only
// insertions cost work: ~K*(1+ln(E/K)) of them).
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

// min over the slot lanes [0, KMAX) of a 16-lane DPP row, broadcast from
// lane 0 (lanes in [K, KMAX) must hold +inf).
template <int KMAX>
__device__ __forceinline__ float slot_min(float v) {
    static_assert(KMAX >= 1 && KMAX <= 16, "slot_min: KMAX <= 16");
    if constexpr (KMAX > 1) v = dpp_min<0xB1>(v);   // quad_perm [1,0,3,2]
    if constexpr (KMAX > 2) v = dpp_min<0x4E>(v);   // quad_perm [2,3,0,1]
    if constexpr (KMAX > 4) v = dpp_min<0x141>(v);  // row_half_mirror
    if constexpr (KMAX > 8) v = dpp_min<0x140>(v);  // row_mirror
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

// Routing of one token by one wave, E <= 256, K <= KMAX <= 16: `v` holds
// the logits of experts lane + 64j (j < 4; -FLT_MAX past E).
// SEQ: the softmax denominator in the reference's order (ascending expert,
// one add at a time), for logits that are bit-identical to the reference's
// (the fp32 gate), so the weights are too.  Otherwise a tree sum over the
// wave (every lane gets the same value): for the MFMA gates, whose logits
// differ from the reference's sequential fp32 sums by rounding anyway.  The
// denominator scales every probability alike, so the order of the
// probabilities, and with it the selection, is the same either way
// wherever distinct logits are farther apart than the rounding of one
// division (always, for the exactly representable logits the parity tests
// use); the weights move by at most a few ulps.
template <int KMAX, bool SEQ = true>
__device__ void wave_route_token_reg(float (&v)[4], int E, int K, int* out_idx, float* out_wts) {
    const int lane = lane_id();
    // softmax (tests/test_moe.cu:14-20)
    float mx = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
    mx = wave_max(mx);
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = lane + 64 * j < E ? expf(v[j] - mx) : 0.0f;
    // SEQ: the denominator is summed in ascending expert order, exactly as
    // the reference does: lane values are read out one by one (v_readlane).
    float s = 0.0f;
    if constexpr (!SEQ) s = wave_sum((v[0] + v[1]) + (v[2] + v[3]));  // 0 past E
#pragma unroll
    for (int j = 0; j < 4 && SEQ; j++) {
        if (64 * j >= E) break;  // uniform
        const int n = min(64, E - 64 * j);
        if (n == 64) {
            // eight reads ahead of the adds that consume them
#pragma unroll
            for (int b = 0; b < 64; b += 8) {
                float r[8];
#pragma unroll
                for (int i = 0; i < 8; i++) r[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[j]), b + i));
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < 8; i++) s = add_rn(s, r[i]);
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            for (int l = 0; l < n; l++) s = add_rn(s, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[j]), l)));
        }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = __fdiv_rn(v[j], s);

    // replace-min top-K (tests/test_moe.cu:52-64).  Lane k < K owns slot k.
    // thr is the smallest slot value and m the first slot holding it; only
    // an expert with p > thr changes anything, and thr never decreases, so
    // the experts of each 64-lane group that beat the current thr are taken
    // in ascending order from a ballot mask, which is re-formed after every
    // insertion from the new thr.
    // Every slot starts at -FLT_MAX, so when the first min(K, E) experts all
    // beat it (finite probabilities are >= 0) they are inserted in order into
    // slots 0, 1, ...: that fill is one step, and the scan resumes at expert
    // min(K, E).  A non-finite logit makes every probability NaN, which
    // beats nothing: then the scan runs from expert 0 and, as in the
    // reference, inserts nothing (indices -1, weights -FLT_MAX).
    int k0 = min(K, E);  // uniform, <= 16: all in group 0
    if (__ballot(lane < k0 && !(v[0] > -FLT_MAX))) k0 = 0;
    float sv = lane < k0 ? v[0] : -FLT_MAX;
    int si = lane < k0 ? lane : -1;
    float thr = slot_min<KMAX>(lane < K ? sv : INFINITY);
    int m = __ffsll(__ballot(lane < K && sv == thr)) - 1;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        if (64 * j >= E) break;  // uniform
        const bool valid = lane + 64 * j < E && (j > 0 || lane >= k0);
        unsigned long long cand = __ballot(valid && v[j] > thr);
        while (cand) {
            const int l = __ffsll(cand) - 1;  // next inserted expert: 64j + l
            const float val = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[j]), l));
            if (lane == m) { sv = val; si = 64 * j + l; }
            thr = slot_min<KMAX>(lane < K ? sv : INFINITY);
            m = __ffsll(__ballot(lane < K && sv == thr)) - 1;
            cand = __ballot(valid && lane > l && v[j] > thr);
        }
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

// Smallest power of two >= K (K <= 16): the slot-lane width of
// wave_route_token_reg.
static inline int route_kmax(int K) { return K <= 1 ? 1 : K <= 2 ? 2 : K <= 4 ? 4 : K <= 8 ? 8 : 16; }

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
    if (E <= 256 && K <= 16) {
        const int lane = lane_id();
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = lane + 64 * j < E ? p[lane + 64 * j] : -FLT_MAX;
        if (K <= 2) wave_route_token_reg<2>(v, E, K, out_idx, out_wts);
        else if (K <= 4) wave_route_token_reg<4>(v, E, K, out_idx, out_wts);
        else if (K <= 8) wave_route_token_reg<8>(v, E, K, out_idx, out_wts);
        else wave_route_token_reg<16>(v, E, K, out_idx, out_wts);
    } else {
        wave_route_token_lds(p, E, K, out_idx, out_wts);
    }
}

template <typename T> __device__ __forceinline__ float load_f(const T* p);
template <> __device__ __forceinline__ float load_f<float>(const float* p) { return *p; }
template <> __device__ __forceinline__ float load_f<uint16_t>(const uint16_t* p) {
    return bf16_to_f32(*p);
}
// eight consecutive elements as fp32 (p 16-byte aligned)
__device__ __forceinline__ void load8_f(const float* p, float (&v)[8]) {
    const f32x4 a = *(const f32x4*)p, b = *(const f32x4*)(p + 4);
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = a[i], v[4 + i] = b[i];
}
__device__ __forceinline__ void load8_f(const uint16_t* p, float (&v)[8]) {
    const u32x4 a = *(const u32x4*)p;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[2 * i] = __uint_as_float(a[i] << 16);
        v[2 * i + 1] = __uint_as_float(a[i] & 0xffff0000u);
    }
}

// 32 consecutive elements of a row, as loaded (16-byte loads, row 16-byte
// aligned); get<i>() converts element i to fp32.  Keeping the raw registers
// lets many chunks' loads be in flight while earlier chunks are consumed.
template <typename T> struct Row32;
template <> struct Row32<uint16_t> {
    u32x4 r[4];
    __device__ __forceinline__ void load(const uint16_t* p) {
#pragma unroll
        for (int i = 0; i < 4; i++) r[i] = *(const u32x4*)(p + 8 * i);
    }
    template <int I> __device__ __forceinline__ float get() const {
        const uint32_t w = r[I / 8][(I % 8) / 2];
        return __uint_as_float(I % 2 ? w & 0xffff0000u : w << 16);
    }
};
template <> struct Row32<float> {
    f32x4 r[8];
    __device__ __forceinline__ void load(const float* p) {
#pragma unroll
        for (int i = 0; i < 8; i++) r[i] = *(const f32x4*)(p + 4 * i);
    }
    template <int I> __device__ __forceinline__ float get() const { return r[I / 4][I % 4]; }
};
// sum += x[i] * w[i] for the 32 elements in ascending order (product, then
// sum, each rounded).  The products are independent and formed first; only
// the adds are a dependent chain.
template <typename XT, typename GT>
__device__ __forceinline__ void mac32(float& sum, const Row32<XT>& x, const Row32<GT>& w) {
    float p[32];
    static_for<32>([&](auto ic) __attribute__((always_inline)) {
        constexpr int i = decltype(ic)::value;
        p[i] = mul_rn(x.template get<i>(), w.template get<i>());
    });
#pragma unroll
    for (int i = 0; i < 32; i++) sum = add_rn(sum, p[i]);
}
// 32-element chunks in flight per lane: 8 (4 for fp32 x and gate, whose
// chunks take twice the registers)
template <typename XT, typename GT>
constexpr int exact_ring() { return sizeof(XT) == 4 && sizeof(GT) == 4 ? 4 : 8; }

// ---------------------------------------------------------------- exact
// Block = 128 threads (E <= 128) or 256.  tpb tokens per block (tpb*E <=
// the block when E fits it; otherwise tpb = 1 and lanes loop over experts).
template <typename XT, typename GT>
__global__ __launch_bounds__(256) void route_exact_kernel(const XT* __restrict__ x,
                                                          const GT* __restrict__ wg,
                                                          const float* __restrict__ bias, int T,
                                                          int E, int K, int D, int tpb,
                                                          bool vec, int* __restrict__ idx,
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
            // the reference's order (d ascending, multiply then add).  When
            // the rows are 16-byte aligned the operands arrive 32 at a time
            // through a ring of chunks in registers: a chunk's loads are
            // issued 4-8 chunks before it is summed (one
            // HBM latency is ~4000 cycles, one chunk's sum ~200), so the
            // dependent adds, not the load latency, are the critical path (a
            // lane waiting for each chunk's loads took 182 us for the
            // Mixtral gate, T=4096, D=4096).  The ring's loads are issued
            // unconditionally (chunks past the row re-read its last chunk)
            // so every wait has the same count.
            int d = 0;
            const int n32 = vec ? D / 32 : 0;  // uniform
            if (n32 > 0) {
                constexpr int kExactRing = exact_ring<XT, GT>();
                Row32<XT> xc[kExactRing];
                Row32<GT> wc[kExactRing];
                static_for<kExactRing>([&](auto jc) __attribute__((always_inline)) {
                    constexpr int jj = decltype(jc)::value;
                    const int c = min(jj, n32 - 1);
                    xc[jj].load(xr + 32 * c);
                    wc[jj].load(wr + 32 * c);
                });
                for (int c0 = 0; c0 < n32; c0 += kExactRing) {
                    static_for<kExactRing>([&](auto jc) __attribute__((always_inline)) {
                        constexpr int jj = decltype(jc)::value;
                        if (c0 + jj < n32) mac32(sum, xc[jj], wc[jj]);  // uniform
                        const int cn = min(c0 + jj + kExactRing, n32 - 1);
                        xc[jj].load(xr + 32 * cn);
                        wc[jj].load(wr + 32 * cn);
                    });
                }
                d = 32 * n32;
            }
            if (vec) {
                for (; d + 8 <= D; d += 8) {
                    float xv[8], wv[8];
                    load8_f(xr + d, xv);
                    load8_f(wr + d, wv);
#pragma unroll
                    for (int i = 0; i < 8; i++) sum = mac_rn(sum, xv[i], wv[i]);
                }
            }
            for (; d < D; d++) sum = mac_rn(sum, load_f(xr + d), load_f(wr + d));
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

// ------------------------------------------------------- exact, LDS-fed
// route_exact_lds_kernel: the same per-(token, expert) sequential sums as
// route_exact_kernel (mac32: d ascending, product then sum, each rounded),
// for an fp32 gate, E in {2, 4, 8, 16} and D a multiple of 256 (fp32 x with
// E = 2 excepted: its stages do not fit three deep).  One wave per block holds
// 64/E tokens x E experts.  The block's x rows and the whole gate stream
// through LDS in 256-element stages: a ring of NST stages, the global -> LDS
// DMA of stage c + NST - 1 issued before stage c is summed.  Each x and gate
// row then crosses L2 -> CU once per block instead of once per lane, and
// NST - 1 stages (5 at the Mixtral gate: 1280 elements, ~8000 cycles of
// adds) are in flight where a lane's register ring held ~4 chunks of 32 --
// short of the load latency, so the dependent adds waited on loads (90-100
// us for the Mixtral gate at T = 256 and at T = 4096).  A row's 16-byte
// pieces sit at piece ^ (row & 15), so the distinct rows one read touches
// (64/E of x, E of the gate) fall on distinct banks.
constexpr int kXch = 256;  // elements per stage

template <typename XT, typename GT, int E>
struct ExactLds {
    static constexpr int XB = kXch * (int)sizeof(XT);   // bytes of an x row per stage
    static constexpr int GB = kXch * (int)sizeof(GT);   // bytes of a gate row per stage
    static constexpr int TPB = 64 / E;                  // tokens per block
    static constexpr int XBYTES = TPB * XB;
    static constexpr int STAGE = XBYTES + E * GB;
    static constexpr int NLD = STAGE / 1024;            // DMA instructions per stage
    static constexpr int NST0 = 73728 / STAGE < 8 ? 73728 / STAGE : 8;
    static constexpr int NST = NST0 < 63 / NLD + 1 ? NST0 : 63 / NLD + 1;  // (NST - 1) * NLD <= 63
    static constexpr int LDS = NST * STAGE + 64 * 4;    // + the block's logits
    // whole DMA instructions per region, at least two stages in flight
    static constexpr bool OK = XBYTES % 1024 == 0 && (E * GB) % 1024 == 0 && NST >= 3;
};

// A Row32's k-th 16-byte vector (its elements 16k/sizeof(T) .. in order).
__device__ __forceinline__ void set16(Row32<uint16_t>& r, int k, u32x4 v) { r.r[k] = v; }
__device__ __forceinline__ void set16(Row32<float>& r, int k, u32x4 v) { r.r[k] = __builtin_bit_cast(f32x4, v); }

// The body is a device template behind plain kernels (below): the host side
// emits no launch stub for a kernel template instantiated this way.
template <typename XT, typename GT, int E>
__device__ __forceinline__ void route_exact_lds_body(const XT* __restrict__ x, const GT* __restrict__ wg,
                                                     const float* __restrict__ bias, int T, int K, int D,
                                                     int* __restrict__ idx, float* __restrict__ wts) {
    using L = ExactLds<XT, GT, E>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    float* s_logit = (float*)(smem + L::NST * L::STAGE);
    const int lane = threadIdx.x;
    const int t0 = blockIdx.x * L::TPB;
    const int nst = D / kXch;  // stages of the row
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (long)T * D * (long)sizeof(XT));
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(wg, (long)E * D * (long)sizeof(GT));
    // DMA instruction n of a stage: this lane's 16 bytes land at LDS offset
    // 1024 n + 16 lane of the stage; the piece it loads is the one that
    // offset holds under the XOR layout (stage c adds c * kXch elements)
    uint32_t voff[L::NLD];
#pragma unroll
    for (int n = 0; n < L::NLD; n++) {
        const int o = 1024 * n + 16 * lane;
        if (1024 * n < L::XBYTES) {
            const int row = o / L::XB, piece = ((o % L::XB) >> 4) ^ (row & 15);
            const long t = min(t0 + row, T - 1);  // rows past T re-read the last token
            voff[n] = (uint32_t)(t * D * (long)sizeof(XT) + 16 * piece);
        } else {
            const int ow = o - L::XBYTES;
            const int row = ow / L::GB, piece = ((ow % L::GB) >> 4) ^ (row & 15);
            voff[n] = (uint32_t)((long)row * D * (long)sizeof(GT) + 16 * piece);
        }
    }
    auto issue = [&](int c) __attribute__((always_inline)) {
        const int cc = min(c, nst - 1);  // stages past the row re-read its last one
        uint8_t* st = smem + (c % L::NST) * L::STAGE;
#pragma unroll
        for (int n = 0; n < L::NLD; n++) {
            if (1024 * n < L::XBYTES)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr_t)(st + 1024 * n), 16, voff[n],
                                                         cc * kXch * (int)sizeof(XT), 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t)(st + 1024 * n), 16, voff[n],
                                                         cc * kXch * (int)sizeof(GT), 0, 0);
        }
    };
    const int lt = lane / E, e = lane % E;
    constexpr int XP = 32 * (int)sizeof(XT) / 16, GP = 32 * (int)sizeof(GT) / 16;  // pieces per 32 elements
    float sum = 0.0f;
#pragma unroll
    for (int c = 0; c < L::NST - 1; c++) issue(c);
    for (int c = 0; c < nst; c++) {
        issue(c + L::NST - 1);        // into the stage summed at c - 1 (its reads are done)
        wait_vmcnt<(L::NST - 1) * L::NLD>();  // stage c has landed
        const uint8_t* st = smem + (c % L::NST) * L::STAGE;
        const uint8_t* xs = st + lt * L::XB;
        const uint8_t* ws = st + L::XBYTES + e * L::GB;
#pragma unroll
        for (int s32 = 0; s32 < kXch / 32; s32++) {
            Row32<XT> xr;
            Row32<GT> wr;
            // Row32 holds its 32 elements as 16-byte vectors in order
#pragma unroll
            for (int k = 0; k < XP; k++) set16(xr, k, *(const u32x4*)(xs + 16 * ((s32 * XP + k) ^ (lt & 15))));
#pragma unroll
            for (int k = 0; k < GP; k++) set16(wr, k, *(const u32x4*)(ws + 16 * ((s32 * GP + k) ^ (e & 15))));
            mac32(sum, xr, wr);
        }
    }
    wait_vmcnt<0>();  // the trailing re-reads
    if (bias) sum = add_rn(sum, bias[e]);
    s_logit[lane] = sum;
    __syncthreads();
    for (int j = 0; j < L::TPB; j++) {
        const int t = t0 + j;
        if (t >= T) break;
        wave_route_token(s_logit + j * E, E, K, idx + (size_t)t * K, wts + (size_t)t * K);
    }
}

template <typename XT, typename GT, int E> struct ExactLdsKernel {
    static constexpr void (*fn)(const XT*, const GT*, const float*, int, int, int, int*, float*) = nullptr;
};
#define AMDMOE_EXACT_LDS_KERNEL(NAME, XT, GT, E)                                                            \
    __global__ __launch_bounds__(64) void NAME(const XT* __restrict__ x, const GT* __restrict__ wg,         \
                                               const float* __restrict__ bias, int T, int K, int D,         \
                                               int* __restrict__ idx, float* __restrict__ wts) {            \
        route_exact_lds_body<XT, GT, E>(x, wg, bias, T, K, D, idx, wts);                                     \
    }                                                                                                        \
    template <> struct ExactLdsKernel<XT, GT, E> {                                                           \
        static constexpr void (*fn)(const XT*, const GT*, const float*, int, int, int, int*, float*) = NAME; \
    };
AMDMOE_EXACT_LDS_KERNEL(route_exact_lds_f32_f32_e4, float, float, 4)
AMDMOE_EXACT_LDS_KERNEL(route_exact_lds_f32_f32_e8, float, float, 8)
AMDMOE_EXACT_LDS_KERNEL(route_exact_lds_f32_f32_e16, float, float, 16)
AMDMOE_EXACT_LDS_KERNEL(route_exact_lds_bf16_f32_e2, uint16_t, float, 2)
AMDMOE_EXACT_LDS_KERNEL(route_exact_lds_bf16_f32_e4, uint16_t, float, 4)
AMDMOE_EXACT_LDS_KERNEL(route_exact_lds_bf16_f32_e8, uint16_t, float, 8)
AMDMOE_EXACT_LDS_KERNEL(route_exact_lds_bf16_f32_e16, uint16_t, float, 16)
// (a bf16 gate whose D is a multiple of 64 routes on the MFMA path)
#undef AMDMOE_EXACT_LDS_KERNEL

// -1: this (types, E) has no LDS-fed form (its stages do not fit three deep)
template <typename XT, typename GT, int E>
static int launch_exact_lds(const XT* x, const GT* wg, const float* bias, int T, int K, int D, int* idx,
                            float* wts, hipStream_t st) {
    using L = ExactLds<XT, GT, E>;
    constexpr auto kern = ExactLdsKernel<XT, GT, E>::fn;
    if constexpr (!L::OK || kern == nullptr) {
        return -1;
    } else {
        const int rc = ensure_dynamic_lds((const void*)kern, L::LDS);
        if (rc != AMDMOE_OK) return rc;
        hipLaunchKernelGGL(kern, dim3((unsigned)ceil_div(T, L::TPB)), dim3(64), L::LDS, st, x, wg, bias, T, K, D, idx,
                           wts);
        AMDMOE_LAUNCH_CHECK();
        return AMDMOE_OK;
    }
}

// ---------------------------------------------------------------- MFMA
// bf16 x [T,D] and bf16 Wg [E,D], E <= 256, D % 64 == 0.  Two launches:
//
// route_logits_kernel: the gate GEMM, split along D.  Block = 512 threads,
//   a 64-token x 256-expert tile over one K-chunk (wave w owns experts
//   [32w, 32w+32): 4 row tiles x 2 column tiles of 16x16 MFMA).  Each K-step
//   (64 bf16 = 128 bytes of every row) streams the x rows (8 KB) and the
//   gate rows (32 KB) global -> LDS through a 3-stage direct-load ring; rows
//   past T or E read as zeros.  LDS rows are 128 bytes, 16-byte chunks
//   XOR-swizzled by (row & 7).  The grid is (token tiles) x (K-chunks),
//   with as many chunks as it takes to give every CU a block (4 at
//   T=4096; at most 16, 14 at T=1), so no block walks all of D alone; every x element is
//   read by exactly one block.  Blocks of one chunk share an XCD (its L2
//   holds the chunk's gate rows).  Each chunk's partial logits go to
//   part[chunk][T][E] (fp32).
//   Fused x quantisation (fp8 layer): a chunk covers whole 128-column
//   blocks (two K-steps), so the block that reads a token's columns also
//   writes their e4m3 codes and 1x128 scale -- the even K-step's 64 values
//   are held in registers until the odd one arrives.  Same arithmetic as
//   quant_rows_kernel (scale = amax/448, q = e4m3_rne_sat(v/scale)), so the
//   codes are bit-identical.
// route_topk_kernel: one wave per token: sums the chunk partials in chunk
//   order, then softmax + replace-min top-K + renormalisation
//   (wave_route_token_reg).
// LDS: an 8-stage ring of x slabs (64 tokens x 64 columns, 8 KB) and a
// 3-stage ring of gate slabs (256 experts x 64 columns, 32 KB).  x comes from
// HBM (every element is read by one block), the gate from L2 (the blocks of
// a K-chunk share it), so x is loaded 7 K-steps ahead and the gate 2: 56 KB
// of x in flight per CU, 14 MB over the chip, which the HBM latency needs
// (with x and the gate in one 2-ahead ring, 16 KB of x per CU was in flight
// and the gate GEMM ran at ~2.4 TB/s).
constexpr int kRtTok = 64;
constexpr int kRtExp = 256;
constexpr int kRtXStage = kRtTok * 128;            // 8192
constexpr int kRtWStage = kRtExp * 128;            // 32768
constexpr int kRtNX = 8;
constexpr int kRtNW = 3;
constexpr int kRtWOff = kRtNX * kRtXStage;         // 65536
constexpr int kRtLds = kRtWOff + kRtNW * kRtWStage;  // 163840
constexpr int kRtMinBlocks = 256;                  // one per CU
constexpr int kRtMaxSplit = 16;                    // partials summed per logit (one wave per token)
// Decode-sized batches (one 64-token tile) split the gate into up to 64
// chunks of one 128-column block each, so 56 workgroups share the gate's
// 3.7 MB at DeepSeek-V3's shape; route_topk_block_kernel then sums them.
constexpr int kRtMaxSplitSmall = 64;

// K-steps (64 columns) per chunk and number of chunks.  With quantisation
// a chunk is a whole number of 128-column blocks.
struct RouteSplit {
    int kc, nsplit;
};
static RouteSplit route_split(int T, int D, bool quant) {
    const int nk = D / 64, unit = quant ? 2 : 1;
    const int units = nk / unit;
    const int tiles = (T + kRtTok - 1) / kRtTok;
    int want = (kRtMinBlocks + tiles - 1) / tiles;
    const int cap = tiles == 1 ? kRtMaxSplitSmall : kRtMaxSplit;
    want = want > cap ? cap : want;
    want = want < 1 ? 1 : (want > units ? units : want);
    const int kc = ((units + want - 1) / want) * unit;
    return {kc, (nk + kc - 1) / kc};
}

// max over the 8 lanes of a DPP half-row
template <int CTRL>
__device__ __forceinline__ float dpp_fmax(float v) {
    return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v),
                                                                CTRL, 0xF, 0xF, false)));
}

__global__ __launch_bounds__(512) void route_logits_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ wg, int T,
                                                           int E, int D, int kc, int nsplit,
                                                           float* __restrict__ part,
                                                           uint8_t* __restrict__ xq,
                                                           float* __restrict__ xs) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // work item (chunk-major, token tile fastest), dealt to the 8 XCDs in
    // contiguous ranges (workgroup b runs on XCD b % 8): the blocks of one
    // K-chunk share an XCD, whose L2 then holds that chunk's gate rows
    // instead of every chunk's
    const int ntile = (T + kRtTok - 1) / kRtTok;
    const int per = gridDim.x >> 3;
    const int item = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (item >= ntile * nsplit) return;  // grid padding
    const int split = item / ntile;
    const int t0 = (item - split * ntile) * kRtTok;
    const int nk = D / 64;
    const int kb0 = split * kc;
    const int nloc = min(nk, kb0 + kc) - kb0;  // >= 1 (even with quantisation)
    const long row_bytes = (long)D * 2;

    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (long)T * row_bytes);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(wg, (long)E * row_bytes);
    const int lrow = lane >> 3, lchunk = (lane & 7) ^ lrow;
    // x: 8 slabs of 8 rows (one per wave); Wg: 32 slabs (4 per wave)
    const int xr = t0 + 8 * wave + lrow;
    const uint32_t voff_x = xr < T ? (uint32_t)(xr * row_bytes + 16 * lchunk) : kOob;
    uint32_t voff_w[4];
    for (int j = 0; j < 4; j++) {
        const int r = 32 * wave + 8 * j + lrow;
        voff_w[j] = r < E ? (uint32_t)(r * row_bytes + 16 * lchunk) : kOob;
    }
    // rotated K order per block (by whole 128-column blocks): gate rows are
    // 128-byte slices at a fixed stride, so blocks in lockstep would all hit
    // the same memory channels
    const int npair = nloc >> 1;
    const int kt0 = npair > 1 ? 2 * (int)(((unsigned)(t0 / kRtTok) * 13u) % (unsigned)npair) : 0;
    auto kloc = [&](int kt) {
        int k = kt + kt0;
        return k >= nloc ? k - nloc : k;
    };
    // every issue is unconditional (a K-step past the chunk reads zeros into
    // a stage nobody reads again), so each wait below has a fixed count
    auto issue_x = [&](int kt) {
        uint8_t* base = smem + (kt % kRtNX) * kRtXStage;
        const bool live = kt < nloc;
        const int soff = live ? (kb0 + kloc(kt)) * 128 : 0;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr_t)(base + 8 * wave * 128), 16,
                                                 live ? voff_x : kOob, soff, 0, 0);
    };
    auto issue_w = [&](int kt) {
        uint8_t* base = smem + kRtWOff + (kt % kRtNW) * kRtWStage;
        const bool live = kt < nloc;
        const int soff = live ? (kb0 + kloc(kt)) * 128 : 0;
        for (int j = 0; j < 4; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t)(base + (32 * wave + 8 * j) * 128), 16,
                                                     live ? voff_w[j] : kOob, soff, 0, 0);
    };

    const int q = lane >> 4, r16 = lane & 15;
    const int off_lo = 16 * (q ^ (r16 & 7)), off_hi = 16 * ((4 + q) ^ (r16 & 7));
    f32x4 acc[4][2];
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 2; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // quantisation: thread (token tq, chunk qc) owns 8 columns of each half
    const int tq = tid >> 3, qc = tid & 7;
    const int qtok = t0 + tq;
    float qv[8];
    float qam = 0.0f;

    // issue order: x(0..6), gate(0), gate(1), then per K-step kt: x(kt+7),
    // gate(kt+2).  Waiting for x(kt) and gate(kt) leaves the 4 loads of
    // gate(1) outstanding at kt = 0 and the 5 of step kt-1 after that.
    for (int j = 0; j < kRtNX - 1; j++) issue_x(j);
    issue_w(0);
    issue_w(1);
    for (int kt = 0; kt < nloc; kt++) {
        if (kt == 0) wait_vmcnt<4>();
        else wait_vmcnt<5>();
        bare_barrier();  // step kt landed; steps kt-1 (x, gate) and their stages free
        issue_x(kt + kRtNX - 1);
        issue_w(kt + 2);
        const uint8_t* base = smem + (kt % kRtNX) * kRtXStage;
        const uint8_t* wbase = smem + kRtWOff + (kt % kRtNW) * kRtWStage;
        u32x4 alo[4], ahi[4];
        for (int rt = 0; rt < 4; rt++) {
            const uint8_t* p = base + (16 * rt + r16) * 128;
            alo[rt] = *(const u32x4*)(p + off_lo);
            ahi[rt] = *(const u32x4*)(p + off_hi);
        }
        for (int ct = 0; ct < 2; ct++) {
            const uint8_t* p = wbase + (32 * wave + 16 * ct + r16) * 128;
            const u32x4 blo = *(const u32x4*)(p + off_lo), bhi = *(const u32x4*)(p + off_hi);
            for (int rt = 0; rt < 4; rt++) {
                acc[rt][ct] = mfma_bf16(alo[rt], blo, acc[rt][ct]);
                acc[rt][ct] = mfma_bf16(ahi[rt], bhi, acc[rt][ct]);
            }
        }
        if (xq) {
            const u32x4 raw = *(const u32x4*)(base + tq * 128 + 16 * (qc ^ (tq & 7)));
            float f[8];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                f[2 * k] = __uint_as_float(raw[k] << 16);
                f[2 * k + 1] = __uint_as_float(raw[k] & 0xffff0000u);
            }
            float am = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; k++) am = fmaxf(am, fabsf(f[k]));
            am = dpp_fmax<0x141>(dpp_fmax<0x4E>(dpp_fmax<0xB1>(am)));  // 8-lane max
            const int kg = kb0 + kloc(kt);                              // global K-step
            if ((kg & 1) == 0) {
#pragma unroll
                for (int k = 0; k < 8; k++) qv[k] = f[k];
                qam = am;
            } else if (qtok < T) {
                am = fmaxf(am, qam);
                const float sc = am > 0.0f ? __fdiv_rn(am, 448.0f) : 1.0f;
                const BlockDivisor dv = block_divisor(sc);
                const int blk = kg >> 1;
                uint8_t* dst = xq + (size_t)qtok * D + blk * 128 + 8 * qc;
                u32x2 c0, c1;
                c0[0] = f32x4_to_e4m3x4(div_rn(dv, qv[0]), div_rn(dv, qv[1]), div_rn(dv, qv[2]), div_rn(dv, qv[3]));
                c0[1] = f32x4_to_e4m3x4(div_rn(dv, qv[4]), div_rn(dv, qv[5]), div_rn(dv, qv[6]), div_rn(dv, qv[7]));
                c1[0] = f32x4_to_e4m3x4(div_rn(dv, f[0]), div_rn(dv, f[1]), div_rn(dv, f[2]), div_rn(dv, f[3]));
                c1[1] = f32x4_to_e4m3x4(div_rn(dv, f[4]), div_rn(dv, f[5]), div_rn(dv, f[6]), div_rn(dv, f[7]));
                *(u32x2*)dst = c0;
                *(u32x2*)(dst + 64) = c1;
                if (qc == 0) xs[(size_t)qtok * (D / 128) + blk] = sc;
            }
        }
    }
    // lane (q, r16) holds logits of tokens 16rt + 4q + i, expert 32w + 16ct + r16
    float* dst = part + (size_t)split * T * E;
    for (int rt = 0; rt < 4; rt++)
        for (int ct = 0; ct < 2; ct++) {
            const int e = 32 * wave + 16 * ct + r16;
            for (int i = 0; i < 4; i++) {
                const int t = t0 + 16 * rt + 4 * q + i;
                if (e < E && t < T) dst[(size_t)t * E + e] = acc[rt][ct][i];
            }
        }
}

template <int KMAX>
__global__ __launch_bounds__(256) void route_topk_kernel(const float* __restrict__ part, int nsplit,
                                                         int T, int E, int K, int* __restrict__ idx,
                                                         float* __restrict__ wts) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;  // whole wave
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = lane + 64 * j < E ? 0.0f : -FLT_MAX;
    // every chunk's partials (nsplit <= kRtMaxSplit) are loaded before any
    // is added -- one round trip -- then summed in chunk order
    static_assert(kRtMaxSplit == 16, "one batch of 16 chunk loads");
    float pv[kRtMaxSplit][4];
#pragma unroll
    for (int i = 0; i < kRtMaxSplit; i++) {
        const float* row = part + ((size_t)i * T + t) * E;
#pragma unroll
        for (int j = 0; j < 4; j++) pv[i][j] = i < nsplit && lane + 64 * j < E ? row[lane + 64 * j] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < kRtMaxSplit; i++)
        if (i < nsplit)
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (lane + 64 * j < E) v[j] = add_rn(v[j], pv[i][j]);
    wave_route_token_reg<KMAX, false>(v, E, K, idx + (size_t)t * K, wts + (size_t)t * K);
}

// route_topk_block_kernel: one 256-thread workgroup per token for gates
// split into more than kRtMaxSplit chunks.  Thread e sums expert e's chunk
// partials in chunk order (every chunk's load in flight at once, each load
// instruction 1 KB contiguous across the workgroup), the logits go through
// LDS, and wave 0 routes the token (wave_route_token_reg).
template <int KMAX>
__global__ __launch_bounds__(256) void route_topk_block_kernel(const float* __restrict__ part, int nsplit,
                                                               int T, int E, int K, int* __restrict__ idx,
                                                               float* __restrict__ wts) {
    __shared__ float s_logit[256];
    const int t = blockIdx.x, e = threadIdx.x;
    // every load unconditional (chunks past nsplit re-read the last one and
    // are not added; experts past E re-read expert E-1 and are not used):
    // no per-load branch, no exec masks held across the batch
    const int ec = min(e, E - 1);
    float pv[kRtMaxSplitSmall];
#pragma unroll
    for (int i = 0; i < kRtMaxSplitSmall; i++)
        pv[i] = part[((size_t)min(i, nsplit - 1) * T + t) * E + ec];
    float v = 0.0f;
#pragma unroll
    for (int i = 0; i < kRtMaxSplitSmall; i++)
        if (i < nsplit) v = add_rn(v, pv[i]);
    s_logit[e] = v;
    __syncthreads();
    if (threadIdx.x >= 64) return;  // wave 0 routes
    const int lane = threadIdx.x;
    float r[4];
#pragma unroll
    for (int j = 0; j < 4; j++) r[j] = lane + 64 * j < E ? s_logit[lane + 64 * j] : -FLT_MAX;
    wave_route_token_reg<KMAX, false>(r, E, K, idx + (size_t)t * K, wts + (size_t)t * K);
}

// ---------------------------------------------------------------- launch
template <typename XT, typename GT>
int launch_route_exact(const XT* x, const GT* wg, const float* bias, int T, int E, int K, int D,
                       int* idx, float* wts, hipStream_t st) {
    // 128-thread blocks for E <= 128: the (token, expert) lanes of a token
    // batch then spread over twice the CUs, halving each CU's load volume
    // (every lane streams its x row and gate row through the CU)
    const int threads = E <= 128 ? 128 : 256;
    int tpb = E <= threads ? threads / E : 1;
    if (tpb > 64) tpb = 64;
    size_t lds = sizeof(float) * (size_t)tpb * E;
    AMDMOE_CHECK_ARG(lds <= 64 * 1024, "routing: E=%d too large for the exact gate", E);
    int grid = (int)ceil_div(T, tpb);
    // every row 16-byte aligned: base pointers aligned, rows a multiple of 16 bytes
    const bool vec = ((uintptr_t)x & 15) == 0 && ((uintptr_t)wg & 15) == 0 && (D * sizeof(XT)) % 16 == 0 &&
                     (D * sizeof(GT)) % 16 == 0;
    // the LDS-fed form: few experts, whole 256-element stages, x and the gate
    // within a buffer descriptor's 32-bit range
    if (vec && T > 0 && D % kXch == 0 && K <= 16 && (long)T * D * (long)sizeof(XT) < (1L << 31) &&
        (long)E * D * (long)sizeof(GT) < (1L << 31)) {
        int rc = -1;
        switch (E) {
            case 2: rc = launch_exact_lds<XT, GT, 2>(x, wg, bias, T, K, D, idx, wts, st); break;
            case 4: rc = launch_exact_lds<XT, GT, 4>(x, wg, bias, T, K, D, idx, wts, st); break;
            case 8: rc = launch_exact_lds<XT, GT, 8>(x, wg, bias, T, K, D, idx, wts, st); break;
            case 16: rc = launch_exact_lds<XT, GT, 16>(x, wg, bias, T, K, D, idx, wts, st); break;
            default: break;
        }
        if (rc != -1) return rc;
    }
    hipLaunchKernelGGL((route_exact_kernel<XT, GT>), dim3(grid), dim3(threads), lds, st, x, wg, bias,
                       T, E, K, D, tpb, vec, idx, wts);
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

bool route_mfma_supported(int E, int K, int D) { return E >= 1 && E <= 256 && K <= 16 && D % 64 == 0; }

size_t route_mfma_scratch_bytes(int T, int E, int D, bool quant) {
    return (size_t)route_split(T, D, quant).nsplit * T * E * sizeof(float);
}

int launch_route_mfma(const uint16_t* x, const uint16_t* wg, int T, int E, int K, int D, int* idx,
                      float* wts, float* part, uint8_t* xq, float* xs, hipStream_t st) {
    AMDMOE_CHECK_ARG(route_mfma_supported(E, K, D), "routing: MFMA gate needs E <= 256, K <= 16 and D %% 64 == 0");
    const bool quant = xq != nullptr;
    AMDMOE_CHECK_ARG(!quant || (xs && D % 128 == 0), "routing: fused quantisation needs D %% 128 == 0");
    const RouteSplit sp = route_split(T, D, quant);
    AMDMOE_CHECK_ARG(sp.nsplit >= 1 && sp.nsplit <= kRtMaxSplitSmall && (sp.nsplit <= kRtMaxSplit || T <= kRtTok),
                     "routing: %d gate splits", sp.nsplit);
    {
        const int rc = ensure_dynamic_lds((const void*)route_logits_kernel, kRtLds);
        if (rc != AMDMOE_OK) return rc;
    }
    // one linear grid, padded to a multiple of 8 for the XCD dealing
    const long items = ceil_div(T, kRtTok) * (long)sp.nsplit;
    hipLaunchKernelGGL(route_logits_kernel, dim3((unsigned)(ceil_div(items, 8) * 8)), dim3(512), kRtLds,
                       st, x, wg, T, E, D, sp.kc, sp.nsplit, part, xq, xs);
    AMDMOE_LAUNCH_CHECK();
    auto topk = route_topk_kernel<16>;
    switch (route_kmax(K)) {
        case 1: topk = route_topk_kernel<1>; break;
        case 2: topk = route_topk_kernel<2>; break;
        case 4: topk = route_topk_kernel<4>; break;
        case 8: topk = route_topk_kernel<8>; break;
        default: break;
    }
    if (sp.nsplit > kRtMaxSplit) {
        auto topkb = route_topk_block_kernel<16>;
        switch (route_kmax(K)) {
            case 1: topkb = route_topk_block_kernel<1>; break;
            case 2: topkb = route_topk_block_kernel<2>; break;
            case 4: topkb = route_topk_block_kernel<4>; break;
            case 8: topkb = route_topk_block_kernel<8>; break;
            default: break;
        }
        hipLaunchKernelGGL(topkb, dim3((unsigned)T), dim3(256), 0, st, part, sp.nsplit, T, E, K, idx, wts);
    } else {
        hipLaunchKernelGGL(topk, dim3((unsigned)ceil_div(T, 4)), dim3(256), 0, st, part, sp.nsplit, T, E,
                           K, idx, wts);
    }
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

}  // namespace amdmoe
