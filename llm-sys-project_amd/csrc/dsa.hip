// D1 -- DeepSeek sparse attention (MLA absorbed) decode.
//
// Reference: dsa_forward (kernels/dsa/naive_dsa.cu:435-474) gathers the
// selected K_c/K_p/V rows into [Q,S,*] fp32 buffers, materialises a
// [Q,H,S] score matrix, scales it, softmaxes it serially per (q,h) and
// multiplies by the gathered V; the CPU copy is tests/test_dsa.cu:23-68:
//   s = (dot(q_nope,K_c[i]) + dot(q_pe,K_p[i])) * (1/sqrt(Dc+Dp))
//   P = softmax_S(s);  out = sum_s P*V[i]
//
// dsa_f32_kernel: the fp32 entry point, one workgroup per (q,h).  Lanes own
//   tokens for the scores (each lane runs the reference's two sequential
//   sums), the softmax denominator is summed in token order by one lane,
//   and lanes own output columns for P.V with a sequential sum over tokens,
//   so every value is computed in the reference's order.
//
// dsa_bf16_paged_kernel: the BASELINE decode (Dc=512, Dp=64, bf16 paged
//   latent cache, V = K_c).  Nothing is materialised: one workgroup per
//   (query, 32 heads) translates the query's indices through the page table
//   into LDS, streams 32-token tiles of 1152-byte latent rows into LDS, and
//   per wave (16 heads x one token half) computes
//     S^T = K . Q^T      (bf16 MFMA; K rows from LDS, q held in registers)
//     online softmax per head (lane = head; reduction over lanes/regs)
//     O^T += V^T . P^T   (bf16 MFMA; P^T is already in the B-operand layout
//                         because S^T's output layout gives each lane the
//                         8 tokens {4g..4g+3, 16+4g..16+4g+3} of its head)
//   V^T fragments are read from the same row-major tile with the gfx950
//   transposing LDS read.  The two token halves merge through LDS at the end.
#include "internal.hpp"

#include <float.h>

namespace amdmoe {

// ---------------------------------------------------------------- fp32
// An index outside [0, N) selects no row: it takes no part in the softmax
// (score -inf, weight 0) and nothing is read for it, so the result is the
// attention over the valid indices (0 when there is none).  The scores of
// one (q,h) row live in LDS for S <= kF32LdsS; beyond that in `gscore`
// ([Q*H, S] fp32 scratch), with the same arithmetic.
constexpr int kF32LdsS = 16384;

template <bool GLOBAL>
__global__ __launch_bounds__(64) void dsa_f32_kernel(const float* __restrict__ qn,
                                                     const float* __restrict__ qp,
                                                     const float* __restrict__ kc,
                                                     const float* __restrict__ kp,
                                                     const float* __restrict__ v,
                                                     const int* __restrict__ idx,
                                                     float* __restrict__ out, int H, int Dc,
                                                     int Dp, int S, long N,
                                                     float* __restrict__ gscore) {
    extern __shared__ float s_lds[];  // [S] (LDS form)
    const int qh = blockIdx.x;
    const int q = qh / H;
    const int lane = threadIdx.x;
    float* s_score = GLOBAL ? gscore + (size_t)qh * S : s_lds;
    const float scale = 1.0f / sqrtf((float)(Dc + Dp));
    const float* qnr = qn + (size_t)qh * Dc;
    const float* qpr = qp + (size_t)qh * Dp;
    const int* ir = idx + (size_t)q * S;
    for (int s = lane; s < S; s += 64) {
        const long row = ir[s];
        if (row < 0 || row >= N) {
            s_score[s] = -INFINITY;
            continue;
        }
        const float* kcr = kc + row * Dc;
        const float* kpr = kp + row * Dp;
        float sc = 0.0f, sp = 0.0f;
        for (int d = 0; d < Dc; d++) sc = mac_rn(sc, qnr[d], kcr[d]);
        for (int d = 0; d < Dp; d++) sp = mac_rn(sp, qpr[d], kpr[d]);
        s_score[s] = mul_rn(add_rn(sc, sp), scale);
    }
    __syncthreads();
    float mx = -INFINITY;
    for (int s = lane; s < S; s += 64) mx = fmaxf(mx, s_score[s]);
    mx = wave_max(mx);
    if (mx == -INFINITY) {  // no valid index
        for (int d = lane; d < Dc; d += 64) out[(size_t)qh * Dc + d] = 0.0f;
        return;
    }
    for (int s = lane; s < S; s += 64) s_score[s] = expf(s_score[s] - mx);
    __syncthreads();
    float tot = 0.0f;
    if (lane == 0)
        for (int s = 0; s < S; s++) tot = add_rn(tot, s_score[s]);
    tot = __shfl(tot, 0, 64);
    for (int s = lane; s < S; s += 64) s_score[s] = __fdiv_rn(s_score[s], tot);
    __syncthreads();
    for (int d = lane; d < Dc; d += 64) {
        float acc = 0.0f;
        for (int s = 0; s < S; s++) {
            const long row = ir[s];
            if (row >= 0 && row < N) acc = mac_rn(acc, s_score[s], v[row * Dc + d]);
        }
        out[(size_t)qh * Dc + d] = acc;
    }
}

size_t dsa_f32_scratch_bytes(int Q, int H, int S) {
    return S > kF32LdsS ? (size_t)Q * H * S * 4 : 0;
}

int launch_dsa_f32(const float* qn, const float* qp, const float* kc, const float* kp,
                   const float* v, const int* idx, float* out, int Q, int H, int Dc, int Dp, int S,
                   int N, float* scratch, hipStream_t st) {
    if (Q == 0 || H == 0) return AMDMOE_OK;
    if (S <= kF32LdsS) {
        hipLaunchKernelGGL(dsa_f32_kernel<false>, dim3(Q * H), dim3(64), sizeof(float) * (size_t)S, st,
                           qn, qp, kc, kp, v, idx, out, H, Dc, Dp, S, (long)N, nullptr);
    } else {
        AMDMOE_CHECK_ARG(scratch != nullptr, "dsa_forward: no score scratch for S=%d", S);
        hipLaunchKernelGGL(dsa_f32_kernel<true>, dim3(Q * H), dim3(64), 0, st, qn, qp, kc, kp, v, idx,
                           out, H, Dc, Dp, S, (long)N, scratch);
    }
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

// ---------------------------------------------------------------- bf16 paged
// Geometry: Dc = 512, Dp = 64, one latent row = 576 bf16 = 1152 bytes = 72
// chunks of 16 bytes.  A stage holds 32 token rows densely (36 KB), chunk j
// of token r stored at chunk position j ^ (r & 7) (conflict-free 16-row
// reads).  Workgroup = one query x 32 heads, 4 waves: wave (hg, th) owns
// heads [16hg, 16hg+16) of the group and tokens [16th, 16th+16) of every
// stage.  The stages are filled by direct global->LDS loads (36 per stage,
// 9 per wave) through a 3-stage ring; each lane loads the chunk of the
// token whose physical row the page table gives.
//   S^T (16 tok x 16 heads) = K . Q^T : 18 MFMA 16x16x32, A = K rows (LDS),
//                                       B = q (registers, loaded once)
//   online softmax per head in the exp2 domain; the running max is raised
//   only when a tile's max exceeds it by more than 8 (p <= 256 in bf16),
//   so the O rescale is rare
//   O^T (512 d x 16 heads) += V^T . P^T : 32 MFMA 16x16x16; P^T comes
//   straight from S^T's output layout (lane = head, 4 tokens), V^T
//   fragments from the row-major K_c tile with ds_read_b64_tr_b16.
// Out-of-range voffset for the cache loads: at least the buffer size (the
// cache is at most kMaxCacheBytes) and far enough below 2^32 that adding the
// largest soffset and the 16-byte access cannot wrap back into range.
constexpr uint32_t kOobDsa = 0xFFFFF000u;
constexpr long kMaxCacheBytes = 0xFFFFE000L;
constexpr int kDc = 512, kDp = 64, kDt = 576;
constexpr int kRowBytes = kDt * 2;               // 1152
constexpr int kRowChunks = kRowBytes / 16;       // 72
constexpr int kTileTok = 32;
constexpr int kStageB = kTileTok * kRowBytes;    // 36864
constexpr int kDsaNS = 3;
constexpr int kMaxS = 4096;
constexpr int kRowsOff = kDsaNS * kStageB;       // 110592
constexpr int kMaskOff = kRowsOff + kMaxS * 4;   // 126976: validity bits, 64 tokens per word
constexpr int kDsaLds = kMaskOff + kMaxS / 8;    // 127488
constexpr int kLoadsPerWave = kStageB / 1024 / 4;  // 9

typedef short s16x4 __attribute__((ext_vector_type(4)));

// Reductions over the lanes l, l^16 (resp. l^32) with the gfx950 lane
// swaps: permlane16_swap exchanges the odd 16-lane rows of its first operand
// with the even rows of its second, permlane32_swap the upper half of the
// first with the lower half of the second; with both operands the same
// value the two results hold, at every lane, the values of l and l^16
// (resp. l^32) in some order.
__device__ __forceinline__ float xor16_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
typedef __attribute__((address_space(3))) s16x4* lds_s16x4_ptr;

// Physical cache row of each of a query's S selected tokens -> LDS, by the
// 256 threads of the block (paged latent cache: logical token i lives in
// row page_table[i / page] * page + i % page).  All index loads are issued
// before any page-table load, so the prologue costs two load latencies.
// A selected token is valid when its logical index lies in [0, seq) (seq =
// pages_per_seq * page, the page-table row's capacity), its page id is >= 0
// and its row lies inside the cache; an invalid token (e.g. the -1 padding
// of a sequence shorter than the selection) reads no page-table entry, gets
// row -1 and takes no part in the softmax.  Validity of tokens 64b..64b+63
// goes to bit i of s_mask[b] (wave w of round k writes mask 4k + w).
template <int N>
__device__ __forceinline__ void translate_rows(const int* __restrict__ lg, const int* __restrict__ pt,
                                               int S, int page, long seq, long cache_rows,
                                               int* s_rows, unsigned long long* s_mask) {
    const int tid = threadIdx.x;
    int li[N], pg[N];
#pragma unroll
    for (int k = 0; k < N; k++) li[k] = tid + 256 * k < S ? lg[tid + 256 * k] : -1;
#pragma unroll
    for (int k = 0; k < N; k++) {
        if (li[k] >= seq) li[k] = -1;
        pg[k] = li[k] >= 0 ? pt[li[k] / page] : -1;
    }
#pragma unroll
    for (int k = 0; k < N; k++) {
        const long row = (long)pg[k] * page + (li[k] >= 0 ? li[k] % page : 0);
        const bool ok = li[k] >= 0 && pg[k] >= 0 && row < cache_rows;
        if (tid + 256 * k < S) s_rows[tid + 256 * k] = ok ? (int)row : -1;
        const unsigned long long m = __ballot(ok);
        if ((tid & 63) == 0) s_mask[4 * k + (tid >> 6)] = m;
    }
}

__global__ __launch_bounds__(256, 1) void dsa_bf16_paged_kernel(
    const uint16_t* __restrict__ qn, const uint16_t* __restrict__ qp,
    const uint16_t* __restrict__ cache, long cache_bytes, const int* __restrict__ page_table,
    const int* __restrict__ logical, uint16_t* __restrict__ out, int Q, int H, int S, int page,
    int pages_per_seq, float scale_log2) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    int* s_rows = (int*)(smem + kRowsOff);
    unsigned long long* s_mask = (unsigned long long*)(smem + kMaskOff);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // query-major block order, 4 head groups of one query adjacent: with
    // block b on XCD b % 8, remap so a query's 4 blocks share an XCD (its
    // latent rows are then read from HBM once and served to all 4 from L2)
    const int nblk = gridDim.x, per = nblk / 8;
    const int lin = (blockIdx.x % 8) * per + blockIdx.x / 8;
    const int hgroups = H / 32;
    const int qi = lin / hgroups;
    if (qi >= Q) return;  // padding block of the XCD remap
    const int h0 = (lin % hgroups) * 32;
    const int hg = wave & 1, th = wave >> 1;
    const int g = lane >> 4, c16 = lane & 15;
    const int my_head = h0 + 16 * hg + c16;

    // page-table translation of this query's indices: physical row, or -1
    translate_rows<kMaxS / 256>(logical + (size_t)qi * S, page_table + (size_t)qi * pages_per_seq,
                                S, page, (long)pages_per_seq * page, cache_bytes / kRowBytes, s_rows,
                                s_mask);

    // q of my head as B fragments: 18 K-steps of 32 dims, group g holds 8
    u32x4 qf[18];
    {
        const uint16_t* qnr = qn + ((size_t)qi * H + my_head) * kDc;
        const uint16_t* qpr = qp + ((size_t)qi * H + my_head) * kDp;
        for (int ks = 0; ks < 16; ks++) qf[ks] = *(const u32x4*)(qnr + 32 * ks + 8 * g);
        for (int ks = 0; ks < 2; ks++) qf[16 + ks] = *(const u32x4*)(qpr + 32 * ks + 8 * g);
    }
    __syncthreads();  // s_rows visible; regular loads complete

    const __amdgpu_buffer_rsrc_t rc = make_rsrc(cache, cache_bytes);
    // Lane chunk n of this wave's share of a stage: chunk c = 64*(9w+n)+lane
    // of the 32x72-chunk tile, row c / 72, swizzled column.  The 9 physical
    // rows are read from LDS together, then the 9 loads go out.
    auto issue = [&](int st, int tile) {
        uint8_t* base = smem + st * kStageB;
        int row[kLoadsPerWave];
#pragma unroll
        for (int n = 0; n < kLoadsPerWave; n++) {
            const int c = 64 * (kLoadsPerWave * wave + n) + lane;
            const int tok = tile * kTileTok + c / kRowChunks;
            row[n] = tok < S ? s_rows[tok] : -1;
        }
#pragma unroll
        for (int n = 0; n < kLoadsPerWave; n++) {
            const int c = 64 * (kLoadsPerWave * wave + n) + lane;
            const int r = c / kRowChunks, jp = c - r * kRowChunks;
            const int j = jp ^ (r & 7);
            const uint32_t vo = row[n] >= 0 ? (uint32_t)((long)row[n] * kRowBytes + 16 * j) : kOobDsa;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rc, (lds_ptr_t)(base + 1024 * (kLoadsPerWave * wave + n)), 16, vo, 0, 0, 0);
        }
    };

    f32x4 o[32];
#pragma unroll
    for (int i = 0; i < 32; i++) o[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.0f;
    const int ntiles = (S + kTileTok - 1) / kTileTok;

    // per-lane LDS addresses (bytes within a stage)
    const int r_s = 16 * th + c16;  // token row read for S^T (A operand)
    // V^T transposed read: lane (g, s) supplies token 4g + (s>>2) of this
    // half, dims d0 + 4(s&3) .. +3
    const int r_v = 16 * th + 4 * g + (c16 >> 2);
    const int vsub = 4 * (c16 & 3);

    issue(0, 0);
    if (ntiles > 1) issue(1, 1);
    for (int t = 0; t < ntiles; t++) {
        if (t + 1 < ntiles) wait_vmcnt<kLoadsPerWave>();
        else wait_vmcnt<0>();
        bare_barrier();
        if (t + 2 < ntiles) issue((t + 2) % kDsaNS, t + 2);
        const uint8_t* kb = smem + (t % kDsaNS) * kStageB;

        // S^T: two independent accumulation chains over the 18 K-steps; the
        // K fragments are read from LDS four steps ahead of their MFMA
        f32x4 sa = {0.f, 0.f, 0.f, 0.f}, sb2 = {0.f, 0.f, 0.f, 0.f};
        {
            const uint8_t* krow = kb + r_s * kRowBytes;
            auto kfrag = [&](int ks) __attribute__((always_inline)) {
                return *(const u32x4*)(krow + 16 * ((4 * ks + g) ^ (r_s & 7)));
            };
            u32x4 a[18];
#pragma unroll
            for (int ks = 0; ks < 4; ks++) a[ks] = kfrag(ks);
#pragma unroll
            for (int ks = 0; ks < 18; ks++) {
                if (ks + 4 < 18) a[ks + 4] = kfrag(ks + 4);
                if (ks & 1) sb2 = mfma_bf16(a[ks], qf[ks], sb2);
                else sa = mfma_bf16(a[ks], qf[ks], sa);
            }
        }
        // lane: head c16, tokens 16th + 4g + i of this tile (an invalid
        // token, or one past S, scores -inf)
        float sv[4];
        float tmax = -INFINITY;
        const uint32_t vmask = (uint32_t)(s_mask[t >> 1] >> (32 * (t & 1) + 16 * th + 4 * g));
        for (int i = 0; i < 4; i++) {
            sv[i] = (vmask >> i) & 1u ? (sa[i] + sb2[i]) * scale_log2 : -INFINITY;
            tmax = fmaxf(tmax, sv[i]);
        }
        tmax = xor16_max(tmax);
        tmax = xor32_max(tmax);
        const bool raise = tmax > m_run + 8.0f;
        if (__ballot(raise)) {  // rare after the first tile: rescale O
            const float m_new = raise ? tmax : m_run;
            const float corr = m_run == -INFINITY ? 0.0f : exp2f(m_run - m_new);
            l_run *= corr;
#pragma unroll
            for (int i = 0; i < 32; i++) o[i] *= corr;
            m_run = m_new;
        }
        float pv[4], psum = 0.0f;
        for (int i = 0; i < 4; i++) {
            pv[i] = sv[i] == -INFINITY ? 0.0f : exp2f(sv[i] - m_run);
            psum += pv[i];
        }
        psum = xor16_sum(psum);
        psum = xor32_sum(psum);
        l_run += psum;
        const u32x2 pb2 = {pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3])};
        const s16x4 pb = __builtin_bit_cast(s16x4, pb2);
        {
            const uint8_t* vrow = kb + r_v * kRowBytes;
            auto vfrag = [&](int mt) __attribute__((always_inline)) {
                const int dd = 16 * mt + vsub;
                return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s16x4_ptr)(vrow + 16 * ((dd >> 3) ^ (r_v & 7)) + 8 * ((dd >> 2) & 1)));
            };
            s16x4 va[32];
#pragma unroll
            for (int mt = 0; mt < 6; mt++) va[mt] = vfrag(mt);
#pragma unroll
            for (int mt = 0; mt < 32; mt++) {
                if (mt + 6 < 32) va[mt + 6] = vfrag(mt + 6);
                o[mt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va[mt], pb, o[mt], 0, 0, 0);
            }
        }
    }
    __syncthreads();  // ring no longer read; reuse it for the merge

    // merge the two token halves: wave (hg, 1) hands (m, l, O) to wave (hg, 0)
    float* xch = (float*)smem;                              // [hg][32 mt][4][64 lanes]
    float* xml = (float*)(smem + 2 * 32 * 4 * 64 * 4);      // [hg][2][64]
    if (th == 1) {
#pragma unroll
        for (int mt = 0; mt < 32; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) xch[((hg * 32 + mt) * 4 + i) * 64 + lane] = o[mt][i];
        xml[(hg * 2 + 0) * 64 + lane] = m_run;
        xml[(hg * 2 + 1) * 64 + lane] = l_run;
    }
    __syncthreads();
    if (th == 0) {
        const float m1 = xml[(hg * 2 + 0) * 64 + lane], l1 = xml[(hg * 2 + 1) * 64 + lane];
        const float m = fmaxf(m_run, m1);
        const float c0 = m_run == -INFINITY ? 0.0f : exp2f(m_run - m);
        const float c1 = m1 == -INFINITY ? 0.0f : exp2f(m1 - m);
        const float l = l_run * c0 + l1 * c1;
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        uint16_t* orow = out + ((size_t)qi * H + my_head) * kDc;
#pragma unroll
        for (int mt = 0; mt < 32; mt++) {
            float r[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                r[i] = (o[mt][i] * c0 + xch[((hg * 32 + mt) * 4 + i) * 64 + lane] * c1) * inv;
            const u32x2 pk = {pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3])};
            *(u32x2*)(orow + 16 * mt + 4 * g) = pk;
        }
    }
}

// ------------------------------------------------------ 64-token tiles
// dsa_bf16_paged64_kernel (S <= 2048): one workgroup per (query, 32
// heads), 4 waves, 64-token tiles in a 2-stage LDS ring.  Every token row
// is read from LDS once for S and once for V:
//   wave w computes S^T for tokens 16w..16w+15 of the tile and all 32 heads
//     (two MFMA column tiles; q of the 32 heads held in registers);
//   the 4 waves share one running max per head (tile maxima exchanged
//     through LDS) and write their P (bf16) to LDS;
//   wave w then computes O^T += V^T . P^T for output dims 128w..128w+127
//     over all 64 tokens (16x16x32 MFMA, K = 32 tokens, two K halves).
// No merge is needed at the end: each wave owns a quarter of the output.
// Tile layout in LDS (tile64_off): 1 KB blocks of 16 tokens x 4 chunks
// (16-byte chunk j of the 1152-byte row), [token][chunk slot] with slot =
// (j & 3) ^ ((token >> 2) & 3).  The DMA of wave w, instruction n, lane l
// fills block (w, n) at 16 l, so the 4 lanes of a token read one 64-byte run
// of its row (coalesced); a 16-token S^T fragment read (lane = token, one
// chunk) and a transposed V^T read (4 tokens x 2 chunks per 16 lanes) both
// hit distinct banks; all loop addresses are a base plus an immediate.
constexpr int kT64 = 64;
constexpr int kStage64 = kT64 * kRowBytes;                 // 73728
constexpr int kMaxS64 = 2048;
constexpr int kRows64Off = 2 * kStage64;                   // 147456
constexpr int kP64Off = kRows64Off + kMaxS64 * 4;          // 155648
constexpr int kMax64Off = kP64Off + 4 * 1024;              // 159744
constexpr int kMask64Off = kMax64Off + 4 * 32 * 4;         // 160256: validity bits per tile
constexpr int kDsa64Lds = kMask64Off + kMaxS64 / 8;        // 160512

__device__ __forceinline__ int tile64_off(int t, int j) {  // token t (0..63), chunk j (0..71)
    return ((t >> 4) * 18 + (j >> 2)) * 1024 + (t & 15) * 64 + ((j & 3) ^ ((t >> 2) & 3)) * 16;
}

__global__ __launch_bounds__(256, 1) void dsa_bf16_paged64_kernel(
    const uint16_t* __restrict__ qn, const uint16_t* __restrict__ qp,
    const uint16_t* __restrict__ cache, long cache_bytes, const int* __restrict__ page_table,
    const int* __restrict__ logical, uint16_t* __restrict__ out, int Q, int H, int S, int page,
    int pages_per_seq, float scale_log2) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    int* s_rows = (int*)(smem + kRows64Off);
    uint16_t* s_p = (uint16_t*)(smem + kP64Off);    // [ht][head 16][token 64] bf16
    float* s_max = (float*)(smem + kMax64Off);      // [wave][32 heads]
    unsigned long long* s_mask = (unsigned long long*)(smem + kMask64Off);  // [tile] token bits
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // XCD remap as in dsa_bf16_paged_kernel: a query's head groups share an XCD
    const int nblk = gridDim.x, per = nblk / 8;
    const int lin = (blockIdx.x % 8) * per + blockIdx.x / 8;
    const int hgroups = H / 32;
    const int qi = lin / hgroups;
    if (qi >= Q) return;
    const int h0 = (lin % hgroups) * 32;
    const int g = lane >> 4, c16 = lane & 15;

    translate_rows<kMaxS64 / 256>(logical + (size_t)qi * S, page_table + (size_t)qi * pages_per_seq,
                                  S, page, (long)pages_per_seq * page, cache_bytes / kRowBytes,
                                  s_rows, s_mask);
    // q of heads h0 + 16ht + c16 as B fragments: K-step ks = 32 dims, group g holds 8
    u32x4 qf[2][18];
#pragma unroll
    for (int ht = 0; ht < 2; ht++) {
        const size_t hrow = (size_t)qi * H + h0 + 16 * ht + c16;
        const uint16_t* qnr = qn + hrow * kDc;
        const uint16_t* qpr = qp + hrow * kDp;
#pragma unroll
        for (int ks = 0; ks < 16; ks++) qf[ht][ks] = *(const u32x4*)(qnr + 32 * ks + 8 * g);
#pragma unroll
        for (int ks = 0; ks < 2; ks++) qf[ht][16 + ks] = *(const u32x4*)(qpr + 32 * ks + 8 * g);
    }
    __syncthreads();  // s_rows visible; regular loads complete

    const __amdgpu_buffer_rsrc_t rc = make_rsrc(cache, cache_bytes);
    // DMA lane l: token 16w + (l >> 2), chunk 4n + ((l & 3) ^ ((l >> 4) & 3))
    const int my_tok = 16 * wave + (lane >> 2);
    const int my_chunk = (lane & 3) ^ ((lane >> 4) & 3);
    // Tile loads: 18 per wave, one per 64-byte chunk group n.  The row
    // offset of group n goes in soffset: an instruction immediate would also
    // shift the LDS destination.
    auto tile_vo = [&](int tile) {
        const int tok = tile * kT64 + my_tok;
        const int r = tok < S ? s_rows[tok] : -1;
        return r >= 0 ? (uint32_t)((long)r * kRowBytes + 16 * my_chunk) : kOobDsa;
    };
    auto issue_n = [&](int st, uint32_t vo, int n) __attribute__((always_inline)) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rc, (lds_ptr_t)(smem + st * kStage64 + wave * 18 * 1024 + n * 1024), 16, vo, 64 * n, 0, 0);
    };

    f32x4 o[8][2];  // dims 128w + 16mt + 4g + i, head c16 of tile ht
#pragma unroll
    for (int i = 0; i < 8; i++)
        for (int j = 0; j < 2; j++) o[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
    const int ntiles = (S + kT64 - 1) / kT64;

    // V^T transposed reads: K half kh (tokens 32kh..), group g of 8 tokens,
    // half r: lane (g, s) supplies token 32kh + 8g + 4r + (s >> 2), dims
    // d0 + 4(s & 3) .. +3; dim tile mt sits at voff[kh][r][mt & 1] + 1024 (mt >> 1)
    int voff[2][2][2];
#pragma unroll
    for (int kh = 0; kh < 2; kh++)
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int d = 128 * wave + 16 * e + 4 * (c16 & 3);
                voff[kh][r][e] = tile64_off(32 * kh + 8 * g + 4 * r + (c16 >> 2), d >> 3) + (d & 7) * 2;
            }
    const int koff = tile64_off(16 * wave + c16, g);  // S^T fragment of K-step ks: + 1024 ks

    {
        const uint32_t vo0 = tile_vo(0);
#pragma unroll
        for (int n = 0; n < 18; n++) issue_n(0, vo0, n);
    }
    for (int t = 0; t < ntiles; t++) {
        // the next tile's loads are spread over this tile's S^T steps (one
        // per K-step) instead of issued in one burst
        const bool more = t + 1 < ntiles;
        const uint32_t vo_next = tile_vo(more ? t + 1 : t);
        wait_vmcnt<0>();
        bare_barrier();  // tile t landed everywhere; stage (t+1)&1 is free
        const uint8_t* kb = smem + (t & 1) * kStage64;

        // S^T for tokens 16w + (0..15), heads h0 + 16ht + (0..15): four
        // accumulation chains (head tile x even/odd K-step)
        f32x4 sacc[2][2];
#pragma unroll
        for (int i = 0; i < 2; i++)
            for (int j = 0; j < 2; j++) sacc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
        {
            const uint8_t* krow = kb + koff;
            // 10 fragment reads in flight: with one wave per SIMD the LDS
            // only streams at full rate with many reads outstanding
            constexpr int kPre = 10;
            u32x4 a[18];
#pragma unroll
            for (int ks = 0; ks < kPre; ks++) a[ks] = *(const u32x4*)(krow + ks * 1024);
#pragma unroll
            for (int ks = 0; ks < 18; ks++) {
                if (ks + kPre < 18) a[ks + kPre] = *(const u32x4*)(krow + (ks + kPre) * 1024);
                sacc[0][ks & 1] = mfma_bf16(a[ks], qf[0][ks], sacc[0][ks & 1]);
                sacc[1][ks & 1] = mfma_bf16(a[ks], qf[1][ks], sacc[1][ks & 1]);
                if (more) issue_n((t + 1) & 1, vo_next, ks);
            }
        }
        float sv[2][4], tm[2];
        const uint32_t vmask = (uint32_t)(s_mask[t] >> (16 * wave + 4 * g));  // invalid: -inf
#pragma unroll
        for (int ht = 0; ht < 2; ht++) {
            tm[ht] = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sv[ht][i] = (vmask >> i) & 1u ? (sacc[ht][0][i] + sacc[ht][1][i]) * scale_log2 : -INFINITY;
                tm[ht] = fmaxf(tm[ht], sv[ht][i]);
            }
            tm[ht] = xor32_max(xor16_max(tm[ht]));
        }
        if (g == 0) {
            s_max[wave * 32 + c16] = tm[0];
            s_max[wave * 32 + 16 + c16] = tm[1];
        }
        lds_barrier();
        // the tile max over all 64 tokens; the running max is raised only
        // when it grows by more than 8 (p <= 256 in bf16), so the O rescale
        // is rare.  Every wave reads the same values: the same decision.
        bool raise = false;
        float mt4[2];
#pragma unroll
        for (int ht = 0; ht < 2; ht++) {
            mt4[ht] = fmaxf(fmaxf(s_max[16 * ht + c16], s_max[32 + 16 * ht + c16]),
                            fmaxf(s_max[64 + 16 * ht + c16], s_max[96 + 16 * ht + c16]));
            raise |= mt4[ht] > m_run[ht] + 8.0f;
        }
        if (__ballot(raise)) {
#pragma unroll
            for (int ht = 0; ht < 2; ht++) {
                const float m_new = fmaxf(m_run[ht], mt4[ht]);
                const float corr = m_run[ht] == -INFINITY ? 0.0f : exp2f(m_run[ht] - m_new);
                l_run[ht] *= corr;
#pragma unroll
                for (int mt = 0; mt < 8; mt++) o[mt][ht] *= corr;
                m_run[ht] = m_new;
            }
        }
        // P (bf16), head-major [ht][c16][token 0..63]; l over this wave's tokens
#pragma unroll
        for (int ht = 0; ht < 2; ht++) {
            float pv[4], psum = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                pv[i] = sv[ht][i] == -INFINITY ? 0.0f : exp2f(sv[ht][i] - m_run[ht]);
                psum += pv[i];
            }
            l_run[ht] += xor32_sum(xor16_sum(psum));
            const u32x2 pk = {pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3])};
            *(u32x2*)(s_p + (ht * 16 + c16) * 64 + 16 * wave + 4 * g) = pk;
        }
        lds_barrier();
        // O^T (dims 128w + 16mt + 4g + i, head c16) += V^T . P^T over 64 tokens
        u32x4 pb[2][2];  // [K half][ht]
#pragma unroll
        for (int kh = 0; kh < 2; kh++)
#pragma unroll
            for (int ht = 0; ht < 2; ht++)
                pb[kh][ht] = *(const u32x4*)(s_p + (ht * 16 + c16) * 64 + 32 * kh + 8 * g);
        auto vfrag = [&](int i) __attribute__((always_inline)) {  // i = 2 mt + kh
            const int mt = i >> 1, kh = i & 1;
            const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s16x4_ptr)(kb + voff[kh][0][mt & 1] + 1024 * (mt >> 1)));
            const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s16x4_ptr)(kb + voff[kh][1][mt & 1] + 1024 * (mt >> 1)));
            const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
            return (u32x4){l2[0], l2[1], h2[0], h2[1]};
        };
        constexpr int kPreV = 6;
        u32x4 va[16];
#pragma unroll
        for (int i = 0; i < kPreV; i++) va[i] = vfrag(i);
#pragma unroll
        for (int i = 0; i < 16; i++) {
            if (i + kPreV < 16) va[i + kPreV] = vfrag(i + kPreV);
            const int mt = i >> 1, kh = i & 1;
            o[mt][0] = mfma_bf16(va[i], pb[kh][0], o[mt][0]);
            o[mt][1] = mfma_bf16(va[i], pb[kh][1], o[mt][1]);
        }
    }
    __syncthreads();  // every wave is done with s_p / s_max

    // l over all 64 tokens of each tile: sum of the 4 waves' shares
    float* xs = (float*)smem;                          // ring no longer read
#pragma unroll
    for (int ht = 0; ht < 2; ht++) xs[(wave * 2 + ht) * 64 + lane] = l_run[ht];
    __syncthreads();
#pragma unroll
    for (int ht = 0; ht < 2; ht++) {
        float l = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; w++) l += xs[(w * 2 + ht) * 64 + lane];
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        uint16_t* orow = out + ((size_t)qi * H + h0 + 16 * ht + c16) * kDc + 128 * wave;
#pragma unroll
        for (int mt = 0; mt < 8; mt++) {
            const u32x2 pk = {pack_bf16x2(o[mt][ht][0] * inv, o[mt][ht][1] * inv),
                              pack_bf16x2(o[mt][ht][2] * inv, o[mt][ht][3] * inv)};
            *(u32x2*)(orow + 16 * mt + 4 * g) = pk;
        }
    }
}

// ------------------------------------------------------ split kernel
// dsa_split_kernel (H a multiple of 128): one workgroup per (query, group
// of 128 heads, token split), 8 waves; wave w owns heads 16w..16w+15 of the
// group for all of the split's tokens, so its softmax state is private (no
// exchange between waves) and P goes from the S^T accumulators straight
// into the PV MFMA operand.  32-token tiles stream through a 4-stage LDS
// ring (each tile's loads go out two tiles ahead), filled by direct
// global->LDS loads; each wave reads every tile once for S and once for V.
//   S^T (16 tokens x 16 heads) = K . Q^T   16x16x32 bf16, 2 token tiles,
//                                          q of the wave's 16 heads in
//                                          registers
//   online softmax per head in the exp2 domain; l is kept per lane and
//     reduced once at the end
//   O^T (512 dims x 16 heads) += V^T . P^T  16x16x32 bf16 in the token
//     order of S^T's output layout: lane (head c, group g) holds tokens
//     4g..4g+3 and 16+4g..16+4g+3, and the transposed LDS reads of V^T
//     fetch the same tokens
// Registers: O is 128 accumulators and q 72, so a wave fits in 256
// registers and two waves share each SIMD (one wave's softmax, LDS waits
// and barrier run under the other's MFMAs).  The price is LDS traffic:
// every wave reads each tile for its 16 heads, 544 KB per CU per tile.  The
// running max m is raised only when a tile max exceeds it by more than 8
// (so p <= 256), and then O and l are multiplied by 2^(m_old - m_new) in
// registers; with O(1) scores the first tile's max is never exceeded by 8.
// Every split writes its unnormalised O (bf16: the output is bf16 and the
// merge sums at most a few splits in fp32) and (max, sum) per head;
// dsa_merge_kernel combines the splits and writes bf16.
//
// Tile layout (tile32_off): 1 KB blocks of 16 tokens x 4 chunks (16-byte
// chunk j of the 1152-byte row), blocks [token group][chunk group], within a
// block [token][slot] with slot = (j & 3) ^ (token bits 1-2).  Measured with
// the bank-conflict counter on gfx950, this is free of conflicts for both the
// 16-token S fragment reads (ds_read_b128, lane = token, one chunk) and the
// transposed V^T reads (ds_read_b64_tr_b16, 4 tokens x 2 chunks per 16
// lanes); XOR-ing token bits 2-3 instead (the plain 64-bank model's answer)
// cost the S reads 4 conflict cycles each.
constexpr int kT32 = 32;
constexpr int kStage32 = kT32 * kRowBytes;                // 36864
constexpr int kRing32 = 4;
constexpr int kMaxChunk = 2048;                           // tokens per split
constexpr int kMaxSplitS = 65536;                         // selected positions per query (32 splits)
constexpr int kRows32Off = kRing32 * kStage32;            // 147456
constexpr int kMask32Off = kRows32Off + kMaxChunk * 4;    // 155648: validity bits, 64 tokens per word
constexpr int kDsaSplitLds = kMask32Off + kMaxChunk / 8;  // 155904

__device__ __forceinline__ int tile32_off(int t, int j) {  // token t (0..31), chunk j (0..71)
    return ((t >> 4) * 18 + (j >> 2)) * 1024 + (t & 15) * 64 + (((j & 3) ^ ((t >> 1) & 3)) << 4);
}

// 1152 zero bytes: the latent row an invalid position reads when the cache
// is addressed with 64-bit pointers (caches beyond the 4 GiB that a buffer
// descriptor's 32-bit offsets reach)
static __device__ __align__(16) uint16_t g_dsa_zero_row[kDt];

// WIDE: the cache is addressed with 64-bit per-lane pointers
// (global_load_lds_dwordx4) instead of a buffer descriptor's 32-bit offsets.
// The body is a device template behind two plain kernels (the host side
// dropped the launch stub of a templated kernel instantiation using buffer
// descriptors).
constexpr int kRowsPer8 = kMaxChunk / 512;  // split positions per thread

template <bool WIDE>
__device__ __forceinline__ void dsa_split_body(
    const uint16_t* __restrict__ qn, const uint16_t* __restrict__ qp,
    const uint16_t* __restrict__ cache, long cache_bytes, const int* __restrict__ page_table,
    const int* __restrict__ logical, uint16_t* __restrict__ part_b, float* __restrict__ part_ml, int Q,
    int H, int S, int page, int pages_per_seq, int nsplit, int chunk, float scale_log2) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    int* s_rows = (int*)(smem + kRows32Off);
    unsigned long long* s_mask = (unsigned long long*)(smem + kMask32Off);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // work item lin = (query, head group, split), dealt to the 8 XCDs in
    // contiguous chunks (workgroup b runs on XCD b % 8): the splits of a
    // query share an XCD, so its q rows come from HBM once and its partials
    // are written and merged within one L2
    const int hgroups = H / 128;
    const int per = gridDim.x / 8;
    const int lin = (blockIdx.x % 8) * per + blockIdx.x / 8;
    const int sp = lin % nsplit;
    const int qh = lin / nsplit;
    const int hg = qh % hgroups, qi = qh / hgroups;
    if (qi >= Q) return;  // padding of the grid to a multiple of 8
    const int t0 = sp * chunk;
    const int len = max(0, min(S, t0 + chunk) - t0);
    const int g = lane >> 4, c16 = lane & 15;
    const int hbase = 128 * hg + 16 * wave;  // this wave's first head

    // Prologue, ordered so the q loads overlap the two dependent loads of
    // the page-table translation: logical indices, then page-table entries,
    // then q (18 loads per lane), then wait for all but the q loads.  The
    // q loads are waited for (by the compiler) at tile 0's first S step.
    // A token is valid when its logical index lies in [0, pages_per_seq *
    // page), its page id is >= 0 and its row inside the cache; an invalid
    // one (e.g. the -1 padding of a sequence shorter than the selection)
    // reads no page-table entry, loads a zero row and scores -inf.
    int li[kRowsPer8], pg[kRowsPer8];
    {
        const int* lg = logical + (size_t)qi * S + t0;
        const int* pt = page_table + (size_t)qi * pages_per_seq;
        const long seq = (long)pages_per_seq * page;
#pragma unroll
        for (int k = 0; k < kRowsPer8; k++) li[k] = tid + 512 * k < len ? lg[tid + 512 * k] : -1;
#pragma unroll
        for (int k = 0; k < kRowsPer8; k++) {
            const bool ok = li[k] >= 0 && li[k] < seq;
            if (!ok) li[k] = -1;
            pg[k] = ok ? pt[li[k] / page] : -1;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // q of head hbase + c16 as B fragments: K-step ks = 32 dims, group g holds 8
    u32x4 qf[18];
    {
        const size_t hrow = (size_t)qi * H + hbase + c16;
        const uint16_t* qnr = qn + hrow * kDc;
        const uint16_t* qpr = qp + hrow * kDp;
#pragma unroll
        for (int ks = 0; ks < 16; ks++) qf[ks] = *(const u32x4*)(qnr + 32 * ks + 8 * g);
#pragma unroll
        for (int ks = 0; ks < 2; ks++) qf[16 + ks] = *(const u32x4*)(qpr + 32 * ks + 8 * g);
    }
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<18>();  // every page-table entry has arrived
    {
        const long cache_rows = cache_bytes / kRowBytes;
#pragma unroll
        for (int k = 0; k < kRowsPer8; k++) {
            const long row = (long)pg[k] * page + (li[k] >= 0 ? li[k] % page : 0);
            const bool ok = li[k] >= 0 && pg[k] >= 0 && row < cache_rows;
            if (tid + 512 * k < len) s_rows[tid + 512 * k] = ok ? (int)row : -1;
            // validity of split tokens 64(8k + w) .. +63 (none past len)
            const unsigned long long m = __ballot(ok);
            if (lane == 0) s_mask[8 * k + wave] = m;
        }
    }
    lds_barrier();  // s_rows, s_mask visible (the q loads stay in flight)

    const __amdgpu_buffer_rsrc_t rc = make_rsrc(cache, cache_bytes);
    // DMA: block b of a tile is filled by one instruction, lane l taking
    // token 16 (b / 18) + (l >> 2), chunk 4 (b % 18) + ((l & 3) ^ ((l >> 3) & 3));
    // the chunk-group offset goes in soffset (an instruction immediate would
    // also move the LDS address)
    const uint32_t lane_c16 = 16u * (uint32_t)((lane & 3) ^ ((lane >> 3) & 3));
    using RowAddr = std::conditional_t<WIDE, const uint8_t*, uint32_t>;
    auto row_vo = [&](int tok) __attribute__((always_inline)) -> RowAddr {
        if constexpr (WIDE) {
            const uint8_t* a = (const uint8_t*)g_dsa_zero_row + lane_c16;
            if (tok < len) {
                const long r = s_rows[tok];
                const long off = r * kRowBytes + lane_c16;
                if (r >= 0 && off < cache_bytes) a = (const uint8_t*)cache + off;
            }
            return a;
        } else {
            uint32_t vo = kOobDsa;
            if (tok < len) {
                const long r = s_rows[tok];
                const long off = r * kRowBytes + lane_c16;
                if (r >= 0 && off < cache_bytes) vo = (uint32_t)off;
            }
            return vo;
        }
    };
    // a tile's 36 blocks: wave w issues b = w + 8n, n < 5 for waves 0-3 and
    // n < 4 for waves 4-7
    auto issue_blk = [&](int st, RowAddr vo0, RowAddr vo1, int n) __attribute__((always_inline)) {
        const int b = wave + 8 * n;
        const int tg = b >= 18 ? 1 : 0;
        if constexpr (WIDE)
            __builtin_amdgcn_global_load_lds((gptr_t)((tg ? vo1 : vo0) + 64 * (b - 18 * tg)),
                                             (lds_ptr_t)(smem + st * kStage32 + b * 1024), 16, 0, 0);
        else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rc, (lds_ptr_t)(smem + st * kStage32 + b * 1024), 16, tg ? vo1 : vo0, 64 * (b - 18 * tg), 0, 0);
    };
    const bool five = wave < 4;  // uniform: this wave issues a fifth block per tile

    f32x4 o[32];  // dims 16mt + 4g + i, head hbase + c16
#pragma unroll
    for (int i = 0; i < 32; i++) o[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_lane = 0.0f;
    const int ntiles = (len + kT32 - 1) / kT32;

    const int koff = tile32_off(c16, g);  // S fragment (token tile tt, K-step ks): + 1024 (18 tt + ks)
    int vlo[2];                           // V^T read, dim tile mt: vlo[mt & 1] + 1024 (mt >> 1)
#pragma unroll
    for (int e = 0; e < 2; e++)
        vlo[e] = tile32_off(4 * g + (c16 >> 2), 2 * e + ((c16 >> 1) & 1)) + 8 * (c16 & 1);

    // The two waves of a SIMD (w and w + 4) run half a tile apart: waves
    // 0-3 pass the tile barrier at the start of a tile, waves 4-7 between
    // their S^T and PV phases, so one wave's S^T fragment reads, softmax and
    // barrier wait run under the other's PV MFMAs.  Barrier n is where waves
    // 0-3 start tile n and waves 4-7 finish S^T of tile n-1, so tile n's
    // stage is read between barriers n and n+2; the DMA of tile n+2 goes out
    // after barrier n into the stage of tile n-2 (read until barrier n), and
    // every wave waits for its blocks of tile n before barrier n.  Each wave
    // passes ntiles + 1 barriers.
    const bool lag = wave >= 4;  // uniform
    // prologue: tiles 0 and 1 (tiles past the end read zeros into their stage)
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const RowAddr a = row_vo(kT32 * i + (lane >> 2)), b = row_vo(kT32 * i + 16 + (lane >> 2));
#pragma unroll
        for (int n = 0; n < 4; n++) issue_blk(i, a, b, n);
        if (five) issue_blk(i, a, b, 4);
    }
    // this wave's blocks of the older of its two tiles in flight have landed
    auto wait_older = [&]() __attribute__((always_inline)) {
        if (five) wait_vmcnt<5>();
        else wait_vmcnt<4>();
    };

    // S^T (2 token tiles x 16 heads) of the tile in stage soff, 18 K-steps,
    // fragment reads kPre steps ahead; with ISSUE, one block of tile tn goes
    // out per step for the first 5
    auto s_phase = [&](auto issuec, uint32_t soff, int stn, RowAddr nvo0, RowAddr nvo1,
                       f32x4 (&sacc)[2]) __attribute__((always_inline)) {
        constexpr bool ISSUE = decltype(issuec)::value;
        const uint8_t* kb = smem + soff;
        constexpr int kPre = 2;
        u32x4 a[18][2];
#pragma unroll
        for (int ks = 0; ks < kPre; ks++)
#pragma unroll
            for (int tt = 0; tt < 2; tt++) a[ks][tt] = *(const u32x4*)(kb + koff + 1024 * (18 * tt + ks));
        static_for<18>([&](auto ksc) __attribute__((always_inline)) {
            constexpr int ks = decltype(ksc)::value;
            if constexpr (ks + kPre < 18)
#pragma unroll
                for (int tt = 0; tt < 2; tt++)
                    a[ks + kPre][tt] = *(const u32x4*)(kb + koff + 1024 * (18 * tt + ks + kPre));
#pragma unroll
            for (int tt = 0; tt < 2; tt++)
                sacc[tt] = mfma_bf16(a[ks][tt], qf[ks], ks == 0 ? (f32x4){0.f, 0.f, 0.f, 0.f} : sacc[tt]);
            if constexpr (ISSUE && ks < 4) issue_blk(stn, nvo0, nvo1, ks);
            if constexpr (ISSUE && ks == 4)
                if (five) issue_blk(stn, nvo0, nvo1, 4);
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    // online softmax of tile t's scores; returns P^T as the PV B operand.
    // Lane: head c16, tokens 16tt + 4g + i of the tile; an invalid token (or
    // one past the split) scores -inf
    auto softmax = [&](int t, const f32x4 (&sacc)[2]) __attribute__((always_inline)) -> u32x4 {
        float sv[2][4], tm = -INFINITY;
        const uint32_t vmask = (uint32_t)(s_mask[t >> 1] >> (32 * (t & 1) + 4 * g));
#pragma unroll
        for (int tt = 0; tt < 2; tt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sv[tt][i] = (vmask >> (16 * tt + i)) & 1u ? sacc[tt][i] * scale_log2 : -INFINITY;
                tm = fmaxf(tm, sv[tt][i]);
            }
        tm = xor32_max(xor16_max(tm));
        // uniform: no valid token so far (validity is per token, the same
        // for every head)
        if (m_run == -INFINITY) {
            m_run = tm;
        } else if (__ballot(tm > m_run + 8.0f)) {
            // rare: rescale O and l to a new running max
            const float m_new = fmaxf(m_run, tm);
            const float corr = exp2f(m_run - m_new);
            l_lane *= corr;
            m_run = m_new;
#pragma unroll
            for (int mt = 0; mt < 32; mt++) o[mt] *= corr;
        }
        float p[2][4];
        // with no valid token yet every score is -inf: subtract 0, not -inf
        const float m_use = m_run == -INFINITY ? 0.0f : m_run;
#pragma unroll
        for (int tt = 0; tt < 2; tt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                p[tt][i] = __builtin_amdgcn_exp2f(sv[tt][i] - m_use);  // 0 for a masked -inf score
                l_lane += p[tt][i];
            }
        return (u32x4){pack_bf16x2(p[0][0], p[0][1]), pack_bf16x2(p[0][2], p[0][3]),
                       pack_bf16x2(p[1][0], p[1][1]), pack_bf16x2(p[1][2], p[1][3])};
    };
    // O^T += V^T . P^T over the tile in stage soff; with ISSUE, one block of
    // tile tn goes out after each of the first 5 dim tiles
    auto pv_phase = [&](auto issuec, uint32_t soff, int stn, RowAddr nvo0, RowAddr nvo1,
                        const u32x4& pb) __attribute__((always_inline)) {
        constexpr bool ISSUE = decltype(issuec)::value;
        const uint8_t* kb = smem + soff;
        auto vfrag = [&](int mt) __attribute__((always_inline)) {
            const uint8_t* p = kb + vlo[mt & 1] + 1024 * (mt >> 1);
            const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)p);
            const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(p + 18 * 1024));
            const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
            return (u32x4){l2[0], l2[1], h2[0], h2[1]};
        };
        constexpr int kPreV = 6;
        u32x4 va[32];
#pragma unroll
        for (int mt = 0; mt < kPreV; mt++) va[mt] = vfrag(mt);
        static_for<32>([&](auto mtc) __attribute__((always_inline)) {
            constexpr int mt = decltype(mtc)::value;
            if constexpr (mt + kPreV < 32) va[mt + kPreV] = vfrag(mt + kPreV);
            o[mt] = mfma_bf16(va[mt], pb, o[mt]);
            if constexpr (ISSUE && mt < 4) issue_blk(stn, nvo0, nvo1, mt);
            if constexpr (ISSUE && mt == 4)
                if (five) issue_blk(stn, nvo0, nvo1, 4);
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    auto stage_of = [](int t) __attribute__((always_inline)) -> uint32_t {
        uint32_t soff = (uint32_t)(t % kRing32) * kStage32;
        asm volatile("" : "+s"(soff));
        return soff;
    };
    using on = std::integral_constant<bool, true>;
    using off = std::integral_constant<bool, false>;

    if (!lag) {
        // the q loads (older than the tile DMA) have landed: without this the
        // compiler waits for every load in flight, tile 1's included
        wait_older();
        for (int t = 0; t < ntiles; t++) {
            const int tn = t + 2;
            const RowAddr nvo0 = row_vo(kT32 * tn + (lane >> 2)), nvo1 = row_vo(kT32 * tn + 16 + (lane >> 2));
            wait_older();    // tile t landed (this wave's part); tile t+1 may stay in flight
            bare_barrier();  // barrier t
            const uint32_t soff = stage_of(t);
            f32x4 sacc[2];
            s_phase(on{}, soff, tn % kRing32, nvo0, nvo1, sacc);
            const u32x4 pb = softmax(t, sacc);
            pv_phase(off{}, soff, 0, nvo0, nvo1, pb);
        }
        bare_barrier();  // barrier ntiles
    } else {
        wait_older();
        bare_barrier();  // barrier 0
        {
            const RowAddr a = row_vo(kT32 * 2 + (lane >> 2)), b = row_vo(kT32 * 2 + 16 + (lane >> 2));
#pragma unroll
            for (int n = 0; n < 4; n++) issue_blk(2, a, b, n);
            if (five) issue_blk(2, a, b, 4);
        }
        for (int t = 0; t < ntiles; t++) {
            const int tn = t + 3;
            const RowAddr nvo0 = row_vo(kT32 * tn + (lane >> 2)), nvo1 = row_vo(kT32 * tn + 16 + (lane >> 2));
            const uint32_t soff = stage_of(t);
            f32x4 sacc[2];
            s_phase(off{}, soff, 0, nvo0, nvo1, sacc);
            const u32x4 pb = softmax(t, sacc);
            wait_older();    // tile t+1 landed (this wave's part); tile t+2 may stay in flight
            bare_barrier();  // barrier t+1
            pv_phase(on{}, soff, tn % kRing32, nvo0, nvo1, pb);
        }
    }
    wait_vmcnt<0>();  // the trailing (out-of-range) tile loads

    // the split's partial, bf16 in the accumulator order (512 contiguous
    // bytes per store), and (max, sum) per head
    const size_t prow0 = ((size_t)qi * nsplit + sp) * H + hbase;
    uint16_t* pb_base = part_b + prow0 * kDc + (size_t)lane * 4;
#pragma unroll
    for (int mt = 0; mt < 32; mt++)
        *(u32x2*)(pb_base + 256 * mt) =
            (u32x2){pack_bf16x2(o[mt][0], o[mt][1]), pack_bf16x2(o[mt][2], o[mt][3])};
    const float l = xor32_sum(xor16_sum(l_lane));
    if (g == 0) *(float2*)(part_ml + 2 * (prow0 + c16)) = make_float2(m_run, l);
}

#define AMDMOE_DSA_SPLIT_KERNEL(NAME, W)                                                             \
    __global__ __launch_bounds__(512, 1) void NAME(                                                   \
        const uint16_t* __restrict__ qn, const uint16_t* __restrict__ qp,                             \
        const uint16_t* __restrict__ cache, long cache_bytes, const int* __restrict__ page_table,     \
        const int* __restrict__ logical, uint16_t* __restrict__ part_b, float* __restrict__ part_ml,  \
        int Q, int H, int S, int page, int pages_per_seq, int nsplit, int chunk, float scale_log2) {  \
        dsa_split_body<W>(qn, qp, cache, cache_bytes, page_table, logical, part_b, part_ml, Q, H, S, \
                           page, pages_per_seq, nsplit, chunk, scale_log2);                           \
    }
AMDMOE_DSA_SPLIT_KERNEL(dsa_split_kernel, false)
AMDMOE_DSA_SPLIT_KERNEL(dsa_split_wide_kernel, true)
#undef AMDMOE_DSA_SPLIT_KERNEL

// Combines the splits of dsa_split_kernel: per (query, head), m = max of
// the split maxima, weights c_j = 2^(m_j - m), out = (sum c_j O_j) /
// (sum c_j l_j), bf16.  Workgroup = one query x 16 heads (one partial block),
// wave w = dim tiles 8w..8w+7 in the block's accumulator order: every load
// is 512 bytes contiguous, and lane (g, c) holds dims 16mt + 4g + i of head c.
// Splits are read four at a time, every load of the four in flight at once
// (one round trip for up to four splits); a later group whose maximum is
// higher rescales the sums so far by 2^(m_old - m_new).
__global__ __launch_bounds__(256) void dsa_merge_kernel(const uint16_t* __restrict__ part_b,
                                                        const float* __restrict__ part_ml,
                                                        uint16_t* __restrict__ out, int Q,
                                                        int H, int nsplit) {
    // same XCD dealing as dsa_split_kernel: a query's blocks on the XCD
    // whose L2 holds its partials
    const int h16 = H / 16;
    const int per = gridDim.x / 8;
    const int lin = (blockIdx.x % 8) * per + blockIdx.x / 8;
    const int qi = lin / h16, hb = lin % h16;
    if (qi >= Q) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int h = 16 * hb + c16;
    constexpr int kGroup = 4;
    f32x4 acc[8];
#pragma unroll
    for (int k = 0; k < 8; k++) acc[k] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, L = 0.0f;
    for (int j0 = 0; j0 < nsplit; j0 += kGroup) {
        float2 ml[kGroup];
        u32x2 pv[kGroup][8];
#pragma unroll
        for (int u = 0; u < kGroup; u++) {
            const int j = min(j0 + u, nsplit - 1);  // in bounds; splits past the end get weight 0
            const size_t blk = ((size_t)qi * nsplit + j) * H + 16 * hb;  // first row of the block
            ml[u] = *(const float2*)(part_ml + 2 * (blk + c16));
            const u32x2* po = (const u32x2*)(part_b + blk * kDc) + 64 * 8 * wave + lane;
#pragma unroll
            for (int k = 0; k < 8; k++) pv[u][k] = po[64 * k];
        }
        float mg = m;
#pragma unroll
        for (int u = 0; u < kGroup; u++)
            if (j0 + u < nsplit) mg = fmaxf(mg, ml[u].x);
        if (mg == -INFINITY) continue;  // no valid position so far: the sums stay 0
        // the sums so far are 0 while m = -inf
        const float r = m == -INFINITY ? 0.0f : exp2f(m - mg);
        L *= r;
#pragma unroll
        for (int k = 0; k < 8; k++) acc[k] *= r;
        m = mg;
#pragma unroll
        for (int u = 0; u < kGroup; u++) {
            const float c = j0 + u < nsplit && ml[u].x != -INFINITY ? exp2f(ml[u].x - m) : 0.0f;
            L += c * ml[u].y;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                acc[k][0] += c * __uint_as_float(pv[u][k][0] << 16);
                acc[k][1] += c * __uint_as_float(pv[u][k][0] & 0xffff0000u);
                acc[k][2] += c * __uint_as_float(pv[u][k][1] << 16);
                acc[k][3] += c * __uint_as_float(pv[u][k][1] & 0xffff0000u);
            }
        }
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    uint16_t* orow = out + ((size_t)qi * H + h) * kDc + 4 * g;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int mt = 8 * wave + k;
        const u32x2 pk = {pack_bf16x2(acc[k][0] * inv, acc[k][1] * inv),
                          pack_bf16x2(acc[k][2] * inv, acc[k][3] * inv)};
        *(u32x2*)(orow + 16 * mt) = pk;
    }
}

// Splits per query for dsa_split_kernel: enough workgroups to cover the
// chip (256 CUs), at most 2048 tokens per split, at least 32.
static int dsa_nsplit(int Q, int H, int S) {
    const long wg = (long)Q * (H / 128);
    int ns = (int)std::min<long>((256 + wg - 1) / wg, (S + kT32 - 1) / kT32);
    return std::max(ns, (S + kMaxChunk - 1) / kMaxChunk);
}

size_t dsa_paged_scratch_bytes(int Q, int H, int S) {
    if (Q <= 0 || H % 128 != 0 || S < 1) return 0;  // the kernels without splits
    const size_t rows = (size_t)Q * dsa_nsplit(Q, H, S) * H;
    // the bf16 partials, (m, l)
    return align_up(rows * kDc * 2, 256) + align_up(rows * 8, 256);
}

int launch_dsa_bf16_paged(const uint16_t* qn, const uint16_t* qp, const uint16_t* cache,
                          long cache_tokens, const int* page_table, const int* logical,
                          uint16_t* out, int Q, int H, int Dc, int Dp, int S, int page,
                          int pages_per_seq, void* scratch, size_t scratch_bytes, hipStream_t st) {
    AMDMOE_CHECK_ARG(Dc == kDc && Dp == kDp, "dsa_decode_bf16_paged: needs Dc=512, Dp=64 (got %d, %d)", Dc, Dp);
    AMDMOE_CHECK_ARG(H % 32 == 0 && H > 0, "dsa_decode_bf16_paged: H=%d not a multiple of 32", H);
    // the split kernel (H a multiple of 128) takes any S up to kMaxSplitS in
    // more splits; the others hold a query's rows in LDS
    AMDMOE_CHECK_ARG(S >= 1 && S <= (H % 128 == 0 ? kMaxSplitS : kMaxS),
                     "dsa_decode_bf16_paged: S=%d outside [1, %d] for H=%d", S,
                     H % 128 == 0 ? kMaxSplitS : kMaxS, H);
    AMDMOE_CHECK_ARG(page >= 1 && pages_per_seq >= 1, "dsa_decode_bf16_paged: bad paging");
    // caches beyond 4 GiB: the split kernel addresses them with 64-bit
    // pointers; the kernels for H not a multiple of 128 use 32-bit offsets
    AMDMOE_CHECK_ARG(cache_tokens >= 1 && (cache_tokens * kRowBytes <= kMaxCacheBytes || H % 128 == 0),
                     "dsa_decode_bf16_paged: cache of %ld tokens outside (0, 4 GiB) (larger caches need H a "
                     "multiple of 128)", cache_tokens);
    const bool wide = cache_tokens * kRowBytes > kMaxCacheBytes;
    if (Q == 0) return AMDMOE_OK;
    const float scale_log2 = 1.0f / sqrtf((float)(Dc + Dp)) * 1.4426950408889634f;
    if (H % 128 == 0) {
        const int ns = dsa_nsplit(Q, H, S);
        const int chunk = (int)ceil_div(ceil_div(S, ns), kT32) * kT32;
        const size_t need = dsa_paged_scratch_bytes(Q, H, S);
        AMDMOE_CHECK_ARG(scratch != nullptr && scratch_bytes >= need,
                         "dsa_decode_bf16_paged: scratch of %zu bytes, %zu needed", scratch_bytes, need);
        const long grid = ceil_div((long)Q * (H / 128) * ns, 8) * 8;
        AMDMOE_CHECK_ARG(grid < (1L << 31), "dsa_decode_bf16_paged: grid too large");
        uint16_t* part_b = (uint16_t*)scratch;
        float* part_ml = (float*)((uint8_t*)scratch + align_up((size_t)Q * ns * H * kDc * 2, 256));
        auto split = wide ? dsa_split_wide_kernel : dsa_split_kernel;
        const int rc = ensure_dynamic_lds((const void*)split, kDsaSplitLds);
        if (rc != AMDMOE_OK) return rc;
        hipLaunchKernelGGL(split, dim3((unsigned)grid), dim3(512), kDsaSplitLds, st, qn, qp, cache,
                           cache_tokens * kRowBytes, page_table, logical, part_b, part_ml, Q, H, S, page,
                           pages_per_seq, ns, chunk, scale_log2);
        AMDMOE_LAUNCH_CHECK();
        hipLaunchKernelGGL(dsa_merge_kernel, dim3((unsigned)(ceil_div((long)Q * (H / 16), 8) * 8)),
                           dim3(256), 0, st, (const uint16_t*)part_b, (const float*)part_ml, out, Q, H, ns);
        AMDMOE_LAUNCH_CHECK();
        return AMDMOE_OK;
    }
    // H not a multiple of 128: one workgroup per (query, 32 heads)
    const int nblk = Q * (H / 32);
    const int grid = (nblk + 7) / 8 * 8;  // padded for the XCD remap; padding blocks exit
    if (S <= kMaxS64) {
        const int rc = ensure_dynamic_lds((const void*)dsa_bf16_paged64_kernel, kDsa64Lds);
        if (rc != AMDMOE_OK) return rc;
        hipLaunchKernelGGL(dsa_bf16_paged64_kernel, dim3(grid), dim3(256), kDsa64Lds, st, qn, qp,
                           cache, cache_tokens * kRowBytes, page_table, logical, out, Q, H, S, page,
                           pages_per_seq, scale_log2);
        AMDMOE_LAUNCH_CHECK();
        return AMDMOE_OK;
    }
    {
        const int rc = ensure_dynamic_lds((const void*)dsa_bf16_paged_kernel, kDsaLds);
        if (rc != AMDMOE_OK) return rc;
    }
    hipLaunchKernelGGL(dsa_bf16_paged_kernel, dim3(grid), dim3(256), kDsaLds, st, qn, qp, cache,
                       cache_tokens * kRowBytes, page_table, logical, out, Q, H, S, page,
                       pages_per_seq, scale_log2);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

}  // namespace amdmoe
