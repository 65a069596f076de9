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
//   V^T fragments come from a 4-token-interleaved copy of the K_c part, so
//   each MFMA operand is two 8-byte LDS reads.  The two token halves merge
//   through LDS at the end.
#include "internal.hpp"

#include <float.h>

namespace amdmoe {

// ---------------------------------------------------------------- fp32
__global__ __launch_bounds__(64) void dsa_f32_kernel(const float* __restrict__ qn,
                                                     const float* __restrict__ qp,
                                                     const float* __restrict__ kc,
                                                     const float* __restrict__ kp,
                                                     const float* __restrict__ v,
                                                     const int* __restrict__ idx,
                                                     float* __restrict__ out, int H, int Dc,
                                                     int Dp, int S) {
    extern __shared__ float s_score[];  // [S]
    const int qh = blockIdx.x;
    const int q = qh / H;
    const int lane = threadIdx.x;
    const float scale = 1.0f / sqrtf((float)(Dc + Dp));
    const float* qnr = qn + (size_t)qh * Dc;
    const float* qpr = qp + (size_t)qh * Dp;
    const int* ir = idx + (size_t)q * S;
    for (int s = lane; s < S; s += 64) {
        const long row = ir[s];
        const float* kcr = kc + row * Dc;
        const float* kpr = kp + row * Dp;
        float sc = 0.0f, sp = 0.0f;
        for (int d = 0; d < Dc; d++) sc = __fadd_rn(sc, __fmul_rn(qnr[d], kcr[d]));
        for (int d = 0; d < Dp; d++) sp = __fadd_rn(sp, __fmul_rn(qpr[d], kpr[d]));
        s_score[s] = __fmul_rn(__fadd_rn(sc, sp), scale);
    }
    __syncthreads();
    float mx = -FLT_MAX;
    for (int s = lane; s < S; s += 64) mx = fmaxf(mx, s_score[s]);
    mx = wave_max(mx);
    for (int s = lane; s < S; s += 64) s_score[s] = expf(s_score[s] - mx);
    __syncthreads();
    float tot = 0.0f;
    if (lane == 0)
        for (int s = 0; s < S; s++) tot = __fadd_rn(tot, s_score[s]);
    tot = __shfl(tot, 0, 64);
    for (int s = lane; s < S; s += 64) s_score[s] = __fdiv_rn(s_score[s], tot);
    __syncthreads();
    for (int d = lane; d < Dc; d += 64) {
        float acc = 0.0f;
        for (int s = 0; s < S; s++) acc = __fadd_rn(acc, __fmul_rn(s_score[s], v[(long)ir[s] * Dc + d]));
        out[(size_t)qh * Dc + d] = acc;
    }
}

int launch_dsa_f32(const float* qn, const float* qp, const float* kc, const float* kp,
                   const float* v, const int* idx, float* out, int Q, int H, int Dc, int Dp, int S,
                   int N, hipStream_t st) {
    size_t lds = sizeof(float) * (size_t)S;
    AMDMOE_CHECK_ARG(lds <= 64 * 1024, "dsa_forward: S=%d exceeds 16384", S);
    if (Q == 0 || H == 0) return AMDMOE_OK;
    hipLaunchKernelGGL(dsa_f32_kernel, dim3(Q * H), dim3(64), lds, st, qn, qp, kc, kp, v, idx, out,
                       H, Dc, Dp, S);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

// ---------------------------------------------------------------- bf16 paged
constexpr int kDc = 512, kDp = 64, kDt = 576;
constexpr int kRowBytes = kDt * 2;            // 1152
constexpr int kKPitch = kRowBytes + 16;       // 1168: conflict-free 16-row b128 reads
constexpr int kTileTok = 32;
constexpr int kKBuf = kTileTok * kKPitch;     // 37376
constexpr int kVBuf = (kTileTok / 4) * kDc * 8;  // 32768: [quad][d][4 tokens] bf16
constexpr int kBuf = kKBuf + kVBuf;           // 70144
constexpr int kMaxS = 4096;
constexpr int kDsaLds = 2 * kBuf + kMaxS * 4;  // 156672

__global__ __launch_bounds__(256, 1) void dsa_bf16_paged_kernel(
    const uint16_t* __restrict__ qn, const uint16_t* __restrict__ qp,
    const uint16_t* __restrict__ cache, const int* __restrict__ page_table,
    const int* __restrict__ logical, uint16_t* __restrict__ out, int H, int S, int page,
    int pages_per_seq, float scale) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    int* s_rows = (int*)(smem + 2 * kBuf);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int hgroups = H / 32;
    const int qi = blockIdx.x / hgroups;
    const int h0 = (blockIdx.x % hgroups) * 32;
    const int hg = wave & 1, th = wave >> 1;
    const int g = lane >> 4, c16 = lane & 15;
    const int my_head = h0 + 16 * hg + c16;

    // page-table translation of all of this query's indices
    for (int s = tid; s < S; s += 256) {
        int i = logical[(size_t)qi * S + s];
        s_rows[s] = page_table[(size_t)qi * pages_per_seq + i / page] * page + i % page;
    }

    // q of my head as MFMA B fragments: 18 K-steps of 32 dims, lane group g
    // holds dims 32ks + 8g .. +7.
    u32x4 qf[18];
    {
        const uint16_t* qnr = qn + ((size_t)qi * H + my_head) * kDc;
        const uint16_t* qpr = qp + ((size_t)qi * H + my_head) * kDp;
        for (int ks = 0; ks < 16; ks++) qf[ks] = *(const u32x4*)(qnr + 32 * ks + 8 * g);
        for (int ks = 0; ks < 2; ks++) qf[16 + ks] = *(const u32x4*)(qpr + 32 * ks + 8 * g);
    }
    __syncthreads();

    // load assignment per 64-token step: Kc units (buffer b, quad, dchunk)
    // = 2*8*64 = 1024 -> 4 per thread (4 tokens x 16 B each); Kp chunks
    // 2*32*8 = 512 -> 2 per thread.
    const uint8_t* cbase = (const uint8_t*)cache;
    u32x4 rk[4][4], rp[2];
    auto tok_row = [&](int s) -> long { return s < S ? (long)s_rows[s] : -1L; };
    const u32x4 zero4 = {0u, 0u, 0u, 0u};
    auto gload = [&](int step) {
        const int tbase = step * 64;
        for (int j = 0; j < 4; j++) {
            int u = tid + 256 * j;
            int b = u >> 9, quad = (u >> 6) & 7, dch = u & 63;
            for (int t4 = 0; t4 < 4; t4++) {
                long r = tok_row(tbase + 32 * b + 4 * quad + t4);
                rk[j][t4] = r >= 0 ? *(const u32x4*)(cbase + r * kRowBytes + dch * 16) : zero4;
            }
        }
        for (int j = 0; j < 2; j++) {
            int u = tid + 256 * j;
            int b = u >> 8, t = (u >> 3) & 31, dch = u & 7;
            long r = tok_row(tbase + 32 * b + t);
            rp[j] = r >= 0 ? *(const u32x4*)(cbase + r * kRowBytes + 1024 + dch * 16) : zero4;
        }
    };
    auto sstore = [&]() {
        for (int j = 0; j < 4; j++) {
            int u = tid + 256 * j;
            int b = u >> 9, quad = (u >> 6) & 7, dch = u & 63;
            uint8_t* kb = smem + b * kBuf;
            for (int t4 = 0; t4 < 4; t4++)
                *(u32x4*)(kb + (4 * quad + t4) * kKPitch + dch * 16) = rk[j][t4];
            // interleave: for each of the 8 dims, the 4 tokens' values
            uint8_t* vb = kb + kKBuf + ((size_t)quad * kDc + dch * 8) * 8;
            for (int dd = 0; dd < 8; dd++) {
                const int w = dd >> 1, sh = (dd & 1) * 16;
                uint32_t v0 = (rk[j][0][w] >> sh) & 0xffffu, v1 = (rk[j][1][w] >> sh) & 0xffffu;
                uint32_t v2 = (rk[j][2][w] >> sh) & 0xffffu, v3 = (rk[j][3][w] >> sh) & 0xffffu;
                u32x2 pk = {v0 | (v1 << 16), v2 | (v3 << 16)};
                *(u32x2*)(vb + dd * 8) = pk;
            }
        }
        for (int j = 0; j < 2; j++) {
            int u = tid + 256 * j;
            int b = u >> 8, t = (u >> 3) & 31, dch = u & 7;
            *(u32x4*)(smem + b * kBuf + t * kKPitch + 1024 + dch * 16) = rp[j];
        }
    };

    f32x4 o[32];
    for (int i = 0; i < 32; i++) o[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.0f;
    const int nsteps = (S + 63) / 64;
    const float kLog2e = 1.4426950408889634f;

    gload(0);
    for (int step = 0; step < nsteps; step++) {
        sstore();
        __syncthreads();
        if (step + 1 < nsteps) gload(step + 1);
        const uint8_t* kb = smem + th * kBuf;
        const int tok0 = step * 64 + 32 * th;
        // S^T tiles: tokens 0-15 and 16-31 of this half
        f32x4 sacc[2] = {(f32x4){0.f, 0.f, 0.f, 0.f}, (f32x4){0.f, 0.f, 0.f, 0.f}};
        for (int ks = 0; ks < 18; ks++) {
            for (int mt = 0; mt < 2; mt++) {
                u32x4 a = *(const u32x4*)(kb + (16 * mt + c16) * kKPitch + (32 * ks + 8 * g) * 2);
                sacc[mt] = mfma_bf16(a, qf[ks], sacc[mt]);
            }
        }
        // lane: head c16, tokens 16*mt + 4g + i
        float sv[8];
        float tmax = -INFINITY;
        for (int mt = 0; mt < 2; mt++)
            for (int i = 0; i < 4; i++) {
                int tk = tok0 + 16 * mt + 4 * g + i;
                float s = tk < S ? sacc[mt][i] * scale : -INFINITY;
                sv[4 * mt + i] = s;
                tmax = fmaxf(tmax, s);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float m_new = fmaxf(m_run, tmax);
        const float corr = m_new == -INFINITY ? 1.0f : exp2f((m_run - m_new) * kLog2e);
        float psum = 0.0f;
        float pv[8];
        for (int j = 0; j < 8; j++) {
            pv[j] = m_new == -INFINITY ? 0.0f : exp2f((sv[j] - m_new) * kLog2e);
            psum += pv[j];
        }
        psum += __shfl_xor(psum, 16, 64);
        psum += __shfl_xor(psum, 32, 64);
        l_run = l_run * corr + psum;
        m_run = m_new;
        u32x4 pb = {pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3]),
                    pack_bf16x2(pv[4], pv[5]), pack_bf16x2(pv[6], pv[7])};
        const uint8_t* vb = kb + kKBuf;
        for (int mt = 0; mt < 32; mt++) {
            o[mt] *= corr;
            const int d = 16 * mt + c16;
            u32x2 lo = *(const u32x2*)(vb + ((size_t)g * kDc + d) * 8);
            u32x2 hi = *(const u32x2*)(vb + ((size_t)(4 + g) * kDc + d) * 8);
            u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
            o[mt] = mfma_bf16(a, pb, o[mt]);
        }
        __syncthreads();
    }

    // merge the two token halves: wave (hg, 1) hands (m, l, O) to wave (hg, 0)
    float* xch = (float*)smem;  // [hg][32 mt][4][64 lanes] + m/l
    float* xml = (float*)(smem + 2 * 32 * 4 * 64 * 4);
    if (th == 1) {
        for (int mt = 0; mt < 32; mt++)
            for (int i = 0; i < 4; i++) xch[((hg * 32 + mt) * 4 + i) * 64 + lane] = o[mt][i];
        xml[(hg * 2 + 0) * 64 + lane] = m_run;
        xml[(hg * 2 + 1) * 64 + lane] = l_run;
    }
    __syncthreads();
    if (th == 0) {
        const float m1 = xml[(hg * 2 + 0) * 64 + lane], l1 = xml[(hg * 2 + 1) * 64 + lane];
        const float m = fmaxf(m_run, m1);
        const float c0 = m_run == -INFINITY ? 0.0f : exp2f((m_run - m) * kLog2e);
        const float c1 = m1 == -INFINITY ? 0.0f : exp2f((m1 - m) * kLog2e);
        const float l = l_run * c0 + l1 * c1;
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        uint16_t* orow = out + ((size_t)qi * H + my_head) * kDc;
        for (int mt = 0; mt < 32; mt++) {
            float r[4];
            for (int i = 0; i < 4; i++)
                r[i] = (o[mt][i] * c0 + xch[((hg * 32 + mt) * 4 + i) * 64 + lane] * c1) * inv;
            u32x2 pk = {pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3])};
            *(u32x2*)(orow + 16 * mt + 4 * g) = pk;
        }
    }
}

int launch_dsa_bf16_paged(const uint16_t* qn, const uint16_t* qp, const uint16_t* cache,
                          const int* page_table, const int* logical, uint16_t* out, int Q, int H,
                          int Dc, int Dp, int S, int page, int pages_per_seq, hipStream_t st) {
    AMDMOE_CHECK_ARG(Dc == kDc && Dp == kDp, "dsa_decode_bf16_paged: needs Dc=512, Dp=64 (got %d, %d)", Dc, Dp);
    AMDMOE_CHECK_ARG(H % 32 == 0 && H > 0, "dsa_decode_bf16_paged: H=%d not a multiple of 32", H);
    AMDMOE_CHECK_ARG(S >= 1 && S <= kMaxS, "dsa_decode_bf16_paged: S=%d outside [1, %d]", S, kMaxS);
    AMDMOE_CHECK_ARG(page >= 1 && pages_per_seq >= 1, "dsa_decode_bf16_paged: bad paging");
    if (Q == 0) return AMDMOE_OK;
    static bool attr_set = false;
    if (!attr_set) {
        AMDMOE_HIP_TRY(hipFuncSetAttribute((const void*)dsa_bf16_paged_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kDsaLds));
        attr_set = true;
    }
    const float scale = 1.0f / sqrtf((float)(Dc + Dp));
    hipLaunchKernelGGL(dsa_bf16_paged_kernel, dim3(Q * (H / 32)), dim3(256), kDsaLds, st, qn, qp,
                       cache, page_table, logical, out, H, S, page, pages_per_seq, scale);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

}  // namespace amdmoe
