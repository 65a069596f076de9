// R3/R4/R5 -- single-launch grouped expert GEMMs on MFMA.
//
// Reference: the per-expert host loop of moe_forward
// (kernels/moe/naive_moe.cu:424-470): per expert, GEMM1 [cnt,D]x[2I,D]^T
// (tiled_gemm_bt_kernel, 246-280), swiglu_strided_kernel (297-310), GEMM2
// [cnt,I]x[D,I]^T, then scatter_kernel (315-335) with the routing weight.
//
// Here each GEMM is ONE launch over every expert.  The permutation kernel
// emits M-tiles {expert, first sorted row, rows}; a workgroup owns one
// (M-tile, N-tile) work item:
//   UP   (GEMM1 + SwiGLU): A rows are gathered straight from x through
//        sorted_token (no permuted copy of x exists); the B tile holds 128
//        gate rows n0.. and the 128 matching up rows I+n0.., so the epilogue
//        has g and u of the same column in the same lane and writes
//        act = silu(g)*u (fp8: requantised per 128 columns, the tile width).
//   DOWN (GEMM2 + combine weight): A = act rows (contiguous, sorted order),
//        B = 256 rows of W2; the epilogue multiplies by the routing weight of
//        the row's slot and writes the row to ypair[slot] (slot = t*K+k), from
//        where the combine kernel sums each token's rows in ascending expert
//        order -- the reference's scatter order, deterministic, no atomics.
// fp8 block scales (128x128 weights, 1x128 activations): a K-step is exactly
// one 128-wide K block, so each 16x16x128 MFMA yields a fresh partial that
// is folded into the fp32 accumulator as acc += partial * (s_a[row]*s_b).
//
// Tile: 128 rows x 256 weight rows x 128 bytes of K per step; 512 threads =
// 8 waves in a 4 (rows) x 2 (cols) grid, each wave 32 rows x 8 MFMA column
// tiles of 16.  Operands are staged global -> registers -> LDS (double
// buffered, one barrier per K-step); LDS rows are padded to 144 bytes so
// the 16 rows read by a quarter-wave fall in distinct banks.
//
// Work items are laid out M-tile-major (all N-tiles of an M-tile are
// consecutive) and dealt to XCDs in contiguous chunks (workgroup b runs on
// XCD b % 8), so the A rows of an M-tile and the weight tiles shared by
// the two M-tiles of an expert stay in one XCD's L2.
#include "internal.hpp"

namespace amdmoe {

constexpr int kBM = 128;
constexpr int kBRows = 256;
constexpr int kPitch = 144;
constexpr int kAStage = kBM * kPitch;
constexpr int kBStage = kBRows * kPitch;
constexpr int kStage = kAStage + kBStage + kBM * 4;
constexpr int kEpiPitch = 132;  // floats
constexpr int kGemmLds = (2 * kStage > kBM * kEpiPitch * 4) ? 2 * kStage : kBM * kEpiPitch * 4;

template <int DT> struct DtTraits;
template <> struct DtTraits<DT_F32> { static constexpr int es = 4; };
template <> struct DtTraits<DT_BF16> { static constexpr int es = 2; };
template <> struct DtTraits<DT_FP8> { static constexpr int es = 1; };

template <int DT, int MODE>
__global__ __launch_bounds__(512, 1) void grouped_gemm_kernel(GemmArgs g) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int ES = DtTraits<DT>::es;
    constexpr int KE = 128 / ES;  // elements per K-step
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // ---- work item (XCD-chunked) ----
    const int W = (*g.num_tiles) * g.n_tiles_n;
    const int per = (W + 7) >> 3;
    const int slot = blockIdx.x >> 3;
    if (slot >= per) return;
    const int w = (blockIdx.x & 7) * per + slot;
    if (w >= W) return;
    const int mt = w / g.n_tiles_n, nt = w - mt * g.n_tiles_n;
    const int4 tile = g.tiles[mt];
    const int e = tile.x, row0 = tile.y, rows = tile.z;
    const int nk = g.K / KE;
    const int kb_per_row = g.K / 128;  // fp8 scale blocks along K

    // ---- global source pointers of this thread ----
    const u32x4 zero4 = {0u, 0u, 0u, 0u};
    const uint8_t* asrc[2];
    int aoff[2];
    for (int j = 0; j < 2; j++) {
        int c = tid + 512 * j, r = c >> 3, ch = c & 7;
        aoff[j] = r * kPitch + ch * 16;
        asrc[j] = nullptr;
        if (r < rows) {
            long ar = MODE == MODE_UP ? (long)g.a_map[row0 + r] : (long)(row0 + r);
            asrc[j] = g.a + ar * g.a_row_bytes + ch * 16;
        }
    }
    const uint8_t* bexp = g.b + (size_t)e * g.b_expert_bytes;
    const uint8_t* bsrc[4];
    int boff[4];
    for (int j = 0; j < 4; j++) {
        int c = tid + 512 * j, r = c >> 3, ch = c & 7;
        boff[j] = kAStage + r * kPitch + ch * 16;
        long n;
        bool ok;
        if (MODE == MODE_UP) {
            int col = nt * 128 + (r & 127);
            ok = col < g.n_out;
            n = r < 128 ? col : (long)g.n_out + col;
        } else {
            n = (long)nt * 256 + r;
            ok = n < g.n_out;
        }
        bsrc[j] = ok ? bexp + n * g.b_row_bytes + ch * 16 : nullptr;
    }
    const float* assrc = nullptr;
    if (DT == DT_FP8 && tid < kBM && tid < rows) {
        long ar = MODE == MODE_UP ? (long)g.a_map[row0 + tid] : (long)(row0 + tid);
        assrc = g.a_scale + ar * kb_per_row;
    }

    u32x4 ra[2], rb[4];
    float ras = 0.0f;
    auto gload = [&](int kt) {
        const size_t off = (size_t)kt * 128;
        for (int j = 0; j < 2; j++) ra[j] = asrc[j] ? *(const u32x4*)(asrc[j] + off) : zero4;
        for (int j = 0; j < 4; j++) rb[j] = bsrc[j] ? *(const u32x4*)(bsrc[j] + off) : zero4;
        if (DT == DT_FP8) ras = assrc ? assrc[kt] : 0.0f;
    };
    auto sstore = [&](int st) {
        uint8_t* base = smem + st * kStage;
        for (int j = 0; j < 2; j++) *(u32x4*)(base + aoff[j]) = ra[j];
        for (int j = 0; j < 4; j++) *(u32x4*)(base + boff[j]) = rb[j];
        if (DT == DT_FP8 && tid < kBM) ((float*)(base + kAStage + kBStage))[tid] = ras;
    };

    // ---- wave geometry ----
    const int wr = wave & 3, wc = wave >> 2;
    const int q = lane >> 4, r16 = lane & 15;
    int bcol[8];
    for (int ct = 0; ct < 8; ct++)
        bcol[ct] = MODE == MODE_UP ? (ct < 4 ? 64 * wc + 16 * ct : 128 + 64 * wc + 16 * (ct - 4))
                                   : 128 * wc + 16 * ct;
    const bool rt_on[2] = {32 * wr < rows, 32 * wr + 16 < rows};

    // fp8 weight-scale rows of this wave
    const float* bs0 = nullptr;
    const float* bs1 = nullptr;
    if (DT == DT_FP8) {
        const float* bse = g.b_scale + (size_t)e * (g.b_rows / 128) * kb_per_row;
        if (MODE == MODE_UP) {
            bs0 = bse + (size_t)nt * kb_per_row;                       // gate block
            bs1 = bse + (size_t)(g.n_out / 128 + nt) * kb_per_row;     // up block
        } else {
            int nb = 2 * nt + wc;
            if (nb >= g.b_rows / 128) nb = g.b_rows / 128 - 1;         // masked columns
            bs0 = bs1 = bse + (size_t)nb * kb_per_row;
        }
    }

    f32x4 acc[2][8];
    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 8; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        if (kt + 1 < nk) gload(kt + 1);
        const uint8_t* base = smem + (kt & 1) * kStage;
        u32x4 alo[2], ahi[2];
        float sa[2][4];
        for (int rt = 0; rt < 2; rt++) {
            if (!rt_on[rt]) continue;
            const uint8_t* p = base + (32 * wr + 16 * rt + r16) * kPitch + 16 * q;
            alo[rt] = *(const u32x4*)p;
            ahi[rt] = *(const u32x4*)(p + 64);
            if (DT == DT_FP8) {
                f32x4 s4 = *(const f32x4*)(base + kAStage + kBStage + 4 * (32 * wr + 16 * rt + 4 * q));
                for (int i = 0; i < 4; i++) sa[rt][i] = s4[i];
            }
        }
        float sb0 = 0.f, sb1 = 0.f;
        if (DT == DT_FP8) { sb0 = bs0[kt]; sb1 = bs1[kt]; }
        for (int ct = 0; ct < 8; ct++) {
            const uint8_t* p = base + kAStage + (bcol[ct] + r16) * kPitch + 16 * q;
            u32x4 blo = *(const u32x4*)p, bhi = *(const u32x4*)(p + 64);
            for (int rt = 0; rt < 2; rt++) {
                if (!rt_on[rt]) continue;
                if (DT == DT_F32) {
                    for (int j = 0; j < 4; j++)
                        acc[rt][ct] = mfma_f32(__uint_as_float(alo[rt][j]), __uint_as_float(blo[j]), acc[rt][ct]);
                    for (int j = 0; j < 4; j++)
                        acc[rt][ct] = mfma_f32(__uint_as_float(ahi[rt][j]), __uint_as_float(bhi[j]), acc[rt][ct]);
                } else if (DT == DT_BF16) {
                    acc[rt][ct] = mfma_bf16(alo[rt], blo, acc[rt][ct]);
                    acc[rt][ct] = mfma_bf16(ahi[rt], bhi, acc[rt][ct]);
                } else {
                    i32x8 av, bv;
                    for (int j = 0; j < 4; j++) {
                        av[j] = (int)alo[rt][j]; av[4 + j] = (int)ahi[rt][j];
                        bv[j] = (int)blo[j];     bv[4 + j] = (int)bhi[j];
                    }
                    f32x4 pr = mfma_fp8(av, bv, (f32x4){0.f, 0.f, 0.f, 0.f});
                    const float sb = (MODE == MODE_UP && ct >= 4) ? sb1 : sb0;
                    for (int i = 0; i < 4; i++) acc[rt][ct][i] += pr[i] * (sa[rt][i] * sb);
                }
            }
        }
        if (kt + 1 < nk) sstore((kt + 1) & 1);
        __syncthreads();
    }

    // ---- epilogues (LDS staging for coalesced 16-byte stores) ----
    float* T = (float*)smem;
    const int er = tid >> 2, pp = tid & 3;  // output row, 32-column part
    if (MODE == MODE_UP) {
        for (int rt = 0; rt < 2; rt++) {
            if (!rt_on[rt]) continue;
            for (int j = 0; j < 4; j++)
                for (int i = 0; i < 4; i++) {
                    float gv = acc[rt][j][i], uv = acc[rt][j + 4][i];
                    float silu = gv / (1.0f + expf(-gv));
                    T[(32 * wr + 16 * rt + 4 * q + i) * kEpiPitch + 64 * wc + 16 * j + r16] = silu * uv;
                }
        }
        __syncthreads();
        const int col = nt * 128 + 32 * pp;
        const bool ok = er < rows && col < g.n_out;
        float v[32];
        for (int j = 0; j < 32; j++) v[j] = ok ? T[er * kEpiPitch + 32 * pp + j] : 0.0f;
        const size_t pos = (size_t)row0 + er;
        if (DT == DT_FP8) {
            float amax = 0.0f;
            for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
            amax = fmaxf(amax, __shfl_xor(amax, 1, kWave));
            amax = fmaxf(amax, __shfl_xor(amax, 2, kWave));
            const float s = amax > 0.0f ? __fdiv_rn(amax, 448.0f) : 1.0f;
            if (ok) {
                u32x4 o0, o1;
                for (int k = 0; k < 4; k++) {
                    o0[k] = f32x4_to_e4m3x4(__fdiv_rn(v[4 * k], s), __fdiv_rn(v[4 * k + 1], s),
                                            __fdiv_rn(v[4 * k + 2], s), __fdiv_rn(v[4 * k + 3], s));
                    o1[k] = f32x4_to_e4m3x4(__fdiv_rn(v[16 + 4 * k], s), __fdiv_rn(v[16 + 4 * k + 1], s),
                                            __fdiv_rn(v[16 + 4 * k + 2], s), __fdiv_rn(v[16 + 4 * k + 3], s));
                }
                uint8_t* dst = g.out + pos * g.n_out + col;
                *(u32x4*)dst = o0;
                *(u32x4*)(dst + 16) = o1;
                if (pp == 0) g.out_scale[pos * (g.n_out / 128) + nt] = s;
            }
        } else if (DT == DT_BF16) {
            if (ok) {
                uint8_t* dst = g.out + (pos * g.n_out + col) * 2;
                for (int k = 0; k < 4; k++) {
                    u32x4 o;
                    for (int m = 0; m < 4; m++) o[m] = pack_bf16x2(v[8 * k + 2 * m], v[8 * k + 2 * m + 1]);
                    *(u32x4*)(dst + 16 * k) = o;
                }
            }
        } else {
            if (ok) {
                float* dst = (float*)g.out + pos * g.n_out + col;
                for (int k = 0; k < 8; k++)
                    *(f32x4*)(dst + 4 * k) = (f32x4){v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
            }
        }
    } else {
        for (int h = 0; h < 2; h++) {
            if (h) __syncthreads();
            if (wc == h) {
                for (int rt = 0; rt < 2; rt++) {
                    if (!rt_on[rt]) continue;
                    for (int ct = 0; ct < 8; ct++)
                        for (int i = 0; i < 4; i++)
                            T[(32 * wr + 16 * rt + 4 * q + i) * kEpiPitch + 16 * ct + r16] = acc[rt][ct][i];
                }
            }
            __syncthreads();
            const int n = nt * 256 + 128 * h + 32 * pp;
            if (er < rows && n < g.n_out) {
                const size_t pos = (size_t)row0 + er;
                const int sl = g.sorted_slot[pos];
                const float wgt = g.wts[sl];
                float v[32];
                for (int j = 0; j < 32; j++) v[j] = wgt * T[er * kEpiPitch + 32 * pp + j];
                if (DT == DT_F32) {
                    float* dst = (float*)g.out + (size_t)sl * g.n_out + n;
                    for (int k = 0; k < 8; k++)
                        *(f32x4*)(dst + 4 * k) = (f32x4){v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
                } else {
                    uint8_t* dst = g.out + ((size_t)sl * g.n_out + n) * 2;
                    for (int k = 0; k < 4; k++) {
                        u32x4 o;
                        for (int m = 0; m < 4; m++) o[m] = pack_bf16x2(v[8 * k + 2 * m], v[8 * k + 2 * m + 1]);
                        *(u32x4*)(dst + 16 * k) = o;
                    }
                }
            }
        }
    }
}

// ---------------------------------------------------------------- launch
// Upper bound of M-tiles for P routed rows over E experts.
long max_mtiles(long P, int E) { return P / kBM + (P < E ? P : E); }

template <int DT, int MODE>
static int launch_one(const GemmArgs& g, long max_tiles, hipStream_t st) {
    static bool attr_set = false;
    if (!attr_set) {
        AMDMOE_HIP_TRY(hipFuncSetAttribute((const void*)grouped_gemm_kernel<DT, MODE>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kGemmLds));
        attr_set = true;
    }
    long work = max_tiles * g.n_tiles_n;
    long grid = 8 * ceil_div(work, 8);
    if (grid == 0) return AMDMOE_OK;
    AMDMOE_CHECK_ARG(grid < (1L << 31), "grouped gemm: grid too large (%ld)", grid);
    hipLaunchKernelGGL((grouped_gemm_kernel<DT, MODE>), dim3((unsigned)grid), dim3(512), kGemmLds,
                       st, g);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

int launch_grouped_gemm(int dt, int mode, const GemmArgs& g, long max_tiles, hipStream_t st) {
    if (dt == DT_F32) return mode == MODE_UP ? launch_one<DT_F32, MODE_UP>(g, max_tiles, st)
                                             : launch_one<DT_F32, MODE_DOWN>(g, max_tiles, st);
    if (dt == DT_BF16) return mode == MODE_UP ? launch_one<DT_BF16, MODE_UP>(g, max_tiles, st)
                                              : launch_one<DT_BF16, MODE_DOWN>(g, max_tiles, st);
    return mode == MODE_UP ? launch_one<DT_FP8, MODE_UP>(g, max_tiles, st)
                           : launch_one<DT_FP8, MODE_DOWN>(g, max_tiles, st);
}

}  // namespace amdmoe
