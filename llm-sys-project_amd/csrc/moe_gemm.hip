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
// Memory pipeline.  The kernel is bound by streaming expert weights from
// HBM, so what matters is bytes in flight per CU.  Operands go global -> LDS
// with buffer_load ... lds (no staging registers) into a 3-stage ring: while
// a K-step is consumed, the next two are in flight (~96 KB per CU).  Buffer
// descriptors bound every operand, so rows outside the tile (masked M rows,
// N columns past the end) are fetched as zeros without branches.  LDS rows
// are 128 bytes, XOR-swizzled in 16-byte chunks (chunk c of row r lives at
// c ^ (r & 7)) so the 16 rows an MFMA fragment reads hit distinct banks.
// Waits are explicit (vmcnt) and the barrier is a bare s_barrier, so the
// ring is never drained mid-loop.
//
// Tile: 128 rows x 256 weight rows x 128 bytes of K per step; 512 threads =
// 8 waves in a 2 (rows) x 4 (cols) grid, each wave 64 rows (4 MFMA row tiles
// of 16) x 64 weight rows (4 column tiles): the square wave tile minimises
// LDS fragment traffic, (64 + 64) x 128 bytes per wave per K-step.  In the
// up-projection a wave's 64 weight rows are 32 gate rows and the 32 matching
// up rows.
//
// Work items are laid out M-tile-major (all N-tiles of an M-tile are
// consecutive) and dealt to XCDs in contiguous chunks (workgroup b runs on
// XCD b % 8), so the A rows of an M-tile and the weight tiles shared by
// the two M-tiles of an expert stay in one XCD's L2.
#include "internal.hpp"

#include <type_traits>

namespace amdmoe {

constexpr int kBM = 128;
constexpr int kNS = 3;                                 // pipeline stages
constexpr int kATile = kBM * 128;                      // 16 KB
constexpr int kBTile = 256 * 128;                      // 32 KB
constexpr int kSTile = 8 * 256;                        // A-scale slots, 256 B per wave
constexpr int kStageBytes = kATile + kBTile + kSTile;  // 51200
constexpr int kBScaleOff = kNS * kStageBytes;          // fp8 weight scales [2][kMaxKb]
constexpr int kMaxKb = 128;                            // K <= 16384 on the fp8 path
constexpr int kEpiPitch = 132;                         // floats per staged output row
constexpr int kGemmLds = kBScaleOff + 2 * kMaxKb * 4;  // 154624
static_assert(kBM * kEpiPitch * 4 <= kNS * kStageBytes, "epilogue staging fits the ring");

template <int DT> struct DtTraits;
template <> struct DtTraits<DT_F32> { static constexpr int es = 4; };
template <> struct DtTraits<DT_BF16> { static constexpr int es = 2; };
template <> struct DtTraits<DT_FP8> { static constexpr int es = 1; };

template <int DT, int MODE>
__global__ __launch_bounds__(512, 1) void grouped_gemm_kernel(GemmArgs g) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int ES = DtTraits<DT>::es;
    constexpr int kLoadsPerStage = 6 + (DT == DT_FP8 ? 1 : 0);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)

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
    const int nk = (int)((long)g.K * ES / 128);
    const int kb_per_row = g.K / 128;  // fp8 scale blocks along K

    // ---- buffer descriptors ----
    const uint8_t* bexp = g.b + (size_t)e * g.b_expert_bytes;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc((void*)g.a, (short)0, (int)g.a_bytes, kRsrcFlags);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc((void*)bexp, (short)0, (int)g.b_expert_bytes, kRsrcFlags);

    // ---- per-lane source offsets (fixed over K; the K-step is the soffset) ----
    const int lrow = lane >> 3;                  // row within an 8-row, 1 KB slab
    const int lchunk = (lane & 7) ^ lrow;        // global chunk landing at lane's LDS slot
    uint32_t voff_a[2], voff_b[4];
    for (int j = 0; j < 2; j++) {
        const int r = 16 * wave + 8 * j + lrow;
        voff_a[j] = kOob;
        if (r < rows) {
            const long ar = MODE == MODE_UP ? (long)g.a_map[row0 + r] : (long)(row0 + r);
            voff_a[j] = (uint32_t)(ar * g.a_row_bytes + 16 * lchunk);
        }
    }
    for (int j = 0; j < 4; j++) {
        const int r = 32 * wave + 8 * j + lrow;  // weight row within the 256-row tile
        long n;
        bool ok;
        if (MODE == MODE_UP) {
            const int col = nt * 128 + (r & 127);
            ok = col < g.n_out;
            n = r < 128 ? col : (long)g.n_out + col;
        } else {
            n = (long)nt * 256 + r;
            ok = n < g.n_out;
        }
        voff_b[j] = ok ? (uint32_t)(n * g.b_row_bytes + 16 * lchunk) : kOob;
    }
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(DT == DT_FP8 ? (const void*)g.a_scale : (const void*)g.a), (short)0,
        DT == DT_FP8 ? (int)g.a_scale_bytes : 0, kRsrcFlags);
    uint32_t voff_s = kOob;
    if (DT == DT_FP8) {
        const int r = 16 * wave + lane;
        if (lane < 16 && r < rows) {
            const long ar = MODE == MODE_UP ? (long)g.a_map[row0 + r] : (long)(row0 + r);
            voff_s = (uint32_t)(ar * kb_per_row * 4);
        }
        // weight scales of this work item for every K block -> LDS
        float* sbs = (float*)(smem + kBScaleOff);
        const float* bse = g.b_scale + (size_t)e * (g.b_rows / 128) * kb_per_row;
        for (int i = tid; i < 2 * kb_per_row; i += 512) {
            const int which = i / kb_per_row, kb = i - which * kb_per_row;
            int nb;
            if (MODE == MODE_UP) nb = which == 0 ? nt : g.n_out / 128 + nt;
            else nb = min(2 * nt + which, g.b_rows / 128 - 1);
            sbs[which * kMaxKb + kb] = bse[(size_t)nb * kb_per_row + kb];
        }
    }

    auto issue = [&](int st, int kt) {
        uint8_t* base = smem + st * kStageBytes;
        const int soff = kt * 128;
        for (int j = 0; j < 2; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (lds_ptr_t)(base + (16 * wave + 8 * j) * 128), 16, voff_a[j], soff, 0, 0);
        for (int j = 0; j < 4; j++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (lds_ptr_t)(base + kATile + (32 * wave + 8 * j) * 128), 16, voff_b[j], soff, 0, 0);
        if (DT == DT_FP8)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs, (lds_ptr_t)(base + kATile + kBTile + wave * 256), 4, voff_s, kt * 4, 0, 0);
    };

    // ---- wave geometry ----
    const int wr = wave & 1, wc = wave >> 1;
    const int q = lane >> 4, r16 = lane & 15;
    const int off_lo = 16 * (q ^ (r16 & 7)), off_hi = 16 * ((4 + q) ^ (r16 & 7));
    int bcol[4];
    for (int ct = 0; ct < 4; ct++)
        bcol[ct] = MODE == MODE_UP ? (ct < 2 ? 32 * wc + 16 * ct : 128 + 32 * wc + 16 * (ct - 2))
                                   : 64 * wc + 16 * ct;
    int nrt = (rows - 64 * wr + 15) / 16;  // live row tiles of this wave (uniform)
    nrt = nrt < 0 ? 0 : (nrt > 4 ? 4 : nrt);

    f32x4 acc[4][4];
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    __syncthreads();  // weight scales in LDS; every regular load has completed
    issue(0, 0);
    if (nk > 1) issue(1, 1);
    for (int kt = 0; kt < nk; kt++) {
        if (kt + 1 < nk) wait_vmcnt<kLoadsPerStage>();
        else wait_vmcnt<0>();
        bare_barrier();
        if (kt + 2 < nk) issue((kt + 2) % kNS, kt + 2);

        const uint8_t* base = smem + (kt % kNS) * kStageBytes;
        float sb0 = 0.f, sb1 = 0.f;
        if (DT == DT_FP8) {
            const float* sbs = (const float*)(smem + kBScaleOff);
            if (MODE == MODE_UP) { sb0 = sbs[kt]; sb1 = sbs[kMaxKb + kt]; }
            else { sb0 = sb1 = sbs[(wc >> 1) * kMaxKb + kt]; }
        }
        // one K-step for NRT (1..4) live row tiles of 16, straight-line so
        // the scheduler can overlap MFMAs with fragment loads and scaling
        auto step = [&](auto nrt_tag) {
            constexpr int NRT = decltype(nrt_tag)::value;
            u32x4 alo[NRT], ahi[NRT];
            float sa[NRT][4];
            for (int rt = 0; rt < NRT; rt++) {
                const uint8_t* p = base + (64 * wr + 16 * rt + r16) * 128;
                alo[rt] = *(const u32x4*)(p + off_lo);
                ahi[rt] = *(const u32x4*)(p + off_hi);
                if (DT == DT_FP8) {
                    const int r = 64 * wr + 16 * rt + 4 * q;  // 4 rows inside one 16-row slot
                    const f32x4 s4 = *(const f32x4*)(base + kATile + kBTile + (r >> 4) * 256 + (r & 15) * 4);
                    for (int i = 0; i < 4; i++) sa[rt][i] = s4[i];
                }
            }
            for (int ct = 0; ct < 4; ct++) {
                const uint8_t* p = base + kATile + (bcol[ct] + r16) * 128;
                const u32x4 blo = *(const u32x4*)(p + off_lo), bhi = *(const u32x4*)(p + off_hi);
                for (int rt = 0; rt < NRT; rt++) {
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
                        const f32x4 pr = mfma_fp8(av, bv, (f32x4){0.f, 0.f, 0.f, 0.f});
                        const float sb = (MODE == MODE_UP && ct >= 2) ? sb1 : sb0;
                        for (int i = 0; i < 4; i++) acc[rt][ct][i] += pr[i] * (sa[rt][i] * sb);
                    }
                }
            }
        };
        if (nrt == 4) step(std::integral_constant<int, 4>{});
        else if (nrt == 3) step(std::integral_constant<int, 3>{});
        else if (nrt == 2) step(std::integral_constant<int, 2>{});
        else if (nrt == 1) step(std::integral_constant<int, 1>{});
    }
    __syncthreads();  // every wave is done with the ring before it is reused

    // ---- epilogues (LDS staging for coalesced 16-byte stores) ----
    float* T = (float*)smem;
    const int er = tid >> 2, pp = tid & 3;  // output row, 32-column part
    if (MODE == MODE_UP) {
        for (int rt = 0; rt < 4; rt++) {
            if (rt >= nrt) continue;  // constant bound keeps acc[] in registers
            for (int j = 0; j < 2; j++)
                for (int i = 0; i < 4; i++) {
                    const float gv = acc[rt][j][i], uv = acc[rt][j + 2][i];
                    const float silu = gv / (1.0f + expf(-gv));
                    T[(64 * wr + 16 * rt + 4 * q + i) * kEpiPitch + 32 * wc + 16 * j + r16] = silu * uv;
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
            if ((wc >> 1) == h) {
                for (int rt = 0; rt < 4; rt++) {
                    if (rt >= nrt) continue;
                    for (int ct = 0; ct < 4; ct++)
                        for (int i = 0; i < 4; i++)
                            T[(64 * wr + 16 * rt + 4 * q + i) * kEpiPitch + 64 * (wc & 1) + 16 * ct + r16] =
                                acc[rt][ct][i];
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
    // buffer descriptors address at most 4 GiB - 1 bytes per operand
    const long lim = 0xFFFFFFF0L;
    AMDMOE_CHECK_ARG(g.a_bytes <= lim && g.b_expert_bytes <= lim && g.a_scale_bytes <= lim,
                     "grouped gemm: an operand exceeds 4 GiB (A %ld, expert %ld bytes)", g.a_bytes,
                     g.b_expert_bytes);
    AMDMOE_CHECK_ARG(dt != DT_FP8 || g.K / 128 <= kMaxKb, "grouped gemm: K=%d too large for fp8", g.K);
    if (dt == DT_F32) return mode == MODE_UP ? launch_one<DT_F32, MODE_UP>(g, max_tiles, st)
                                             : launch_one<DT_F32, MODE_DOWN>(g, max_tiles, st);
    if (dt == DT_BF16) return mode == MODE_UP ? launch_one<DT_BF16, MODE_UP>(g, max_tiles, st)
                                              : launch_one<DT_BF16, MODE_DOWN>(g, max_tiles, st);
    return mode == MODE_UP ? launch_one<DT_FP8, MODE_UP>(g, max_tiles, st)
                           : launch_one<DT_FP8, MODE_DOWN>(g, max_tiles, st);
}

}  // namespace amdmoe
