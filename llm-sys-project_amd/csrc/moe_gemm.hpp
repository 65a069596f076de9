// R3/R4/R5 -- single-launch grouped expert GEMMs on MFMA.
//
// Reference: the per-expert host loop of moe_forward
// (kernels/moe/naive_moe.cu:424-470): per expert, GEMM1 [cnt,D]x[2I,D]^T
// (tiled_gemm_bt_kernel, 246-280), swiglu_strided_kernel (297-310), GEMM2
// [cnt,I]x[D,I]^T, then scatter_kernel (315-335) with the routing weight.
//
// Here each GEMM is ONE launch over every expert.  The permutation kernel
// emits M-tiles {expert, first sorted row, rows} of up to 256 rows; a
// workgroup owns one (M-tile, N-tile) work item:
//   UP   (GEMM1 + SwiGLU): A rows are gathered straight from x through
//        sorted_token (no permuted copy of x exists); the weight tile is 128
//        gate rows n0.. and the 128 matching up rows I+n0.., so each wave has
//        g and u of the same columns and writes act = silu(g)*u (fp8:
//        requantised per 128 columns, the tile width).
//   DOWN (GEMM2 + combine weight): A = act rows (contiguous, sorted order),
//        256 rows of W2; the epilogue multiplies by the routing weight of the
//        row's slot and writes the row to ypair[slot] (slot = t*K+k), from
//        where the combine kernel sums each token's rows in ascending expert
//        order -- the reference's scatter order, deterministic, no atomics.
// fp8 block scales (128x128 weights, 1x128 activations): a K-step is exactly
// one 128-wide K block, so each 16x16x128 MFMA yields a fresh partial that
// is folded into the fp32 accumulator as acc += partial * (s_a[row]*s_w).
//
// Why the tile is 256 rows.  The layer is bound by streaming expert weights
// from HBM.  With top-8 of 256 experts at T=4096 an expert sees 128 +- 11
// tokens, so 128-row tiles split half the experts in two and those experts'
// weights are streamed twice (measured: 1.7x the algorithmic bytes).  A
// 256-row tile covers every expert at T <= ~7000 in one pass.
//
// Memory pipeline.  Activations: 256 rows x 128 bytes per K-step, global ->
// LDS with buffer_load ... lds into a 3-stage ring (rows past the tile read
// as zeros through the buffer descriptor); LDS rows are XOR-swizzled in
// 16-byte chunks so 16-row fragment reads hit distinct banks.  Weights:
// each of the 8 waves owns 32 weight rows and loads them straight into
// registers in MFMA operand layout (a register ring of 4 K-step sets, 3 for
// a full 16-tile M-tile), so the weight stream needs no LDS: three K-steps
// (~96 KB per CU) are in flight while one is consumed.  Waits are explicit vmcnt counts and the barrier is a bare
// s_barrier, so nothing drains mid-loop.
//
// Work items are laid out expert by expert, N-tile major over the expert's
// M-tiles (the M-tiles that read one weight tile are consecutive), and dealt
// to XCDs in contiguous chunks (workgroup b runs on XCD b % 8), so an
// expert's activation rows and weight tiles stay in one XCD's L2.
//
// The kernel template lives in this header; each moe_gemm_<type>.hip file
// instantiates some of its variants (the fp8 ones are large: one main loop
// per live token-tile count), so they compile in parallel.  Built: fp8 and
// MX (both projections), fp32.  The bf16 GEMMs run
// grouped_gemm_bf16_w4_kernel (moe_gemm_bf16_w4.hip: same items and
// arithmetic, 4 waves x 64 weight rows); this template has no bf16 form.
#pragma once

#include <type_traits>
#include <utility>

#include "internal.hpp"

namespace amdmoe {

constexpr int kBM = kMTile;                            // 256
constexpr int kNS = 3;                                 // ring stages (activations and weights)
static_assert(kNS == 3, "activations are prefetched two K-steps ahead");
constexpr int kATile = kBM * 128;                      // 32 KB
constexpr int kSTile = 8 * 256;                        // A-scale slots, 256 B per wave
constexpr int kStageBytes = kATile + kSTile;           // 34816
constexpr int kBScaleOff = kNS * kStageBytes;          // fp8 weight scales [2][kMaxKb]
constexpr int kMaxKb = 128;                            // K <= 16384 on the fp8 path
// weight register sets of the main loop's ring (RB - 1 K-steps of weights in
// flight) for up to 12 live token tiles and for more
constexpr int kRbSmall = 4, kRbLarge = 3;
// fp8 / MX M-tiles of up to this many 16-row token tiles stage their
// activations through registers (global -> VGPR -> ds_write) instead of the
// LDS DMA: measured cheaper per byte, and the registers are there while the
// accumulators are few
constexpr int kVgMaxR = 12;
constexpr int kVgMaxRMx = 0;   // MX: none (its fragments hold scale registers too; the register path spilled)
constexpr float kNegLog2e = -1.4426950408889634f;  // -log2(e)
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kEpiPitch = 132;                         // floats per staged output row
constexpr int kEpiRows = 128;                          // epilogue stages 128 rows at a time
constexpr int kRowInfoOff = kBScaleOff + 2 * kMaxKb * 4;  // DOWN: [256] slot, [256] weight
constexpr int kGemmLds = kRowInfoOff + kBM * 8;           // 107520
static_assert(kEpiRows * kEpiPitch * 4 <= kNS * kStageBytes, "epilogue staging fits the ring");
static_assert(kBM == 256, "the wave layout assumes 256-row tiles");
static_assert(128 * 528 <= kNS * kStageBytes, "DOWN epilogue staging fits the ring");

template <int DT> struct DtTraits;
template <> struct DtTraits<DT_F32> { static constexpr int es = 4; };
template <> struct DtTraits<DT_FP8> { static constexpr int es = 1; };
template <> struct DtTraits<DT_MX> { static constexpr int es = 1; };  // activation bytes per element

// One K-step of a wave's weights in registers: per column tile the lane's
// 32 bytes, lo 16 B at K offset 16q and hi 16 B at 64 + 16q (the fp8 MFMA
// consumes them as one 8-dword tuple).
struct BFrag {
    u32x4 q[2][2];  // [column tile][lo, hi]
};

// MXFP4: per column tile the lane's 16 bytes of E2M1 weights (32 elements,
// one E8M0 block) and that block's scale byte.
struct BFragMx {
    u32x4 w[2];
    uint32_t s[2];
};

// An empty asm that reads and redefines the fragment: no use of it can move
// above this point, and the compiler must assume its value changes here.
__device__ __forceinline__ void pin(BFrag& f) {
    asm volatile("" : "+v"(f.q[0][0]), "+v"(f.q[0][1]), "+v"(f.q[1][0]), "+v"(f.q[1][1]));
}
__device__ __forceinline__ void pin(BFragMx& f) {
    asm volatile("" : "+v"(f.w[0]), "+v"(f.w[1]), "+v"(f.s[0]), "+v"(f.s[1]));
}

typedef int i32x4 __attribute__((ext_vector_type(4)));

// the first N registers of a register-path activation set
template <int N>
__device__ __forceinline__ void pin_av(u32x4 (&a)[4]) {
    static_assert(N >= 1 && N <= 4, "one to four slabs");
    asm volatile("" : "+v"(a[0]));
    if constexpr (N > 1) asm volatile("" : "+v"(a[1]));
    if constexpr (N > 2) asm volatile("" : "+v"(a[2]));
    if constexpr (N > 3) asm volatile("" : "+v"(a[3]));
}

// 16-byte buffer load into registers, issued as inline asm so the compiler
// does not insert its own vector-memory waits before the (much later) use;
// the kernel's explicit vmcnt wait at the top of each K-step covers it.
// OFF is the immediate offset; an out-of-range voffset reads zeros.
// The buffer descriptor of make_rsrc() as four scalar words: base address,
// stride 0, byte count, raw-buffer flags.
__device__ __forceinline__ i32x4 make_rsrc_words(const void* base, long bytes) {
    const uint64_t p = (uint64_t)base;
    return (i32x4){__builtin_amdgcn_readfirstlane((int)(uint32_t)p),
                   __builtin_amdgcn_readfirstlane((int)((p >> 32) & 0xffff)),
                   __builtin_amdgcn_readfirstlane((int)bytes), kRsrcFlags};
}

// NT: a streaming (non-temporal) load -- GEMM2's weights, read once: DOWN
// 4.5% and the combine that follows 8% faster at DSV3 T=4096 (GEMM1's
// weights are not marked: an expert's paired M-tiles share them in L2).
template <int OFF, bool NT = false>
__device__ __forceinline__ u32x4 buffer_load_b128_async(i32x4 rsrc, uint32_t voff, int soff) {
    u32x4 r;
    if constexpr (NT)
        asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen offset:%4 nt"
                     : "=v"(r)
                     : "v"(voff), "s"(rsrc), "s"(soff), "i"(OFF));
    else
        asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen offset:%4"
                     : "=v"(r)
                     : "v"(voff), "s"(rsrc), "s"(soff), "i"(OFF));
    return r;
}

// One byte, zero-extended (the MX weight scale of the lane's block), as
// asm for the same reason.
__device__ __forceinline__ uint32_t buffer_load_u8_async(i32x4 rsrc, uint32_t voff, int soff) {
    uint32_t r;
    asm volatile("buffer_load_ubyte %0, %1, %2, %3 offen"
                 : "=v"(r)
                 : "v"(voff), "s"(rsrc), "s"(soff));
    return r;
}

// 16x16x128 MFMA, A = MXFP4 weights (E2M1, 4 registers used), B = MXFP8
// activations, with the hardware applying each operand's E8M0 block scale
// (byte 0 of sa / sb): scale j belongs to K elements 32j..32j+31 of the
// step for both operands (the lanes of group j supply it).
__device__ __forceinline__ f32x4 mfma_mx(const u32x4& w, const i32x8& x, uint32_t sa, uint32_t sb, f32x4 c) {
    const i32x8 a = {(int)w[0], (int)w[1], (int)w[2], (int)w[3], 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, x, c, 4, 0, 0, (int)sa, 0, (int)sb);
}

__device__ __forceinline__ i32x8 frag8(const BFrag& f, int ct) {
    const u32x4 a = f.q[ct][0], b = f.q[ct][1];
    return (i32x8){(int)a[0], (int)a[1], (int)a[2], (int)a[3], (int)b[0], (int)b[1], (int)b[2], (int)b[3]};
}

__device__ __forceinline__ u32x4 lo4(const i32x8& x) {
    return (u32x4){(uint32_t)x[0], (uint32_t)x[1], (uint32_t)x[2], (uint32_t)x[3]};
}
__device__ __forceinline__ u32x4 hi4(const i32x8& x) {
    return (u32x4){(uint32_t)x[4], (uint32_t)x[5], (uint32_t)x[6], (uint32_t)x[7]};
}

// PK: weights in fragment-block order (pack_weights), a separate
// instantiation so the two layouts are distinct kernels
template <int DT, int MODE, bool PK>
__global__ __launch_bounds__(512, 1) void grouped_gemm_kernel(GemmArgs g) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    constexpr int ES = DtTraits<DT>::es;
    // vector-memory instructions per K-step per wave ("slots"): 4
    // activation slabs (+1 scale slot on fp8 / MX) into LDS, then 4 weight
    // loads into registers (MX: per column tile 16 bytes of E2M1 and one
    // scale byte); a wave whose activation rows are all past the live token
    // tiles issues only the weight loads
    static_assert(DT != DT_BF16, "the bf16 GEMMs are grouped_gemm_bf16_w4_kernel");
    constexpr bool kScaledA = DT == DT_FP8 || DT == DT_MX;  // activations carry row scales
    static_assert(DT != DT_MX || PK, "MX weights exist in fragment order only");
    using Frag = std::conditional_t<DT == DT_MX, BFragMx, BFrag>;
    // per K-step and wave: ceil(R/4) activation slabs of 8 rows (the 2R slabs
    // of R live token tiles dealt round-robin over the 8 waves: slab s of
    // wave w holds rows 64s + 8w .. +7), one scale slot (fp8 / MX), 4
    // weight slots -- the same count for every wave, so no wave branches
    // around its loads
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)

    // ---- work item (XCD-chunked) ----
    // DOWN with fp32 rows may split K over S items per (M-tile, N-tile):
    // virtual N-tile v = S * nt + ks (uniform)
    constexpr bool kCanSplit = MODE == MODE_DOWN && DT == DT_F32;
    const int S = kCanSplit ? max(g.k_splits, 1) : 1;
    const int W = (*g.num_tiles) * g.n_tiles_n * S;
    const int per = (W + 7) >> 3;
    const int slot = blockIdx.x >> 3;
    if (slot >= per) return;
    const int w = (blockIdx.x & 7) * per + slot;
    if (w >= W) return;
    // An expert with m M-tiles owns items [f*ntn, (f+m)*ntn) (f its first
    // tile), ordered N-tile major: item f*ntn + m*nt + j is (tile f+j, nt),
    // so the m tiles that read the same weight tile are dispatched back to
    // back on one XCD and share its weight stream through L2.
    const int ntn = g.n_tiles_n * S;
    const int mt0 = w / ntn;  // a tile of the owning expert
    const int4 tile0 = g.tiles[mt0];
    const int m_tiles = tile0.w & 0xffff, first_tile = mt0 - (tile0.w >> 16);
    const int l_item = w - first_tile * ntn;
    const int ntv = __builtin_amdgcn_readfirstlane(l_item / m_tiles);
    const int mt = first_tile + (l_item - ntv * m_tiles);
    const int nt = S == 1 ? ntv : ntv / S, ks = ntv - nt * S;
    const int4 tile = m_tiles == 1 ? tile0 : g.tiles[mt];
    // uniform values (SGPRs): the asm loads take their soffsets from them
    const int e = __builtin_amdgcn_readfirstlane(tile.x), row0 = __builtin_amdgcn_readfirstlane(tile.y),
              rows = __builtin_amdgcn_readfirstlane(tile.z);
    const int nk_all = (int)((long)g.K * ES / 128);  // K-steps of the whole reduction
    const int nk = nk_all / S;                          // K-steps of this item: [ks nk, ks nk + nk)
    const int kbase = ks * nk;
    const int kb_per_row = g.K / 128;  // fp8 scale blocks along K

    // ---- buffer descriptors ----
    const uint8_t* bexp = g.b + (size_t)e * g.b_expert_bytes;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(g.a, g.a_bytes);
    const i32x4 rb = make_rsrc_words(bexp, g.b_expert_bytes);
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc(kScaledA ? (const void*)g.a_scale : (const void*)g.a,
                  kScaledA ? g.a_scale_bytes : 0);
    const i32x4 rbs = DT == DT_MX ? make_rsrc_words(g.b_mx_scale + (size_t)e * g.b_mx_scale_expert_bytes,
                                                    g.b_mx_scale_expert_bytes)
                                  : rb;

    // ---- activation DMA offsets: wave w fills rows [32w, 32w+32) ----
    const int lrow = lane >> 3;              // row within an 8-row, 1 KB slab
    const int lchunk = (lane & 7) ^ lrow;    // global chunk landing at lane's LDS slot
    // Prologue loads: the weight scales of this work item for every K block
    // (fp8: [which][kMaxKb] dwords in LDS, kb < kb_per_row), UP's row
    // indices (a_map), and DOWN's slot and routing weight of each row, which
    // only the epilogue needs: those stay in flight through the main loop.
    // DOWN loads the scales straight into LDS by the LDS DMA of waves 0-3
    // (lane l of wave w writes dword 64w + l: waves 0-1 fill block 0, waves
    // 2-3 block 1 at dword kMaxKb = 128), with no register wait: they
    // are the oldest loads of those waves, so the first K-step's vmcnt wait
    // and barrier cover them, and the weight ring goes out one round trip
    // earlier (DSV3 DOWN -0.3% at T=4096, -1.7% at T=8192).  UP waits for
    // a_map before its ring anyway, so it loads one scale per thread into
    // registers and then LDS, behind a barrier.  The register loads are
    // unconditional, from clamped in-range addresses: in a branch, each
    // would be waited for on its own.
    float sb_val = 0.0f;
    int sb_pos = -1;
    if (DT == DT_FP8 && MODE == MODE_UP) {
        const float* bse = g.b_scale + (size_t)e * (g.b_rows / 128) * kb_per_row;
        const int i = min(tid, 2 * kb_per_row - 1);
        const int which = i / kb_per_row, kb = i - which * kb_per_row;
        const int nb = which == 0 ? nt : g.n_out / 128 + nt;
        sb_val = bse[(size_t)nb * kb_per_row + kb];
        sb_pos = tid < 2 * kb_per_row ? which * kMaxKb + kb : -1;
    }
    if (DT == DT_FP8 && MODE == MODE_DOWN && wave < 4) {
        const int nbr = g.b_rows / 128;  // 128-row scale blocks per expert
        const __amdgpu_buffer_rsrc_t rsb =
            make_rsrc(g.b_scale + (size_t)e * nbr * kb_per_row, (long)nbr * kb_per_row * 4);
        const int which = wave >> 1, kb = 64 * (wave & 1) + lane;
        const int nb = 2 * nt + which;  // waves 0-3 of the loop use block 2nt, waves 4-7 block 2nt + 1
        const uint32_t vo = kb < kb_per_row && nb < nbr ? (uint32_t)((nb * kb_per_row + kb) * 4) : kOob;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsb, (lds_ptr_t)(smem + kBScaleOff + 256 * wave), 4, vo, 0, 0, 0);
    }
    // UP gathers the rows through a_map (index clamped to a live row; the
    // offset of a row past the tile is replaced by the out-of-range one)
    long arow[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int r = 64 * j + 8 * wave + lrow;
        arow[j] = MODE == MODE_UP ? (long)g.a_map[row0 + min(r, rows - 1)] : (long)(row0 + r);
    }
    uint32_t voff_a[4];  // slab j of this wave: rows 64j + 8w .. +7
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int r = 64 * j + 8 * wave + lrow;
        voff_a[j] = r < rows ? (uint32_t)(arow[j] * g.a_row_bytes + 16 * lchunk) : kOob;
    }
    // activation scales of a K-step: fp8 one fp32 per row, MX the row's four
    // E8M0 bytes -- both one dword per row and step, stored K-step major in
    // sorted row order ([K/128][a_scale_rows] dwords), so the 32 rows of a
    // wave's scale slot are one 128-byte line (row-major, every gathered
    // row's scale was a line of its own: UP 8% slower)
    uint32_t voff_s = kOob;
    if (kScaledA) {
        const int r = 32 * wave + lane;
        if (lane < 32 && r < rows) voff_s = (uint32_t)((row0 + r) * 4);
    }
    const int scale_kstride = (int)(g.a_scale_rows * 4);  // bytes per K-step of a_scale

    // ---- weight rows of this wave: two MFMA column tiles of 16 ----
    //   UP:   ct 0 = gate rows n0 + 16w + c, ct 1 = up rows I + n0 + 16w + c
    //   DOWN: ct = rows n0 + 32w + 16ct + c
    const int q = lane >> 4, r16 = lane & 15;
    uint32_t voff_b[2], voff_bs[2];
    for (int ct = 0; ct < 2; ct++) {
        long n;
        bool ok;
        if (MODE == MODE_UP) {
            const int col = nt * 128 + 16 * wave + r16;
            ok = col < g.n_out;
            n = ct == 0 ? col : (long)g.n_out + col;
        } else {
            n = (long)nt * 256 + 32 * wave + 16 * ct + r16;
            ok = n < g.n_out;
        }
        // row-major: lane (q, r16) reads row n at K offset 16q (+64 for the
        // hi half); fragment blocks: the 16 rows' 2 KB K-step is stored as
        // [half][lane][16 B], so each load is 1 KB contiguous
        const long nb = PK ? (n - r16) * g.b_row_bytes + 16 * lane : n * g.b_row_bytes + 16 * q;
        voff_b[ct] = ok ? (uint32_t)nb : kOob;
        // MX: E8M0 scales of the 16 rows' K-step, [lane] bytes per block of 64
        voff_bs[ct] = ok ? (uint32_t)((n - r16) / 16 * nk_all * 64 + lane) : kOob;
    }
    __builtin_amdgcn_sched_barrier(0);
    int row_slot = 0;
    float row_w = 0.0f;
    if (MODE == MODE_DOWN) {
        const size_t r = (size_t)row0 + min(tid, rows - 1);  // rows >= 1
        row_slot = g.sorted_slot[r];
        row_w = tid < rows ? g.sorted_w[r] : 0.0f;
    }
    __builtin_amdgcn_sched_barrier(0);
    if (sb_pos >= 0) ((float*)(smem + kBScaleOff))[sb_pos] = sb_val;

    // K-steps run in a rotated order starting at kt0, keyed by the expert:
    // the N-tiles of one M-tile run together on one XCD and read the same
    // activation K-slice at the same time (one fetch, the rest L2 hits), an
    // expert's M-tiles (evenly sized, adjacent in the item order) read the
    // same weight K-slices together, and different experts start at
    // different K offsets.
    const int kt0 = (int)(((unsigned)e * 7u) % (unsigned)nk);
    auto kblk = [&](int kt) __attribute__((always_inline)) {
        int k = kt + kt0;
        k = k >= nk ? k - nk : k;
        return kbase + (k >= nk ? k - nk : k);
    };

    // Loads for a K-step past the end (kt >= nk) are still issued, through
    // a descriptor of zero bytes (they read zeros and touch no memory), so
    // every step waits for the same vmcnt and no path through the loop skips
    // a wait.  The scalar part of a step's addressing (rotated K block,
    // soffsets, LDS stage, live or null descriptors) is formed once per step
    // (STEP_ADDR); issue_slot(sl, ...) then issues slot sl of kSl: the
    // activation slabs of K-step kt_a into ring stage kt_a % kNS, the scale
    // slot, then the weight slots of K-step kt_b into register set f.
    const __amdgpu_buffer_rsrc_t ra0 = make_rsrc(g.a, 0), rs0 = make_rsrc(g.a, 0);
    i32x4 rb0 = rb, rbs0 = rbs;
    rb0[2] = 0;
    rbs0[2] = 0;
    // the activation descriptor as words, for the register path's asm loads
    const i32x4 rav = make_rsrc_words(g.a, g.a_bytes);
    i32x4 rav0 = rav;
    rav0[2] = 0;
    // (the step's scalars: descriptors ra_/rs_/rb_/rbs_, soffsets so_*, LDS
    // stage st_ -- declared by STEP_ADDR(kt_a, kt_b) where a slot is issued)
#define STEP_ADDR(KT_A, KT_B, KT_V)                                                        \
    const bool live_a_ = (KT_A) < nk, live_b_ = (KT_B) < nk, live_v_ = (KT_V) < nk;        \
    const int ka_ = kblk(KT_A), kb_ = kblk(KT_B), kv_ = kblk(KT_V);                        \
    const __amdgpu_buffer_rsrc_t ra_ = live_a_ ? ra : ra0, rs_ = live_a_ ? rs : rs0;       \
    const i32x4 rb_ = live_b_ ? rb : rb0, rbs_ = live_b_ ? rbs : rbs0;                     \
    const i32x4 rv_ = live_v_ ? rav : rav0;                                                \
    const int so_a = ka_ * 128, so_s = ka_ * scale_kstride, so_bs = kb_ * 64, so_v = kv_ * 128; \
    const int so_b = DT == DT_MX ? kb_ * 1024 : (PK ? kb_ * 2048 : kb_ * 128);             \
    uint8_t* const st_ = smem + ((KT_A) % kNS) * kStageBytes
    auto issue_slot = [&](auto rc, int sl, __amdgpu_buffer_rsrc_t ra_, __amdgpu_buffer_rsrc_t rs_,
                          i32x4 rb_, i32x4 rbs_, i32x4 rv_, int so_a, int so_s, int so_b, int so_bs,
                          int so_v, uint8_t* st_, Frag& f, u32x4 (&av)[4]) __attribute__((always_inline)) {
        constexpr int R = decltype(rc)::value;
        constexpr int NS = (R + 3) / 4;
        constexpr int kAS = NS + (kScaledA ? 1 : 0);
        if (sl < NS) {
            if constexpr ((kScaledA && R <= (DT == DT_MX ? kVgMaxRMx : kVgMaxR)) || (DT == DT_FP8 && R > kVgMaxR))  // register path: K-step KT_V into av
                av[sl < 4 ? sl : 0] = buffer_load_b128_async<0>(rv_, voff_a[sl], so_v);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    ra_, (lds_ptr_t)(st_ + (64 * sl + 8 * wave) * 128), 16, voff_a[sl], so_a, 0, 0);
        } else if (sl < kAS) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rs_, (lds_ptr_t)(st_ + kATile + wave * 256), 4, voff_s, so_s, 0, 0);
        } else {
            const int ct = (sl - kAS) >> 1;
            if constexpr (DT == DT_MX) {
                // 1 KB of E2M1 (16 rows x 128 K) and the 64 scale bytes of the block
                if ((sl - kAS) & 1) f.s[ct] = buffer_load_u8_async(rbs_, voff_bs[ct], so_bs);
                else f.w[ct] = buffer_load_b128_async<0, MODE == MODE_DOWN>(rb_, voff_b[ct], so_b);
            } else {
                if ((sl - kAS) & 1)
                    f.q[ct][1] = buffer_load_b128_async<0, MODE == MODE_DOWN>(rb_, voff_b[ct], so_b + (PK ? 1024 : 64));
                else
                    f.q[ct][0] = buffer_load_b128_async<0, MODE == MODE_DOWN>(rb_, voff_b[ct], so_b);
            }
        }
    };
#define SLOT_ARGS ra_, rs_, rb_, rbs_, rv_, so_a, so_s, so_b, so_bs, so_v, st_

    const int off_lo = 16 * (q ^ (r16 & 7)), off_hi = 16 * ((4 + q) ^ (r16 & 7));

    // acc[rt][ct] is the transposed output tile: lane (q, r16) holds weight
    // columns 4q..4q+3 of column tile ct for token 16*rt + r16.
    f32x4 acc[16][2];

    // One K-step on ring stage ST with weights `bf`.  The MFMA computes
    // C^T = W x^T: weights are operand A (rows = weight columns), tokens
    // operand B, so each lane owns a single token and the activation block
    // scale is one float per lane, while the weight block scale is uniform.
    auto compute = [&](auto rc, const Frag& bf, int kt, auto&& tile_issued) __attribute__((always_inline)) {
        constexpr int R = decltype(rc)::value;
        // the stage offset is made opaque so the compiler forms the LDS
        // addresses here (one add, then immediate offsets) rather than
        // hoisting one address register per stage and tile out of the loop
        uint32_t soff_st = (kt % kNS) * kStageBytes;
        asm volatile("" : "+s"(soff_st));
        const uint8_t* base = smem + soff_st;
        float sb0 = 0.f, sb1 = 0.f;
        if (DT == DT_FP8) {
            const float* sbs = (const float*)(smem + kBScaleOff);
            const int kb = kblk(kt);
            // UP: the gate rows accumulate -log2(e) * g (the exponent the
            // epilogue's exp2 takes), folded into their block scale here
            if (MODE == MODE_UP) { sb0 = sbs[kb] * kNegLog2e; sb1 = sbs[kMaxKb + kb]; }
            else { sb0 = sb1 = sbs[(wave >> 2) * kMaxKb + kb]; }
        }
        auto load_x = [&](int rt, i32x8& xv, float& sx) __attribute__((always_inline)) {
            const uint8_t* p = base + (16 * rt + r16) * 128;
            const u32x4 lo = *(const u32x4*)(p + off_lo), hi = *(const u32x4*)(p + off_hi);
            xv = (i32x8){(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                         (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
            if (kScaledA) {  // fp8: the row's fp32 scale; MX: its four E8M0 bytes
                const int r = 16 * rt + r16;
                sx = *(const float*)(base + kATile + (r >> 5) * 256 + (r & 31) * 4);
            }
        };
        auto mma = [&](int rt, const i32x8& xv, float sx) __attribute__((always_inline)) {
            const u32x4 xlo = lo4(xv), xhi = hi4(xv);
            if constexpr (DT == DT_MX) {
                // block scales applied by the MFMA: the weights' from the
                // lane's scale byte, the token's from byte q of its dword
                const uint32_t sbx = __float_as_uint(sx) >> (8 * q);
#pragma unroll
                for (int ct = 0; ct < 2; ct++) acc[rt][ct] = mfma_mx(bf.w[ct], xv, bf.s[ct], sbx, acc[rt][ct]);
            } else if constexpr (DT == DT_FP8) {
                const float s0 = sx * sb0;
                const float s1 = MODE == MODE_UP ? sx * sb1 : s0;
#pragma unroll
                for (int ct = 0; ct < 2; ct++) {
                    const f32x4 pr = mfma_fp8(frag8(bf, ct), xv, (f32x4){0.f, 0.f, 0.f, 0.f});
                    const float sc = ct == 0 ? s0 : s1;
                    for (int i = 0; i < 4; i++) acc[rt][ct][i] += pr[i] * sc;
                }
            } else {
#pragma unroll
                for (int ct = 0; ct < 2; ct++) {
                    const u32x4 wlo = bf.q[ct][0], whi = bf.q[ct][1];  // f32
                    for (int j = 0; j < 4; j++)
                        acc[rt][ct] = mfma_f32(__uint_as_float(wlo[j]), __uint_as_float(xlo[j]), acc[rt][ct]);
                    for (int j = 0; j < 4; j++)
                        acc[rt][ct] = mfma_f32(__uint_as_float(whi[j]), __uint_as_float(xhi[j]), acc[rt][ct]);
                }
            }
            // pin the products here: without it the MFMAs float to their
            // last use and every tile's operands stay live at once
            asm volatile("" : "+v"(acc[rt][0]), "+v"(acc[rt][1]));
        };
        // fp8: the block-scale fold of a tile's products is deferred until
        // the next tile's MFMAs are issued, so the VALU never waits on an
        // MFMA it just issued (products of two tiles live, 16 registers).
        auto mfma_pair = [&](const i32x8& xv, f32x4& p0, f32x4& p1) __attribute__((always_inline)) {
            if constexpr (DT == DT_FP8) {
                p0 = mfma_fp8(frag8(bf, 0), xv, (f32x4){0.f, 0.f, 0.f, 0.f});
                p1 = mfma_fp8(frag8(bf, 1), xv, (f32x4){0.f, 0.f, 0.f, 0.f});
                asm volatile("" : "+v"(p0), "+v"(p1));
            }
        };
        auto fold = [&](int rt, const f32x4& p0, const f32x4& p1, float sx) __attribute__((always_inline)) {
            const float s0 = sx * sb0;
            const float s1 = MODE == MODE_UP ? sx * sb1 : s0;
            for (int i = 0; i < 4; i++) acc[rt][0][i] += p0[i] * s0;
            for (int i = 0; i < 4; i++) acc[rt][1][i] += p1[i] * s1;
            asm volatile("" : "+v"(acc[rt][0]), "+v"(acc[rt][1]));
        };
        // R token tiles, straight-line code (the main loop is instantiated
        // per live tile count, so nothing here branches), software-pipelined:
        // a tile's fragments are read from LDS two tiles ahead of its MFMAs
        // and (fp8) its products are folded after the next tile's MFMAs are
        // issued.  Scheduling fences keep operands of at most three tiles
        // live -- with 128 accumulators and the weight ring live, more would
        // spill.
        auto fence = []() __attribute__((always_inline)) {
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
        };
        i32x8 xs[3];
        float ss[3] = {0.f, 0.f, 0.f};
        f32x4 pp[2][2];
        load_x(0, xs[0], ss[0]);
        if (R > 1) load_x(1, xs[1], ss[1]);
        fence();
        static_for<R>([&](auto tc) __attribute__((always_inline)) {
            constexpr int t = decltype(tc)::value;
            if constexpr (DT == DT_FP8) {
                mfma_pair(xs[t % 3], pp[t & 1][0], pp[t & 1][1]);
                tile_issued(t);
                if constexpr (t >= 1) fold(t - 1, pp[(t - 1) & 1][0], pp[(t - 1) & 1][1], ss[(t - 1) % 3]);
            } else {
                mma(t, xs[t % 3], ss[t % 3]);
                tile_issued(t);
            }
            if constexpr (t + 2 < R) load_x(t + 2, xs[(t + 2) % 3], ss[(t + 2) % 3]);
            fence();
        });
        if (DT == DT_FP8) {
            fold(R - 1, pp[(R - 1) & 1][0], pp[(R - 1) & 1][1], ss[(R - 1) % 3]);
            fence();
        }
    };

    static_assert(kMaxKb == 128, "DOWN's scale DMA: two waves of 64 lanes per 128-row block");
    if (!(DT == DT_FP8 && MODE == MODE_DOWN)) lds_barrier();  // UP's weight scales in LDS
    // Prefetch distances: activations 2 K-steps ahead (a 3-stage LDS ring;
    // they come from L2), weights RB-1 K-steps ahead in a ring of RB
    // register sets -- as deep as the registers left by the live
    // accumulators allow (RB = 4 for up to 12 token tiles, else 3).  The
    // loop is unrolled by RB so each weight set keeps a fixed name.
    //
    // The prefetch is spread over the step: the vector-memory unit accepts
    // a wave's loads only as fast as it drains them, so issuing all of a
    // step's loads at once parks every wave at the issue for most of the
    // step.  Slot s goes out right after the MFMAs of token tile
    // (s * tiles) / kSl, so the activation slots go first.
    auto step = [&](auto stc, auto rc, auto rbc, int kt, Frag& cur, Frag& refill, u32x4 (&av_w)[4],
                    u32x4 (&av_l)[4]) __attribute__((always_inline)) {
        constexpr int R = decltype(rc)::value;  // token tiles per step
        constexpr int RB = decltype(rbc)::value;
        constexpr int NS = (R + 3) / 4;
        constexpr int kSl = NS + (kScaledA ? 1 : 0) + 4;
        constexpr bool kVg = kScaledA && R <= (DT == DT_MX ? kVgMaxRMx : kVgMaxR);
        constexpr bool kVg1 = DT == DT_FP8 && R > kVgMaxR;  // one register set (MX: registers run out)
        // Issue order per step: activation slots of step kt+2, then the 4
        // weight loads of step kt+RB-1.  Everything of step kt has landed
        // once at most kWait vector-memory instructions are outstanding:
        //   RB == 3: the weights of step kt+1 (4), which follow the
        //            activations of step kt+1 (those are thus waited for
        //            one step early).
        //   RB == 4: the last 8 issued (the weights of step kt+2 and the
        //            newest activation slots of step kt+1): the weights of
        //            step kt and the activations of step kt precede them.
        //   RB == 2: the weights of step kt were the last loads issued, so
        //            nothing may be outstanding (the activations of step
        //            kt+1, issued before them, are waited for one step early).
        //   register path (kVg, RB == 4): per step the activations of
        //            step kt+3 go to registers (NS loads), the scale slot of
        //            step kt+2, the weights of step kt+3.  At the top of step
        //            kt the activations of step kt+1 (issued at step kt-2) are
        //            written to LDS, so at most the NS + 5 loads of step kt-1
        //            and the 4 weight loads of step kt-2 may be outstanding.
        //   register path with one set (kVg1, RB == 3): per step the
        //            activations of step kt+2 (registers), the scale slot of
        //            step kt+2, the weights of step kt+2.  At the top of step
        //            kt the activations of step kt+1 (issued at step kt-1, the
        //            step's oldest loads) are written to LDS: only the scale
        //            and the 4 weight loads of step kt-1 may be outstanding.
        static_assert(RB >= 2 && RB <= 4, "wait counts are derived for rings of 2 to 4 sets");
        static_assert(!kVg || RB == 4, "the register path's wait count is derived for RB == 4");
        static_assert(!kVg1 || RB == 3, "the one-set register path's wait count is derived for RB == 3");
        wait_vmcnt<kVg ? NS + 9 : (kVg1 ? 5 : (RB == 4 ? 8 : (RB == 3 ? 4 : 0)))>();
        // the weights of this step have landed: pin every use of them below
        // the wait (the loads were asm, invisible to the compiler's waits)
        pin(cur);
        if constexpr (kVg || kVg1) {
            // activations of step kt+1 -> LDS stage (kt+1) % 3, the slab
            // layout the DMA would give (lane l's 16 bytes at 16 l); that
            // stage was last read at step kt-2, which every wave has left
            pin_av<NS>(av_w);
            uint8_t* stw = smem + ((kt + 1) % kNS) * kStageBytes + 8 * wave * 128 + 16 * lane;
#pragma unroll
            for (int sl = 0; sl < NS; sl++) *(u32x4*)(stw + 64 * sl * 128) = av_w[sl];
        }
        bare_barrier();
        STEP_ADDR(kt + 2, kt + RB - 1, kt + (kVg1 ? 2 : 3));
        auto tile_issued = [&](int rt) __attribute__((always_inline)) {
            for (int sl = 0; sl < kSl; sl++)
                if ((sl * R) / kSl == rt) issue_slot(rc, sl, SLOT_ARGS, refill, av_l);
        };
        compute(rc, cur, kt, tile_issued);
    };
    // The weight registers are written by asm loads the compiler cannot see
    // as pending, so nothing may copy them before their wait: the prologue
    // sits inside each instantiation, next to its loop, so the register
    // sets are defined and consumed in one place with no moves between.
    auto main_loop = [&](auto rc) __attribute__((always_inline)) {
        constexpr int R = decltype(rc)::value;
        constexpr int RB = R <= 12 ? kRbSmall : kRbLarge;
        const std::integral_constant<int, RB> rbc;
        // only the live token tiles' accumulators exist during the loop
#pragma unroll
        for (int i = 0; i < R; i++)
            for (int j = 0; j < 2; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
        Frag bs[RB];
        constexpr int NS = (R + 3) / 4;
        constexpr bool kVg = kScaledA && R <= (DT == DT_MX ? kVgMaxRMx : kVgMaxR);
        constexpr bool kVg1 = DT == DT_FP8 && R > kVgMaxR;
        u32x4 av[2][4];  // register path: activations of odd / even K-steps (kVg1: set 0 only)
        if constexpr (kVg1) {
            // prologue of the one-set register path: activations, scale and
            // weights of step 0; the activations -> LDS stage 0 once landed
            // (the scale and weight loads may be outstanding); then those of
            // step 1.  Step j then issues the activations, scale and weights
            // of step j+2.
            {
                STEP_ADDR(0, 0, 0);
                for (int sl = 0; sl < NS + 5; sl++) issue_slot(rc, sl, SLOT_ARGS, bs[0], av[0]);
            }
            wait_vmcnt<5>();
            pin_av<NS>(av[0]);
            {
                uint8_t* stw = smem + 8 * wave * 128 + 16 * lane;
#pragma unroll
                for (int sl = 0; sl < NS; sl++) *(u32x4*)(stw + 64 * sl * 128) = av[0][sl];
            }
            {
                STEP_ADDR(1, 1, 1);
                for (int sl = 0; sl < NS + 5; sl++) issue_slot(rc, sl, SLOT_ARGS, bs[1], av[0]);
            }
            lds_wait();  // stage 0 written before step 0's barrier
        } else if constexpr (kVg) {
            // prologue of the register path: groups (activations, scale,
            // weights) of steps 0 and 1; the activations of step 0 -> LDS
            // stage 0 once landed (the NS + 10 newer loads may be
            // outstanding); then the activations and weights of step 2
            // (set 0 is free again).  Step j then issues the activations
            // and weights of step j+3 and the scale of step j+2.
            static_for<2>([&](auto ic) __attribute__((always_inline)) {
                constexpr int i = decltype(ic)::value;
                STEP_ADDR(i, i, i);
                for (int sl = 0; sl < NS + 5; sl++) issue_slot(rc, sl, SLOT_ARGS, bs[i], av[i]);
            });
            wait_vmcnt<NS + 10>();
            pin_av<NS>(av[0]);
            {
                uint8_t* stw = smem + 8 * wave * 128 + 16 * lane;
#pragma unroll
                for (int sl = 0; sl < NS; sl++) *(u32x4*)(stw + 64 * sl * 128) = av[0][sl];
            }
            {
                STEP_ADDR(2, 2, 2);
                for (int sl = 0; sl < NS + 5; sl++)
                    if (sl != NS) issue_slot(rc, sl, SLOT_ARGS, bs[2], av[0]);
            }
            lds_wait();  // stage 0 written before step 0's barrier
        } else {
            // prologue, in the steady-state issue order: per step the
            // activation slots (steps 0, 1) before the weight slots (steps
            // 0..RB-2)
            static_for<(RB - 1 > 2 ? RB - 1 : 2)>([&](auto ic) __attribute__((always_inline)) {
                constexpr int i = decltype(ic)::value;
                constexpr int kAS = NS + (kScaledA ? 1 : 0);
                STEP_ADDR(i, i, i);
                for (int sl = 0; sl < kAS + 4; sl++)
                    if (sl < kAS ? i < 2 : i < RB - 1) issue_slot(rc, sl, SLOT_ARGS, bs[i < RB ? i : 0], av[0]);
            });
        }
        // whole groups of RB steps, then the < RB remaining ones (the loop's
        // back edge is taken only after a full group, so no path re-enters
        // it with a ring set still in flight that the next group reuses);
        // kt is a multiple of RB at every group start (RB is even on the
        // register path, so kt's parity is ST's)
        int kt = 0;
        for (; kt + RB <= nk; kt += RB) {
            static_for<RB>([&](auto stc) __attribute__((always_inline)) {
                constexpr int ST = decltype(stc)::value;
                step(stc, rc, rbc, kt + ST, bs[ST], bs[(ST + RB - 1) % RB], av[kVg1 ? 0 : (ST + 1) & 1],
                     av[kVg1 ? 0 : (ST + 1) & 1]);
            });
        }
        // the tail, nested: tail step ST runs only after tail step ST-1 (no
        // control-flow path reaches a step without the loads of the one
        // before it)
        auto tail = [&](auto self, auto stc) __attribute__((always_inline)) {
            constexpr int ST = decltype(stc)::value;
            if constexpr (ST < RB - 1) {
                if (kt + ST < nk) {
                    step(stc, rc, rbc, kt + ST, bs[ST], bs[(ST + RB - 1) % RB], av[kVg1 ? 0 : (ST + 1) & 1],
                         av[kVg1 ? 0 : (ST + 1) & 1]);
                    self(self, std::integral_constant<int, ST + 1>());
                }
            }
        };
        tail(tail, std::integral_constant<int, 0>());
        // drain the trailing (out-of-range) prefetches before the ring and
        // the weight registers are reused
        wait_vmcnt<0>();
        static_for<RB>([&](auto ic) __attribute__((always_inline)) { pin(bs[decltype(ic)::value]); });
        if constexpr (kVg || kVg1) {
            pin_av<NS>(av[0]);
            if constexpr (kVg) pin_av<NS>(av[1]);
        }
#pragma unroll
        for (int i = R; i < 16; i++)
            for (int j = 0; j < 2; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    };
#undef STEP_ADDR
#undef SLOT_ARGS
    // The loop is instantiated per live token-tile count: fp8 and MX (the
    // layer's headline paths, where an expert's 128 +- 11 rows would
    // otherwise be rounded up to 192) in steps of one 16-row tile, the fp32
    // path in groups of four.
    const int ntiles = (rows + 15) / 16;  // 1..16, uniform
    if constexpr (kScaledA) {
        static_for<16>([&](auto ic) __attribute__((always_inline)) {
            constexpr int R = decltype(ic)::value + 1;
            if (ntiles == R) main_loop(std::integral_constant<int, R>());
        });
    } else {
        switch ((ntiles + 3) / 4) {
            case 1: main_loop(std::integral_constant<int, 4>()); break;
            case 2: main_loop(std::integral_constant<int, 8>()); break;
            case 3: main_loop(std::integral_constant<int, 12>()); break;
            default: main_loop(std::integral_constant<int, 16>()); break;
        }
    }
    if (MODE == MODE_DOWN && tid < kBM) {
        ((int*)(smem + kRowInfoOff))[tid] = row_slot;
        ((float*)(smem + kRowInfoOff))[kBM + tid] = row_w;
    }
    __syncthreads();  // every wave is done with the ring before it is reused; row info in LDS

    // ---- epilogues (LDS staging for coalesced 16-byte stores), 128 rows
    //      per pass; every wave holds all rows of its columns ----
    float* Tb = (float*)smem;
    const int er = tid >> 2, pp = tid & 3;  // staged row, 32-column part
    if (MODE == MODE_UP) {
#pragma unroll
        for (int half = 0; half < 2; half++) {
            if (128 * half >= rows) continue;  // uniform; unrolled so acc[] stays in registers
            if (half) __syncthreads();
#pragma unroll
            for (int r8 = 0; r8 < 8; r8++) {
                const int rt = 8 * half + r8;
                if (rt >= ntiles) continue;  // uniform: no live row in this tile
                f32x4 hv;
                for (int i = 0; i < 4; i++) {
                    const float gv = acc[rt][0][i], uv = acc[rt][1][i];
                    if constexpr (DT == DT_FP8) {
                        // gv = -log2(e) g: h' = gv u / (1 + 2^gv) = -log2(e) h
                        // (the quantisation below takes the constant back)
                        hv[i] = gv * uv * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gv));
                    } else {
                        // fp32 keeps the reference's expf and IEEE division
                        // (naive_moe.cu:297-310); MX uses the hardware exp2
                        // and reciprocal (~1 ulp each)
                        const float silu = DT == DT_F32 ? gv / (1.0f + expf(-gv))
                                                        : gv * __builtin_amdgcn_rcpf(1.0f + __expf(-gv));
                        hv[i] = silu * uv;
                    }
                }
                *(f32x4*)&Tb[(16 * r8 + r16) * kEpiPitch + 16 * wave + 4 * q] = hv;
            }
            __syncthreads();
            const int rr = 128 * half + er;
            // the four lanes of a row (one quad: the shuffles below stay in
            // it) take the branch together; a wave past the live rows skips
            // the reads, the requantisation and the stores
            if (rr >= rows) continue;
            const int col = nt * 128 + 32 * pp;
            const bool ok = col < g.n_out;
            // eight unconditional 16-byte reads (the staged row is in LDS
            // whether or not it is stored), zeroed where not stored.  Parts
            // pp and pp + 2 of a row lie 128 bytes apart, on the same banks,
            // so parts 2 and 3 read their columns rotated by 16: v[s] holds
            // column (s + 16 rot) mod 32, and the stores below undo it
            const int rot = pp >> 1;
            float v[32];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const f32x4 t = *(const f32x4*)&Tb[er * kEpiPitch + 32 * pp + 4 * ((j + 4 * rot) & 7)];
                for (int i = 0; i < 4; i++) v[4 * j + i] = ok ? t[i] : 0.0f;
            }
            const size_t pos = (size_t)row0 + rr;
            if (DT == DT_FP8) {
                // the staged values are h' = -log2(e) h: amax(h) = ln2 amax(h'),
                // and h * inv = h' * (-ln2 inv)
                float amax = 0.0f;
                for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
                amax = fmaxf(amax, __shfl_xor(amax, 1, kWave));
                amax = fmaxf(amax, __shfl_xor(amax, 2, kWave));
                amax *= kLn2;
                const float s = amax > 0.0f ? __fdiv_rn(amax, 448.0f) : 1.0f;
                // q = h * (1/s): one correctly rounded reciprocal per block
                // instead of 32 divisions (codes may differ from h / s by one
                // step where h / s lies within an ulp of an e4m3 midpoint);
                // |h / s| <= 448 up to rounding, which RNE takes to 448, so the
                // conversion needs no clamp
                const float inv = -kLn2 * __fdiv_rn(1.0f, s);
                if (ok) {
                    u32x4 o0, o1;
                    for (int k = 0; k < 4; k++) {
                        o0[k] = f32x4_to_e4m3x4_noclamp(v[4 * k] * inv, v[4 * k + 1] * inv,
                                                        v[4 * k + 2] * inv, v[4 * k + 3] * inv);
                        o1[k] = f32x4_to_e4m3x4_noclamp(v[16 + 4 * k] * inv, v[16 + 4 * k + 1] * inv,
                                                        v[16 + 4 * k + 2] * inv, v[16 + 4 * k + 3] * inv);
                    }
                    uint8_t* dst = g.out + pos * g.n_out + col;
                    *(u32x4*)(dst + 16 * rot) = o0;
                    *(u32x4*)(dst + 16 - 16 * rot) = o1;
                    if (pp == 0) g.out_scale[(size_t)nt * g.out_scale_rows + pos] = s;
                }
            } else if (DT == DT_MX) {
                // MXFP8 (OCP MX): the thread's 32 columns are one block;
                // E8M0 exponent = floor(log2 amax) - 8 (E4M3's largest
                // binade), clamped to [0, 254]; codes = e4m3(v * 2^(127 - E)),
                // an exact power-of-two scaling
                float amax = 0.0f;
                for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
                const int e8 = min(max((int)((__float_as_uint(amax) >> 23) & 0xff) - 8, 0), 254);
                const float inv = __builtin_amdgcn_ldexpf(1.0f, 127 - e8);
                if (ok) {
                    u32x4 o0, o1;
                    for (int k = 0; k < 4; k++) {
                        o0[k] = f32x4_to_e4m3x4(v[4 * k] * inv, v[4 * k + 1] * inv,
                                                v[4 * k + 2] * inv, v[4 * k + 3] * inv);
                        o1[k] = f32x4_to_e4m3x4(v[16 + 4 * k] * inv, v[16 + 4 * k + 1] * inv,
                                                v[16 + 4 * k + 2] * inv, v[16 + 4 * k + 3] * inv);
                    }
                    uint8_t* dst = g.out + pos * g.n_out + col;
                    *(u32x4*)(dst + 16 * rot) = o0;
                    *(u32x4*)(dst + 16 - 16 * rot) = o1;
                    ((uint8_t*)g.out_scale)[((size_t)(col / 128) * g.out_scale_rows + pos) * 4 + (col / 32) % 4] =
                        (uint8_t)e8;
                }
            } else {
                if (ok) {
                    float* dst = (float*)g.out + pos * g.n_out + col;
                    for (int k = 0; k < 8; k++)
                        *(f32x4*)(dst + 4 * ((k + 4 * rot) & 7)) =
                            (f32x4){v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
                }
            }
        }
    } else {
        // lane (q, r16) holds output columns n0 + 32w + 16ct + 4q .. +3 of
        // token row 16 rt + r16; the row's slot and routing weight come from
        // LDS (staged in the prologue)
        const int* s_slot = (const int*)(smem + kRowInfoOff);
        const float* s_wt = (const float*)(smem + kRowInfoOff) + kBM;
        if (DT == DT_F32) {
            // fp32 rows (the fp32 layer, the reference's format): 16-byte
            // stores straight from the accumulators
#pragma unroll
            for (int rt = 0; rt < 16; rt++) {
                if (16 * rt >= rows) continue;  // uniform; unrolled so acc[] stays in registers
                const int r = 16 * rt + r16;
                if (r >= rows) continue;
                const size_t sl = (size_t)s_slot[r];
                const float wgt = s_wt[r];
#pragma unroll
                for (int ct = 0; ct < 2; ct++) {
                    const int n = nt * 256 + 32 * wave + 16 * ct + 4 * q;
                    if (n >= g.n_out) continue;
                    *(f32x4*)((float*)g.out + ks * g.out_split_stride + sl * g.n_out + n) = acc[rt][ct] * wgt;
                }
            }
        } else {
            // fp8 / MX (bf16 rows): the weighted rows are staged through the (now idle) ring,
            // 128 rows per pass as bf16, then every thread stores 16
            // contiguous bytes: one instruction writes two full 512-byte row
            // segments instead of 16 rows x 32 bytes.
            // Staging write: lane (q, r16) holds columns 4q..4q+3 of both
            // column tiles.  v_permlane16_swap exchanges lane group q = 1's
            // ct = 0 half with group q = 0's ct = 1 half (and likewise 3 / 2),
            // so each lane then holds 8 consecutive columns, 16 * (q & 1) +
            // 8 * (q >> 1) onwards, of one tile, and writes them as one 16-byte
            // piece.  With a 528-byte pitch (132 dwords, 4 mod 64) the 16 rows
            // of a lane group land on 16 distinct 4-bank groups.
            constexpr int kPitch = 528;
            uint8_t* stg = smem;
            const int col = 32 * wave + 16 * (q & 1) + 8 * (q >> 1);
#pragma unroll
            for (int half = 0; half < 2; half++) {
                if (128 * half >= rows) continue;  // uniform
                if (half) __syncthreads();          // pass 0's reads are done
#pragma unroll
                for (int r8 = 0; r8 < 8; r8++) {
                    const int rt = 8 * half + r8;
                    if (rt >= ntiles) continue;  // uniform: no live row in this tile
                    const float wgt = s_wt[16 * rt + r16];
                    const f32x4 v0 = acc[rt][0] * wgt, v1 = acc[rt][1] * wgt;
                    const auto s0 = __builtin_amdgcn_permlane16_swap(pack_bf16x2(v0[0], v0[1]),
                                                                     pack_bf16x2(v1[0], v1[1]), false, false);
                    const auto s1 = __builtin_amdgcn_permlane16_swap(pack_bf16x2(v0[2], v0[3]),
                                                                     pack_bf16x2(v1[2], v1[3]), false, false);
                    *(u32x4*)(stg + (16 * r8 + r16) * kPitch + col * 2) = (u32x4){s0[0], s1[0], s0[1], s1[1]};
                }
                lds_barrier();
    #pragma unroll
                for (int j = 0; j < 8; j++) {
                    if (128 * half + 16 * j >= rows) break;  // uniform: rows 16j.. of the pass are past the tile
                    const int c = tid + 512 * j;       // 16-byte chunk of the pass
                    const int rr = c >> 5, ch = c & 31;  // row in the pass, chunk in the row
                    const int r = 128 * half + rr;
                    const int n = nt * 256 + 8 * ch;
                    if (r < rows && n < g.n_out) {
                        const u32x4 v = *(const u32x4*)(stg + rr * kPitch + 16 * ch);
                        *(u32x4*)(g.out + ((size_t)s_slot[r] * g.n_out + n) * 2) = v;
                    }
                }
            }
        }
    }
}

// ---------------------------------------------------------------- launch
template <int DT, int MODE, bool PK>
int launch_gemm_variant(const GemmArgs& g, long max_tiles, hipStream_t st) {
    {
        const int rc = ensure_dynamic_lds((const void*)grouped_gemm_kernel<DT, MODE, PK>, kGemmLds);
        if (rc != AMDMOE_OK) return rc;
    }
    long work = max_tiles * g.n_tiles_n * (MODE == MODE_DOWN && DT == DT_F32 ? max(g.k_splits, 1) : 1);
    long grid = 8 * ceil_div(work, 8);
    if (grid == 0) return AMDMOE_OK;
    AMDMOE_CHECK_ARG(grid < (1L << 31), "grouped gemm: grid too large (%ld)", grid);
    hipLaunchKernelGGL((grouped_gemm_kernel<DT, MODE, PK>), dim3((unsigned)grid), dim3(512), kGemmLds,
                       st, g);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

// defined (explicitly instantiated) in the moe_gemm_<type>.hip files
#define AMDMOE_GEMM_VARIANT(DT, MODE, PK) \
    extern template int launch_gemm_variant<DT, MODE, PK>(const GemmArgs&, long, hipStream_t);
AMDMOE_GEMM_VARIANT(DT_F32, MODE_UP, false)
AMDMOE_GEMM_VARIANT(DT_F32, MODE_DOWN, false)
AMDMOE_GEMM_VARIANT(DT_FP8, MODE_UP, false)
AMDMOE_GEMM_VARIANT(DT_FP8, MODE_UP, true)
AMDMOE_GEMM_VARIANT(DT_FP8, MODE_DOWN, false)
AMDMOE_GEMM_VARIANT(DT_FP8, MODE_DOWN, true)
AMDMOE_GEMM_VARIANT(DT_MX, MODE_UP, true)
AMDMOE_GEMM_VARIANT(DT_MX, MODE_DOWN, true)
#undef AMDMOE_GEMM_VARIANT

}  // namespace amdmoe
