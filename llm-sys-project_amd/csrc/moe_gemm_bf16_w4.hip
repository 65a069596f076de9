// Grouped GEMM for bf16 weights (packed or row-major), one wave per SIMD:
// 4 waves x 64 weight rows per work item (the bf16 layers' GEMMs: Mixtral,
// the medium bf16 configuration).
//
// Work items, K-step order, weight fragments, activation slabs and the
// arithmetic are those of the template grouped_gemm_kernel in moe_gemm.hpp
// (same bf16 16x16x32 MFMA, same operand lanes, same K-step rotation and the
// same epilogue arithmetic), whose bf16 instantiations it replaced with
// bit-identical outputs; what differs is the wave layout.  There every one
// of 8 waves multiplies 32 weight rows
// by all of the tile's token rows, so each token fragment read from LDS
// feeds 4 MFMAs: per 64-element K-step of a full M-tile a CU reads 8 x 32 KB
// of fragments (2048 cycles at 128 B per clock) against 2048 MFMA cycles per
// SIMD.  Here a wave owns 64 weight rows (4 column tiles), every fragment
// feeds 8 MFMAs, and a K-step reads 4 x 32 KB.  The 16 x 4 accumulator tiles
// (256 registers) live in AGPRs: one wave per SIMD may use all 512
// registers of the lane.  Measured at Mixtral T=4096: UP 1.59 -> 1.52-1.54
// ms, DOWN 0.92 -> 0.83-0.84 ms.  A full-tile K-step then takes ~2630
// cycles against 2048 of MFMAs: the single wave's MFMA issue alone (a loop
// of just the MFMAs) takes ~2290, the fragment reads add ~245, the loads ~90.
#include "moe_gemm.hpp"

namespace amdmoe {

constexpr int kW4Threads = 256;
constexpr int kW4Stage = kMTile * 128;              // 256 rows x one 64-element bf16 K-step
constexpr int kW4Ring = 3;                          // activations run 2 K-steps ahead
constexpr int kW4RowInfo = kW4Ring * kW4Stage;      // DOWN: [256] slot, [256] weight
constexpr int kW4Lds = kW4RowInfo + kMTile * 8;     // 100352 bytes
constexpr int kW4Pitch = 272;                       // UP staging: bytes per bf16 row of 128 columns
constexpr int kW4Rb = 3;                            // weight register sets (2 K-steps in flight)
constexpr int kW4La = 2;                            // token tiles the fragment reads run ahead
static_assert(kMTile * kW4Pitch <= kW4Ring * kW4Stage, "UP staging fits the ring");

// One K-step of a wave's weights: per column tile the lane's 32 bytes (lo
// 16 B = K elements 8q..8q+7, hi = 32 + 8q.., of row r16).
struct WFrag4 {
    u32x4 q[4][2];
};
__device__ __forceinline__ void pin(WFrag4& f) {
    asm volatile("" : "+v"(f.q[0][0]), "+v"(f.q[0][1]), "+v"(f.q[1][0]), "+v"(f.q[1][1]),
                      "+v"(f.q[2][0]), "+v"(f.q[2][1]), "+v"(f.q[3][0]), "+v"(f.q[3][1]));
}

// c += a b^T (bf16 16x16x32) in place: the accumulator is one AGPR tuple,
// source C and destination alike.  With the builtin the compiler gave the
// unrolled steps' products different AGPRs and copied them back on every
// loop iteration (~65 v_accvgpr moves per K-step).  The compiler does not
// see this as an MFMA: the only readers of the accumulators outside these
// MFMAs (the zeroing writes, the epilogue) are separated from the last MFMA
// by mfma_drain().
__device__ __forceinline__ void mfma_bf16_acc(f32x4& c, const u32x4& a, const u32x4& b) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
// wait states between an MFMA writing an accumulator and any other
// instruction reading or writing it (the ISA asks for at most 18 after an
// 8-pass XDL op; 3 x 8 + 3 issue slots)
__device__ __forceinline__ void mfma_drain() {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
}

// a K-step's scalar addressing: activation (KT_A) and weight (KT_B) steps
struct W4Step {
    __amdgpu_buffer_rsrc_t ra;
    i32x4 rb;
    int so_a, so_b;
    uint8_t* st;
};

// PK: weights in fragment-block order (pack_weights_bf16: each 16-row
// group's K-step is 2 KB, [half][lane][16 B], one 1 KB load per half);
// otherwise row-major (lane (q, r16) reads 16 bytes of row r16 at K offset
// 16q, and 64 + 16q for the hi half)
template <int MODE, bool PK>
__global__ __launch_bounds__(kW4Threads, 1) void grouped_gemm_bf16_w4_kernel(GemmArgs g) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // 0..3

    // ---- work item (XCD-chunked; DOWN may split K over S items) ----
    const int S = MODE == MODE_DOWN ? max(g.k_splits, 1) : 1;
    const int W = (*g.num_tiles) * g.n_tiles_n * S;
    const int per = (W + 7) >> 3;
    const int slot = blockIdx.x >> 3;
    if (slot >= per) return;
    const int w = (blockIdx.x & 7) * per + slot;
    if (w >= W) return;
    const int ntn = g.n_tiles_n * S;
    const int mt0 = w / ntn;
    const int4 tile0 = g.tiles[mt0];
    const int m_tiles = tile0.w & 0xffff, first_tile = mt0 - (tile0.w >> 16);
    const int l_item = w - first_tile * ntn;
    const int ntv = __builtin_amdgcn_readfirstlane(l_item / m_tiles);
    const int mt = first_tile + (l_item - ntv * m_tiles);
    const int nt = S == 1 ? ntv : ntv / S, ks = ntv - nt * S;
    const int4 tile = m_tiles == 1 ? tile0 : g.tiles[mt];
    const int e = __builtin_amdgcn_readfirstlane(tile.x), row0 = __builtin_amdgcn_readfirstlane(tile.y),
              rows = __builtin_amdgcn_readfirstlane(tile.z);
    const int nk_all = (int)((long)g.K * 2 / 128);  // 64-element K-steps of the whole reduction
    const int nk = nk_all / S;
    const int kbase = ks * nk;

    const uint8_t* bexp = g.b + (size_t)e * g.b_expert_bytes;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(g.a, g.a_bytes), ra0 = make_rsrc(g.a, 0);
    const i32x4 rb = make_rsrc_words(bexp, g.b_expert_bytes);
    i32x4 rb0 = rb;
    rb0[2] = 0;

    // ---- activation slabs: slab s of wave w holds rows 32s + 8w .. +7
    //      (1 KB, one 16-byte DMA per lane; chunk c of row r lands at slot
    //      c ^ (r & 7), so a fragment read touches distinct banks) ----
    const int lrow = lane >> 3, lchunk = (lane & 7) ^ lrow;
    uint32_t voff_a[8];
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const int r = 32 * s + 8 * wave + lrow;
        const long arow = MODE == MODE_UP ? (long)g.a_map[row0 + min(r, rows - 1)] : (long)(row0 + r);
        voff_a[s] = r < rows ? (uint32_t)(arow * g.a_row_bytes + 16 * lchunk) : kOob;
    }
    // ---- weight rows of this wave: four column tiles of 16 ----
    //   UP:   ct 0, 1 = gate rows n0 + 32w + 16ct + c, ct 2, 3 = the up rows
    //         I + n0 + 32w + 16(ct - 2) + c of the same output columns
    //   DOWN: ct = rows n0 + 64w + 16ct + c
    const int q = lane >> 4, r16 = lane & 15;
    uint32_t voff_b[4];
#pragma unroll
    for (int ct = 0; ct < 4; ct++) {
        long n;
        bool ok;
        if (MODE == MODE_UP) {
            const int col = nt * 128 + 32 * wave + 16 * (ct & 1) + r16;
            ok = col < g.n_out;
            n = ct < 2 ? col : (long)g.n_out + col;
        } else {
            n = (long)nt * 256 + 64 * wave + 16 * ct + r16;
            ok = n < g.n_out;
        }
        const long nb = PK ? (n - r16) * g.b_row_bytes + 16 * lane : n * g.b_row_bytes + 16 * q;
        voff_b[ct] = ok ? (uint32_t)nb : kOob;
    }
    // DOWN: each row's slot and routing weight, only needed by the epilogue
    // (the loads stay in flight through the main loop)
    int row_slot = 0;
    float row_w = 0.0f;
    if (MODE == MODE_DOWN) {
        const size_t r = (size_t)row0 + min(tid, rows - 1);  // rows >= 1
        row_slot = g.sorted_slot[r];
        row_w = tid < rows ? g.sorted_w[r] : 0.0f;
    }
    __builtin_amdgcn_sched_barrier(0);

    // K-steps in the rotated order of grouped_gemm_kernel (kt0 keyed by the
    // expert); steps past the end (prefetches) read through null descriptors
    const int kt0 = (int)(((unsigned)e * 7u) % (unsigned)nk);
    auto kblk = [&](int kt) __attribute__((always_inline)) {
        int k = kt + kt0;
        k = k >= nk ? k - nk : k;
        return kbase + (k >= nk ? k - nk : k);
    };
    auto addr = [&](int kta, int ktb) __attribute__((always_inline)) {
        W4Step s;
        s.ra = kta < nk ? ra : ra0;
        s.rb = ktb < nk ? rb : rb0;
        s.so_a = kblk(kta) * 128;
        s.so_b = kblk(ktb) * (PK ? 2048 : 128);
        s.st = smem + (kta % kW4Ring) * kW4Stage;
        return s;
    };
    const int off_lo = 16 * (q ^ (r16 & 7)), off_hi = 16 * ((4 + q) ^ (r16 & 7));

    // acc[rt][ct]: lane (q, r16) holds weight rows 4q..4q+3 of column tile
    // ct for token row 16 rt + r16 (C^T = W x^T, as in grouped_gemm_kernel)
    f32x4 acc[16][4];

    auto fence = []() __attribute__((always_inline)) {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    };

    auto main_loop = [&](auto rc) __attribute__((always_inline)) {
        constexpr int R = decltype(rc)::value;  // live token tiles (a multiple of 4)
        constexpr int NS = R / 2;               // activation slabs per wave and step
        constexpr int kSl = NS + 8;             // vector-memory slots per wave and step
        constexpr int RB = kW4Rb;
#pragma unroll
        for (int i = 0; i < R; i++)
            for (int j = 0; j < 4; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
        mfma_drain();  // the zeroing writes before the first MFMA reads them
        WFrag4 bs[RB];
        // slot sl of a step: the activation slabs, then per column tile the
        // lo and hi 1 KB weight loads
        auto issue_slot = [&](auto slc, const W4Step& s, WFrag4& f) __attribute__((always_inline)) {
            constexpr int sl = decltype(slc)::value;
            if constexpr (sl < NS) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    s.ra, (lds_ptr_t)(s.st + (32 * sl + 8 * wave) * 128), 16, voff_a[sl], s.so_a, 0, 0);
            } else {
                constexpr int j = sl - NS, ct = j >> 1;
                if constexpr (j & 1)
                    f.q[ct][1] = buffer_load_b128_async<PK ? 1024 : 64, MODE == MODE_DOWN>(s.rb, voff_b[ct], s.so_b);
                else
                    f.q[ct][0] = buffer_load_b128_async<0, MODE == MODE_DOWN>(s.rb, voff_b[ct], s.so_b);
            }
        };
        // One K-step on ring stage kt % 3 with weights `bf`; the step's
        // prefetch slots go out spread over its token tiles (slot s after
        // tile (s * R) / kSl), activations first.
        auto compute = [&](int kt, const WFrag4& bf, const W4Step& s, WFrag4& refill) __attribute__((always_inline)) {
            uint32_t soff_st = (kt % kW4Ring) * kW4Stage;
            asm volatile("" : "+s"(soff_st));
            const uint8_t* base = smem + soff_st;
            auto load_x = [&](int rt, u32x4& lo, u32x4& hi) __attribute__((always_inline)) {
                const uint8_t* p = base + (16 * rt + r16) * 128;
                lo = *(const u32x4*)(p + off_lo);
                hi = *(const u32x4*)(p + off_hi);
            };
            // fragments are read kW4La tiles ahead of their MFMAs (kW4La + 1
            // register sets)
            constexpr int LA = kW4La < R ? kW4La : R, NB = LA + 1;
            u32x4 xl[NB], xh[NB];
            static_for<LA>([&](auto ic) __attribute__((always_inline)) {
                constexpr int i = decltype(ic)::value;
                load_x(i, xl[i], xh[i]);
            });
            fence();
            static_for<R>([&](auto tc) __attribute__((always_inline)) {
                constexpr int t = decltype(tc)::value;
#pragma unroll
                for (int ct = 0; ct < 4; ct++) mfma_bf16_acc(acc[t][ct], bf.q[ct][0], xl[t % NB]);
#pragma unroll
                for (int ct = 0; ct < 4; ct++) mfma_bf16_acc(acc[t][ct], bf.q[ct][1], xh[t % NB]);
                static_for<kSl>([&](auto slc) __attribute__((always_inline)) {
                    constexpr int sl = decltype(slc)::value;
                    if constexpr ((sl * R) / kSl == t) issue_slot(slc, s, refill);
                });
                if constexpr (t + LA < R) load_x(t + LA, xl[(t + LA) % NB], xh[(t + LA) % NB]);
                fence();
            });
        };
        // Issue order per step kt: the activations of step kt+2, then the
        // weights of step kt+RB-1.
        //   RB == 3: at the top of step kt the loads issued after the
        //            weights of step kt (the last loads of step kt-2, which
        //            follow its activations of step kt) are those of step
        //            kt-1: NS + 8.  The prologue issues A0 W0 A1 W1.
        //   RB == 4: the loads issued after the activations of step kt
        //            (issued at step kt-2) are the weights of step kt+1,
        //            the activations of step kt+1 and the weights of step
        //            kt+2: NS + 16, and the weights of step kt precede the
        //            activations of step kt.  The prologue issues A0 W0 A1
        //            W1 W2; for steps 0 and 1 the same count also waits for
        //            W0 / W1, which the step needs anyway.
        static_assert(RB == 3 || RB == 4, "wait counts are derived for rings of 3 and 4 sets");
        auto step = [&](auto stc, int kt, WFrag4& cur, WFrag4& refill) __attribute__((always_inline)) {
            wait_vmcnt<RB == 3 ? NS + 8 : NS + 16>();
            pin(cur);
            bare_barrier();  // every wave's slabs of step kt have landed; stage (kt+2) % 3 is free
            const W4Step s = addr(kt + 2, kt + RB - 1);
            compute(kt, cur, s, refill);
        };
        {
            const W4Step s = addr(0, 0);
            static_for<kSl>([&](auto slc) __attribute__((always_inline)) { issue_slot(slc, s, bs[0]); });
        }
        {
            const W4Step s = addr(1, 1);
            static_for<kSl>([&](auto slc) __attribute__((always_inline)) { issue_slot(slc, s, bs[1]); });
        }
        if constexpr (RB == 4) {
            const W4Step s = addr(2, 2);
            static_for<kSl>([&](auto slc) __attribute__((always_inline)) {
                if constexpr (decltype(slc)::value >= NS) issue_slot(slc, s, bs[2]);
            });
        }
        int kt = 0;
        for (; kt + RB <= nk; kt += RB) {
            static_for<RB>([&](auto stc) __attribute__((always_inline)) {
                constexpr int ST = decltype(stc)::value;
                step(stc, kt + ST, bs[ST], bs[(ST + RB - 1) % RB]);
            });
        }
        // the < RB remaining steps, nested (a step runs only after the one before it)
        auto tail = [&](auto self, auto stc) __attribute__((always_inline)) {
            constexpr int ST = decltype(stc)::value;
            if constexpr (ST < RB - 1) {
                if (kt + ST < nk) {
                    step(stc, kt + ST, bs[ST], bs[(ST + RB - 1) % RB]);
                    self(self, std::integral_constant<int, ST + 1>());
                }
            }
        };
        tail(tail, std::integral_constant<int, 0>());
        wait_vmcnt<0>();  // the trailing (null) prefetches, before the ring and the registers are reused
        mfma_drain();
        static_for<RB>([&](auto ic) __attribute__((always_inline)) { pin(bs[decltype(ic)::value]); });
#pragma unroll
        for (int i = R; i < 16; i++)
            for (int j = 0; j < 4; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    };
    const int ntiles = (rows + 15) / 16;  // 1..16, uniform
    switch ((ntiles + 3) / 4) {
        case 1: main_loop(std::integral_constant<int, 4>()); break;
        case 2: main_loop(std::integral_constant<int, 8>()); break;
        case 3: main_loop(std::integral_constant<int, 12>()); break;
        default: main_loop(std::integral_constant<int, 16>()); break;
    }
    int* s_slot = (int*)(smem + kW4RowInfo);
    float* s_wt = (float*)(smem + kW4RowInfo) + kMTile;
    if (MODE == MODE_DOWN) {
        s_slot[tid] = row_slot;
        s_wt[tid] = row_w;
    }
    __syncthreads();  // every wave is done with the ring; row info in LDS

    if (MODE == MODE_UP) {
        // h = silu(g) * u (the arithmetic of grouped_gemm_kernel's bf16
        // epilogue), staged as bf16 rows of the N-tile's 128 columns, then
        // 16-byte stores: 16 rows of 16 pieces per pass
        uint8_t* stg = smem;
#pragma unroll
        for (int rt = 0; rt < 16; rt++) {
            if (rt >= ntiles) continue;  // uniform
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const f32x4 gv = acc[rt][c], uv = acc[rt][c + 2];
                float h[4];
                for (int i = 0; i < 4; i++)
                    h[i] = gv[i] * __builtin_amdgcn_rcpf(1.0f + __expf(-gv[i])) * uv[i];
                *(uint2*)(stg + (16 * rt + r16) * kW4Pitch + (32 * wave + 16 * c + 4 * q) * 2) =
                    make_uint2(pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3]));
            }
        }
        __syncthreads();
        const int ch = tid & 15, col = nt * 128 + 8 * ch;
        for (int it = 0; 16 * it < rows; it++) {
            const int rr = 16 * it + (tid >> 4);
            if (rr < rows && col < g.n_out) {
                const u32x4 v = *(const u32x4*)(stg + rr * kW4Pitch + 16 * ch);
                *(u32x4*)(g.out + ((size_t)(row0 + rr) * g.n_out + col) * 2) = v;
            }
        }
    } else {
        // fp32 rows (output rounded once, in the combine): 16-byte stores
        // straight from the accumulators, each row at its slot
#pragma unroll
        for (int rt = 0; rt < 16; rt++) {
            if (16 * rt >= rows) continue;  // uniform
            const int r = 16 * rt + r16;
            if (r >= rows) continue;
            const size_t sl = (size_t)s_slot[r];
            const float wgt = s_wt[r];
#pragma unroll
            for (int ct = 0; ct < 4; ct++) {
                const int n = nt * 256 + 64 * wave + 16 * ct + 4 * q;
                if (n >= g.n_out) continue;
                *(f32x4*)((float*)g.out + ks * g.out_split_stride + sl * g.n_out + n) = acc[rt][ct] * wgt;
            }
        }
    }
}

int launch_gemm_bf16_w4(int mode, const GemmArgs& g, long max_tiles, hipStream_t st) {
    const void* fn = mode == MODE_UP ? (g.b_packed ? (const void*)grouped_gemm_bf16_w4_kernel<MODE_UP, true>
                                                   : (const void*)grouped_gemm_bf16_w4_kernel<MODE_UP, false>)
                                     : (g.b_packed ? (const void*)grouped_gemm_bf16_w4_kernel<MODE_DOWN, true>
                                                   : (const void*)grouped_gemm_bf16_w4_kernel<MODE_DOWN, false>);
    {
        const int rc = ensure_dynamic_lds(fn, kW4Lds);
        if (rc != AMDMOE_OK) return rc;
    }
    const long work = max_tiles * g.n_tiles_n * (mode == MODE_DOWN ? max(g.k_splits, 1) : 1);
    const long grid = 8 * ceil_div(work, 8);
    if (grid == 0) return AMDMOE_OK;
    AMDMOE_CHECK_ARG(grid < (1L << 31), "grouped gemm: grid too large (%ld)", grid);
    void* args[] = {(void*)&g};
    AMDMOE_HIP_TRY(hipLaunchKernel(fn, dim3((unsigned)grid), dim3(kW4Threads), args, kW4Lds, st));
    return AMDMOE_OK;
}

}  // namespace amdmoe
