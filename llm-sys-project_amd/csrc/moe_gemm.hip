// R3/R4/R5 -- grouped expert GEMM launch: validates the operands and picks
// the kernel variant (the kernel itself is in moe_gemm.hpp).
#include "moe_gemm.hpp"

namespace amdmoe {

// ---------------------------------------------------------------- launch
// Upper bound of M-tiles of at most BM rows for P routed rows over E experts.
long max_mtiles(long P, int E, int BM) { return P / BM + (P < E ? P : E); }

int launch_grouped_gemm(int dt, int mode, const GemmArgs& g, long max_tiles, hipStream_t st) {
    // operands stay below 2 GiB so the out-of-range voffset (2^31) always
    // fails the buffer range check
    const long lim = 0x7FFFFFF0L;
    AMDMOE_CHECK_ARG(g.a_bytes <= lim && g.b_expert_bytes <= lim && g.a_scale_bytes <= lim,
                     "grouped gemm: an operand exceeds 4 GiB (A %ld, expert %ld bytes)", g.a_bytes,
                     g.b_expert_bytes);
    AMDMOE_CHECK_ARG((dt != DT_FP8 && dt != DT_MX) || g.K / 128 <= kMaxKb, "grouped gemm: K=%d too large for fp8 / MX", g.K);
    AMDMOE_CHECK_ARG(!g.b_packed || dt == DT_FP8 || dt == DT_MX || dt == DT_BF16, "grouped gemm: packed weights are fp8 / bf16 / MX only");
    AMDMOE_CHECK_ARG(dt != DT_MX || g.b_packed, "grouped gemm: MX weights must be packed");
    {
        const int es = dt == DT_F32 ? 4 : (dt == DT_BF16 ? 2 : 1);
        const long nk = (long)g.K * es / 128;
        AMDMOE_CHECK_ARG(g.k_splits <= 1 || (mode == MODE_DOWN && (dt == DT_F32 || dt == DT_BF16) &&
                                             nk % g.k_splits == 0 && g.out_split_stride > 0),
                         "grouped gemm: a K split (%d) needs DOWN with fp32 rows and whole K-steps per split",
                         g.k_splits);
    }
    AMDMOE_CHECK_ARG(dt != DT_MX || g.b_mx_scale_expert_bytes <= lim, "grouped gemm: MX scales exceed 2 GiB");
    if (dt == DT_MX) return mode == MODE_UP ? launch_gemm_variant<DT_MX, MODE_UP, true>(g, max_tiles, st)
                                            : launch_gemm_variant<DT_MX, MODE_DOWN, true>(g, max_tiles, st);
    if (dt == DT_F32) return mode == MODE_UP ? launch_gemm_variant<DT_F32, MODE_UP, false>(g, max_tiles, st)
                                             : launch_gemm_variant<DT_F32, MODE_DOWN, false>(g, max_tiles, st);
    if (dt == DT_BF16) return launch_gemm_bf16_w4(mode, g, max_tiles, st);
    if (g.b_packed) return mode == MODE_UP ? launch_gemm_variant<DT_FP8, MODE_UP, true>(g, max_tiles, st)
                                           : launch_gemm_variant<DT_FP8, MODE_DOWN, true>(g, max_tiles, st);
    return mode == MODE_UP ? launch_gemm_variant<DT_FP8, MODE_UP, false>(g, max_tiles, st)
                           : launch_gemm_variant<DT_FP8, MODE_DOWN, false>(g, max_tiles, st);
}

}  // namespace amdmoe
