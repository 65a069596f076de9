// Declarations shared by the library's translation units (kernel launchers
// and the grouped-GEMM argument block).  Not part of the public ABI.
#pragma once

#include <mutex>
#include <set>
#include <utility>

#include "common.hpp"

namespace amdmoe {

// Raises a kernel's dynamic-LDS limit to `bytes` on the current device, once
// per (kernel, device) -- the attribute is per device -- under a lock, so
// concurrent first launches from several threads are safe.
inline int ensure_dynamic_lds(const void* fn, int bytes) {
    static std::mutex mu;
    static std::set<std::pair<const void*, int>> done;
    int dev = -1;
    AMDMOE_HIP_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(mu);
    if (done.count({fn, dev})) return AMDMOE_OK;
    AMDMOE_HIP_TRY(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
    done.insert({fn, dev});
    return AMDMOE_OK;
}

enum { DT_F32 = 0, DT_BF16 = 1, DT_FP8 = 2, DT_MX = 3 };  // DT_MX: MXFP4 weights x MXFP8 activations
enum { MODE_UP = 0, MODE_DOWN = 1 };

constexpr int kMTile = 256;  // rows of one grouped-GEMM M-tile

struct GemmArgs {
    const uint8_t* a;        // A base
    long a_bytes;            // bytes of the whole A array (buffer range)
    long a_row_bytes;        // bytes per A row
    const int* a_map;        // UP: sorted_token (A row of sorted position); DOWN: unused
    const float* a_scale;    // fp8 / MX: [K/128][a_scale_rows] dwords, rows in sorted order
    long a_scale_bytes;      // fp8 / MX: bytes of the whole a_scale array
    long a_scale_rows;       // fp8 / MX: dwords per K-step of a_scale
    const uint8_t* b;        // expert weights base
    long b_expert_bytes;     // bytes per expert
    long b_row_bytes;        // bytes per weight row (K * element size)
    int b_packed;            // weights in 16-row x 128-byte fragment blocks (pack_weights)
    const float* b_scale;    // fp8: [E][b_rows/128][K/128]
    int b_rows;              // weight rows per expert (2I or D)
    int K;                   // reduction length in elements
    int n_out;               // UP: I, DOWN: D
    const int4* tiles;       // M-tiles {expert, first sorted row, rows, 0}
    const int* num_tiles;    // device count of M-tiles
    int n_tiles_n;           // N-tiles per M-tile
    uint8_t* out;            // UP: act [P, I]; DOWN: ypair [T*K, D]
    float* out_scale;        // UP fp8 / MX: act scales [I/128][out_scale_rows] dwords
    long out_scale_rows;     // UP fp8 / MX: dwords per 128-column block of out_scale
    const int* sorted_slot;  // DOWN: flat slot t*K+k of each sorted row
    const float* sorted_w;   // DOWN: routing weight of each sorted row
    int k_splits;            // DOWN with fp32 rows (fp32 / bf16): K split over this many work
                             // items (0 or 1: none); split s writes its partial rows at
                             // out + s * out_split_stride floats
    long out_split_stride;
    // MX only: E8M0 weight scales in fragment order [E][b_rows/16][K/128][64]
    // (a_scale then holds the activations' E8M0 scales, four bytes -- the
    // 32-blocks of a 128-K step -- per dword)
    const uint8_t* b_mx_scale;
    long b_mx_scale_expert_bytes;
};

// moe_permute.hip: dst[kb * P + p] = src[sorted_token[p] * nkb + kb] (4-byte
// elements, p < P): per-row block scales gathered into sorted row order,
// K-step major (the grouped GEMM's a_scale layout)
int launch_gather_row_scales(const uint32_t* src, const int* sorted_token, long P, int T, int nkb,
                             uint32_t* dst, hipStream_t st);

// moe_route.hip
template <typename XT, typename GT>
int launch_route_exact(const XT* x, const GT* wg, const float* bias, int T, int E, int K, int D,
                       int* idx, float* wts, hipStream_t st);
bool route_mfma_supported(int E, int K, int D);
// part: scratch of route_mfma_scratch_bytes(T, E, D, quant) bytes (split-K
// partial logits).  quant: xq [T,D] e4m3 and xs [T,D/128] are also written
// (the 1x128 activation quantisation of x, D % 128 == 0); else both null.
size_t route_mfma_scratch_bytes(int T, int E, int D, bool quant);
int launch_route_mfma(const uint16_t* x, const uint16_t* wg, int T, int E, int K, int D, int* idx,
                      float* wts, float* part, uint8_t* xq, float* xs, hipStream_t st);

// moe_permute.hip
// scratch: permute_scratch_bytes(T, E) bytes, or nullptr (single-launch
// kernel); permute_scratch_bytes returns 0 where only the latter applies
size_t permute_scratch_bytes(int T, int E);
// wts / sorted_w: optional (both or neither): sorted_w[row] = wts[slot of row]
// rs_src / rs_dst: optional (both or neither): the row scales of
// launch_gather_row_scales (rs_nkb per token) in sorted row order, fused
// into the decode-sized single-launch permutation
int launch_permute(const int* idx, int T, int K, int E, int BM, int* counts, int* offsets,
                   int* sorted_token, int* sorted_slot, int4* tiles, int* num_tiles,
                   int* scratch, const float* wts, float* sorted_w, hipStream_t st,
                   const uint32_t* rs_src = nullptr, int rs_nkb = 0, uint32_t* rs_dst = nullptr);
int launch_gather_one(const float* x, const int* idx, int T, int K, int E, int D, int expert,
                      float* gathered, int* token_map, int* count, hipStream_t st);

// moe_quant.hip
int launch_quant_rows(const uint16_t* x, long rows, int cols, uint8_t* q, float* scale,
                      hipStream_t st);
int launch_quant_weight(const float* w, long rows, int cols, const float* u, uint8_t* q,
                        float* scale, hipStream_t st);

// moe_gemm.hip
long max_mtiles(long P, int E, int BM = kMTile);
int launch_grouped_gemm(int dt, int mode, const GemmArgs& g, long max_tiles, hipStream_t st);
// moe_gemm_bf16_w4.hip: the bf16 packed-weight GEMMs on one wave per SIMD
int launch_gemm_bf16_w4(int mode, const GemmArgs& g, long max_tiles, hipStream_t st);

// moe_generic.hip: fp32 UP + DOWN + combine for any D and I (the forward's
// tail when D or I is not a multiple of 32), over the permutation's M-tiles
int launch_experts_f32_any(const float* x, const float* w1, const float* w2, int T, int E, int K,
                           int D, int I, const int4* tiles, const int* num_tiles, long max_tiles,
                           const int* sorted_token, const int* sorted_slot, const float* sorted_w,
                           const int* idx, float* act, float* ypair, float* y, hipStream_t st);

// moe_mx.hip: OCP MX quantisers and the MXFP4 weight packer
int launch_quant_weight_mxfp4(const float* w, long rows, int cols, uint8_t* q, uint8_t* s,
                              hipStream_t st);
int launch_quant_rows_mxfp8(const uint16_t* x, long rows, int cols, uint8_t* q, uint8_t* s,
                            hipStream_t st);
int launch_pack_mxfp4(const uint8_t* q, const uint8_t* s, long E, int N, int K, uint8_t* qp,
                      uint8_t* sp, hipStream_t st);

// moe_pack.hip: [E][N][K]-byte weights -> fragment-block order (N % 16 == 0,
// K % 128 == 0)
int launch_pack_weights(const uint8_t* w, long E, long N, long K, uint8_t* out, hipStream_t st);

// moe_combine.hip: ypair rows fp32 or bf16 (DT_F32 / DT_BF16), y fp32 or bf16;
// nsplit fp32 partial row sets of T*K*D floats each (a split down projection)
int launch_combine(int ypair_dt, int out_dt, const void* ypair, const int* idx, int T, int K, int E,
                   int D, void* y, hipStream_t st, int nsplit = 1);
int launch_naive_gemm_f32(const float* A, const float* B, float* C, int M, int N, int K,
                          hipStream_t st);
int launch_swiglu_f32(const float* gate, const float* up, float* out, int n, hipStream_t st);
int launch_scatter_f32(const float* expert_out, const int* token_map, const float* wts,
                       const int* idx, int expert, float* out, int count, int T, int K, int D,
                       hipStream_t st);

// dsa.hip
// scratch: dsa_f32_scratch_bytes(Q, H, S) bytes of fp32 scores (0 bytes /
// nullptr when the scores fit in LDS)
size_t dsa_f32_scratch_bytes(int Q, int H, int S);
int launch_dsa_f32(const float* qn, const float* qp, const float* kc, const float* kp,
                   const float* v, const int* idx, float* out, int Q, int H, int Dc, int Dp, int S,
                   int N, float* scratch, hipStream_t st);
// scratch: dsa_paged_scratch_bytes(Q, H, S) bytes (split partials), may be
// 0 bytes / nullptr when that is 0
size_t dsa_paged_scratch_bytes(int Q, int H, int S);
// dsa_indexer.hip: lightning-indexer scores [Q, max_seq] (scratch) and the
// topk positions per query
size_t dsa_indexer_scratch_bytes(int Q, int max_seq, int topk);
int launch_dsa_indexer(const uint8_t* qc, const float* qs, const float* hw, const uint8_t* kc,
                       long kc_rows, const float* ks, const int* page_table, const int* seq_len,
                       int Q, int Hi, int page, int pages_per_seq, int max_seq, int topk,
                       float* scores, int* out, void* scratch, size_t scratch_bytes, hipStream_t st);
int launch_dsa_bf16_paged(const uint16_t* qn, const uint16_t* qp, const uint16_t* cache,
                          long cache_tokens, const int* page_table, const int* logical,
                          uint16_t* out, int Q, int H, int Dc, int Dp, int S, int page,
                          int pages_per_seq, void* scratch, size_t scratch_bytes, hipStream_t st);

// dsa_stages.hip: the reference's DSA stage functions (fp32)
int launch_dsa_gather(const float* kc, const float* kp, const float* v, const int* idx, float* gkc,
                      float* gkp, float* gv, int Q, int S, int Dc, int Dp, long N, hipStream_t st);
// parts: 1 = the K_c dot, 2 = the K_p dot, 3 = both in one accumulator
int launch_dsa_dot(const float* qn, const float* qp, const float* kc, const float* kp,
                   float* scores, int Q, int H, int S, int Dc, int Dp, int parts, hipStream_t st);
int launch_dsa_softmax(float* scores, long rows, int S, hipStream_t st);
int launch_dsa_output_proj(const float* attn, const float* v, float* out, int Q, int H, int S,
                           int Dc, hipStream_t st);

}  // namespace amdmoe
