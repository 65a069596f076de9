/*
 * amdmoe.h -- C ABI of the MI355X (gfx950) MoE forward and DSA decode library.
 *
 * Plain C: POD structs, raw device pointers, sizes, a hipStream_t passed as
 * void* (NULL = the null stream).  No torch types, no C++ in the signatures.
 *
 * Conventions shared by every entry point:
 *   - All tensor pointers are DEVICE pointers owned by the caller, row-major,
 *     laid out as the reference documents (kernels/moe/naive_moe.cuh:21-76,
 *     kernels/dsa/naive_dsa.cuh:20-87).
 *   - Every call is asynchronous on `stream`; none synchronises the host.
 *   - Return 0 (AMDMOE_OK) on success, a positive AMDMOE_ERR_* code
 *     otherwise; amdmoe_last_error() then holds a message (per host thread).
 *     The reference aborts instead (utils/cuda_utils.cuh:13-21); the C++
 *     drop-in header include/naive_moe.h restores that behaviour.
 *   - `workspace` may be NULL: the library then uses its own per-device
 *     workspace, grown on demand (that first call allocates).  A non-NULL
 *     workspace must hold amdmoe_moe_workspace_bytes() bytes; calls that
 *     share one workspace must be ordered on one stream.
 *   - Entry points without a workspace argument that need scratch (the
 *     split-K routing of amdmoe_moe_gate_bf16/_fp8, amdmoe_moe_permute,
 *     amdmoe_dsa_decode_bf16_paged, amdmoe_dsa_forward_f32 with S > 16384,
 *     amdmoe_dsa_indexer_topk_fp8 selecting in parts)
 *     use a per-device buffer of their own family (routing, permutation,
 *     decode, fp32 DSA, indexer; none is shared with the MoE forward's workspace or
 *     with another family).  A call that must grow that buffer frees and
 *     allocates it, which waits for the device; calls of one family that use
 *     the buffer must be ordered on one stream (concurrent calls of one
 *     family on two streams race on it).
 *   - bf16 tensors are passed as uint16_t (bfloat16 bit patterns), fp8 as
 *     uint8_t OCP e4m3 ("E4M3FN") codes.
 */
#ifndef AMDMOE_H
#define AMDMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AMDMOE_OK 0
#define AMDMOE_ERR_INVALID 1   /* bad argument / unsupported shape            */
#define AMDMOE_ERR_HIP 2       /* a HIP runtime call or kernel launch failed   */
#define AMDMOE_ERR_WORKSPACE 3 /* caller workspace smaller than required      */

/* Same member order and types as the reference (naive_moe.cuh:9-15), so a
 * positional aggregate initialiser {T, E, K, D, I} means the same thing. */
typedef struct MoeConfig {
    int num_tokens;       /* T */
    int num_experts;      /* E */
    int top_k;            /* K */
    int hidden_dim;       /* D */
    int intermediate_dim; /* I */
} MoeConfig;

/* Same member order and types as the reference (naive_dsa.cuh:9-17). */
typedef struct DsaConfig {
    int num_queries;         /* Q  */
    int num_heads;           /* H  */
    int head_dim_compressed; /* Dc */
    int head_dim_positional; /* Dp */
    int num_selected_kv;     /* S  */
    int page_size;           /* P  */
    int total_kv_tokens;     /* N  */
} DsaConfig;

/* Arithmetic of a forward call. */
#define AMDMOE_DTYPE_F32 0      /* fp32 in/out, fp32 intermediates            */
#define AMDMOE_DTYPE_BF16 1     /* bf16 x/W1/W2/y, fp32 gate, bf16 activation */
#define AMDMOE_DTYPE_FP8 2      /* e4m3 block-scaled experts, bf16 x/gate/y   */
#define AMDMOE_DTYPE_MXFP4 3    /* OCP MXFP4 experts, MXFP8 activations, bf16 x/gate/y */

/* Message of the last failing call on this host thread ("" if none). */
const char* amdmoe_last_error(void);

/* Library version string. */
const char* amdmoe_version(void);

/* ------------------------------------------------------------------ MoE */

/* Bytes of device workspace a forward of `dtype` needs for `cfg`. */
int amdmoe_moe_workspace_bytes(const MoeConfig* cfg, int dtype, size_t* bytes);

/* Full MoE layer, fp32.  Replaces moe_forward (kernels/moe/naive_moe.cuh:74-76,
 * kernels/moe/naive_moe.cu:400-471): x [T,D], Wg [E,D], W1 [E,2I,D] (gate rows
 * 0..I-1, up rows I..2I-1), W2 [E,D,I]; y [T,D] is overwritten.  Any D and I
 * (D and I multiples of 32 run on MFMA, other shapes on bounds-checked fp32
 * kernels). */
int amdmoe_moe_forward_f32(const float* x, const float* gate_weight, const float* w1,
                           const float* w2, float* y, const MoeConfig* cfg,
                           void* workspace, size_t workspace_bytes, void* stream);

/* The fp32 layer with a per-expert logit bias (BASELINE medium-fp32 config,
 * whose skewed expert loads come from the bias).  No counterpart in the
 * reference (moe_forward has no bias, naive_moe.cuh:74-76); same arguments
 * and result as amdmoe_moe_forward_f32, with gate_bias fp32 [E] added to
 * each token's logits before the softmax (NULL = no bias). */
int amdmoe_moe_forward_f32_bias(const float* x, const float* gate_weight, const float* gate_bias,
                                const float* w1, const float* w2, float* y, const MoeConfig* cfg,
                                void* workspace, size_t workspace_bytes, void* stream);

/* Full MoE layer, bf16 storage with fp32 accumulation (BASELINE medium-bf16
 * and Mixtral configs; same layouts as moe_forward).  gate_weight is fp32,
 * gate_bias fp32 [E] is added to the logits before the softmax (NULL = no
 * bias, as in the reference).  y bf16 [T,D] is overwritten. */
int amdmoe_moe_forward_bf16(const uint16_t* x, const float* gate_weight, const float* gate_bias,
                            const uint16_t* w1, const uint16_t* w2, uint16_t* y,
                            const MoeConfig* cfg, void* workspace, size_t workspace_bytes,
                            void* stream);

/* The bf16 layer with pre-packed expert weights.  No counterpart in the
 * reference (whose moe_forward is fp32 only): the same computation and
 * arguments as amdmoe_moe_forward_bf16, but W1 and W2 are given in the
 * fragment-block order written by amdmoe_pack_weights_bf16, so each of the
 * grouped GEMMs' weight loads reads 1 KB contiguous instead of 16 rows x
 * 64 bytes.  Results are bit-identical to the row-major entry. */
int amdmoe_moe_forward_bf16_packed(const uint16_t* x, const float* gate_weight, const float* gate_bias,
                                   const uint16_t* w1_packed, const uint16_t* w2_packed, uint16_t* y,
                                   const MoeConfig* cfg, void* workspace, size_t workspace_bytes,
                                   void* stream);

/* Full MoE layer, FP8 block-scale (BASELINE DeepSeek-V3 config).
 *   x bf16 [T,D] (quantised internally to e4m3 with one fp32 scale per token
 *   per 128 columns); gate_weight bf16 [E,D];
 *   w1 e4m3 [E,2I,D] with w1_scale fp32 [E,2I/128,D/128];
 *   w2 e4m3 [E,D,I]  with w2_scale fp32 [E,D/128,I/128];
 *   y bf16 [T,D] overwritten.  D and I must be multiples of 128. */
int amdmoe_moe_forward_fp8(const uint16_t* x, const uint16_t* gate_weight, const uint8_t* w1,
                           const float* w1_scale, const uint8_t* w2, const float* w2_scale,
                           uint16_t* y, const MoeConfig* cfg, void* workspace,
                           size_t workspace_bytes, void* stream);

/* The fp8 layer with pre-packed expert weights.  No counterpart in the
 * reference (whose moe_forward, naive_moe.cuh:74-76, is fp32 only): the
 * same computation and arguments as amdmoe_moe_forward_fp8, but W1 and W2
 * are given in the fragment-block order written by amdmoe_pack_weights_fp8
 * (scales unchanged).  Results are bit-identical to the row-major entry. */
int amdmoe_moe_forward_fp8_packed(const uint16_t* x, const uint16_t* gate_weight,
                                  const uint8_t* w1_packed, const float* w1_scale,
                                  const uint8_t* w2_packed, const float* w2_scale, uint16_t* y,
                                  const MoeConfig* cfg, void* workspace, size_t workspace_bytes,
                                  void* stream);

/* The MoE layer with OCP MXFP4 expert weights (OCP Microscaling spec v1.0;
 * no counterpart in the reference, whose layer is fp32 only -- the AMD
 * analogue of its roadmap's NVFP4 experts): every 32 consecutive weights
 * along K share one E8M0 scale 2^(E-127), elements are FP4 E2M1.  x bf16
 * [T,D] is quantised in the forward to MXFP8 (E4M3, one E8M0 scale per 32
 * columns), as is the SwiGLU output; the MFMA applies all block scales.
 * Weights in the fragment order of amdmoe_pack_weights_mxfp4:
 * w1_packed [E, 2I*D/2] bytes with w1_scale_packed [E, 2I*D/32],
 * w2_packed [E, D*I/2] with w2_scale_packed [E, D*I/32].  gate_weight bf16
 * [E,D]; routing as amdmoe_moe_forward_fp8; y bf16 [T,D] overwritten.
 * D and I multiples of 128; workspace as amdmoe_moe_workspace_bytes with
 * AMDMOE_DTYPE_MXFP4. */
int amdmoe_moe_forward_mxfp4(const uint16_t* x, const uint16_t* gate_weight,
                             const uint8_t* w1_packed, const uint8_t* w1_scale_packed,
                             const uint8_t* w2_packed, const uint8_t* w2_scale_packed, uint16_t* y,
                             const MoeConfig* cfg, void* workspace, size_t workspace_bytes,
                             void* stream);

/* MXFP4 quantisation of fp32 rows w [rows, cols] (cols % 32 == 0): q
 * [rows, cols/2] E2M1 codes, two per byte, even column in the low nibble;
 * scale [rows, cols/32] E8M0 = floor(log2 max|block|) - 2 + 127 clamped to
 * [0, 254] (0 for an all-zero block); q = RNE(w / 2^(scale-127)) saturated
 * at 6.  No counterpart in the reference. */
int amdmoe_quant_weight_mxfp4(const float* w, long rows, int cols, uint8_t* q, uint8_t* scale,
                              void* stream);

/* MXFP8 quantisation of bf16 rows x [rows, cols] (cols % 32 == 0): q
 * [rows, cols] E4M3, scale [rows, cols/32] E8M0 = floor(log2 max|block|) - 8
 * + 127 clamped to [0, 254].  No counterpart in the reference. */
int amdmoe_quant_rows_mxfp8(const uint16_t* x, long rows, int cols, uint8_t* q, uint8_t* scale,
                            void* stream);

/* One-time repacking of row-major MXFP4 expert weights (q [E][rows][cols/2],
 * scale [E][rows][cols/32], as amdmoe_quant_weight_mxfp4 writes them) into
 * the forward's fragment order: per expert, per 16 rows x 128 columns, 1 KB
 * of codes stored [lane l][16 B] with lane l = 16g + r holding row r,
 * columns 32g .. 32g+31 of the block, and the 64 scales [lane l] = scale of
 * (row r, columns 32g ..); blocks ordered [rows/16][cols/128].  rows % 16
 * == 0, cols % 128 == 0; outputs must not alias inputs. */
int amdmoe_pack_weights_mxfp4(const uint8_t* q, const uint8_t* scale, int num_experts, int rows,
                              int cols, uint8_t* q_packed, uint8_t* scale_packed, void* stream);

/* Bytes of device scratch amdmoe_moe_forward_fp8_packed_noalloc owns per GPU.
 * The array is a static device variable of the library's code object, so it
 * is reserved on every GPU the library is loaded on, when the code object
 * loads there, whether or not the entry is ever called (512 MiB on a host
 * of 8 GPUs), and it is held until the process ends. */
#define AMDMOE_NOALLOC_SCRATCH_BYTES (64u << 20)

/* amdmoe_moe_forward_fp8_packed for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  Same arguments and results as
 * amdmoe_moe_forward_fp8_packed without the workspace: the scratch is a
 * fixed AMDMOE_NOALLOC_SCRATCH_BYTES (64 MiB) device array inside the
 * library, one per GPU, held until the process ends; the call allocates and
 * frees nothing.  Configurations whose workspace (amdmoe_moe_workspace_bytes
 * with AMDMOE_DTYPE_FP8) exceeds it are rejected with AMDMOE_ERR_WORKSPACE
 * (at the DeepSeek-V3 shape, E=256, K=8, D=7168, I=2048: T <= 432).  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (two
 * streams, two host threads) race and must be ordered by the caller. */
int amdmoe_moe_forward_fp8_packed_noalloc(const uint16_t* x, const uint16_t* gate_weight,
                                          const uint8_t* w1_packed, const float* w1_scale,
                                          const uint8_t* w2_packed, const float* w2_scale,
                                          uint16_t* y, const MoeConfig* cfg, void* stream);

/* One-time repacking of row-major expert weights [num_experts][rows][cols]
 * (bytes; W1 [E,2I,D] or W2 [E,D,I] e4m3, naive_moe.cuh:66-72) into
 * fragment-block order: per expert, per 16 rows x 128 bytes, 2 KB stored as
 * [half h][lane l][16 B] with lane l = 16q + r holding row r, bytes
 * 64h + 16q .. +15 of the block; blocks ordered [rows/16][cols/128].  Needs
 * rows % 16 == 0 and cols % 128 == 0; out must not alias w. */
int amdmoe_pack_weights_fp8(const uint8_t* w, int num_experts, int rows, int cols, uint8_t* out,
                            void* stream);

/* The same repacking for bf16 expert weights [num_experts][rows][cols]
 * (W1 [E,2I,D] or W2 [E,D,I], naive_moe.cuh:66-72): the blocks are those of
 * amdmoe_pack_weights_fp8 over the rows' 2*cols bytes (a 128-byte K-step
 * holds 64 elements).  Needs rows % 16 == 0 and cols % 64 == 0; out must
 * not alias w.  Feeds amdmoe_moe_forward_bf16_packed. */
int amdmoe_pack_weights_bf16(const uint16_t* w, int num_experts, int rows, int cols, uint16_t* out,
                             void* stream);

/* --- stage entry points with the reference's semantics --- */

/* Routing: replaces moe_gate (naive_moe.cuh:27-29, naive_moe.cu:341-355).
 * expert_indices int32 [T,K] in the reference's slot order, expert_weights
 * fp32 [T,K] (softmax probabilities of the chosen experts, renormalised). */
int amdmoe_moe_gate_f32(const float* x, const float* gate_weight, int* expert_indices,
                        float* expert_weights, const MoeConfig* cfg, void* stream);

/* Routing for the bf16 layer: bf16 x, fp32 gate (+ optional fp32 bias [E]). */
int amdmoe_moe_gate_bf16x(const uint16_t* x, const float* gate_weight, const float* gate_bias,
                          int* expert_indices, float* expert_weights, const MoeConfig* cfg,
                          void* stream);

/* Routing for the fp8 layer: bf16 x, bf16 gate, logits on bf16 MFMA.  When
 * E <= 256 and D % 64 == 0 the gate GEMM is split along D and its partial
 * logits pass through the library's cached per-device scratch (at most
 * T*E*4*16 bytes, allocated on first use); calls sharing it
 * must be ordered on one stream. */
int amdmoe_moe_gate_bf16(const uint16_t* x, const uint16_t* gate_weight, int* expert_indices,
                         float* expert_weights, const MoeConfig* cfg, void* stream);

/* Routing for the fp8 layer together with the 1x128 quantisation of x, as
 * the fp8 forward runs it: the gate GEMM reads every x element once and
 * also writes xq e4m3 [T,D] and x_scale fp32 [T,D/128] (the format of
 * amdmoe_quant_rows_fp8; D % 128 == 0).  expert_indices / expert_weights as
 * amdmoe_moe_gate_bf16, whose scratch rules apply.  No counterpart in the
 * reference (fp32 only); its routing is moe_gate (naive_moe.cuh:27-29). */
int amdmoe_moe_gate_fp8(const uint16_t* x, const uint16_t* gate_weight, int* expert_indices,
                        float* expert_weights, uint8_t* xq, float* x_scale, const MoeConfig* cfg,
                        void* stream);

/* Per-expert gather: replaces moe_gather (naive_moe.cuh:38-41,
 * naive_moe.cu:357-366).  Tokens routed to expert_id in ascending token
 * order: gathered [cnt,D], token_map [cnt], *count (device int). */
int amdmoe_moe_gather_f32(const float* x, const int* expert_indices, const float* expert_weights,
                          int expert_id, float* gathered, int* token_map, int* count,
                          const MoeConfig* cfg, void* stream);

/* All-expert permutation (the batched form of moe_gather's index work):
 * counts [E], offsets [E+1] (exclusive scan), sorted_token / sorted_slot
 * [offsets[E]] = token id / flat slot t*K+k, experts ascending, tokens
 * ascending within an expert (the reference gather order). */
int amdmoe_moe_permute(const int* expert_indices, const MoeConfig* cfg, int* counts,
                       int* offsets, int* sorted_token, int* sorted_slot, void* stream);

/* C[M,N] = A[M,K] * B[K,N], row-major, B not transposed: replaces
 * naive_gemm (naive_moe.cuh:44-45, naive_moe.cu:368-374). */
int amdmoe_naive_gemm_f32(const float* A, const float* B, float* C, int M, int N, int K,
                          void* stream);

/* out[i] = silu(gate[i]) * up[i]: replaces swiglu (naive_moe.cuh:50-51,
 * naive_moe.cu:376-382). */
int amdmoe_swiglu_f32(const float* gate, const float* up, float* out, int n, void* stream);

/* output[token_map[m], :] += w(token_map[m], expert_id) * expert_out[m, :]
 * for m < count (host int): replaces moe_scatter (naive_moe.cuh:59-62,
 * naive_moe.cu:384-395).  Accumulates; count == 0 is a no-op. */
int amdmoe_moe_scatter_f32(const float* expert_out, const int* token_map,
                           const float* expert_weights, const int* expert_indices, int expert_id,
                           float* output, int count, const MoeConfig* cfg, void* stream);

/* --- weight / activation formats (BASELINE fp8 layout) --- */

/* Row quantisation, 1x128 blocks: scale = amax/448 (1 for an all-zero
 * block), q = e4m3_rne_sat(x/scale).  x bf16 [rows, cols], q [rows, cols],
 * scale [rows, cols/128]. */
int amdmoe_quant_rows_fp8(const uint16_t* x, long rows, int cols, uint8_t* q, float* scale,
                          void* stream);

/* Weight quantisation, 128x128 blocks, with a per-block multiplier u:
 * scale = u * amax / 448, q = e4m3_rne_sat(w/scale).  w fp32 [rows, cols],
 * u fp32 [rows/128, cols/128], q [rows, cols], scale [rows/128, cols/128]. */
int amdmoe_quant_weight_fp8(const float* w, long rows, int cols, const float* u, uint8_t* q,
                            float* scale, void* stream);

/* Instrumentation (no reference counterpart; the reference times whole
 * calls with events on stream 0, utils/cuda_utils.cuh:27-50).  While
 * `events` is non-NULL, each MoE forward records events[0..6] (hipEvent_t,
 * owned by the caller) on its stream: [0] start, [1] after routing,
 * [2] after x quantisation (fp8 with E > 256 or K > 16, where it is a launch
 * of its own; otherwise -- including the fp8 layer, whose gate GEMM quantises x
 * -- recorded right after [1]),
 * [3] after the permutation, [4] after the up-projection GEMM, [5] after
 * the down-projection GEMM, [6] after the combine.  Per host thread;
 * NULL turns it off. */
int amdmoe_set_stage_events(void** events);

/* ------------------------------------------------------------------ DSA */

/* Sparse MLA decode, fp32: replaces dsa_forward (naive_dsa.cuh:81-87,
 * naive_dsa.cu:435-474).  q_nope [Q,H,Dc], q_pe [Q,H,Dp], kv_c [N,Dc],
 * kv_p [N,Dp], v [N,Dc], sparse_indices [Q,S] (flat rows); out [Q,H,Dc].
 * Any S (S > 16384 keeps the scores in the entry's cached scratch).  An
 * index outside [0, N) (N = cfg->total_kv_tokens) selects nothing: it takes
 * no part in the softmax and no row is read for it; a query with no valid
 * index gets 0 (the reference reads such an index out of bounds). */
int amdmoe_dsa_forward_f32(const float* q_nope, const float* q_pe, const float* kv_cache_compressed,
                           const float* kv_cache_positional, const float* v_cache,
                           const int* sparse_indices, float* output, const DsaConfig* cfg,
                           void* stream);

/* Sparse MLA decode, bf16, paged latent cache (BASELINE DSA config).
 * cache bf16 [num_pages * page_size, Dc+Dp]: columns 0..Dc-1 are K_c and
 * also V (MLA absorbed), Dc..Dc+Dp-1 are K_p.  page_table int32
 * [Q, pages_per_seq]; logical_indices int32 [Q,S] are positions in the
 * query's sequence, physical row = page_table[q][i/page]*page + i%page.
 * q_nope bf16 [Q,H,Dc], q_pe bf16 [Q,H,Dp]; out bf16 [Q,H,Dc].
 * cfg->total_kv_tokens is the number of rows of `cache`; cfg->page_size is
 * the page length.  A selected position selects nothing when it lies
 * outside [0, pages_per_seq * page), when its page-table entry is negative
 * or when its row is at or past total_kv_tokens: no page-table entry or
 * cache row is read for it and it takes no part in the softmax, so the
 * output is attention over the valid positions only (0 for a query with
 * none).  The -1 padding of amdmoe_dsa_indexer_topk_fp8 (sequences shorter
 * than the selection) is therefore decoded correctly.
 * Requires Dc == 512, Dp == 64, H a multiple of 32, 1 <= S <= 4096; for H a
 * multiple of 128, S up to 65536 and caches of more than 4 GiB (about 3.7 M
 * tokens) are accepted. */
int amdmoe_dsa_decode_bf16_paged(const uint16_t* q_nope, const uint16_t* q_pe,
                                 const uint16_t* cache, const int* page_table,
                                 const int* logical_indices, uint16_t* output,
                                 const DsaConfig* cfg, int pages_per_seq, void* stream);

/* Lightning indexer of DeepSeek-V3.2: the producer of the sparse indices
 * amdmoe_dsa_decode_bf16_paged consumes.  No counterpart in the reference
 * (its tests draw the indices at random, tests/test_dsa.cu:73-85); the
 * formula is the published one, I = sum_j w_j * ReLU(q_j . k), in fp8:
 *   score[q,s] = k_scale[row] * sum_j head_w[q,j] * q_scale[q,j]
 *                * relu(q_codes[q,j,:] . k_codes[row,:]),  s < seq_len[q],
 *   row = page_table[q][s / page] * page + s % page.
 * q_codes e4m3 [Q,Hi,128], q_scale / head_w fp32 [Q,Hi] (scales > 0);
 * k_codes e4m3 [cache_rows,128] with k_scale fp32 [cache_rows] (> 0), in
 * pages of `page` rows; page_table int32 [Q, pages_per_seq]; seq_len int32
 * [Q] (device).  out int32 [Q, topk]: the topk positions with the largest
 * scores (ties: the lower position), in ascending position order; a query
 * with fewer than topk positions lists all of them, then -1.  scores fp32
 * [Q, max_seq] is caller scratch (left holding the scores, -inf past
 * seq_len).  Hi in {16, 32, 64, 128}; max_seq <= 131072, and above 32768
 * only while the row splits into parts of at most 32768 positions, each
 * longer than topk, with parts * topk <= 32768.  Rows are selected in parts
 * when that fills the device (few queries) or the row is long; the parts'
 * candidates then live in the indexer's own per-device scratch (see the
 * scratch rules above). */
int amdmoe_dsa_indexer_topk_fp8(const uint8_t* q_codes, const float* q_scale, const float* head_w,
                                const uint8_t* k_codes, const float* k_scale, long cache_rows,
                                const int* page_table, const int* seq_len, int num_queries,
                                int num_heads, int page, int pages_per_seq, int max_seq, int topk,
                                float* scores, int* out, void* stream);

/* The reference's DSA stage functions (fp32), same semantics; dsa_forward
 * above does not go through them.  Shapes follow cfg: gathered_kc/v
 * [Q,S,Dc], gathered_kp [Q,S,Dp], scores/attn [Q,H,S], output [Q,H,Dc].
 * Every value is formed in the reference kernel's order (sequential fp32
 * sums, no contraction). */

/* Replaces dsa_kv_gather (naive_dsa.cuh:31-36, naive_dsa.cu:336-367):
 * gathered_*[q,s,:] = cache row sparse_indices[q,s].  An index outside
 * [0, cfg->total_kv_tokens) gathers a row of zeros. */
int amdmoe_dsa_kv_gather_f32(const float* kv_cache_compressed, const float* kv_cache_positional,
                             const float* v_cache, const int* sparse_indices, float* gathered_kc,
                             float* gathered_kp, float* gathered_v, const DsaConfig* cfg,
                             void* stream);

/* Replaces dsa_dot_compressed (naive_dsa.cuh:42-43, naive_dsa.cu:89-134,
 * 369-380): scores[q,h,s] += dot(q_nope[q,h,:], kc[q,s,:]). */
int amdmoe_dsa_dot_compressed_f32(const float* q_nope, const float* kc, float* scores,
                                  const DsaConfig* cfg, void* stream);

/* Replaces dsa_dot_positional (naive_dsa.cuh:49-50, naive_dsa.cu:157-206,
 * 382-393): scores[q,h,s] += dot(q_pe[q,h,:], kp[q,s,:]). */
int amdmoe_dsa_dot_positional_f32(const float* q_pe, const float* kp, float* scores,
                                  const DsaConfig* cfg, void* stream);

/* Replaces dsa_dot_fused (naive_dsa.cuh:54-57, naive_dsa.cu:208-276,
 * 395-409): scores[q,h,s] += dot over the concatenation [q_nope|q_pe] .
 * [kc|kp], one accumulator. */
int amdmoe_dsa_dot_fused_f32(const float* q_nope, const float* q_pe, const float* kc,
                             const float* kp, float* scores, const DsaConfig* cfg, void* stream);

/* Replaces dsa_softmax (naive_dsa.cuh:61, naive_dsa.cu:278-296, 411-418):
 * per (q,h) row, in place: e = expf(x - max), x = e * (1/sum e). */
int amdmoe_dsa_softmax_f32(float* scores, const DsaConfig* cfg, void* stream);

/* Replaces dsa_output_proj (naive_dsa.cuh:67-68, naive_dsa.cu:300-316,
 * 420-429): output[q,h,d] = sum_s attn[q,h,s] * v[q,s,d] (overwritten). */
int amdmoe_dsa_output_proj_f32(const float* attn, const float* v, float* output,
                               const DsaConfig* cfg, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AMDMOE_H */
