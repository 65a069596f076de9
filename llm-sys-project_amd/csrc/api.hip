// C ABI of the library (include/amdmoe.h): argument validation, workspace
// layout, and the forward orchestration.  A forward is a fixed sequence of
// launches on the caller's stream with no host synchronisation and no
// allocation when a workspace is supplied:
//   route (R1; fp8: the gate GEMM also quantises x 1x128) -> permute (R2)
//   -> grouped GEMM up + SwiGLU (R3/R4) -> grouped GEMM down + weight (R5)
//   -> combine (ascending-expert sum per token)
// The reference's moe_forward (kernels/moe/naive_moe.cu:400-471) instead
// loops over experts on the host with a blocking device-to-host copy per
// expert and eight cudaMalloc/cudaFree pairs per call.
#include "internal.hpp"

#include <mutex>
#include <stdarg.h>
#include <stdio.h>

namespace amdmoe {

static thread_local char g_err[1024] = "";
static thread_local hipEvent_t* g_stage_events = nullptr;

// Records stage boundary `i` when instrumentation is on.
static int mark(int i, hipStream_t st) {
    if (g_stage_events) AMDMOE_HIP_TRY(hipEventRecord(g_stage_events[i], st));
    return AMDMOE_OK;
}

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

// ---------------------------------------------------------------- workspace
struct MoeWs {
    int* idx;
    float* wts;
    int* counts;
    int* offsets;
    int* num_tiles;
    int4* tiles;
    int* sorted_token;
    int* sorted_slot;
    float* sorted_w;
    uint8_t* xq;
    float* xs;
    float* xs_sorted;  // xs gathered to sorted row order, K-step major (the UP GEMM's scales)
    uint8_t* act;
    float* act_s;
    uint8_t* ypair;
    float* logits;  // gate logits scratch of the MFMA routing (fp8 path)
    int* perm;      // permutation scratch (per-block counts and offsets)
    size_t total;
};

static int elem_size(int dtype) { return dtype == AMDMOE_DTYPE_F32 ? 4 : (dtype == AMDMOE_DTYPE_BF16 ? 2 : 1); }
static bool is_8bit(int dtype) { return dtype == AMDMOE_DTYPE_FP8 || dtype == AMDMOE_DTYPE_MXFP4; }

// fp32 D and I the MFMA kernels tile (whole 32-element K steps); other
// shapes take the bounds-checked kernels of moe_generic.hip
static bool f32_mfma_shape(const MoeConfig& c) {
    return c.hidden_dim % 32 == 0 && c.intermediate_dim % 32 == 0;
}

// M-tile rows.  The fp32 GEMMs are bound by MFMA work per CU, so a small
// layer whose 256-row M-tiles give fewer than 256 UP work items (the medium
// configuration: 8 experts of ~128 rows x 16 N-tiles = 128 items) leaves CUs
// idle; halving the tile rows (down to 64) doubles its items.  The bf16,
// fp8 and MX GEMMs stream weights, and keep 256 rows (fewer weight passes).
static int mtile_rows(const MoeConfig& c, int dtype) {
    if (dtype != AMDMOE_DTYPE_F32 || !f32_mfma_shape(c)) return kMTile;
    const long P = (long)c.num_tokens * c.top_k;
    const long up_ntiles = ceil_div((long)c.intermediate_dim, 128L);
    int bm = kMTile;
    while (bm > 64 && (P / bm) * up_ntiles < 256) bm /= 2;
    return bm;
}

// K splits of the fp32 / bf16 down projection.  Its work items are (M-tile,
// 256-column N-tile) pairs.  With few experts and a long I (Mixtral: 8
// experts x 16 N-tiles x 4-5 M-tiles = 512-640 items of 224 K-steps) they
// fill the 256 CUs only two-and-a-bit times, so the last round runs on a
// fraction of the chip: I is split in two when there are at most 1024
// items.  A small layer (the medium configuration: 8 experts x 4 N-tiles)
// fills only part of the chip even then, so the splits keep doubling while
// the items would not fill the 256 CUs once, each split keeping at least 8
// whole K-steps, up to 8 splits.  The s fp32 partial rows of a slot are
// added in the combine, in split order.  (More splits where the items
// already fill the chip cost the partial rows' traffic: Mixtral T=256 with
// 8 splits, 0.530 -> 0.587 ms.)
static int down_splits(const MoeConfig& c, int dtype) {
    if (is_8bit(dtype)) return 1;
    const long P = (long)c.num_tokens * c.top_k;
    const long items = max_mtiles(P, c.num_experts, mtile_rows(c, dtype)) * ceil_div((long)c.hidden_dim, 256L);
    const long nk = (long)c.intermediate_dim * elem_size(dtype) / 128;  // K-steps
    int s = items <= 1024 && nk >= 32 && nk % 2 == 0 ? 2 : 1;
    while (2 * s <= 8 && items * s < 256 && nk % (2 * s) == 0 && nk / (2 * s) >= 8) s *= 2;
    return s;
}

// Lays the workspace out from `base` (nullptr: sizes only).
static MoeWs ws_layout(const MoeConfig& c, int dtype, uint8_t* base) {
    MoeWs w{};
    size_t off = 0;
    auto take = [&](size_t bytes) -> uint8_t* {
        uint8_t* p = base ? base + off : nullptr;
        off += align_up(bytes ? bytes : 1, 256);
        return p;
    };
    const size_t T = c.num_tokens, E = c.num_experts, K = c.top_k, D = c.hidden_dim,
                 I = c.intermediate_dim;
    const size_t P = T * K;
    w.idx = (int*)take(4 * P);
    w.wts = (float*)take(4 * P);
    w.counts = (int*)take(4 * E);
    w.offsets = (int*)take(4 * (E + 1));
    w.num_tiles = (int*)take(4);
    w.tiles = (int4*)take(16 * (size_t)max_mtiles((long)P, (int)E, mtile_rows(c, dtype)));
    w.sorted_token = (int*)take(4 * P);
    w.sorted_slot = (int*)take(4 * P);
    w.sorted_w = (float*)take(4 * P);
    w.perm = (int*)take(permute_scratch_bytes((int)T, (int)E));
    if (is_8bit(dtype)) {
        // activation scales: fp8 one fp32 per 128 columns, MX one E8M0 byte
        // per 32 -- the same bytes per row
        w.xq = take(T * D);
        w.xs = (float*)take(4 * T * (D / 128));
        w.xs_sorted = (float*)take(4 * P * (D / 128));
        w.act = take(P * I);
        w.act_s = (float*)take(4 * P * (I / 128));
        w.ypair = take(2 * P * D);
        w.logits = (float*)take(route_mfma_scratch_bytes((int)T, (int)E, (int)D, dtype == AMDMOE_DTYPE_FP8));
    } else {
        // the down-projection's weighted rows stay fp32 on the fp32 and bf16
        // paths, so a bf16 output is rounded once (in the combine); one set
        // of rows per K split
        w.act = take(elem_size(dtype) * P * I);
        w.ypair = take(4 * P * D * (size_t)down_splits(c, dtype));
    }
    w.total = off;
    return w;
}

// Per-device cached scratch for calls that take no workspace (or pass
// workspace == NULL), one buffer per entry-point family, so that calls of
// different families (an MoE forward on one stream, a decode on another)
// never share memory.  Calls of one family that use it must be ordered on
// one stream; the call that grows a buffer frees and allocates (hipFree
// waits for the device).
enum ScratchKind { SCR_MOE = 0, SCR_GATE, SCR_PERMUTE, SCR_DSA_DECODE, SCR_DSA_F32, SCR_DSA_INDEXER, SCR_KINDS };
struct CachedWs {
    std::mutex m;
    void* ptr = nullptr;
    size_t bytes = 0;
};
static CachedWs g_cache[64][SCR_KINDS];

static int cached_workspace(size_t need, void** out, int kind = SCR_MOE) {
    int dev = 0;
    AMDMOE_HIP_TRY(hipGetDevice(&dev));
    AMDMOE_CHECK_ARG(dev >= 0 && dev < 64, "device id %d out of range", dev);
    CachedWs& c = g_cache[dev][kind];
    std::lock_guard<std::mutex> lk(c.m);
    if (c.bytes < need) {
        if (c.ptr) AMDMOE_HIP_TRY(hipFree(c.ptr));  // hipFree waits for pending work
        c.ptr = nullptr;
        c.bytes = 0;
        size_t grow = align_up(need + need / 4, 1 << 20);
        AMDMOE_HIP_TRY(hipMalloc(&c.ptr, grow));
        c.bytes = grow;
    }
    *out = c.ptr;
    return AMDMOE_OK;
}

// ---------------------------------------------------------------- checks
static int check_cfg(const MoeConfig* cfg, int dtype) {
    AMDMOE_CHECK_ARG(cfg != nullptr, "cfg is NULL");
    const MoeConfig& c = *cfg;
    AMDMOE_CHECK_ARG(c.num_tokens >= 0, "num_tokens=%d < 0", c.num_tokens);
    AMDMOE_CHECK_ARG(c.num_experts >= 1 && c.num_experts <= 8192, "num_experts=%d outside [1, 8192]", c.num_experts);
    AMDMOE_CHECK_ARG(c.top_k >= 1 && c.top_k <= 64, "top_k=%d outside [1, 64]", c.top_k);
    AMDMOE_CHECK_ARG(c.hidden_dim >= 1 && c.intermediate_dim >= 1, "hidden_dim=%d / intermediate_dim=%d must be positive", c.hidden_dim, c.intermediate_dim);
    AMDMOE_CHECK_ARG((long)c.num_tokens * c.top_k < (1L << 30), "T*K=%ld too large", (long)c.num_tokens * c.top_k);
    // fp32 (the reference's format) takes any D and I; the bf16 / fp8 tiles
    // need whole 64- / 128-element K steps (and the fp8 block scales 128)
    const int kq = dtype == AMDMOE_DTYPE_F32 ? 1 : (dtype == AMDMOE_DTYPE_BF16 ? 64 : 128);  // fp8, MXFP4: 128
    AMDMOE_CHECK_ARG(c.hidden_dim % kq == 0 && c.intermediate_dim % kq == 0,
                     "hidden_dim=%d and intermediate_dim=%d must be multiples of %d for this dtype",
                     c.hidden_dim, c.intermediate_dim, kq);
    return AMDMOE_OK;
}

// Routing entries: any D (the gate GEMM is not tiled along D there), I unused.
static int check_gate_cfg(const MoeConfig* cfg) {
    AMDMOE_CHECK_ARG(cfg != nullptr, "cfg is NULL");
    MoeConfig c = *cfg;
    c.intermediate_dim = 1;
    return check_cfg(&c, AMDMOE_DTYPE_F32);
}

static int resolve_ws(const MoeConfig& c, int dtype, void* workspace, size_t bytes, MoeWs* out) {
    MoeWs sz = ws_layout(c, dtype, nullptr);
    void* base = workspace;
    if (base) {
        AMDMOE_CHECK_ARG(((uintptr_t)base & 255) == 0, "workspace must be 256-byte aligned");
        if (bytes < sz.total)
            return set_error(AMDMOE_ERR_WORKSPACE, "workspace of %zu bytes < required %zu", bytes, sz.total);
    } else {
        int rc = cached_workspace(sz.total, &base);
        if (rc) return rc;
    }
    *out = ws_layout(c, dtype, (uint8_t*)base);
    return AMDMOE_OK;
}

#define TRY(...)                      \
    do {                              \
        int rc_ = (__VA_ARGS__);      \
        if (rc_) return rc_;          \
    } while (0)

// Shared tail of every forward: permute, both grouped GEMMs, combine.
static int moe_experts(int dt, const MoeConfig& c, const MoeWs& w, const uint8_t* a_x,
                       const float* x_scale, const uint8_t* w1, const float* w1s,
                       const uint8_t* w2, const float* w2s, void* y, hipStream_t st,
                       bool packed = false) {
    const int T = c.num_tokens, E = c.num_experts, K = c.top_k, D = c.hidden_dim,
              I = c.intermediate_dim;
    const long P = (long)T * K;
    // the MoeConfig dtype of this path (tile rows and K splits are chosen on it)
    const int cdt = dt == DT_F32 ? AMDMOE_DTYPE_F32
                                 : (dt == DT_BF16 ? AMDMOE_DTYPE_BF16 : (dt == DT_MX ? AMDMOE_DTYPE_MXFP4 : AMDMOE_DTYPE_FP8));
    const int bm = mtile_rows(c, cdt);
    const long mtiles = max_mtiles(P, E, bm);
    const int es = dt == DT_F32 ? 4 : (dt == DT_BF16 ? 2 : 1);  // activation bytes per element
    const int wdiv = dt == DT_MX ? 2 : 1;                       // MX weights: two E2M1 per byte
    // fp8 / MX: with the permutation, x's block scales K-step major in
    // sorted row order (the grouped GEMM's a_scale layout)
    TRY(launch_permute(w.idx, T, K, E, bm, w.counts, w.offsets, w.sorted_token,
                       w.sorted_slot, w.tiles, w.num_tiles,
                       permute_scratch_bytes(T, E) ? w.perm : nullptr, w.wts, w.sorted_w, st,
                       (const uint32_t*)x_scale, x_scale ? D / 128 : 0, x_scale ? (uint32_t*)w.xs_sorted : nullptr));
    TRY(mark(3, st));
    if (dt == DT_F32 && !f32_mfma_shape(c)) {
        TRY(launch_experts_f32_any((const float*)a_x, (const float*)w1, (const float*)w2, T, E, K,
                                   D, I, w.tiles, w.num_tiles, mtiles, w.sorted_token,
                                   w.sorted_slot, w.sorted_w, w.idx, (float*)w.act,
                                   (float*)w.ypair, (float*)y, st));
        TRY(mark(4, st));
        TRY(mark(5, st));
        return mark(6, st);
    }
    GemmArgs up{};
    up.a = a_x;
    up.a_bytes = (long)T * D * es;
    up.a_row_bytes = (long)D * es;
    up.a_map = w.sorted_token;
    up.a_scale = x_scale ? w.xs_sorted : nullptr;
    up.a_scale_bytes = x_scale ? P * (D / 128) * 4 : 0;
    up.a_scale_rows = P;
    up.b = w1;
    up.b_expert_bytes = 2L * I * D * es / wdiv;
    up.b_row_bytes = (long)D * es / wdiv;
    up.b_mx_scale = dt == DT_MX ? (const uint8_t*)w1s : nullptr;
    up.b_mx_scale_expert_bytes = dt == DT_MX ? 2L * I * (D / 32) : 0;
    up.b_packed = packed;
    up.b_scale = w1s;
    up.b_rows = 2 * I;
    up.K = D;
    up.n_out = I;
    up.tiles = w.tiles;
    up.num_tiles = w.num_tiles;
    up.n_tiles_n = (int)ceil_div(I, 128);
    up.out = w.act;
    up.out_scale = w.act_s;
    up.out_scale_rows = P;
    TRY(launch_grouped_gemm(dt, MODE_UP, up, mtiles, st));
    TRY(mark(4, st));
    GemmArgs dn{};
    dn.a = w.act;
    dn.a_bytes = P * I * es;
    dn.a_row_bytes = (long)I * es;
    dn.a_scale = w.act_s;
    dn.a_scale_bytes = w.act_s ? P * (I / 128) * 4 : 0;
    dn.a_scale_rows = P;
    dn.b = w2;
    dn.b_expert_bytes = (long)D * I * es / wdiv;
    dn.b_row_bytes = (long)I * es / wdiv;
    dn.b_mx_scale = dt == DT_MX ? (const uint8_t*)w2s : nullptr;
    dn.b_mx_scale_expert_bytes = dt == DT_MX ? (long)D * (I / 32) : 0;
    dn.b_packed = packed;
    dn.b_scale = w2s;
    dn.b_rows = D;
    dn.K = I;
    dn.n_out = D;
    dn.tiles = w.tiles;
    dn.num_tiles = w.num_tiles;
    dn.n_tiles_n = (int)ceil_div(D, 256);
    dn.out = w.ypair;
    dn.sorted_slot = w.sorted_slot;
    dn.sorted_w = w.sorted_w;
    const int nsplit = down_splits(c, cdt);
    dn.k_splits = nsplit;
    dn.out_split_stride = P * D;
    TRY(launch_grouped_gemm(dt, MODE_DOWN, dn, mtiles, st));
    TRY(mark(5, st));
    TRY(launch_combine(dt == DT_F32 || dt == DT_BF16 ? DT_F32 : DT_BF16, dt == DT_F32 ? DT_F32 : DT_BF16,
                       w.ypair, w.idx, T, K, E, D, y, st, nsplit));
    return mark(6, st);
}

}  // namespace amdmoe

using namespace amdmoe;

extern "C" {

const char* amdmoe_last_error(void) { return g_err; }

const char* amdmoe_version(void) { return "amdmoe 0.1 gfx950"; }

int amdmoe_set_stage_events(void** events) {
    g_stage_events = (hipEvent_t*)events;
    return AMDMOE_OK;
}

int amdmoe_moe_workspace_bytes(const MoeConfig* cfg, int dtype, size_t* bytes) {
    AMDMOE_CHECK_ARG(dtype >= AMDMOE_DTYPE_F32 && dtype <= AMDMOE_DTYPE_MXFP4, "bad dtype %d", dtype);
    TRY(check_cfg(cfg, dtype));
    AMDMOE_CHECK_ARG(bytes != nullptr, "bytes is NULL");
    *bytes = ws_layout(*cfg, dtype, nullptr).total;
    return AMDMOE_OK;
}

static int forward_f32(const float* x, const float* gate_weight, const float* gate_bias,
                       const float* w1, const float* w2, float* y, const MoeConfig* cfg,
                       void* workspace, size_t workspace_bytes, void* stream) {
    TRY(check_cfg(cfg, AMDMOE_DTYPE_F32));
    const MoeConfig& c = *cfg;
    if (c.num_tokens == 0) return AMDMOE_OK;
    AMDMOE_CHECK_ARG(x && gate_weight && w1 && w2 && y, "null tensor pointer");
    hipStream_t st = (hipStream_t)stream;
    MoeWs w;
    TRY(resolve_ws(c, AMDMOE_DTYPE_F32, workspace, workspace_bytes, &w));
    TRY(mark(0, st));
    TRY(launch_route_exact<float, float>(x, gate_weight, gate_bias, c.num_tokens, c.num_experts,
                                         c.top_k, c.hidden_dim, w.idx, w.wts, st));
    TRY(mark(1, st));
    TRY(mark(2, st));
    return moe_experts(DT_F32, c, w, (const uint8_t*)x, nullptr, (const uint8_t*)w1, nullptr,
                       (const uint8_t*)w2, nullptr, y, st);
}

int amdmoe_moe_forward_f32(const float* x, const float* gate_weight, const float* w1,
                           const float* w2, float* y, const MoeConfig* cfg, void* workspace,
                           size_t workspace_bytes, void* stream) {
    return forward_f32(x, gate_weight, nullptr, w1, w2, y, cfg, workspace, workspace_bytes, stream);
}

int amdmoe_moe_forward_f32_bias(const float* x, const float* gate_weight, const float* gate_bias,
                                const float* w1, const float* w2, float* y, const MoeConfig* cfg,
                                void* workspace, size_t workspace_bytes, void* stream) {
    return forward_f32(x, gate_weight, gate_bias, w1, w2, y, cfg, workspace, workspace_bytes,
                       stream);
}

static int forward_bf16(const uint16_t* x, const float* gate_weight, const float* gate_bias,
                        const uint16_t* w1, const uint16_t* w2, uint16_t* y, const MoeConfig* cfg,
                        void* workspace, size_t workspace_bytes, void* stream, bool packed) {
    TRY(check_cfg(cfg, AMDMOE_DTYPE_BF16));
    const MoeConfig& c = *cfg;
    if (c.num_tokens == 0) return AMDMOE_OK;
    AMDMOE_CHECK_ARG(x && gate_weight && w1 && w2 && y, "null tensor pointer");
    hipStream_t st = (hipStream_t)stream;
    MoeWs w;
    TRY(resolve_ws(c, AMDMOE_DTYPE_BF16, workspace, workspace_bytes, &w));
    TRY(mark(0, st));
    TRY(launch_route_exact<uint16_t, float>(x, gate_weight, gate_bias, c.num_tokens,
                                            c.num_experts, c.top_k, c.hidden_dim, w.idx, w.wts,
                                            st));
    TRY(mark(1, st));
    TRY(mark(2, st));
    return moe_experts(DT_BF16, c, w, (const uint8_t*)x, nullptr, (const uint8_t*)w1, nullptr,
                       (const uint8_t*)w2, nullptr, y, st, packed);
}

int amdmoe_moe_forward_bf16(const uint16_t* x, const float* gate_weight, const float* gate_bias,
                            const uint16_t* w1, const uint16_t* w2, uint16_t* y,
                            const MoeConfig* cfg, void* workspace, size_t workspace_bytes,
                            void* stream) {
    return forward_bf16(x, gate_weight, gate_bias, w1, w2, y, cfg, workspace, workspace_bytes, stream,
                        false);
}

int amdmoe_moe_forward_bf16_packed(const uint16_t* x, const float* gate_weight, const float* gate_bias,
                                   const uint16_t* w1_packed, const uint16_t* w2_packed, uint16_t* y,
                                   const MoeConfig* cfg, void* workspace, size_t workspace_bytes,
                                   void* stream) {
    return forward_bf16(x, gate_weight, gate_bias, w1_packed, w2_packed, y, cfg, workspace,
                        workspace_bytes, stream, true);
}

static int forward_fp8(const uint16_t* x, const uint16_t* gate_weight, const uint8_t* w1,
                       const float* w1_scale, const uint8_t* w2, const float* w2_scale,
                       uint16_t* y, const MoeConfig* cfg, void* workspace,
                       size_t workspace_bytes, void* stream, bool packed) {
    TRY(check_cfg(cfg, AMDMOE_DTYPE_FP8));
    const MoeConfig& c = *cfg;
    if (c.num_tokens == 0) return AMDMOE_OK;
    AMDMOE_CHECK_ARG(x && gate_weight && w1 && w1_scale && w2 && w2_scale && y,
                     "null tensor pointer");
    hipStream_t st = (hipStream_t)stream;
    MoeWs w;
    TRY(resolve_ws(c, AMDMOE_DTYPE_FP8, workspace, workspace_bytes, &w));
    TRY(mark(0, st));
    if (route_mfma_supported(c.num_experts, c.top_k, c.hidden_dim)) {
        // the gate GEMM also quantises x (it reads every x element once)
        TRY(launch_route_mfma(x, gate_weight, c.num_tokens, c.num_experts, c.top_k, c.hidden_dim,
                              w.idx, w.wts, w.logits, w.xq, w.xs, st));
        TRY(mark(1, st));
    } else {
        TRY(launch_route_exact<uint16_t, uint16_t>(x, gate_weight, nullptr, c.num_tokens,
                                                   c.num_experts, c.top_k, c.hidden_dim, w.idx,
                                                   w.wts, st));
        TRY(mark(1, st));
        TRY(launch_quant_rows(x, c.num_tokens, c.hidden_dim, w.xq, w.xs, st));
    }
    TRY(mark(2, st));
    return moe_experts(DT_FP8, c, w, w.xq, w.xs, w1, w1_scale, w2, w2_scale, y, st, packed);
}

int amdmoe_moe_forward_fp8(const uint16_t* x, const uint16_t* gate_weight, const uint8_t* w1,
                           const float* w1_scale, const uint8_t* w2, const float* w2_scale,
                           uint16_t* y, const MoeConfig* cfg, void* workspace,
                           size_t workspace_bytes, void* stream) {
    return forward_fp8(x, gate_weight, w1, w1_scale, w2, w2_scale, y, cfg, workspace,
                       workspace_bytes, stream, false);
}

// ---------------------------------------------------------------- no allocation
// Scratch of amdmoe_moe_forward_fp8_packed_noalloc: a file-scope device
// array, one copy per GPU, held until the process ends.  In host code
// `scratch` names a host-side stand-in, not device memory: its device
// address is taken once per device with hipGetSymbolAddress (the entry's
// first call on that device, with the device current) and only that address
// is ever passed to a kernel.
static __device__ __align__(256) uint8_t scratch[AMDMOE_NOALLOC_SCRATCH_BYTES];
static std::mutex g_scratch_mutex;
static void* g_scratch_dev[64];  // device address of `scratch` per device id

static int noalloc_scratch(void** out) {
    int dev = 0;
    AMDMOE_HIP_TRY(hipGetDevice(&dev));
    AMDMOE_CHECK_ARG(dev >= 0 && dev < 64, "device id %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mutex);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        AMDMOE_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        AMDMOE_CHECK_ARG(p != nullptr, "no device address for the scratch array");
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return AMDMOE_OK;
}

int amdmoe_moe_forward_fp8_packed(const uint16_t* x, const uint16_t* gate_weight,
                                  const uint8_t* w1_packed, const float* w1_scale,
                                  const uint8_t* w2_packed, const float* w2_scale, uint16_t* y,
                                  const MoeConfig* cfg, void* workspace, size_t workspace_bytes,
                                  void* stream) {
    return forward_fp8(x, gate_weight, w1_packed, w1_scale, w2_packed, w2_scale, y, cfg, workspace,
                       workspace_bytes, stream, true);
}

int amdmoe_moe_forward_fp8_packed_noalloc(const uint16_t* x, const uint16_t* gate_weight,
                                          const uint8_t* w1_packed, const float* w1_scale,
                                          const uint8_t* w2_packed, const float* w2_scale,
                                          uint16_t* y, const MoeConfig* cfg, void* stream) {
    TRY(check_cfg(cfg, AMDMOE_DTYPE_FP8));
    const size_t need = ws_layout(*cfg, AMDMOE_DTYPE_FP8, nullptr).total;
    if (need > (size_t)AMDMOE_NOALLOC_SCRATCH_BYTES)
        return set_error(AMDMOE_ERR_WORKSPACE,
                         "moe_forward_fp8_packed_noalloc: T=%d E=%d K=%d D=%d I=%d needs %zu bytes "
                         "of scratch, more than the %zu of the no-allocation buffer",
                         cfg->num_tokens, cfg->num_experts, cfg->top_k, cfg->hidden_dim,
                         cfg->intermediate_dim, need, (size_t)AMDMOE_NOALLOC_SCRATCH_BYTES);
    if (cfg->num_tokens == 0) return AMDMOE_OK;
    void* ws = nullptr;
    TRY(noalloc_scratch(&ws));
    return forward_fp8(x, gate_weight, w1_packed, w1_scale, w2_packed, w2_scale, y, cfg, ws,
                       AMDMOE_NOALLOC_SCRATCH_BYTES, stream, true);
}

int amdmoe_moe_forward_mxfp4(const uint16_t* x, const uint16_t* gate_weight,
                             const uint8_t* w1_packed, const uint8_t* w1_scale_packed,
                             const uint8_t* w2_packed, const uint8_t* w2_scale_packed, uint16_t* y,
                             const MoeConfig* cfg, void* workspace, size_t workspace_bytes,
                             void* stream) {
    TRY(check_cfg(cfg, AMDMOE_DTYPE_MXFP4));
    const MoeConfig& c = *cfg;
    if (c.num_tokens == 0) return AMDMOE_OK;
    AMDMOE_CHECK_ARG(x && gate_weight && w1_packed && w1_scale_packed && w2_packed && w2_scale_packed && y,
                     "null tensor pointer");
    hipStream_t st = (hipStream_t)stream;
    MoeWs w;
    TRY(resolve_ws(c, AMDMOE_DTYPE_MXFP4, workspace, workspace_bytes, &w));
    TRY(mark(0, st));
    if (route_mfma_supported(c.num_experts, c.top_k, c.hidden_dim))
        TRY(launch_route_mfma(x, gate_weight, c.num_tokens, c.num_experts, c.top_k, c.hidden_dim,
                              w.idx, w.wts, w.logits, nullptr, nullptr, st));
    else
        TRY(launch_route_exact<uint16_t, uint16_t>(x, gate_weight, nullptr, c.num_tokens,
                                                   c.num_experts, c.top_k, c.hidden_dim, w.idx,
                                                   w.wts, st));
    TRY(mark(1, st));
    TRY(launch_quant_rows_mxfp8(x, c.num_tokens, c.hidden_dim, w.xq, (uint8_t*)w.xs, st));
    TRY(mark(2, st));
    return moe_experts(DT_MX, c, w, w.xq, w.xs, w1_packed, (const float*)w1_scale_packed, w2_packed,
                       (const float*)w2_scale_packed, y, st, true);
}

int amdmoe_quant_weight_mxfp4(const float* w, long rows, int cols, uint8_t* q, uint8_t* scale,
                              void* stream) {
    return launch_quant_weight_mxfp4(w, rows, cols, q, scale, (hipStream_t)stream);
}

int amdmoe_quant_rows_mxfp8(const uint16_t* x, long rows, int cols, uint8_t* q, uint8_t* scale,
                            void* stream) {
    return launch_quant_rows_mxfp8(x, rows, cols, q, scale, (hipStream_t)stream);
}

int amdmoe_pack_weights_mxfp4(const uint8_t* q, const uint8_t* scale, int num_experts, int rows,
                              int cols, uint8_t* q_packed, uint8_t* scale_packed, void* stream) {
    return launch_pack_mxfp4(q, scale, num_experts, rows, cols, q_packed, scale_packed,
                             (hipStream_t)stream);
}

int amdmoe_pack_weights_fp8(const uint8_t* w, int num_experts, int rows, int cols, uint8_t* out,
                            void* stream) {
    AMDMOE_CHECK_ARG(w && out, "null tensor pointer");
    return launch_pack_weights(w, num_experts, rows, cols, out, (hipStream_t)stream);
}

int amdmoe_pack_weights_bf16(const uint16_t* w, int num_experts, int rows, int cols, uint16_t* out,
                             void* stream) {
    AMDMOE_CHECK_ARG(w && out, "null tensor pointer");
    AMDMOE_CHECK_ARG(cols >= 0 && cols <= (1 << 29), "pack_weights_bf16: cols=%d out of range", cols);
    AMDMOE_CHECK_ARG(cols % 64 == 0, "pack_weights_bf16: cols=%d must be a multiple of 64", cols);
    // the fragment blocks are byte blocks: a bf16 row of cols elements is
    // 2 cols bytes, one 128-byte K-step per 64 elements
    return launch_pack_weights((const uint8_t*)w, num_experts, rows, 2 * cols, (uint8_t*)out,
                               (hipStream_t)stream);
}

int amdmoe_moe_gate_f32(const float* x, const float* gate_weight, int* expert_indices,
                        float* expert_weights, const MoeConfig* cfg, void* stream) {
    TRY(check_gate_cfg(cfg));
    if (cfg->num_tokens == 0) return AMDMOE_OK;
    return launch_route_exact<float, float>(x, gate_weight, nullptr, cfg->num_tokens,
                                            cfg->num_experts, cfg->top_k, cfg->hidden_dim,
                                            expert_indices, expert_weights, (hipStream_t)stream);
}

int amdmoe_moe_gate_bf16x(const uint16_t* x, const float* gate_weight, const float* gate_bias,
                          int* expert_indices, float* expert_weights, const MoeConfig* cfg,
                          void* stream) {
    TRY(check_gate_cfg(cfg));
    if (cfg->num_tokens == 0) return AMDMOE_OK;
    return launch_route_exact<uint16_t, float>(x, gate_weight, gate_bias, cfg->num_tokens,
                                               cfg->num_experts, cfg->top_k, cfg->hidden_dim,
                                               expert_indices, expert_weights,
                                               (hipStream_t)stream);
}

int amdmoe_moe_gate_bf16(const uint16_t* x, const uint16_t* gate_weight, int* expert_indices,
                         float* expert_weights, const MoeConfig* cfg, void* stream) {
    TRY(check_gate_cfg(cfg));
    if (cfg->num_tokens == 0) return AMDMOE_OK;
    if (route_mfma_supported(cfg->num_experts, cfg->top_k, cfg->hidden_dim)) {
        // logits scratch: the library's cached per-device workspace
        void* scratch = nullptr;
        TRY(cached_workspace(route_mfma_scratch_bytes(cfg->num_tokens, cfg->num_experts,
                                                      cfg->hidden_dim, false),
                             &scratch, SCR_GATE));
        return launch_route_mfma(x, gate_weight, cfg->num_tokens, cfg->num_experts, cfg->top_k,
                                 cfg->hidden_dim, expert_indices, expert_weights, (float*)scratch,
                                 nullptr, nullptr, (hipStream_t)stream);
    }
    return launch_route_exact<uint16_t, uint16_t>(x, gate_weight, nullptr, cfg->num_tokens,
                                                  cfg->num_experts, cfg->top_k, cfg->hidden_dim,
                                                  expert_indices, expert_weights,
                                                  (hipStream_t)stream);
}

int amdmoe_moe_gate_fp8(const uint16_t* x, const uint16_t* gate_weight, int* expert_indices,
                        float* expert_weights, uint8_t* xq, float* x_scale, const MoeConfig* cfg,
                        void* stream) {
    TRY(check_gate_cfg(cfg));
    AMDMOE_CHECK_ARG(cfg->hidden_dim % 128 == 0, "moe_gate_fp8: hidden_dim=%d not a multiple of 128",
                     cfg->hidden_dim);
    AMDMOE_CHECK_ARG(x && gate_weight && expert_indices && expert_weights && xq && x_scale,
                     "null tensor pointer");
    const MoeConfig& c = *cfg;
    if (c.num_tokens == 0) return AMDMOE_OK;
    hipStream_t st = (hipStream_t)stream;
    if (route_mfma_supported(c.num_experts, c.top_k, c.hidden_dim)) {
        void* scratch = nullptr;
        TRY(cached_workspace(route_mfma_scratch_bytes(c.num_tokens, c.num_experts, c.hidden_dim, true),
                             &scratch, SCR_GATE));
        return launch_route_mfma(x, gate_weight, c.num_tokens, c.num_experts, c.top_k, c.hidden_dim,
                                 expert_indices, expert_weights, (float*)scratch, xq, x_scale, st);
    }
    TRY(launch_route_exact<uint16_t, uint16_t>(x, gate_weight, nullptr, c.num_tokens, c.num_experts,
                                               c.top_k, c.hidden_dim, expert_indices,
                                               expert_weights, st));
    return launch_quant_rows(x, c.num_tokens, c.hidden_dim, xq, x_scale, st);
}

int amdmoe_moe_gather_f32(const float* x, const int* expert_indices, const float* expert_weights,
                          int expert_id, float* gathered, int* token_map, int* count,
                          const MoeConfig* cfg, void* stream) {
    (void)expert_weights;  // unused, as in the reference (naive_moe.cu:358)
    TRY(check_gate_cfg(cfg));
    AMDMOE_CHECK_ARG(expert_id >= 0 && expert_id < cfg->num_experts, "expert_id=%d out of range", expert_id);
    return launch_gather_one(x, expert_indices, cfg->num_tokens, cfg->top_k, cfg->num_experts,
                             cfg->hidden_dim, expert_id, gathered, token_map, count,
                             (hipStream_t)stream);
}

int amdmoe_moe_permute(const int* expert_indices, const MoeConfig* cfg, int* counts,
                       int* offsets, int* sorted_token, int* sorted_slot, void* stream) {
    AMDMOE_CHECK_ARG(cfg && cfg->num_experts >= 1 && cfg->top_k >= 1 && cfg->num_tokens >= 0,
                     "bad MoeConfig");
    const MoeConfig& c = *cfg;
    // the tile table is not part of this entry's outputs: a private buffer
    // of the cached workspace holds it
    const long mt = max_mtiles((long)c.num_tokens * c.top_k, c.num_experts);
    const size_t tiles_bytes = align_up(16 * (size_t)(mt + 1), 256);
    const size_t perm_bytes = permute_scratch_bytes(c.num_tokens, c.num_experts);
    void* scratch = nullptr;
    TRY(cached_workspace(tiles_bytes + 256 + perm_bytes, &scratch, SCR_PERMUTE));
    int4* tiles = (int4*)scratch;
    int* nt = (int*)((uint8_t*)scratch + tiles_bytes);
    int* perm = perm_bytes ? (int*)((uint8_t*)scratch + tiles_bytes + 256) : nullptr;
    return launch_permute(expert_indices, c.num_tokens, c.top_k, c.num_experts, kMTile, counts,
                          offsets, sorted_token, sorted_slot, tiles, nt, perm, nullptr, nullptr,
                          (hipStream_t)stream);
}

int amdmoe_naive_gemm_f32(const float* A, const float* B, float* C, int M, int N, int K,
                          void* stream) {
    AMDMOE_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "negative GEMM size");
    return launch_naive_gemm_f32(A, B, C, M, N, K, (hipStream_t)stream);
}

int amdmoe_swiglu_f32(const float* gate, const float* up, float* out, int n, void* stream) {
    return launch_swiglu_f32(gate, up, out, n, (hipStream_t)stream);
}

int amdmoe_moe_scatter_f32(const float* expert_out, const int* token_map,
                           const float* expert_weights, const int* expert_indices, int expert_id,
                           float* output, int count, const MoeConfig* cfg, void* stream) {
    AMDMOE_CHECK_ARG(cfg != nullptr, "cfg is NULL");
    return launch_scatter_f32(expert_out, token_map, expert_weights, expert_indices, expert_id,
                              output, count, cfg->num_tokens, cfg->top_k, cfg->hidden_dim,
                              (hipStream_t)stream);
}

int amdmoe_quant_rows_fp8(const uint16_t* x, long rows, int cols, uint8_t* q, float* scale,
                          void* stream) {
    AMDMOE_CHECK_ARG(rows >= 0, "rows < 0");
    return launch_quant_rows(x, rows, cols, q, scale, (hipStream_t)stream);
}

int amdmoe_quant_weight_fp8(const float* w, long rows, int cols, const float* u, uint8_t* q,
                            float* scale, void* stream) {
    return launch_quant_weight(w, rows, cols, u, q, scale, (hipStream_t)stream);
}

int amdmoe_dsa_forward_f32(const float* q_nope, const float* q_pe, const float* kv_cache_compressed,
                           const float* kv_cache_positional, const float* v_cache,
                           const int* sparse_indices, float* output, const DsaConfig* cfg,
                           void* stream) {
    AMDMOE_CHECK_ARG(cfg != nullptr, "cfg is NULL");
    const DsaConfig& c = *cfg;
    AMDMOE_CHECK_ARG(c.num_queries >= 0 && c.num_heads >= 0 && c.head_dim_compressed >= 1 &&
                         c.head_dim_positional >= 0 && c.num_selected_kv >= 1,
                     "bad DsaConfig");
    // scores beyond what LDS holds go to the entry's own cached scratch
    const size_t need = dsa_f32_scratch_bytes(c.num_queries, c.num_heads, c.num_selected_kv);
    void* scratch = nullptr;
    if (need) TRY(cached_workspace(need, &scratch, SCR_DSA_F32));
    return launch_dsa_f32(q_nope, q_pe, kv_cache_compressed, kv_cache_positional, v_cache,
                          sparse_indices, output, c.num_queries, c.num_heads,
                          c.head_dim_compressed, c.head_dim_positional, c.num_selected_kv,
                          c.total_kv_tokens, (float*)scratch, (hipStream_t)stream);
}

static int dsa_cfg_check(const DsaConfig* cfg) {
    AMDMOE_CHECK_ARG(cfg != nullptr, "cfg is NULL");
    const DsaConfig& c = *cfg;
    AMDMOE_CHECK_ARG(c.num_queries >= 0 && c.num_heads >= 0 && c.head_dim_compressed >= 0 &&
                         c.head_dim_positional >= 0 && c.num_selected_kv >= 0 &&
                         c.total_kv_tokens >= 0,
                     "bad DsaConfig");
    return AMDMOE_OK;
}

int amdmoe_dsa_indexer_topk_fp8(const uint8_t* q_codes, const float* q_scale, const float* head_w,
                                const uint8_t* k_codes, const float* k_scale, long cache_rows,
                                const int* page_table, const int* seq_len, int num_queries,
                                int num_heads, int page, int pages_per_seq, int max_seq, int topk,
                                float* scores, int* out, void* stream) {
    AMDMOE_CHECK_ARG(num_queries >= 0, "dsa_indexer: num_queries=%d", num_queries);
    AMDMOE_CHECK_ARG(q_codes && q_scale && head_w && k_codes && k_scale && page_table && seq_len &&
                         scores && out,
                     "null tensor pointer");
    // the two-stage selection's candidates live in the indexer's own cached scratch
    const size_t need = dsa_indexer_scratch_bytes(num_queries, max_seq, topk);
    void* scratch = nullptr;
    if (need) TRY(cached_workspace(need, &scratch, SCR_DSA_INDEXER));
    return launch_dsa_indexer(q_codes, q_scale, head_w, k_codes, cache_rows, k_scale, page_table,
                              seq_len, num_queries, num_heads, page, pages_per_seq, max_seq, topk,
                              scores, out, scratch, need, (hipStream_t)stream);
}

int amdmoe_dsa_kv_gather_f32(const float* kv_cache_compressed, const float* kv_cache_positional,
                             const float* v_cache, const int* sparse_indices, float* gathered_kc,
                             float* gathered_kp, float* gathered_v, const DsaConfig* cfg,
                             void* stream) {
    TRY(dsa_cfg_check(cfg));
    const DsaConfig& c = *cfg;
    return launch_dsa_gather(kv_cache_compressed, kv_cache_positional, v_cache, sparse_indices,
                             gathered_kc, gathered_kp, gathered_v, c.num_queries,
                             c.num_selected_kv, c.head_dim_compressed, c.head_dim_positional,
                             c.total_kv_tokens, (hipStream_t)stream);
}

static int dsa_dot(const float* qn, const float* qp, const float* kc, const float* kp,
                   float* scores, const DsaConfig* cfg, int parts, void* stream) {
    TRY(dsa_cfg_check(cfg));
    const DsaConfig& c = *cfg;
    return launch_dsa_dot(qn, qp, kc, kp, scores, c.num_queries, c.num_heads, c.num_selected_kv,
                          c.head_dim_compressed, c.head_dim_positional, parts,
                          (hipStream_t)stream);
}

int amdmoe_dsa_dot_compressed_f32(const float* q_nope, const float* kc, float* scores,
                                  const DsaConfig* cfg, void* stream) {
    return dsa_dot(q_nope, nullptr, kc, nullptr, scores, cfg, 1, stream);
}

int amdmoe_dsa_dot_positional_f32(const float* q_pe, const float* kp, float* scores,
                                  const DsaConfig* cfg, void* stream) {
    return dsa_dot(nullptr, q_pe, nullptr, kp, scores, cfg, 2, stream);
}

int amdmoe_dsa_dot_fused_f32(const float* q_nope, const float* q_pe, const float* kc,
                             const float* kp, float* scores, const DsaConfig* cfg, void* stream) {
    return dsa_dot(q_nope, q_pe, kc, kp, scores, cfg, 3, stream);
}

int amdmoe_dsa_softmax_f32(float* scores, const DsaConfig* cfg, void* stream) {
    TRY(dsa_cfg_check(cfg));
    const DsaConfig& c = *cfg;
    return launch_dsa_softmax(scores, (long)c.num_queries * c.num_heads, c.num_selected_kv,
                              (hipStream_t)stream);
}

int amdmoe_dsa_output_proj_f32(const float* attn, const float* v, float* output,
                               const DsaConfig* cfg, void* stream) {
    TRY(dsa_cfg_check(cfg));
    const DsaConfig& c = *cfg;
    return launch_dsa_output_proj(attn, v, output, c.num_queries, c.num_heads, c.num_selected_kv,
                                  c.head_dim_compressed, (hipStream_t)stream);
}

int amdmoe_dsa_decode_bf16_paged(const uint16_t* q_nope, const uint16_t* q_pe,
                                 const uint16_t* cache, const int* page_table,
                                 const int* logical_indices, uint16_t* output,
                                 const DsaConfig* cfg, int pages_per_seq, void* stream) {
    AMDMOE_CHECK_ARG(cfg != nullptr, "cfg is NULL");
    const DsaConfig& c = *cfg;
    AMDMOE_CHECK_ARG(c.num_queries >= 0 && c.num_heads >= 1 && c.num_selected_kv >= 1,
                     "bad DsaConfig");
    // the token-split partials live in the decode's own cached scratch
    const size_t need = dsa_paged_scratch_bytes(c.num_queries, c.num_heads, c.num_selected_kv);
    void* scratch = nullptr;
    if (need) TRY(cached_workspace(need, &scratch, SCR_DSA_DECODE));
    return launch_dsa_bf16_paged(q_nope, q_pe, cache, c.total_kv_tokens, page_table,
                                 logical_indices, output, c.num_queries, c.num_heads,
                                 c.head_dim_compressed,
                                 c.head_dim_positional, c.num_selected_kv, c.page_size,
                                 pages_per_seq, scratch, need, (hipStream_t)stream);
}

}  // extern "C"
