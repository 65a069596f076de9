// R2 -- token permutation: histogram, prefix sum, stable compaction into an
// expert-sorted order, plus the M-tile table of the grouped GEMMs.
//
// Reference: moe_gather / gather_kernel (kernels/moe/naive_moe.cu:147-166,
// 357-366; CPU tests/test_moe.cu:76-83): for each expert, one thread scans
// idx[T,K] in ascending token order, lists a token once (first matching
// slot), and the host syncs on the count before every expert.
//
// Here one launch serves every expert with no host round trip.  Workgroup e
// (one per expert):
//   1. builds the full expert histogram in LDS (order-independent counts),
//   2. derives its own row offset = sum of counts of lower experts, and its
//      M-tile offset = sum of ceil(count/BM) of lower experts,
//   3. compacts the slots holding e in flat slot order t*K+k (= ascending
//      token order) with a block-wide ballot prefix sum, so the output is
//      deterministic and equals the reference gather order exactly,
//   4. writes its M-tiles {expert, first row, rows}.
// Work is O(E * T*K) slot reads, all L2-resident (T*K*4 bytes per expert),
// in exchange for zero global atomics and zero inter-block ordering.
#include "internal.hpp"

namespace amdmoe {

constexpr int kPermThreads = 1024;

// M-tile j of an expert with `cnt` rows starting at row_off: the expert's
// ceil(cnt / BM) tiles split its 16-row token tiles as evenly as possible
// (270 rows -> 144 + 126, not 256 + 14), so the tiles of one expert run
// at the same pace and stream its weights side by side.  .w = (j << 16) |
// the expert's tile count: the GEMMs order an expert's work items N-tile
// major over its M-tiles with it.
__device__ __forceinline__ int4 mtile(int e, int row_off, int cnt, int BM, int j) {
    const int nt = (cnt + BM - 1) / BM;
    const int q = (cnt + 15) / 16;  // token tiles
    const int base = q / nt, extra = q % nt;
    const int first = 16 * (j * base + min(j, extra));
    const int rows = min(16 * (base + (j < extra ? 1 : 0)), cnt - first);
    return make_int4(e, row_off + first, rows, (j << 16) | nt);
}

// Slot i = t*K + k counts for expert e = idx[i] only if no earlier slot of
// the same token holds e (the reference's `break`).  Slots with e outside
// [0,E) (the -1 left when K > E) count nowhere.
__device__ __forceinline__ int slot_expert(const int* __restrict__ idx, int i, int K, int E) {
    int e = idx[i];
    if (e < 0 || e >= E) return -1;
    int k = i % K;
    for (int j = i - k; j < i; j++)
        if (idx[j] == e) return -1;
    return e;
}

// First slot k of token t holding expert e, or -1.  A token lists an
// expert at most once, so token order equals flat slot order t*K+k.
__device__ __forceinline__ int token_slot_of(const int* __restrict__ row, int K, int e) {
    for (int k = 0; k < K; k++)
        if (row[k] == e) return k;
    return -1;
}

__global__ __launch_bounds__(kPermThreads) void permute_kernel(
    const int* __restrict__ idx, int T, int K, int E, int BM, int* __restrict__ counts,
    int* __restrict__ offsets, int* __restrict__ sorted_token, int* __restrict__ sorted_slot,
    int4* __restrict__ tiles, int* __restrict__ num_tiles, const float* __restrict__ wts,
    float* __restrict__ sorted_w) {
    extern __shared__ int s_hist[];            // [E]
    __shared__ int s_wave[kPermThreads / 64];  // per-wave totals
    __shared__ int s_red[2];
    const int e = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    for (int j = tid; j < E; j += kPermThreads) s_hist[j] = 0;
    __syncthreads();
    // histogram, one token per thread (first occurrence per token only)
    for (int t = tid; t < T; t += kPermThreads) {
        const int* row = idx + (size_t)t * K;
        for (int k = 0; k < K; k++) {
            const int v = row[k];
            if (v < 0 || v >= E) continue;
            bool dup = false;
            for (int j = 0; j < k; j++) dup |= row[j] == v;
            if (!dup) atomicAdd(&s_hist[v], 1);
        }
    }
    __syncthreads();

    // offsets of this expert (rows and tiles) and, for block 0, the totals
    int row_off = 0, tile_off = 0, rows_all = 0, tiles_all = 0;
    for (int j = tid; j < E; j += kPermThreads) {
        int c = s_hist[j];
        int tl = (c + BM - 1) / BM;
        if (j < e) { row_off += c; tile_off += tl; }
        rows_all += c;
        tiles_all += tl;
    }
    // block reduction of the four partial sums (wave shuffles + LDS)
    auto block_sum = [&](int v) -> int {
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
        __syncthreads();
        if (lane == 0) s_wave[wave] = v;
        __syncthreads();
        if (tid == 0) {
            int s = 0;
            for (int w = 0; w < kPermThreads / 64; w++) s += s_wave[w];
            s_red[0] = s;
        }
        __syncthreads();
        return s_red[0];
    };
    row_off = block_sum(row_off);
    tile_off = block_sum(tile_off);
    rows_all = block_sum(rows_all);
    tiles_all = block_sum(tiles_all);
    const int cnt = s_hist[e];

    // stable compaction over tokens, chunks of kPermThreads tokens
    int base = 0;
    for (int c0 = 0; c0 < T; c0 += kPermThreads) {
        const int t = c0 + tid;
        const int k = t < T ? token_slot_of(idx + (size_t)t * K, K, e) : -1;
        const bool hit = k >= 0;
        unsigned long long b = __ballot(hit);
        int rank_in_wave = __popcll(b & ((1ull << lane) - 1ull));
        __syncthreads();
        if (lane == 0) s_wave[wave] = __popcll(b);
        __syncthreads();
        int before = 0, total = 0;
        for (int w = 0; w < kPermThreads / 64; w++) {
            int n = s_wave[w];
            if (w < wave) before += n;
            total += n;
        }
        if (hit) {
            int pos = row_off + base + before + rank_in_wave;
            sorted_token[pos] = t;
            sorted_slot[pos] = t * K + k;
            if (sorted_w) sorted_w[pos] = wts[(size_t)t * K + k];
        }
        base += total;
    }

    for (int j = tid; j * BM < cnt; j += kPermThreads) tiles[tile_off + j] = mtile(e, row_off, cnt, BM, j);
    if (tid == 0) {
        counts[e] = cnt;
        offsets[e] = row_off;
        if (e == 0) {
            offsets[E] = rows_all;
            *num_tiles = tiles_all;
        }
    }
}

// ------------------------------------------------- three-launch variant
// For E <= 1024 with a scratch of 2 * ceil(T/64) * E ints.  Blocks of 64
// tokens (one wave, lane = token):
//   perm_count_kernel: per block, a 64-bit lane mask per expert in LDS
//     (bit l: token 64b+l lists the expert, first occurrence only);
//     blk_cnt[b][e] = popcount(mask[e]);
//   perm_scan_kernel (one block): per expert, exclusive offsets over blocks
//     and the expert's row / M-tile offsets; counts, offsets, tile table;
//   perm_scatter_kernel: rebuilds the masks; token 64b+l goes to row
//     blk_off[b][e] + popcount(mask[e] & lanes below l).
// Rows of an expert are thus in ascending token order (block, then lane):
// the same order as the single-launch kernel above.
constexpr int kPermTok = 64;

__device__ __forceinline__ void perm_masks(const int* __restrict__ idx, int T, int K, int E,
                                           unsigned long long* s_mask) {
    const int lane = threadIdx.x;
    for (int e = lane; e < E; e += kPermTok) s_mask[e] = 0ull;
    __syncthreads();
    const int t = blockIdx.x * kPermTok + lane;
    if (t < T) {
        const int* row = idx + (size_t)t * K;
        for (int k = 0; k < K; k++) {
            const int v = row[k];
            if (v < 0 || v >= E) continue;
            bool dup = false;
            for (int j = 0; j < k; j++) dup |= row[j] == v;
            if (!dup) atomicOr(&s_mask[v], 1ull << lane);
        }
    }
    __syncthreads();
}

__global__ __launch_bounds__(kPermTok) void perm_count_kernel(const int* __restrict__ idx, int T,
                                                              int K, int E, int* __restrict__ blk_cnt) {
    extern __shared__ unsigned long long s_mask[];  // [E]
    perm_masks(idx, T, K, E, s_mask);
    for (int e = threadIdx.x; e < E; e += kPermTok)
        blk_cnt[(size_t)blockIdx.x * E + e] = __popcll(s_mask[e]);
}

__global__ __launch_bounds__(1024) void perm_scan_kernel(const int* __restrict__ blk_cnt,
                                                         int* __restrict__ blk_off, int nblk, int E,
                                                         int BM, int* __restrict__ counts,
                                                         int* __restrict__ offsets,
                                                         int4* __restrict__ tiles,
                                                         int* __restrict__ num_tiles) {
    // thread (p, e): expert e, block range p of NP = 1024 / Ep ranges, so the
    // per-block counts of an expert are read by NP threads in parallel
    __shared__ int s_part[1024], s_rows[1024], s_tiles[1024];
    int Ep = 1;
    while (Ep < E) Ep <<= 1;
    const int NP = 1024 / Ep;
    const int e = threadIdx.x % Ep, p = threadIdx.x / Ep;
    const int chunk = (nblk + NP - 1) / NP;
    const int b0 = p * chunk, b1 = min(nblk, b0 + chunk);
    int part = 0;
    if (e < E)
        for (int b = b0; b < b1; b++) part += blk_cnt[(size_t)b * E + e];
    s_part[threadIdx.x] = part;
    __syncthreads();
    int before = 0, tot = 0;
    for (int pp = 0; pp < NP; pp++) {
        const int v = s_part[pp * Ep + e];
        if (pp < p) before += v;
        tot += v;
    }
    const int nt = (tot + BM - 1) / BM;
    if (p == 0) {
        s_rows[e] = e < E ? tot : 0;
        s_tiles[e] = e < E ? nt : 0;
    }
    __syncthreads();
    // inclusive scans over experts (Hillis-Steele over Ep entries)
    for (int o = 1; o < Ep; o <<= 1) {
        int r = 0, tl = 0;
        if (p == 0 && e >= o) { r = s_rows[e - o]; tl = s_tiles[e - o]; }
        __syncthreads();
        if (p == 0) { s_rows[e] += r; s_tiles[e] += tl; }
        __syncthreads();
    }
    if (e < E) {
        const int row_off = s_rows[e] - tot;
        int run = row_off + before;
        for (int b = b0; b < b1; b++) {
            blk_off[(size_t)b * E + e] = run;
            run += blk_cnt[(size_t)b * E + e];
        }
        if (p == 0) {
            const int tile_off = s_tiles[e] - nt;
            counts[e] = tot;
            offsets[e] = row_off;
            for (int j = 0; j < nt; j++)
                tiles[tile_off + j] = mtile(e, row_off, tot, BM, j);
            if (e == E - 1) {
                offsets[E] = s_rows[e];
                *num_tiles = s_tiles[e];
            }
        }
    }
}

__global__ __launch_bounds__(kPermTok) void perm_scatter_kernel(const int* __restrict__ idx, int T,
                                                                int K, int E,
                                                                const int* __restrict__ blk_off,
                                                                int* __restrict__ sorted_token,
                                                                int* __restrict__ sorted_slot,
                                                                const float* __restrict__ wts,
                                                                float* __restrict__ sorted_w) {
    extern __shared__ unsigned long long s_mask[];  // [E]
    perm_masks(idx, T, K, E, s_mask);
    const int lane = threadIdx.x;
    const int t = blockIdx.x * kPermTok + lane;
    if (t >= T) return;
    const int* row = idx + (size_t)t * K;
    const unsigned long long below = (1ull << lane) - 1ull;
    for (int k = 0; k < K; k++) {
        const int v = row[k];
        if (v < 0 || v >= E) continue;
        bool dup = false;
        for (int j = 0; j < k; j++) dup |= row[j] == v;
        if (dup) continue;
        const int pos = blk_off[(size_t)blockIdx.x * E + v] + __popcll(s_mask[v] & below);
        sorted_token[pos] = t;
        sorted_slot[pos] = t * K + k;
        if (sorted_w) sorted_w[pos] = wts[(size_t)t * K + k];
    }
}

// Scan and scatter in one launch (nblk <= kFusedMaxBlk): every 64-token
// block derives its own offsets.  Thread (p, e) of NP = 1024 / Ep parts
// (Ep = E rounded up to a power of two) sums expert e's counts over its
// range of blocks, all loads in flight together: in total (tot) and over
// the blocks before this one (pre).  A block-wide exclusive scan of tot
// (and of the M-tile counts) over experts gives the expert's first row
// (and first M-tile); the block's rows for expert e start at
// row_off[e] + pre[e].  Block 0 also writes counts, offsets and the M-tile
// table.  Every block reads all of blk_cnt: nblk * E * 4 bytes of L2 reads
// (64 KB at T=4096, E=256).
constexpr int kFusedMaxBlk = 128;
constexpr int kFusedThreads = 1024;
constexpr int kFusedMaxE = 1024;

__global__ __launch_bounds__(kFusedThreads) void perm_scan_scatter_kernel(
    const int* __restrict__ idx, int T, int K, int E, int BM, const int* __restrict__ blk_cnt,
    int nblk, int* __restrict__ counts, int* __restrict__ offsets, int4* __restrict__ tiles,
    int* __restrict__ num_tiles, int* __restrict__ sorted_token, int* __restrict__ sorted_slot,
    const float* __restrict__ wts, float* __restrict__ sorted_w) {
    __shared__ int s_full[kFusedThreads], s_pre[kFusedThreads];
    __shared__ int s_off[kFusedMaxE];                  // this block's first row per expert
    __shared__ unsigned long long s_mask[kFusedMaxE];  // token lane masks per expert
    __shared__ int s_wr[kFusedThreads / 64], s_wt[kFusedThreads / 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int b = blockIdx.x;
    int Ep = 1;
    while (Ep < E) Ep <<= 1;
    const int NP = kFusedThreads / Ep;
    {
        const int e = tid % Ep, p = tid / Ep;
        const int chunk = (nblk + NP - 1) / NP;
        const int b0 = p * chunk;
        constexpr int kMaxChunk = kFusedMaxBlk;  // NP >= 1 parts cover nblk <= 128 blocks
        int full = 0, pre = 0;
        if (e < E) {
            int v[8];
            for (int c0 = 0; c0 < chunk && c0 < kMaxChunk; c0 += 8) {
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const int bb = b0 + c0 + j;
                    v[j] = c0 + j < chunk && bb < nblk ? blk_cnt[(size_t)bb * E + e] : 0;
                }
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    full += v[j];
                    if (b0 + c0 + j < b) pre += v[j];
                }
            }
        }
        s_full[tid] = full;
        s_pre[tid] = pre;
    }
    __syncthreads();
    // thread e < E: expert totals, then an exclusive scan over experts
    int tot = 0, pre = 0, tl = 0;
    if (tid < E) {
        for (int p = 0; p < NP; p++) {
            tot += s_full[p * Ep + tid];
            pre += s_pre[p * Ep + tid];
        }
        tl = (tot + BM - 1) / BM;
    }
    int rs = tot, ts = tl;  // inclusive wave scans
    for (int o = 1; o < 64; o <<= 1) {
        const int ro = __shfl_up(rs, o, 64), to = __shfl_up(ts, o, 64);
        if (lane >= o) { rs += ro; ts += to; }
    }
    if (lane == 63) { s_wr[wave] = rs; s_wt[wave] = ts; }
    __syncthreads();
    int wr = 0, wt = 0, ar = 0, at = 0;
    for (int w = 0; w < kFusedThreads / 64; w++) {
        if (w < wave) { wr += s_wr[w]; wt += s_wt[w]; }
        ar += s_wr[w];
        at += s_wt[w];
    }
    if (tid < E) {
        const int row_off = wr + rs - tot, tile_off = wt + ts - tl;
        s_off[tid] = row_off + pre;
        if (b == 0) {
            counts[tid] = tot;
            offsets[tid] = row_off;
            for (int j = 0; j < tl; j++)
                tiles[tile_off + j] = mtile(tid, row_off, tot, BM, j);
        }
    }
    if (b == 0 && tid == 0) {
        offsets[E] = ar;
        *num_tiles = at;
    }
    // this block's 64 tokens: lane masks per expert (bit i = token i of the
    // block), then every first occurrence goes to its row -- one thread per
    // (token, slot) pair, token = lane and slot k = wave (+16 per pass for
    // K > 16): the expert's offset plus the block's earlier tokens in it
    for (int e = tid; e < E; e += kFusedThreads) s_mask[e] = 0ull;
    __syncthreads();
    const int t = b * kPermTok + lane;
    const int* row = idx + (size_t)t * K;
    for (int k = wave; k < K; k += kFusedThreads / 64) {
        if (t >= T) break;
        const int v = row[k];
        if (v < 0 || v >= E) continue;
        bool dup = false;
        for (int j = 0; j < k; j++) dup |= row[j] == v;
        if (!dup) atomicOr(&s_mask[v], 1ull << lane);
    }
    __syncthreads();
    const unsigned long long below = (1ull << lane) - 1ull;
    for (int k = wave; k < K; k += kFusedThreads / 64) {
        if (t >= T) break;
        const int v = row[k];
        if (v < 0 || v >= E) continue;
        bool dup = false;
        for (int j = 0; j < k; j++) dup |= row[j] == v;
        if (dup) continue;
        const int pos = s_off[v] + __popcll(s_mask[v] & below);
        sorted_token[pos] = t;
        sorted_slot[pos] = t * K + k;
        if (sorted_w) sorted_w[pos] = wts[(size_t)t * K + k];
    }
}

// perm_small_kernel: decode-sized batches (T*K <= 1024 slots, E <= 256) in
// one workgroup and one launch.  Thread i owns slot i = t*K + k; wave w sets
// bit `lane` of its own 64-bit mask for the slot's expert, so a slot's row
// is its expert's offset + the slots of that expert in earlier waves + in
// lower lanes of its wave: flat slot order = ascending token order, as in
// the multi-block path.
constexpr int kSmallSlots = 1024;
constexpr int kSmallMaxE = 256;

__global__ __launch_bounds__(kSmallSlots) void perm_small_kernel(
    const int* __restrict__ idx, int T, int K, int E, int BM, int* __restrict__ counts,
    int* __restrict__ offsets, int4* __restrict__ tiles, int* __restrict__ num_tiles,
    int* __restrict__ sorted_token, int* __restrict__ sorted_slot, const float* __restrict__ wts,
    float* __restrict__ sorted_w, const uint32_t* __restrict__ rs_src, int rs_nkb,
    uint32_t* __restrict__ rs_dst) {
    constexpr int kWaves = kSmallSlots / 64;
    __shared__ unsigned long long s_mask[kWaves][kSmallMaxE];
    __shared__ int s_off[kSmallMaxE];
    __shared__ int s_wr[kWaves], s_wt[kWaves];
    __shared__ int s_tok[kSmallSlots];  // token of each sorted row (row scales)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < kWaves * kSmallMaxE; i += kSmallSlots) (&s_mask[0][0])[i] = 0ull;
    s_tok[tid] = 0;
    __syncthreads();
    const int e = tid < T * K ? slot_expert(idx, tid, K, E) : -1;
    if (e >= 0) atomicOr(&s_mask[wave][e], 1ull << lane);
    __syncthreads();
    // thread e < E: the expert's rows and M-tiles, exclusive scans over experts
    int tot = 0, tl = 0;
    if (tid < E) {
        for (int w = 0; w < kWaves; w++) tot += __popcll(s_mask[w][tid]);
        tl = (tot + BM - 1) / BM;
    }
    int rs = tot, ts = tl;
    for (int o = 1; o < 64; o <<= 1) {
        const int ro = __shfl_up(rs, o, 64), to = __shfl_up(ts, o, 64);
        if (lane >= o) { rs += ro; ts += to; }
    }
    if (lane == 63) { s_wr[wave] = rs; s_wt[wave] = ts; }
    __syncthreads();
    int wr = 0, wt = 0, ar = 0, at = 0;
    for (int w = 0; w < kWaves; w++) {
        if (w < wave) { wr += s_wr[w]; wt += s_wt[w]; }
        ar += s_wr[w];
        at += s_wt[w];
    }
    if (tid < E) {
        const int row_off = wr + rs - tot, tile_off = wt + ts - tl;
        s_off[tid] = row_off;
        counts[tid] = tot;
        offsets[tid] = row_off;
        for (int j = 0; j < tl; j++) tiles[tile_off + j] = mtile(tid, row_off, tot, BM, j);
    }
    if (tid == 0) {
        offsets[E] = ar;
        *num_tiles = at;
    }
    __syncthreads();
    if (e >= 0) {
        int pos = s_off[e] + __popcll(s_mask[wave][e] & ((1ull << lane) - 1ull));
        for (int w = 0; w < wave; w++) pos += __popcll(s_mask[w][e]);
        sorted_token[pos] = tid / K;
        sorted_slot[pos] = tid;
        if (sorted_w) sorted_w[pos] = wts[tid];
        s_tok[pos] = tid / K;
    }
    if (rs_dst) {
        // the row scales (gather_row_scales_kernel's contract): work unit j =
        // (4-dword chunk c, row p), rows fastest, so each K-step row of
        // rs_dst is written coalesced and every thread has one 16-byte load
        // in flight per round (4-byte loads if a token's row is not 16-byte
        // aligned)
        __syncthreads();
        const int P = T * K;
        const int nc = (rs_nkb + 3) >> 2;
        const bool vec = (rs_nkb & 3) == 0;
        for (int j = tid; j < nc * P; j += kSmallSlots) {
            const int c = j / P, p = j - c * P;
            const uint32_t* row = rs_src + (size_t)s_tok[p] * rs_nkb + 4 * c;
            if (vec) {
                const u32x4 v = *(const u32x4*)row;
#pragma unroll
                for (int i = 0; i < 4; i++) rs_dst[(size_t)(4 * c + i) * P + p] = v[i];
            } else {
                for (int i = 0; i < 4 && 4 * c + i < rs_nkb; i++) rs_dst[(size_t)(4 * c + i) * P + p] = row[i];
            }
        }
    }
}

size_t permute_scratch_bytes(int T, int E) {
    const long nblk = (T + kPermTok - 1) / kPermTok;
    if (E > 1024 || nblk * E > (1L << 22)) return 0;
    return (size_t)(2 * nblk * E) * sizeof(int);
}

int launch_gather_row_scales(const uint32_t* src, const int* sorted_token, long P, int T, int nkb,
                             uint32_t* dst, hipStream_t st);

int launch_permute(const int* idx, int T, int K, int E, int BM, int* counts, int* offsets,
                   int* sorted_token, int* sorted_slot, int4* tiles, int* num_tiles,
                   int* scratch, const float* wts, float* sorted_w, hipStream_t st,
                   const uint32_t* rs_src, int rs_nkb, uint32_t* rs_dst) {
    AMDMOE_CHECK_ARG((wts == nullptr) == (sorted_w == nullptr), "permute: wts and sorted_w go together");
    AMDMOE_CHECK_ARG((rs_src == nullptr) == (rs_dst == nullptr) && (!rs_dst || rs_nkb > 0),
                     "permute: rs_src and rs_dst go together (nkb=%d)", rs_nkb);
    if (T > 0 && (long)T * K <= kSmallSlots && E <= kSmallMaxE) {
        // decode-sized: one launch, the row scales included
        hipLaunchKernelGGL(perm_small_kernel, dim3(1), dim3(kSmallSlots), 0, st, idx, T, K, E, BM, counts,
                           offsets, tiles, num_tiles, sorted_token, sorted_slot, wts, sorted_w, rs_src,
                           rs_nkb, rs_dst);
        AMDMOE_LAUNCH_CHECK();
        return AMDMOE_OK;
    }
    if (rs_dst) {
        // the multi-block scatters write scattered rows: gather the scales
        // after them in a launch of their own (coalesced writes)
        const int rc = launch_permute(idx, T, K, E, BM, counts, offsets, sorted_token, sorted_slot, tiles,
                                      num_tiles, scratch, wts, sorted_w, st, nullptr, 0, nullptr);
        if (rc != AMDMOE_OK) return rc;
        return launch_gather_row_scales(rs_src, sorted_token, (long)T * K, T, rs_nkb, rs_dst, st);
    }
    if (scratch && T > 0 && permute_scratch_bytes(T, E) > 0) {
        const int nblk = (T + kPermTok - 1) / kPermTok;
        int* blk_cnt = scratch;
        int* blk_off = scratch + (size_t)nblk * E;
        const size_t lds = sizeof(unsigned long long) * (size_t)E;
        hipLaunchKernelGGL(perm_count_kernel, dim3(nblk), dim3(kPermTok), lds, st, idx, T, K, E, blk_cnt);
        AMDMOE_LAUNCH_CHECK();
        if (nblk <= kFusedMaxBlk && E <= kFusedMaxE) {
            hipLaunchKernelGGL(perm_scan_scatter_kernel, dim3(nblk), dim3(kFusedThreads), 0, st, idx, T,
                               K, E, BM, blk_cnt, nblk, counts, offsets, tiles, num_tiles,
                               sorted_token, sorted_slot, wts, sorted_w);
            AMDMOE_LAUNCH_CHECK();
            return AMDMOE_OK;
        }
        hipLaunchKernelGGL(perm_scan_kernel, dim3(1), dim3(1024), 0, st, blk_cnt, blk_off, nblk, E, BM,
                           counts, offsets, tiles, num_tiles);
        AMDMOE_LAUNCH_CHECK();
        hipLaunchKernelGGL(perm_scatter_kernel, dim3(nblk), dim3(kPermTok), lds, st, idx, T, K, E,
                           blk_off, sorted_token, sorted_slot, wts, sorted_w);
        AMDMOE_LAUNCH_CHECK();
        return AMDMOE_OK;
    }
    size_t lds = sizeof(int) * (size_t)E;
    AMDMOE_CHECK_ARG(lds <= 48 * 1024, "permute: E=%d too large", E);
    hipLaunchKernelGGL(permute_kernel, dim3(E), dim3(kPermThreads), lds, st, idx, T, K, E, BM,
                       counts, offsets, sorted_token, sorted_slot, tiles, num_tiles, wts, sorted_w);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

// Single-expert gather with the reference's moe_gather contract
// (naive_moe.cuh:31-41): one block compacts the expert's tokens in order,
// then copies their rows.
__global__ __launch_bounds__(kPermThreads) void gather_one_kernel(
    const float* __restrict__ x, const int* __restrict__ idx, int T, int K, int E, int D,
    int expert, float* __restrict__ gathered, int* __restrict__ token_map, int* __restrict__ count) {
    __shared__ int s_wave[kPermThreads / 64];
    __shared__ int s_cnt;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int P = T * K;
    int base = 0;
    for (int c0 = 0; c0 < P; c0 += kPermThreads) {
        int i = c0 + tid;
        bool hit = i < P && slot_expert(idx, i, K, E) == expert;
        unsigned long long b = __ballot(hit);
        int rank = __popcll(b & ((1ull << lane) - 1ull));
        __syncthreads();
        if (lane == 0) s_wave[wave] = __popcll(b);
        __syncthreads();
        int before = 0, total = 0;
        for (int w = 0; w < kPermThreads / 64; w++) {
            int n = s_wave[w];
            if (w < wave) before += n;
            total += n;
        }
        if (hit) token_map[base + before + rank] = i / K;
        base += total;
    }
    if (tid == 0) { s_cnt = base; *count = base; }
    __syncthreads();
    const int cnt = s_cnt;
    for (long j = tid; j < (long)cnt * D; j += kPermThreads) {
        int m = (int)(j / D), d = (int)(j % D);
        gathered[j] = x[(size_t)token_map[m] * D + d];
    }
}

int launch_gather_one(const float* x, const int* idx, int T, int K, int E, int D, int expert,
                      float* gathered, int* token_map, int* count, hipStream_t st) {
    hipLaunchKernelGGL(gather_one_kernel, dim3(1), dim3(kPermThreads), 0, st, x, idx, T, K, E, D,
                       expert, gathered, token_map, count);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

// ------------------------------------------------------- row scales
// One thread per sorted row: its token's nkb scale dwords (contiguous, read
// as 16-byte vectors where aligned) go to nkb K-step rows of dst, so each
// K-step row is written coalesced across the wave.  Rows past the valid
// ones (sorted_token not written there) read token 0: never consumed.
// One thread per (sorted row p, group of G scales): p runs fastest, so a
// wave's stores for one scale block are 64 consecutive dwords; G = 4 (one
// 16-byte load) when nkb is a multiple of 4, else 1.  Every row's gathers
// spread over nkb / G threads, all loads of a thread in one round trip.
template <int G>
__global__ __launch_bounds__(256) void gather_row_scales_kernel(const uint32_t* __restrict__ src,
                                                                const int* __restrict__ sorted_token,
                                                                long P, int T, int nkb,
                                                                uint32_t* __restrict__ dst) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long g = i / P, p = i - g * P;  // scale group, sorted row
    if (g * G >= nkb) return;
    int t = sorted_token[p];
    t = (t >= 0 && t < T) ? t : 0;
    const uint32_t* row = src + (size_t)t * nkb + g * G;
    if constexpr (G == 4) {
        const u32x4 v = *(const u32x4*)row;
#pragma unroll
        for (int k = 0; k < 4; k++) dst[(size_t)(4 * g + k) * P + p] = v[k];
    } else {
        dst[(size_t)g * P + p] = *row;
    }
}

int launch_gather_row_scales(const uint32_t* src, const int* sorted_token, long P, int T, int nkb,
                             uint32_t* dst, hipStream_t st) {
    AMDMOE_CHECK_ARG(P >= 0 && T > 0 && nkb > 0, "gather_row_scales: P=%ld T=%d nkb=%d", P, T, nkb);
    if (P == 0) return AMDMOE_OK;
    const bool vec = (nkb & 3) == 0;
    const long threads = P * (vec ? nkb / 4 : nkb);
    AMDMOE_CHECK_ARG(ceil_div(threads, 256) < (1L << 31), "gather_row_scales: %ld threads", threads);
    if (vec)
        hipLaunchKernelGGL(gather_row_scales_kernel<4>, dim3((unsigned)ceil_div(threads, 256)), dim3(256), 0, st,
                           src, sorted_token, P, T, nkb, dst);
    else
        hipLaunchKernelGGL(gather_row_scales_kernel<1>, dim3((unsigned)ceil_div(threads, 256)), dim3(256), 0, st,
                           src, sorted_token, P, T, nkb, dst);
    AMDMOE_LAUNCH_CHECK();
    return AMDMOE_OK;
}

}  // namespace amdmoe
