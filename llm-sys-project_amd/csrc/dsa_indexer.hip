// DeepSeek-V3.2's lightning indexer: the producer of the sparse indices the
// DSA decode consumes.  The reference has no indexer (its tests draw the
// indices at random, tests/test_dsa.cu:73-85); the formula is the published
// one, I[t,s] = sum_j w[t,j] * ReLU(q[t,j] . k[s]), in fp8:
//   score[q,s] = ks[row] * sum_j (hw[q,j] * qs[q,j]) * relu(q8[q,j,:] . k8[row,:])
//   row = page_table[q][s / page] * page + s % page,  s < seq_len[q]
// (the positive scales ks and qs commute with the ReLU), then the topk
// positions per query by score, ties to the lower position, listed in
// ascending position order -- the logical indices dsa_decode_bf16_paged takes.
//
// indexer_scores_kernel: a workgroup scores every nparts-th 256-position
//   tile of one query (the grid is what the device holds at once), 4
//   waves of 64 positions per tile; a tile's keys are loaded while the one
//   before it is scored, and its page ids one tile earlier still.  Per
//   16-position tile one fp8 MFMA per 16 heads,
//   S (16 positions x 16 heads) = K8 . Q8^T, keys as operand A straight from
//   the paged cache (two 16-byte loads per lane, a 128-byte row per 4
//   lanes), the query's heads as operand B held in registers.  Each lane
//   folds ReLU and the head weight over its heads, a 16-lane butterfly sums
//   the heads; HBM-bound on the keys (128 bytes + a 4-byte scale per
//   position).
// indexer_topk_kernel: one 1024-thread workgroup per query, 32 positions
//   per thread held in registers as order-preserving 32-bit keys.  A
//   most-significant-digit-first radix select (four 8-bit passes) finds the
//   key of the topk-th largest score and how many positions holding exactly
//   it are taken.  For the histogram passes a thread holds positions
//   tid, tid + 1024, ... and each wave counts into its own LDS histogram, so
//   one atomic instruction covers 64 unrelated positions (a shared
//   histogram with consecutive positions serialised on the few leading
//   digits real scores have; in the first pass the lanes sharing a digit
//   also combine their counts with a ballot).  Wave 0 then finds the digit
//   with a suffix scan across its lanes (4 digits per lane).  The selection
//   keeps the same layout: ballots and per-(wave, slice) counts give each
//   selected position its slot in ascending order, with no second read of
//   the row.
#include <algorithm>
#include <atomic>

#include "internal.hpp"

namespace amdmoe {

constexpr int kIdxD = 128;         // index head dim (bytes per fp8 row)
constexpr int kIdxMaxHeads = 128;  // index heads, a multiple of 16
constexpr int kIdxTile = 256;      // positions per workgroup of the scoring kernel
constexpr int kIdxMaxSeq = 32768;  // keys one selection workgroup holds (1024 threads x 32)
constexpr int kIdxMaxRow = 4 * kIdxMaxSeq;  // positions per query (rows above kIdxMaxSeq in parts)
constexpr int kTopkThreads = 1024;

// position -> (page, slot): shifts when the page size is a power of two
template <bool POW2>
__device__ __forceinline__ int page_of(int s, int page, int shift) { return POW2 ? s >> shift : s / page; }
template <bool POW2>
__device__ __forceinline__ int slot_of(int s, int page) { return POW2 ? s & (page - 1) : s % page; }

// sum over the 16 lanes of a row: quad_perm [1,0,3,2], [2,3,0,1], then
// row_half_mirror and row_mirror (every lane of the row ends with the sum)
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float v) {
    return dpp_add<0x140>(dpp_add<0x141>(dpp_add<0x4E>(dpp_add<0xB1>(v))));
}

// the 4 rows of a wave's 16-position tiles for lane r16: page ids of the
// tile are loaded one step ahead of its keys
struct IdxRows {
    int page_id[4];
};

template <bool POW2>
__device__ __forceinline__ void idx_load_pages(IdxRows& r, const int* pt, int tb, int wave, int r16, int page,
                                               int shift, int pages_per_seq) {
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int s = tb * kIdxTile + 64 * wave + 16 * t + r16;
        // loaded unconditionally (clamped index) so every wave issues the
        // same loads and waits can count them; positions past the sequence
        // are dropped by the key load's s < len (len <= pages_per_seq * page)
        r.page_id[t] = pt[min(page_of<POW2>(s, page, shift), pages_per_seq - 1)];
    }
}

template <bool POW2>
__device__ __forceinline__ void idx_load_keys(i32x8 (&kf)[4], float (&ksc)[4], const IdxRows& r,
                                              __amdgpu_buffer_rsrc_t rk, long kc_bytes,
                                              __amdgpu_buffer_rsrc_t rks, int tb, int wave, int g, int r16,
                                              int page, int len) {
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int s = tb * kIdxTile + 64 * wave + 16 * t + r16;
        const int p = r.page_id[t];
        long row = (long)p * page + slot_of<POW2>(s, page);
        if (s >= len || p < 0 || (row + 1) * kIdxD > kc_bytes) row = -1;
        const uint32_t vo = row >= 0 ? (uint32_t)(row * kIdxD + 16 * g) : kOob;
        const u32x4 lo = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, vo, 0, 0));
        const u32x4 hi = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, vo, 64, 0));
        kf[t] = (i32x8){(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                        (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        ksc[t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rks, row >= 0 ? (uint32_t)(row * 4) : kOob, 0, 0));
    }
}

// score one 256-position tile from the wave's keys: lane (g, r16) of the
// MFMA result holds S[4g + i][r16], positions 4g + i of a 16-tile, head r16
template <int HT>
__device__ __forceinline__ void idx_score_tile(const i32x8 (&kf)[4], const float (&ksc)[4], const i32x8 (&qf)[HT],
                                               const float (&wq)[HT], int tb, int wave, int g, int r16, int len,
                                               int max_seq, float* __restrict__ srow) {
#pragma unroll
    for (int t = 0; t < 4; t++) {
        float v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int h = 0; h < HT; h++) {
            const f32x4 c = mfma_fp8(kf[t], qf[h], (f32x4){0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] += wq[h] * fmaxf(c[i], 0.0f);
        }
        // sum over the 16 heads of each head tile: across the 16 lanes of a row
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = row16_sum(v[i]);
        // lane (g, n < 4) writes position 4g + n with the scale of its row,
        // held by the lane that loaded that row (r16 = 4g + n)
        const int n = r16 & 3;
        const float sc = __shfl(ksc[t], 4 * g + n, 64);
        const float tot = n == 0 ? v[0] : (n == 1 ? v[1] : (n == 2 ? v[2] : v[3]));
        const int s = tb * kIdxTile + 64 * wave + 16 * t + 4 * g + n;
        if (r16 < 4 && s < max_seq) srow[s] = s < len ? tot * sc : -INFINITY;
    }
}

template <int HT, bool POW2>  // head tiles of 16; page size a power of two (2^shift)
__global__ __launch_bounds__(256) void indexer_scores_kernel(
    const uint8_t* __restrict__ qc, const float* __restrict__ qs, const float* __restrict__ hw,
    const uint8_t* __restrict__ kc, long kc_bytes, const float* __restrict__ ks,
    const int* __restrict__ page_table, const int* __restrict__ seq_len, int Q, int page, int shift,
    int pages_per_seq, int max_seq, int ntile, int nparts, float* __restrict__ scores) {
    const int qi = blockIdx.x / nparts, part = blockIdx.x - qi * nparts;
    if (qi >= Q) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, r16 = lane & 15;
    const int* pt = page_table + (size_t)qi * pages_per_seq;
    // page ids of the first two tiles go out before anything else
    IdxRows pa, pb;
    idx_load_pages<POW2>(pa, pt, part, wave, r16, page, shift, pages_per_seq);
    idx_load_pages<POW2>(pb, pt, part + nparts, wave, r16, page, shift, pages_per_seq);
    // positions at or past seq_len and past the cache's capacity score -inf
    const int len = min(min(seq_len[qi], max_seq), pages_per_seq * page);
    constexpr int Hi = 16 * HT;

    // the query's heads as B operands: head 16h + r16, bytes 16g.. and 64+16g..
    i32x8 qf[HT];
    float wq[HT];
#pragma unroll
    for (int h = 0; h < HT; h++) {
        const uint8_t* qr = qc + ((size_t)qi * Hi + 16 * h + r16) * kIdxD;
        const u32x4 lo = *(const u32x4*)(qr + 16 * g), hi = *(const u32x4*)(qr + 64 + 16 * g);
        qf[h] = (i32x8){(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3],
                        (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        const size_t hq = (size_t)qi * Hi + 16 * h + r16;
        wq[h] = hw[hq] * qs[hq];
    }

    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kc, kc_bytes), rks = make_rsrc(ks, kc_bytes / kIdxD * 4);
    float* srow = scores + (size_t)qi * max_seq;
    // two key buffers in turn (A for tiles part, part + 2 nparts, ...; B for
    // the ones between): a tile's keys are loaded while the one before it
    // is scored, and its page ids one tile earlier still.  Page ids go out
    // before keys, as loads complete in issue order.
    i32x8 ka[4], kb[4];
    float sa[4], sb[4];
    idx_load_keys<POW2>(ka, sa, pa, rk, kc_bytes, rks, part, wave, g, r16, page, len);
    for (int tb = part; tb < ntile; tb += 2 * nparts) {
        const int t1 = tb + nparts, t2 = t1 + nparts;
        if (t1 < ntile) {
            idx_load_pages<POW2>(pa, pt, t2, wave, r16, page, shift, pages_per_seq);
            idx_load_keys<POW2>(kb, sb, pb, rk, kc_bytes, rks, t1, wave, g, r16, page, len);
        }
        idx_score_tile<HT>(ka, sa, qf, wq, tb, wave, g, r16, len, max_seq, srow);
        if (t1 >= ntile) break;
        if (t2 < ntile) {
            idx_load_pages<POW2>(pb, pt, t2 + nparts, wave, r16, page, shift, pages_per_seq);
            idx_load_keys<POW2>(ka, sa, pa, rk, kc_bytes, rks, t2, wave, g, r16, page, len);
        }
        idx_score_tile<HT>(kb, sb, qf, wq, t1, wave, g, r16, len, max_seq, srow);
    }
}

// order-preserving key of a score (larger score, larger key; -0 as +0)
__device__ __forceinline__ uint32_t score_key(float f) {
    if (f == 0.0f) f = 0.0f;
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// number of set bits of m in the lanes below this one
__device__ __forceinline__ int count_below(unsigned long long m) {
    return __builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0));
}

// x shifted across the lanes of each 16-lane row with DPP (row_shl:n reads
// lane + n, row_shr:n lane - n), 0 where the source lane leaves the row
template <int CTRL>
__device__ __forceinline__ unsigned dpp_row(unsigned x) {
    return (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false);
}
// inclusive sums over the wave: of this lane and every higher lane (suffix)
// or every lower lane (prefix).  Four DPP steps within each row, then the
// totals of the other rows (read from one lane of each) -- no LDS round
// trips, where a shuffle scan takes six.
__device__ __forceinline__ unsigned wave_suffix_sum(unsigned x, int lane) {
    x += dpp_row<0x101>(x);
    x += dpp_row<0x102>(x);
    x += dpp_row<0x104>(x);
    x += dpp_row<0x108>(x);
    const unsigned t1 = __builtin_amdgcn_readlane(x, 16), t2 = __builtin_amdgcn_readlane(x, 32),
                   t3 = __builtin_amdgcn_readlane(x, 48);
    const int row = lane >> 4;
    return x + (row < 1 ? t1 : 0u) + (row < 2 ? t2 : 0u) + (row < 3 ? t3 : 0u);
}
__device__ __forceinline__ unsigned wave_prefix_sum(unsigned x, int lane) {
    x += dpp_row<0x111>(x);
    x += dpp_row<0x112>(x);
    x += dpp_row<0x114>(x);
    x += dpp_row<0x118>(x);
    const unsigned t0 = __builtin_amdgcn_readlane(x, 15), t1 = __builtin_amdgcn_readlane(x, 31),
                   t2 = __builtin_amdgcn_readlane(x, 47);
    const int row = lane >> 4;
    return x + (row > 0 ? t0 : 0u) + (row > 1 ? t1 : 0u) + (row > 2 ? t2 : 0u);
}

// Selection modes: FULL selects a query's row in one workgroup; PART
// selects within one of the row's parts (positions [part * chunk, +chunk))
// and writes its top-k as (key, position) candidates in position order,
// padded with position -1; MERGE selects over a query's parts' candidates,
// read in part order, i.e. in position order.  Every position of the global
// top-k is in its part's top-k (the same order: key, then lower position),
// so PART + MERGE select exactly what FULL does.
enum { kSelFull = 0, kSelPart = 1, kSelMerge = 2 };

template <int kPer, int MODE>  // keys per thread: 1024 * kPer >= the keys one workgroup selects from
__global__ __launch_bounds__(kTopkThreads) void indexer_topk_kernel(const float* __restrict__ scores,
                                                                    const int* __restrict__ seq_len,
                                                                    int max_seq, int cap, int topk,
                                                                    int nparts, int chunk,
                                                                    uint2* __restrict__ cand,
                                                                    int* __restrict__ out) {
    constexpr int kWaves = kTopkThreads / 64;
    __shared__ __align__(16) int s_hist[kWaves][256];  // one histogram per wave
    __shared__ unsigned s_slice[kPer + 1];             // counts before each slice, total
    __shared__ int s_sel[3];                           // digit, remaining count, keys with the digit
    __shared__ int s_nvalid;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int qi = MODE == kSelPart ? blockIdx.x / nparts : blockIdx.x;
    const int part = MODE == kSelPart ? blockIdx.x - qi * nparts : 0;
    // the positions the scoring kernel scored: seq_len, at most max_seq
    // and the page-table row's capacity (cap = min of the two)
    const int n = max(0, min(seq_len[qi], cap));
    const float* row = scores + (size_t)qi * max_seq;
    // key j of this thread is slot j * 1024 + tid of the workgroup's range
    // (positions, or candidates in MERGE), so the 64 lanes of a wave hold 64
    // unrelated slots; pos[j] is its position, -1 when it selects nothing
    uint32_t key[kPer];
    int pos[kPer];
    int nvalid;
    if constexpr (MODE == kSelMerge) {
        const uint2* cq = cand + (size_t)qi * nparts * topk;
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < kPer; j++) {
            const int c = j * kTopkThreads + tid;
            const uint2 v = c < nparts * topk ? cq[c] : make_uint2(0u, 0xffffffffu);
            key[j] = v.x;
            pos[j] = (int)v.y;
            cnt += __popcll(__ballot(pos[j] >= 0));
        }
        if (tid == 0) s_nvalid = 0;
        __syncthreads();
        if (lane == 0) atomicAdd(&s_nvalid, cnt);
        __syncthreads();
        nvalid = s_nvalid;
    } else {
        const int lo = MODE == kSelPart ? part * chunk : 0;
        const int hi = MODE == kSelPart ? min(n, lo + chunk) : n;
        nvalid = max(0, hi - lo);
#pragma unroll
        for (int j = 0; j < kPer; j++) {
            const int s = lo + j * kTopkThreads + tid;
            const bool v = s < hi;
            key[j] = v ? score_key(row[s]) : 0u;
            pos[j] = v ? s : -1;
        }
    }

    // radix select of the topk-th largest key among the valid slots
    uint32_t prefix = 0, mask = 0;
    int need = min(topk, nvalid);
    const bool all = nvalid <= topk;
    if (!all) {
        for (int i = tid; i < kWaves * 256; i += kTopkThreads) (&s_hist[0][0])[i] = 0;
        __syncthreads();
        for (int shift = 24; shift >= 0; shift -= 8) {
#pragma unroll
            for (int j = 0; j < kPer; j++) {
                const int d = (key[j] >> shift) & 0xff;
                bool pending = pos[j] >= 0 && (key[j] & mask) == prefix;
                if (shift == 24) {
                    // leading digits cluster (sign and high exponent bits):
                    // the lanes sharing the first pending lane's digit add
                    // with one atomic
                    const unsigned long long act = __ballot(pending);
                    if (act != 0) {
                        const int leader = __ffsll((long long)act) - 1;
                        const int dl = __builtin_amdgcn_readlane(d, leader);
                        const unsigned long long m = __ballot(pending && d == dl);
                        if (lane == leader) atomicAdd(&s_hist[wave][dl], __popcll(m));
                        pending = pending && d != dl;
                    }
                }
                if (pending) atomicAdd(&s_hist[wave][d], 1);
            }
            __syncthreads();
            if (wave == 0) {
                // lane l owns digits 4l..4l+3: their counts over all waves,
                // zeroed behind it for the next pass
                int c[4] = {0, 0, 0, 0};
#pragma unroll
                for (int w = 0; w < kWaves; w++) {
                    int4* h = (int4*)&s_hist[w][4 * lane];
                    const int4 v = *h;
                    c[0] += v.x; c[1] += v.y; c[2] += v.z; c[3] += v.w;
                    *h = make_int4(0, 0, 0, 0);
                }
                // count of keys with digit >= 4l + i: this lane's suffix plus
                // every higher lane's total
                const int s3 = c[3], s2 = s3 + c[2], s1 = s2 + c[1], s0 = s1 + c[0];
                const int above = (int)wave_suffix_sum((unsigned)s0, lane) - s0;
                const int ge[4] = {above + s0, above + s1, above + s2, above + s3};
                // the digit is the largest d whose count of keys >= d reaches
                // need; the counts fall with d, so it is the number of such
                // digits minus one (digit 0 if none)
                const int cnt = __popcll(__ballot(ge[0] >= need)) + __popcll(__ballot(ge[1] >= need)) +
                                __popcll(__ballot(ge[2] >= need)) + __popcll(__ballot(ge[3] >= need));
                const int d = max(cnt - 1, 0);
                if (lane == (d >> 2)) {
                    const int i = d & 3;
                    const int ge_d = i == 0 ? ge[0] : (i == 1 ? ge[1] : (i == 2 ? ge[2] : ge[3]));
                    const int cd = i == 0 ? c[0] : (i == 1 ? c[1] : (i == 2 ? c[2] : c[3]));
                    s_sel[0] = d;
                    s_sel[1] = need - (ge_d - cd);
                    s_sel[2] = cd;
                }
            }
            __syncthreads();
            prefix |= (uint32_t)s_sel[0] << shift;
            mask |= 0xffu << shift;
            need = s_sel[1];
            // every key under the prefix is taken: the lower digits cannot
            // change the selection (uniform: all threads read the same LDS)
            if (need == s_sel[2]) break;
        }
    }
    // prefix = the threshold key's leading bits under mask; slots above it
    // are all taken, and the first `need` slots equal to it.  Slice j (slots j * 1024 + tid) is in
    // slot order across the workgroup, so each slot's output position is the
    // greater / equal keys of the slices before it, of the waves before it in
    // its slice (LDS counts) and of the lanes below it (ballots).
    unsigned* s_cnt = (unsigned*)&s_hist[0][0];  // [wave][slice]: greater | equal << 16
#pragma unroll
    for (int j = 0; j < kPer; j++) {
        const bool valid = pos[j] >= 0;
        const unsigned long long gm = __ballot(valid && (all || (key[j] & mask) > prefix));
        const unsigned long long em = __ballot(valid && !all && (key[j] & mask) == prefix);
        if (lane == 0) s_cnt[wave * kPer + j] = (unsigned)__popcll(gm) | ((unsigned)__popcll(em) << 16);
    }
    __syncthreads();
    if (wave == 0) {
        // counts before each (wave, slice) within the slice, in place, then
        // before each slice (both halves stay below 2^16: at most 32768 slots)
        unsigned run = 0;
        if (lane < kPer)
            for (int w = 0; w < kWaves; w++) {
                const unsigned v = s_cnt[w * kPer + lane];
                s_cnt[w * kPer + lane] = run;
                run += v;
            }
        const unsigned x = wave_prefix_sum(run, lane);
        if (lane < kPer) s_slice[lane] = x - run;
        if (lane == kPer - 1) s_slice[kPer] = x;
    }
    __syncthreads();
    int* o = out + (size_t)qi * topk;
    uint2* cp = cand + ((size_t)qi * nparts + part) * topk;
#pragma unroll
    for (int j = 0; j < kPer; j++) {
        const bool valid = pos[j] >= 0;
        const bool gt = valid && (all || (key[j] & mask) > prefix), eq = valid && !all && (key[j] & mask) == prefix;
        const unsigned long long gm = __ballot(gt), em = __ballot(eq);
        const unsigned base = s_slice[j] + s_cnt[wave * kPer + j];
        const int gb = (int)(base & 0xffff) + count_below(gm), eb = (int)(base >> 16) + count_below(em);
        if (gt || (eq && eb < need)) {
            if constexpr (MODE == kSelPart) cp[gb + min(eb, need)] = make_uint2(key[j], (uint32_t)pos[j]);
            else o[gb + min(eb, need)] = pos[j];
        }
    }
    const unsigned tot = s_slice[kPer];
    const int total = (int)(tot & 0xffff) + min((int)(tot >> 16), need);
    for (int j = total + tid; j < topk; j += kTopkThreads) {
        if constexpr (MODE == kSelPart) cp[j] = make_uint2(0u, 0xffffffffu);
        else o[j] = -1;
    }
}

// Row parts for the two-stage selection: enough parts for Q * parts to
// cover the device (at most 8), and enough that a part holds at most
// kIdxMaxSeq positions; a part must hold more than topk positions and the
// candidates of all parts (parts * topk) fit one workgroup's 32768 keys.
// Returns the part count (1: one workgroup per row) and the part length.
static int indexer_parts(int Q, int max_seq, int topk, int cus, int* chunk_out) {
    const int minp = (max_seq + kIdxMaxSeq - 1) / kIdxMaxSeq;
    const int want = std::max(minp, std::min(8, (cus + Q - 1) / std::max(Q, 1)));
    for (int p = want; p >= std::max(2, minp); p--) {
        const int chunk = (max_seq + p - 1) / p;
        const int ch = (chunk + kTopkThreads - 1) / kTopkThreads * kTopkThreads;
        const int pe = (max_seq + ch - 1) / ch;
        if (pe >= 2 && topk < ch && (long)pe * topk <= kIdxMaxSeq) {
            *chunk_out = ch;
            return pe;
        }
    }
    *chunk_out = max_seq;
    return minp == 1 ? 1 : -1;
}

// compute units of the current device (256 on MI355X), looked up once per device
static int device_cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// resident workgroups of the scoring kernel per CU (its register use sets it)
template <int HT, bool P2>
static int scores_blocks_per_cu() {
    static std::atomic<int> cache{0};
    int b = cache.load(std::memory_order_relaxed);
    if (b <= 0) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, indexer_scores_kernel<HT, P2>, 256, 0) != hipSuccess || b <= 0)
            b = 1;
        cache.store(b, std::memory_order_relaxed);
    }
    return b;
}

size_t dsa_indexer_scratch_bytes(int Q, int max_seq, int topk) {
    if (Q <= 0 || max_seq < 1 || max_seq > kIdxMaxRow || topk < 1) return 0;
    int chunk = 0;
    const int parts = indexer_parts(Q, max_seq, topk, device_cu_count(), &chunk);
    return parts >= 2 ? (size_t)Q * parts * topk * sizeof(uint2) : 0;
}

int launch_dsa_indexer(const uint8_t* qc, const float* qs, const float* hw, const uint8_t* kc,
                       long kc_rows, const float* ks, const int* page_table, const int* seq_len,
                       int Q, int Hi, int page, int pages_per_seq, int max_seq, int topk,
                       float* scores, int* out, void* scratch, size_t scratch_bytes, hipStream_t st) {
    AMDMOE_CHECK_ARG(Hi >= 16 && Hi <= kIdxMaxHeads && Hi % 16 == 0,
                     "dsa_indexer: Hi=%d must be a multiple of 16 in [16, %d]", Hi, kIdxMaxHeads);
    AMDMOE_CHECK_ARG(max_seq >= 1 && max_seq <= kIdxMaxRow, "dsa_indexer: max_seq=%d outside [1, %d]",
                     max_seq, kIdxMaxRow);
    AMDMOE_CHECK_ARG(topk >= 1 && page >= 1 && pages_per_seq >= 1 && kc_rows >= 1,
                     "dsa_indexer: bad topk / paging");
    int chunk = 0;
    const int parts = indexer_parts(std::max(Q, 1), max_seq, topk, device_cu_count(), &chunk);
    AMDMOE_CHECK_ARG(parts >= 1, "dsa_indexer: max_seq=%d above %d needs topk * parts <= %d (topk=%d)",
                     max_seq, kIdxMaxSeq, kIdxMaxSeq, topk);
    const size_t need = parts >= 2 ? (size_t)Q * parts * topk * sizeof(uint2) : 0;
    AMDMOE_CHECK_ARG(scratch_bytes >= need && (need == 0 || scratch != nullptr),
                     "dsa_indexer: scratch of %zu bytes, %zu needed", scratch_bytes, need);
    AMDMOE_CHECK_ARG(kc_rows * kIdxD < 0x7FFFFFF0L, "dsa_indexer: key cache of %ld rows exceeds 2 GiB", kc_rows);
    if (Q == 0) return AMDMOE_OK;
    const int ntile = (max_seq + kIdxTile - 1) / kIdxTile;
    AMDMOE_CHECK_ARG((long)Q * ntile < (1L << 31), "dsa_indexer: grid too large");
    const long kb = kc_rows * kIdxD;
    // each workgroup scores tiles part, part + nparts, ... of one query, the
    // grid sized to the workgroups the device holds at once
#define AMDMOE_IDX_LAUNCH2(HT, P2)                                                                      \
    do {                                                                                               \
        const long target = (long)scores_blocks_per_cu<HT, P2>() * device_cu_count();                 \
        const int nparts = (int)std::max(1L, std::min((long)ntile, (target + Q - 1) / Q));             \
        hipLaunchKernelGGL((indexer_scores_kernel<HT, P2>), dim3((unsigned)((long)Q * nparts)), dim3(256), \
                           0, st, qc, qs, hw, kc, kb, ks, page_table, seq_len, Q, page, shift,          \
                           pages_per_seq, max_seq, ntile, nparts, scores);                             \
    } while (0)
#define AMDMOE_IDX_LAUNCH(HT)                  \
    do {                                       \
        if (pow2) AMDMOE_IDX_LAUNCH2(HT, true);  \
        else AMDMOE_IDX_LAUNCH2(HT, false);      \
    } while (0)
    const bool pow2 = (page & (page - 1)) == 0;
    const int shift = pow2 ? __builtin_ctz((unsigned)page) : 0;
    switch (Hi / 16) {
        case 1: AMDMOE_IDX_LAUNCH(1); break;
        case 2: AMDMOE_IDX_LAUNCH(2); break;
        case 4: AMDMOE_IDX_LAUNCH(4); break;
        case 8: AMDMOE_IDX_LAUNCH(8); break;
        default: return set_error(AMDMOE_ERR_INVALID, "dsa_indexer: Hi=%d must be 16, 32, 64 or 128", Hi);
    }
#undef AMDMOE_IDX_LAUNCH
#undef AMDMOE_IDX_LAUNCH2
    AMDMOE_LAUNCH_CHECK();
    // registers hold the keys of one selection, rounded up to a power of two per thread
    const int cap = (int)std::min<long>(max_seq, (long)pages_per_seq * page);
    uint2* cand = (uint2*)scratch;
#define AMDMOE_TOPK_LAUNCH(P, MODE, GRID)                                                              \
    hipLaunchKernelGGL((indexer_topk_kernel<P, MODE>), dim3((unsigned)(GRID)), dim3(kTopkThreads), 0, st, \
                       scores, seq_len, max_seq, cap, topk, parts, chunk, cand, out)
#define AMDMOE_TOPK_DISPATCH(KEYS, MODE, GRID)                   \
    do {                                                         \
        const int per = ((KEYS) + kTopkThreads - 1) / kTopkThreads; \
        if (per <= 1) AMDMOE_TOPK_LAUNCH(1, MODE, GRID);         \
        else if (per <= 2) AMDMOE_TOPK_LAUNCH(2, MODE, GRID);    \
        else if (per <= 4) AMDMOE_TOPK_LAUNCH(4, MODE, GRID);    \
        else if (per <= 8) AMDMOE_TOPK_LAUNCH(8, MODE, GRID);    \
        else if (per <= 16) AMDMOE_TOPK_LAUNCH(16, MODE, GRID);  \
        else AMDMOE_TOPK_LAUNCH(32, MODE, GRID);                 \
        AMDMOE_LAUNCH_CHECK();                                   \
    } while (0)
    if (parts == 1) {
        AMDMOE_TOPK_DISPATCH(max_seq, kSelFull, Q);
    } else {
        // each part's top-k (Q * parts workgroups), then the top-k of the
        // parts' candidates
        AMDMOE_TOPK_DISPATCH(chunk, kSelPart, (long)Q * parts);
        AMDMOE_TOPK_DISPATCH(parts * topk, kSelMerge, Q);
    }
#undef AMDMOE_TOPK_DISPATCH
#undef AMDMOE_TOPK_LAUNCH
    return AMDMOE_OK;
}

}  // namespace amdmoe
