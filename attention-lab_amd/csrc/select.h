// Pieces shared by the score and select kernels: the order-preserving score key and the first radix digit, whose
// per-row histogram the score kernel builds for the select kernel in the fused decode step.
#pragma once

#include <algorithm>

#include "common.h"

namespace attnlab {

constexpr int kHistBits = 11;                 // first digit: sign, exponent and the top two mantissa bits
constexpr int kHistBins = 1 << kHistBits;
constexpr int kHistShift = 32 - kHistBits;
// Per-row select state shared by the score, select and attend kernels of the fused step: the first-digit histogram
// (kHistBins words), then kSuperBins counts of 32 consecutive bins each (so the threshold's first digit is found from
// 64 + 32 words instead of 2048), then kArriveWords arrival counters of the attend's partitions (one per head group,
// the in-kernel split-K merge). Zero before the first call; the select leaves every word zero (after the score kernel
// and before the attend), and the attend leaves its counters zero.
constexpr int kSuperBins = kHistBins / 32;
constexpr int kArriveOffset = kHistBins + kSuperBins;
constexpr int kArriveWords = 64;
constexpr int kSelectStateWords = kArriveOffset + kArriveWords;
static_assert(kSelectStateWords == ATTNLAB_SELECT_STATE_WORDS, "ABI: ATTNLAB_SELECT_STATE_WORDS");

// Score order sorts up to this many selected pairs in LDS (64 KB); past it the select stages the picks in position
// order and a radix pass over a scratch buffer lists them by score (only the tiled and single-workgroup selects).
constexpr int kMaxScoreOrderK = ATTNLAB_LDS_SORT_K;
__host__ __device__ inline bool staged_score_order(int order, int k) {
    return order == ATTNLAB_ORDER_SCORE && k > kMaxScoreOrderK;
}

// Order-preserving key: larger float -> larger key; -0 -> +0; NaN -> 0 (below -inf, whose key is 0x007fffff).
__device__ __forceinline__ uint32_t score_key(float f) {
    if (f != f) return 0u;
    uint32_t u = __float_as_uint(f);
    if (u == 0x80000000u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// First-digit histogram of this block's scores (the select kernel's first radix pass), flushed to the row's global
// histogram with one device atomic per non-empty bin. Called by every thread of the block.
template <int BLOCK>
__device__ __forceinline__ void flush_histogram(uint32_t* hsh, uint32_t* ghist, int bg) {
    static_assert(BLOCK >= kSuperBins, "one thread per super-bin");
    __syncthreads();
    uint32_t* row = ghist + (size_t)bg * kSelectStateWords;
    // bins: thread t -> t, t + BLOCK, ...: the lanes of one atomic instruction hit consecutive words (two lines)
    for (int b = threadIdx.x; b < kHistBins; b += BLOCK) {
        const uint32_t c = hsh[b];
        if (c) atomicAdd(row + b, c);
    }
    // super-bins: lane s of the first wave sums bins [32 s, 32 s + 32), starting at a lane-dependent chunk so the
    // lanes spread over the LDS banks
    if (threadIdx.x < kSuperBins) {
        const int sb = threadIdx.x;
        uint32_t sum = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint4 v = *reinterpret_cast<const uint4*>(hsh + 32 * sb + 4 * ((sb + j) & 7));
            sum += v.x + v.y + v.z + v.w;
        }
        if (sum) atomicAdd(row + kHistBins + sb, sum);
    }
}

template <int BLOCK>
__device__ __forceinline__ void clear_histogram(uint32_t* hsh) {
    for (int b = threadIdx.x; b < kHistBins; b += BLOCK) hsh[b] = 0u;
}

// First digit of the rank-th largest key of a block's first-digit histogram in LDS (0 when it holds fewer keys),
// found by one wave on its own: lane l sums the l-th 32 bins from the top (starting at a lane-dependent 16-byte segment,
// so the lanes spread over the LDS banks), a DPP scan finds the chunk, a second scan its bin. No barrier; every lane of
// the calling wave gets the digit.
__device__ __forceinline__ uint32_t wave_digit_of_rank(const uint32_t* hist, uint32_t rank) {
    const int lane = threadIdx.x & 63;
    const int top = kHistBins - 32 * (lane + 1);   // lane 0: the highest 32 bins
    uint32_t sum = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint4 v = *reinterpret_cast<const uint4*>(hist + top + 4 * ((lane + i) & 7));
        sum += (v.x + v.y) + (v.z + v.w);
    }
    const uint32_t inc = wave_incl_scan(sum);
    const uint64_t m = __ballot(inc >= rank);
    if (m == 0) return 0u;
    const int l0 = __ffsll((unsigned long long)m) - 1;
    const uint32_t above = (uint32_t)__builtin_amdgcn_readlane((int)(inc - sum), l0);
    const int hib = kHistBins - 32 * l0 - 1;   // highest bin of that chunk
    const uint32_t c = lane < 32 ? hist[hib - lane] : 0u;
    const uint32_t inc2 = wave_incl_scan(c) + above;
    const uint64_t m2 = __ballot(lane < 32 && inc2 >= rank);
    return (uint32_t)(hib - (__ffsll((unsigned long long)m2) - 1));
}

// The index table a row's candidate scores come from, for the select of the fused step when the score kernel wrote
// only key lists: zT [B*G, 32, C] (bf16 or float32, C % 8 == 0, 16-byte aligned) and u [B*G, 32] as the score kernel
// built and stored it.
struct TableRef {
    const void* zT;
    int dtype;   // ATTNLAB_DT_BF16 or ATTNLAB_DT_F32
    int C;
    const float* u;
};

// Scores of index-table columns c0 .. c0 + 7 (c0 % 8 == 0, c0 + 8 <= C) of row bg, in the exact fp32 operation order
// of the one-launch score kernels (score_scan_fused, score_scan_fused_f32): for each group of eight index rows
// j in [8w, 8w + 8), an fma chain from zero in row order, then (p0 + p1) + (p2 + p3). A key recomputed here is
// therefore bit for bit the key those kernels counted in the histogram and put in the lists.
// One group of eight index rows (wave w of the score kernel): p[i] = fma chain over j in [8w, 8w + 8) of
// u[j] * z[j][c0 + i], from zero in row order. T: uint16_t (bf16 table) or float.
template <typename T>
__device__ __forceinline__ void rescore_rows8(const TableRef& t, int bg, int c0, int w, float (&p)[8]) {
    const float* u = t.u + (size_t)bg * 32 + 8 * w;
    const T* zr = static_cast<const T*>(t.zT) + ((size_t)bg * 32 + 8 * w) * (size_t)t.C + c0;
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
        float z[8];
        if constexpr (sizeof(T) == 4) {
            const float4* src = reinterpret_cast<const float4*>(zr + (size_t)jj * t.C);
            const float4 a = src[0], b = src[1];
            z[0] = a.x; z[1] = a.y; z[2] = a.z; z[3] = a.w;
            z[4] = b.x; z[5] = b.y; z[6] = b.z; z[7] = b.w;
        } else {
            const uint4 v = *reinterpret_cast<const uint4*>(zr + (size_t)jj * t.C);
            z[0] = bf16_lo(v.x); z[1] = bf16_hi(v.x); z[2] = bf16_lo(v.y); z[3] = bf16_hi(v.y);
            z[4] = bf16_lo(v.z); z[5] = bf16_hi(v.z); z[6] = bf16_lo(v.w); z[7] = bf16_hi(v.w);
        }
        const float uj = u[jj];
#pragma unroll
        for (int i = 0; i < 8; ++i) p[i] = __builtin_fmaf(uj, z[i], p[i]);
    }
}

// Rare paths (a tile whose list is incomplete, a row resolved by radix passes): each group of eight index rows is
// loaded and reduced before the next is issued (scheduling barriers), which keeps this off the select's register
// budget.
template <typename T>
__device__ __forceinline__ void rescore8_t(const TableRef& t, int bg, int c0, float (&s)[8]) {
    float a[8], b[8];
    rescore_rows8<T>(t, bg, c0, 0, a);
    __builtin_amdgcn_sched_barrier(0);
    rescore_rows8<T>(t, bg, c0, 1, b);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = a[i] + b[i];   // p0 + p1
    float c[8];
    rescore_rows8<T>(t, bg, c0, 2, b);
    __builtin_amdgcn_sched_barrier(0);
    rescore_rows8<T>(t, bg, c0, 3, c);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 8; ++i) s[i] = a[i] + (b[i] + c[i]);   // (p0 + p1) + (p2 + p3)
}

__device__ __forceinline__ void rescore8(const TableRef& t, int bg, int c0, float (&s)[8]) {
    if (t.dtype == ATTNLAB_DT_F32) rescore8_t<float>(t, bg, c0, s);
    else rescore8_t<uint16_t>(t, bg, c0, s);
}

// A row's candidate scores for the select: read from the stored scores where the score stage wrote them (srow,
// candidate index m at srow[m]), else recomputed from the index table. group8 gives table columns c0 .. c0 + 7
// (c0 % 8 == 0); entries outside [lo, hi) are 0 and must be masked by the caller.
struct RowScores {
    const float* srow;
    TableRef table;
    int bg, lo, hi;

    __device__ __forceinline__ void group8(int c0, float (&s)[8]) const {
        if (srow) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int c = c0 + i;
                s[i] = c >= lo && c < hi ? srow[c - lo] : 0.0f;
            }
        } else {
            rescore8(table, bg, c0, s);
        }
    }
};

// Per-workgroup key lists of the fused decode step (the score kernel writes them, the list select reads them): for
// each score workgroup of a row, every key of its tile whose first digit is at least the digit of its lmin-th largest
// key, as (candidate index, key) pairs, and a header (that digit, the list's length; a length above cap means the
// list was cut and its tile must be read in full).
struct ScoreLists {
    uint2* entries;   // [B*G, tiles, cap]
    uint2* hdr;       // [B*G, tiles]
    int lmin, cap;
};

// The key list of one 256-thread score workgroup (list number `list`), called by every thread once the workgroup's
// first-digit histogram in hsh is complete and synchronised: every valid key of its tile whose first digit is at least
// that of the tile's lmin-th largest key (each wave finds that digit itself, no barrier), in no particular order. A
// wave reserves its entries with one LDS atomic on lcount[0]; the wave that finishes last (lcount[1]) writes the
// header. Both counters start at zero. Thread t's keys: lkey[i] of column cb0 + (i / 2) * sstride + 2 t + i % 2, valid
// where bit i of lvalid is set.
template <int NSUB>
__device__ __forceinline__ void write_key_list(const ScoreLists& L, const uint32_t* hsh, uint32_t* lcount,
                                               const uint32_t (&lkey)[2 * NSUB], uint32_t lvalid, size_t list,
                                               int cb0, int sstride, int lo) {
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t dl = wave_digit_of_rank(hsh, (uint32_t)L.lmin);
    uint32_t m = 0u;
#pragma unroll
    for (int i = 0; i < 2 * NSUB; ++i) m |= (uint32_t)(((lvalid >> i) & 1u) && (lkey[i] >> kHistShift) >= dl) << i;
    const uint32_t n = (uint32_t)__popc(m);
    const uint32_t inc = wave_incl_scan(n);
    const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)inc, 63);
    uint32_t base = 0u;
    if (lane == 0) base = atomicAdd(&lcount[0], tot);
    uint32_t pos = (uint32_t)__builtin_amdgcn_readlane((int)base, 0) + inc - n;
    uint2* ent = L.entries + list * L.cap;
#pragma unroll
    for (int i = 0; i < 2 * NSUB; ++i) {
        if ((m >> i) & 1u) {
            const int c = cb0 + (i >> 1) * sstride + 2 * tid + (i & 1);
            if (pos < (uint32_t)L.cap) ent[pos] = make_uint2((uint32_t)(c - lo), lkey[i]);
            ++pos;
        }
    }
    // acquire-release at workgroup scope: this wave's reservation is ordered before its "done", and the count read
    // after the fourth wave's "done"
    if (lane == 0 && __hip_atomic_fetch_add(&lcount[1], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP) == 3)
        L.hdr[list] = make_uint2(dl, __hip_atomic_load(&lcount[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
}

// The argument checks of attnlab_select_rows (the decode step runs them before its first launch, so a rejected call
// leaves the select state untouched).
// scores_needed = false: the select recomputes its scores from the index table (the list select of the fused step).
int select_check(int B, int G, int lo, int hi, int legal, int k, int C, int order, const int32_t* rows,
                 int64_t rows_stride, const float* scores, int64_t score_stride, bool scores_needed = true);

// attnlab_select_rows: `state` [B*G][kSelectStateWords] (nullable) holds the first-digit histograms the score kernel
// built; with it and a scratch of select_scratch_bytes(B*G, M, k, order) the select runs tiled over the chip.
int select_rows_impl(const float* scores, int64_t score_stride, int B, int G, int lo, int hi, int legal, int k, int C,
                     int order, int32_t* rows, int64_t rows_stride, int64_t* rows_flat, uint32_t* state,
                     void* scratch, int64_t scratch_bytes, hipStream_t stream);

// Scratch bytes of the tiled select for R rows of M candidates, plus the score-order sort's buffers when order is
// score order and k exceeds what the LDS sort holds (no zeroing needed).
int64_t select_scratch_bytes(int R, int M, int k, int order);

// attnlab_score_grouped with an optional select-state output: per row, the first-digit histogram of the scores; and,
// with `lists` (only where fused_geometry applies and hist is given), the per-workgroup key lists.
int score_grouped_impl(uint16_t* zT, const uint16_t* k_new, const uint16_t* wk, const uint16_t* q_cat,
                       const uint16_t* wq_t, const float* u_in, float* u_out, float* out, int64_t out_stride, int B,
                       int G, int r, int C, int d, int hd, int lo, int hi, int write_col, int vector, uint32_t* hist,
                       hipStream_t stream, const ScoreLists* lists = nullptr);

// The one-launch score's tiling of a row (u, z column and scan in one kernel): sub-tiles of 512 columns per workgroup
// and workgroups per row; nsub == 0 when that kernel does not apply (u given, unaligned table, r != 32, h*d > 512).
struct FusedGeometry {
    int nsub, tiles;
};
// Sub-tiles per workgroup: 8, 4 or 2, as many as still leave 256 workgroups (one per CU), else 1. Fewer, longer
// workgroups run each one's tail (the histogram flush and the key list) less often and leave the select fewer lists
// to read: at 32K, per layer, B=2 26.1 against 27.0 us for the earlier rule (as many as leave 1024 workgroups, 2 for
// small grids), B=4 34.1 against 36.5, B=8 49.6 against 50.9; float32 tables B=4 46.3 against 52.5. B=1 (2 sub-tiles,
// 256 workgroups) and B=16 (8 sub-tiles, 1024 workgroups) tile as before.
inline FusedGeometry fused_tiling(int BG, int lo, int hi) {
    const int span = ((hi + 7) & ~7) - (lo & ~7);
    const int64_t blocks512 = (int64_t)BG * ((span + 511) / 512);
    const int nsub = blocks512 >= 8 * 256 ? 8 : blocks512 >= 4 * 256 ? 4 : blocks512 >= 2 * 256 ? 2 : 1;
    return FusedGeometry{nsub, (span + 512 * nsub - 1) / (512 * nsub)};
}
FusedGeometry fused_geometry(int BG, int C, int r, int hd, int lo, int hi, const void* zT, bool u_given);

// The list select's sizing for rows of M candidates and a top-k of k under the score tiling `g`: a workgroup's list
// holds at least lmin keys (its even share s of the k plus 3 sqrt(s) + 16, so that a list misses part of the row's
// selection only when its tile holds several standard deviations more than its share), and at most cap (lmin plus
// 192, for the keys of the first-digit bin holding the lmin-th key). cap == 0: the list select does not apply (rows
// past 32768 candidates or 128 tiles, or lists that would hold half a tile or more).
constexpr int kListMaxM = 32768;
constexpr int kListMaxTiles = 128;
struct ListPlan {
    int lmin, cap;
};
inline ListPlan list_plan(int M, int k, FusedGeometry g) {
    if (g.nsub == 0 || k <= 0 || M > kListMaxM || g.tiles > kListMaxTiles) return ListPlan{0, 0};
    const int nw = 512 * g.nsub;
    const int64_t share = ((int64_t)k * nw + M - 1) / M;
    int64_t root = 0;
    while ((root + 1) * (root + 1) <= share) ++root;
    const int64_t lmin = share + 3 * root + 16;
    if (2 * lmin > nw) return ListPlan{0, 0};
    return ListPlan{(int)lmin, (int)std::min<int64_t>(nw, (lmin + 192 + 63) / 64 * 64)};
}
// Bytes of the lists (entries, then headers, 256-byte aligned) for R rows.
inline int64_t list_entry_bytes(int R, FusedGeometry g, ListPlan p) {
    return ((int64_t)R * g.tiles * p.cap * 8 + 255) / 256 * 256;
}
inline int64_t list_bytes(int R, FusedGeometry g, ListPlan p) {
    return list_entry_bytes(R, g, p) + ((int64_t)R * g.tiles * 8 + 255) / 256 * 256;
}
// The list region of R rows of candidates [lo, hi) with a top-k of k (0: the list select does not apply), and the
// lists laid out in a region at `base`.
inline int64_t list_region_bytes(int64_t R, int lo, int hi, int k) {
    if (hi <= lo || k <= 0) return 0;
    const FusedGeometry g = fused_tiling((int)R, lo, hi);
    const ListPlan p = list_plan(hi - lo, k, g);
    return p.cap > 0 ? list_bytes((int)R, g, p) : 0;
}
inline ScoreLists list_layout(void* base, int R, FusedGeometry g, ListPlan p) {
    char* b = static_cast<char*>(base);
    return ScoreLists{reinterpret_cast<uint2*>(b), reinterpret_cast<uint2*>(b + list_entry_bytes(R, g, p)), p.lmin,
                      p.cap};
}

// One index row's z value at d = 128: of the eight threads of a row, thread t % 8 takes dims 16 (t % 8) .. + 15 (two
// 16-byte words of wk[g, j] and of k_new) as a chain of eight bf16 dot2 from zero, then sum8 adds the eight partial
// sums. Every writer of a z column (write_z and the score kernel's early forms) uses this order, so a column has the
// same bits whichever workgroup writes it. Called by all lanes of the wave (sum8 exchanges).
__device__ __forceinline__ float z_dot16(uint4 w0, uint4 w1, uint4 k0, uint4 k1) {
    float s = 0.0f;
    s = dot2_bf16(w0.x, k0.x, s); s = dot2_bf16(w0.y, k0.y, s);
    s = dot2_bf16(w0.z, k0.z, s); s = dot2_bf16(w0.w, k0.w, s);
    s = dot2_bf16(w1.x, k1.x, s); s = dot2_bf16(w1.y, k1.y, s);
    s = dot2_bf16(w1.z, k1.z, s); s = dot2_bf16(w1.w, k1.w, s);
    return sum8(s);
}

// The list select of the fused decode step: from the score kernel's per-workgroup lists (and the full tile scores of
// any list that cannot hold the row's selection), the top-k and F as attnlab_select_rows writes them; one launch.
// scores may be null when `table` is given (its zT and u): the select then recomputes the scores of a tile whose list
// is incomplete (and of a row resolved by radix passes) from the table, bit-exact; position order only, since score
// order reads the selected keys' scores back.
int select_lists_impl(const float* scores, int64_t score_stride, int B, int G, int lo, int hi, int legal, int k, int C,
                      int order, int32_t* rows, int64_t rows_stride, int64_t* rows_flat, uint32_t* state,
                      const ScoreLists& lists, FusedGeometry geo, hipStream_t stream, TableRef table = TableRef{});

// attnlab_attend with, when `arrive` is given and P > 1, the split-K merge inside the attend kernel instead of the
// combine kernel: per (b, g) row one arrival counter per head group at arrive + bg * arrive_stride, zero on entry and
// left zero (the fused step's select state holds them).
int attend_impl(const uint16_t* K, const uint16_t* V, int64_t kv_bg_stride, int kv_row_stride, const uint16_t* q,
                const int32_t* rows, int64_t rows_stride, int B, int G, int h, int S, int C, int P, float scale,
                void* out, int out_bf16, float* part, uint32_t* arrive, int64_t arrive_stride, hipStream_t stream);

// Head groups of the attend's grid: the h heads split over 2, 4, ... workgroups while the grid is below one workgroup
// per CU (attend.hip).
int attend_head_groups(int BG, int h, int P);

// The fused step's select and attend in one launch (select.hip: select_attend), for position order with no row list
// leaving the call: whether it applies to these sizes (each partition's row-list entries fit its LDS, one, two or four
// heads per workgroup), and the launch. state, lists, geo and table as for select_lists_impl; K, V [B*G, C, 128], q
// [B*G, h, 128], out [B*G, h, 128] bf16; part [B*G, P, h, 130] for P > 1, merged in-kernel with the state's counters.
bool select_attend_applies(int B, int G, int lo, int hi, int legal, int k, int h, int P);
int select_attend_impl(int B, int G, int lo, int hi, int legal, int k, int C, uint32_t* state, const ScoreLists& lists,
                       FusedGeometry geo, TableRef table, const uint16_t* K, const uint16_t* V, const uint16_t* q, int h,
                       int P, float scale, uint16_t* out, float* part, hipStream_t stream);

// attnlab_score_grouped_f32: the same score on float32 tables (trained index banks); two launches (prologue, scan).
int score_grouped_f32_impl(float* zT, const float* k_new, const float* wk, const float* q_cat, const float* wq_t,
                           const float* u_in, float* u_out, float* out, int64_t out_stride, int B, int G, int r,
                           int C, int d, int hd, int lo, int hi, int write_col, uint32_t* hist, hipStream_t stream,
                           const ScoreLists* lists = nullptr);
// The float32 one-launch score's tiling (the bf16 kernel's, fused_tiling), or nsub == 0 where it does not apply:
// r != 32, C % 8 != 0, zT not 16-byte aligned, an empty range, or (u not given) h*d > 512 or wq_t not 16-byte aligned.
FusedGeometry fused_geometry_f32(int BG, int C, int r, int hd, int lo, int hi, const void* zT, const void* wq_t,
                                 bool u_given);

}  // namespace attnlab
