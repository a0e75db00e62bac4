// Top-k selection for gfx950: one 1024-thread workgroup per row of candidate scores.
//
// The reference selects with torch.topk (decode.py:86-93) and leaves ties unspecified; this kernel is the
// never-built "P2" selection step (docs/SCOPING_FUSED_D_KERNEL.md:56) with a defined order: larger score first, equal
// scores resolve to the lower candidate index, NaN ranks below every number, -0.0 equals +0.0.
//
// Algorithm: MSB-first radix select over an order-preserving 32-bit key in three digits of 11, 11 and 10 bits. The
// first digit is coarse enough that fp32 scores spread over tens of bins (an 8-bit first digit puts almost every
// score of one row into 4 bins and the LDS atomics serialize). In the fused decode step the first-digit histogram is
// built by the score kernel, which already holds every score, and arrives here in global memory; this kernel reads it
// and clears it for the next call, so only keys that share the first digit with the threshold are touched again.
// Each thread owns a contiguous segment of the row, so once the threshold key T and the number of ties to keep are
// known, one block-wide exclusive scan of (count > T, count == T) gives every thread the output slot of its first
// selected element and the rank of its first tie: indices come out in ascending order with no sort. The score order
// (the reference's cat(F, topk) row list) sorts the k selected (key, index) pairs once in LDS. Rows up to 1024 x 32
// scores keep their keys in registers; longer rows (L = 64K..128K) re-read the row (L2-resident) in every pass.
#include "common.h"
#include "select.h"

namespace attnlab {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kMaxScoreOrderK = 4096;

struct SelectArgs {
    const float* scores;
    int64_t score_stride;
    int M, k;
    // row-list output (attnlab_select_rows): F = [0, lo) U [hi, legal)
    int lo, hi, legal, G, C, order;
    int32_t* rows;
    int64_t rows_stride;
    int64_t* rows_flat;
    // top-k output (attnlab_topk)
    int32_t* top_idx;
    float* top_val;
    int64_t top_stride;
    // first-digit histograms [R][kHistBins] built by the score kernel (nullable); cleared here after use
    uint32_t* hist;
};

struct SelectShared {
    uint32_t hist[kHistBins];
    uint32_t wave_tot[kSelWaves][2];
    uint32_t digit, krem;
    uint64_t sortbuf[kMaxScoreOrderK];
};

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    return x;
}

// Block-wide exclusive scan of two counters at once (1024 threads). Ends with the block synchronised.
__device__ __forceinline__ void block_excl_scan2(uint32_t a, uint32_t b, uint32_t& ea, uint32_t& eb, SelectShared& sh) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t ia = wave_incl_scan(a, lane), ib = wave_incl_scan(b, lane);
    if (lane == 63) {
        sh.wave_tot[wave][0] = ia;
        sh.wave_tot[wave][1] = ib;
    }
    __syncthreads();
    uint32_t oa = 0, ob = 0;
    for (int w = 0; w < wave; ++w) {
        oa += sh.wave_tot[w][0];
        ob += sh.wave_tot[w][1];
    }
    ea = oa + ia - a;
    eb = ob + ib - b;
    __syncthreads();
}

// With the histogram of one digit complete in sh.hist[0..nbins), find the digit D holding the krem-th largest key:
// count(digit > D) < krem <= count(digit >= D). Thread t owns bins [2t, 2t+1]; the counts above a thread come from
// an exclusive scan over the threads in reverse order. Publishes D and the new krem; ends synchronised.
__device__ __forceinline__ void find_digit(SelectShared& sh, uint32_t krem, int nbins) {
    const int tid = threadIdx.x;
    const int rt = kSelThreads - 1 - tid;       // reverse rank: thread 1023 owns the lowest bins
    const int b0 = 2 * rt;
    const uint32_t c0 = b0 < nbins ? sh.hist[b0] : 0u, c1 = b0 + 1 < nbins ? sh.hist[b0 + 1] : 0u;
    uint32_t above, unused;
    block_excl_scan2(c0 + c1, 0u, above, unused, sh);   // keys in bins owned by lower tids = higher bins
    if (above < krem && above + c1 >= krem) {
        sh.digit = (uint32_t)(b0 + 1);
        sh.krem = krem - above;
    } else if (above + c1 < krem && above + c1 + c0 >= krem) {
        sh.digit = (uint32_t)b0;
        sh.krem = krem - above - c1;
    }
    __syncthreads();
}

// Threshold search. `for_each_key(fn)` calls fn(key) for every valid key of this thread. Returns T; sets krem_out to
// the number of keys equal to T that are selected. `ghist` (nullable) is the first digit's histogram of this row.
template <typename ForEach>
__device__ __forceinline__ uint32_t radix_threshold(int k, int M, ForEach for_each_key, SelectShared& sh,
                                                    const uint32_t* ghist, uint32_t& krem_out) {
    const int tid = threadIdx.x;
    if (k >= M) {  // every key is selected: threshold below every key, all ties taken
        krem_out = 0xffffffffu;
        return 0u;
    }
    constexpr int kShift[3] = {21, 10, 0};
    constexpr int kBins[3] = {2048, 2048, 1024};
    uint32_t prefix = 0, pmask = 0, krem = (uint32_t)k;
#pragma unroll
    for (int pass = 0; pass < 3; ++pass) {
        const int shift = kShift[pass], nb = kBins[pass];
        const uint32_t dmask = (uint32_t)nb - 1u;
        if (pass == 0 && ghist) {
            for (int i = tid; i < nb; i += kSelThreads) sh.hist[i] = ghist[i];
            __syncthreads();
        } else {
            for (int i = tid; i < nb; i += kSelThreads) sh.hist[i] = 0u;
            __syncthreads();
            for_each_key([&](uint32_t key) {
                if ((key & pmask) == prefix) atomicAdd(&sh.hist[(key >> shift) & dmask], 1u);
            });
            __syncthreads();
        }
        find_digit(sh, krem, nb);
        prefix |= sh.digit << shift;
        pmask |= dmask << shift;
        krem = sh.krem;
    }
    krem_out = krem;
    return prefix;
}

// Score order: fill sortbuf[0, next_pow2(k)) with 0, below every staged (key, ~index) pair (~index > 0 for any
// index < 2^32 - 1), so the padding sorts last. Ordered before the emission by the barriers of the block scan that
// follows.
__device__ __forceinline__ void init_sortbuf(const SelectArgs& a, SelectShared& sh) {
    if (a.order != ATTNLAB_ORDER_SCORE) return;
    int n = 1;
    while (n < a.k) n <<= 1;
    for (int i = threadIdx.x; i < n; i += kSelThreads) sh.sortbuf[i] = 0ull;
}

// F positions and, in score order, the sorted candidates (the selected pairs are staged in sh.sortbuf).
__device__ __forceinline__ void finish_row(const SelectArgs& a, int row, SelectShared& sh) {
    const int tid = threadIdx.x;
    const int lo = a.lo, hi = a.hi, k = a.k, order = a.order;
    const int nrec = a.legal - hi;
    const int S = lo + nrec + k;
    int32_t* rows = a.rows ? a.rows + (size_t)row * a.rows_stride : nullptr;
    int64_t* flat = a.rows_flat ? a.rows_flat + (size_t)row * S : nullptr;
    const int64_t base = (int64_t)row * a.C;
    const int nf = lo + nrec;
    if (rows || flat) {
        for (int f = tid; f < nf; f += kSelThreads) {
            const int pos = f < lo ? f : hi + (f - lo);
            const int s_out = (f < lo || order == ATTNLAB_ORDER_SCORE) ? f : lo + k + (f - lo);
            if (rows) rows[s_out] = pos;
            if (flat) flat[s_out] = base + pos;
        }
    }
    if (order != ATTNLAB_ORDER_SCORE || k == 0) return;
    // bitonic sort, descending on (key, ~index): larger score first, then lower index (sortbuf[0, n) was pre-filled
    // by init_sortbuf before the emission)
    int n = 1;
    while (n < k) n <<= 1;
    __syncthreads();
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < n / 2; i += kSelThreads) {
                const int lo_i = 2 * i - (i & (stride - 1));
                const int hi_i = lo_i + stride;
                const bool desc = ((lo_i & size) == 0);
                const uint64_t x = sh.sortbuf[lo_i], y = sh.sortbuf[hi_i];
                if ((x < y) == desc) {
                    sh.sortbuf[lo_i] = y;
                    sh.sortbuf[hi_i] = x;
                }
            }
            __syncthreads();
        }
    }
    const float* srow = a.scores + (size_t)row * a.score_stride;
    int32_t* ti = a.top_idx ? a.top_idx + (size_t)row * a.top_stride : nullptr;
    float* tv = a.top_val ? a.top_val + (size_t)row * a.top_stride : nullptr;
    for (int j = tid; j < k; j += kSelThreads) {
        const uint64_t e = sh.sortbuf[j];
        // clamped: a slot left as padding (only possible with a histogram that does not match the scores) must
        // still name a position of this row
        const int idx = min(max((int)(0xffffffffu - (uint32_t)(e & 0xffffffffu)), 0), a.M - 1);
        if (ti) ti[j] = idx;
        if (tv) tv[j] = srow[idx];
        if (rows) rows[nf + j] = lo + idx;
        if (flat) flat[nf + j] = base + lo + idx;
    }
}

// Emission of one thread's selected keys in ascending index order, starting at output slot `slot`. Slots at or past
// k are dropped: with consistent inputs exactly k keys are selected, and a first-digit histogram that does not belong
// to the scores can then only give a wrong selection, never a write outside the k output slots.
struct Emitter {
    int order, lo;
    uint32_t k;
    int32_t* ti;
    float* tv;
    const float* srow;
    int32_t* rows;       // already offset to this row and to slot lo
    int64_t* flat;       // likewise
    int64_t base;
    uint64_t* sortbuf;

    __device__ __forceinline__ void put(uint32_t slot, int idx, uint32_t key) const {
        if (slot >= k) return;
        if (order == ATTNLAB_ORDER_SCORE) {
            sortbuf[slot] = ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)idx);
            return;
        }
        if (ti) ti[slot] = idx;
        if (tv) tv[slot] = srow[idx];
        if (rows) rows[slot] = lo + idx;
        if (flat) flat[slot] = base + lo + idx;
    }
};

__device__ __forceinline__ Emitter make_emitter(const SelectArgs& a, int row, SelectShared& sh) {
    Emitter e;
    e.order = a.order;
    e.lo = a.lo;
    e.k = (uint32_t)a.k;
    e.ti = a.top_idx ? a.top_idx + (size_t)row * a.top_stride : nullptr;
    e.tv = a.top_val ? a.top_val + (size_t)row * a.top_stride : nullptr;
    e.srow = a.scores + (size_t)row * a.score_stride;
    e.rows = a.rows ? a.rows + (size_t)row * a.rows_stride + a.lo : nullptr;
    const int S = a.lo + (a.legal - a.hi) + a.k;
    e.flat = a.rows_flat ? a.rows_flat + (size_t)row * S + a.lo : nullptr;
    e.base = (int64_t)row * a.C;
    e.sortbuf = sh.sortbuf;
    return e;
}

// Keys of this thread's segment held in registers (M <= 1024 * KPT).
template <int KPT>
__global__ __launch_bounds__(kSelThreads) void select_reg(SelectArgs a) {
    __shared__ SelectShared sh;
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const float* s = a.scores + (size_t)row * a.score_stride;
    const int M = a.M;
    const int seg = tid * KPT;
    const int nvalid = max(0, min(KPT, M - seg));
    uint32_t* ghist = a.hist ? a.hist + (size_t)row * kHistBins : nullptr;
    uint32_t key[KPT];
    const bool vec = ((reinterpret_cast<uintptr_t>(s) & 15) == 0) && (KPT % 4 == 0);
    if (vec && nvalid == KPT) {
#pragma unroll
        for (int i = 0; i < KPT; i += 4) {
            const float4 f = *reinterpret_cast<const float4*>(s + seg + i);
            key[i] = score_key(f.x);
            key[i + 1] = score_key(f.y);
            key[i + 2] = score_key(f.z);
            key[i + 3] = score_key(f.w);
        }
    } else {
#pragma unroll
        for (int i = 0; i < KPT; ++i) key[i] = (i < nvalid) ? score_key(s[seg + i]) : 0u;
    }
    if (a.k > 0) {
        uint32_t krem = 0;
        const uint32_t T = radix_threshold(a.k, M, [&](auto fn) {
#pragma unroll
            for (int i = 0; i < KPT; ++i)
                if (i < nvalid) fn(key[i]);
        }, sh, ghist, krem);
        init_sortbuf(a, sh);
        uint32_t cgt = 0, ceq = 0;
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            if (i < nvalid) {
                cgt += key[i] > T;
                ceq += key[i] == T;
            }
        }
        uint32_t egt, eeq;
        block_excl_scan2(cgt, ceq, egt, eeq, sh);
        if (cgt + ceq > 0) {
            const Emitter em = make_emitter(a, row, sh);
            uint32_t slot = egt + min(eeq, krem);
            uint32_t ties = eeq;
#pragma unroll
            for (int i = 0; i < KPT; ++i) {
                const uint32_t kk = key[i];
                const bool eq = (i < nvalid) && kk == T;
                const bool take = (i < nvalid) && (kk > T || (eq && ties < krem));
                ties += eq;
                if (take) em.put(slot++, seg + i, kk);
            }
        }
    }
    if (ghist)  // leave the first-digit histogram zeroed for the next score/select pair
        for (int i = tid; i < kHistBins; i += kSelThreads) ghist[i] = 0u;
    __syncthreads();
    finish_row(a, row, sh);
}

// Long rows: keys are re-read from global memory in every pass.
__global__ __launch_bounds__(kSelThreads) void select_stream(SelectArgs a, int seglen) {
    __shared__ SelectShared sh;
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const float* s = a.scores + (size_t)row * a.score_stride;
    const int seg = tid * seglen;
    const int nvalid = max(0, min(seglen, a.M - seg));
    uint32_t* ghist = a.hist ? a.hist + (size_t)row * kHistBins : nullptr;
    if (a.k > 0) {
        uint32_t krem = 0;
        const uint32_t T = radix_threshold(a.k, a.M, [&](auto fn) {
            for (int i = 0; i < nvalid; ++i) fn(score_key(s[seg + i]));
        }, sh, ghist, krem);
        init_sortbuf(a, sh);
        uint32_t cgt = 0, ceq = 0;
        for (int i = 0; i < nvalid; ++i) {
            const uint32_t kk = score_key(s[seg + i]);
            cgt += kk > T;
            ceq += kk == T;
        }
        uint32_t egt, eeq;
        block_excl_scan2(cgt, ceq, egt, eeq, sh);
        if (cgt + ceq > 0) {
            const Emitter em = make_emitter(a, row, sh);
            uint32_t slot = egt + min(eeq, krem);
            uint32_t ties = eeq;
            for (int i = 0; i < nvalid; ++i) {
                const uint32_t kk = score_key(s[seg + i]);
                const bool eq = kk == T;
                const bool take = kk > T || (eq && ties < krem);
                ties += eq;
                if (take) em.put(slot++, seg + i, kk);
            }
        }
    }
    if (ghist)
        for (int i = tid; i < kHistBins; i += kSelThreads) ghist[i] = 0u;
    __syncthreads();
    finish_row(a, row, sh);
}

static int launch_select(const SelectArgs& a, int R, hipStream_t s) {
    const int kpt = (a.M + kSelThreads - 1) / kSelThreads;
    const dim3 grid(R), block(kSelThreads);
    if (kpt <= 4) hipLaunchKernelGGL(select_reg<4>, grid, block, 0, s, a);
    else if (kpt <= 8) hipLaunchKernelGGL(select_reg<8>, grid, block, 0, s, a);
    else if (kpt <= 16) hipLaunchKernelGGL(select_reg<16>, grid, block, 0, s, a);
    else if (kpt <= 32) hipLaunchKernelGGL(select_reg<32>, grid, block, 0, s, a);
    else hipLaunchKernelGGL(select_stream, grid, block, 0, s, a, kpt);
    return check_launch("select");
}

int select_rows_impl(const float* scores, int64_t score_stride, int B, int G, int lo, int hi, int legal, int k, int C,
                     int order, int32_t* rows, int64_t rows_stride, int64_t* rows_flat, uint32_t* hist,
                     hipStream_t stream) {
    ATTNLAB_REQUIRE(B >= 1 && G >= 1, "B and G must be positive (B=%d G=%d)", B, G);
    ATTNLAB_REQUIRE(0 <= lo && lo <= hi && hi <= legal && legal <= C, "need 0 <= lo <= hi <= legal <= C, got %d %d %d %d",
                    lo, hi, legal, C);
    const int M = hi - lo;
    ATTNLAB_REQUIRE(0 <= k && k <= M, "need 0 <= k <= hi - lo, got k=%d M=%d", k, M);
    ATTNLAB_REQUIRE(order == ATTNLAB_ORDER_POSITION || order == ATTNLAB_ORDER_SCORE, "unknown order %d", order);
    ATTNLAB_REQUIRE(order != ATTNLAB_ORDER_SCORE || k <= kMaxScoreOrderK, "score order supports k <= %d, got %d",
                    kMaxScoreOrderK, k);
    const int S = lo + (legal - hi) + k;
    ATTNLAB_REQUIRE(S >= 1, "empty row list");
    ATTNLAB_REQUIRE(rows == nullptr || rows_stride >= S, "rows_stride=%lld smaller than S=%d", (long long)rows_stride, S);
    ATTNLAB_REQUIRE(k == 0 || (scores != nullptr && score_stride >= M), "scores must hold M=%d values per row", M);
    if (!rows && !rows_flat && !hist) return ATTNLAB_OK;
    SelectArgs a{scores, score_stride, M, k, lo, hi, legal, G, C, order, rows, rows_stride, rows_flat, nullptr, nullptr, 0,
                 hist};
    return launch_select(a, B * G, stream);
}

}  // namespace attnlab

using namespace attnlab;

extern "C" int attnlab_topk(const float* scores, int64_t score_stride, int R, int M, int k, int order, int32_t* top_idx,
                            float* top_val, int64_t top_stride, void* stream) {
    ATTNLAB_REQUIRE(R >= 0 && M >= 0, "R=%d and M=%d must be non-negative", R, M);
    ATTNLAB_REQUIRE(0 <= k && k <= M, "need 0 <= k <= M, got k=%d M=%d", k, M);
    ATTNLAB_REQUIRE(order == ATTNLAB_ORDER_POSITION || order == ATTNLAB_ORDER_SCORE, "unknown order %d", order);
    ATTNLAB_REQUIRE(order != ATTNLAB_ORDER_SCORE || k <= kMaxScoreOrderK, "score order supports k <= %d, got %d",
                    kMaxScoreOrderK, k);
    if (R == 0 || k == 0) return ATTNLAB_OK;
    ATTNLAB_REQUIRE(scores != nullptr && score_stride >= M, "scores must hold M=%d values per row", M);
    ATTNLAB_REQUIRE(top_stride >= k, "top_stride=%lld smaller than k=%d", (long long)top_stride, k);
    SelectArgs a{scores, score_stride, M, k, 0, 0, 0, 1, 0, order, nullptr, 0, nullptr, top_idx, top_val, top_stride,
                 nullptr};
    return launch_select(a, R, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int attnlab_select_rows(const float* scores, int64_t score_stride, int B, int G, int lo, int hi, int legal,
                                   int k, int C, int order, int32_t* rows, int64_t rows_stride, int64_t* rows_flat,
                                   uint32_t* hist, void* stream) {
    return select_rows_impl(scores, score_stride, B, G, lo, hi, legal, k, C, order, rows, rows_stride, rows_flat, hist,
                            reinterpret_cast<hipStream_t>(stream));
}
