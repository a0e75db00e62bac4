// Top-k selection for gfx950: one 1024-thread workgroup per row of candidate scores.
//
// The reference selects with torch.topk (decode.py:86-93) and leaves ties unspecified; this kernel is the
// never-built "P2" selection step (docs/SCOPING_FUSED_D_KERNEL.md:56) with a defined order: larger score first, equal
// scores resolve to the lower candidate index, NaN ranks below every number, -0.0 equals +0.0.
//
// Algorithm: MSB-first radix select over an order-preserving 32-bit key, 8 bits per pass. Each thread owns a
// contiguous segment of the row, so after the threshold key T and the number of ties to keep are known, one
// block-wide exclusive scan of (count > T, count == T) gives every thread the output slot of its first selected
// element and the rank of its first tie: the selected indices come out in ascending index order with no sort. The
// score order (for the reference's cat(F, topk) row list) sorts the k selected (key, index) pairs once in LDS.
// Rows up to 1024 x 32 scores keep their keys in registers; longer rows (L = 64K..128K) re-read the row
// (L2-resident) in every pass.
#include "common.h"

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
};

// Order-preserving key: larger float -> larger key; -0 -> +0; NaN -> 0 (below -inf, whose key is 0x007fffff).
__device__ __forceinline__ uint32_t score_key(float f) {
    if (f != f) return 0u;
    uint32_t u = __float_as_uint(f);
    if (u == 0x80000000u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

struct SelectShared {
    uint32_t hist[kSelWaves][256];
    uint32_t wave_tot[kSelWaves][2];
    uint32_t digit, krem;
    uint64_t sortbuf[kMaxScoreOrderK];
};

// Inclusive scan over the 64 lanes of a wave.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    return x;
}

// Block-wide exclusive scan of two counters at once (1024 threads).
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
}

// After the histograms of one pass are complete, wave 0 finds the digit D holding the krem-th largest key among the
// keys that match the current prefix: count(digit > D) < krem <= count(digit >= D). Publishes D and the new krem.
__device__ __forceinline__ void find_digit(SelectShared& sh, uint32_t krem) {
    const int tid = threadIdx.x;
    if (tid >= 64) return;
    const int lane = tid;
    uint32_t c[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        uint32_t s = 0;
#pragma unroll
        for (int w = 0; w < kSelWaves; ++w) s += sh.hist[w][lane * 4 + b];
        c[b] = s;
    }
    const uint32_t tot = c[0] + c[1] + c[2] + c[3];
    // suffix sum over lanes: count in bins owned by lanes > lane
    uint32_t x = tot;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_down(x, o, 64);
        if (lane + o < 64) x += y;
    }
    uint32_t above = x - tot;
#pragma unroll
    for (int b = 3; b >= 0; --b) {
        if (above < krem && above + c[b] >= krem) {
            sh.digit = (uint32_t)(lane * 4 + b);
            sh.krem = krem - above;
        }
        above += c[b];
    }
}

// Threshold search shared by both kernels. `for_each_key(fn)` calls fn(key) for every valid key of this thread.
// Returns T; sets krem_out to the number of keys equal to T that are selected.
template <typename ForEach>
__device__ __forceinline__ uint32_t radix_threshold(int k, int M, ForEach for_each_key, SelectShared& sh, uint32_t& krem_out) {
    const int tid = threadIdx.x, wave = tid >> 6;
    if (k >= M) {  // every key is selected: threshold below every key, all ties taken
        krem_out = 0xffffffffu;
        return 0u;
    }
    uint32_t prefix = 0, pmask = 0, krem = (uint32_t)k;
    uint32_t* hflat = &sh.hist[0][0];
#pragma unroll 1
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        for (int i = tid; i < kSelWaves * 256; i += kSelThreads) hflat[i] = 0u;
        __syncthreads();
        for_each_key([&](uint32_t key) {
            if ((key & pmask) == prefix) atomicAdd(&sh.hist[wave][(key >> shift) & 255u], 1u);
        });
        __syncthreads();
        find_digit(sh, krem);
        __syncthreads();
        prefix |= sh.digit << shift;
        pmask |= 255u << shift;
        krem = sh.krem;
        __syncthreads();
    }
    krem_out = krem;
    return prefix;
}

// Writes selected candidate j (0 <= slot < k, ascending-index slot) or, in score order, stages it for the sort.
__device__ __forceinline__ void emit(const SelectArgs& a, int row, uint32_t slot, int idx, uint32_t key, SelectShared& sh) {
    if (a.order == ATTNLAB_ORDER_SCORE) {
        sh.sortbuf[slot] = ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)idx);
        return;
    }
    if (a.top_idx) a.top_idx[(size_t)row * a.top_stride + slot] = idx;
    if (a.top_val) a.top_val[(size_t)row * a.top_stride + slot] = a.scores[(size_t)row * a.score_stride + idx];
    if (a.rows || a.rows_flat) {
        const int s_out = a.lo + (int)slot;  // ascending positions: [0, lo) then the candidates then [hi, legal)
        const int pos = a.lo + idx;
        if (a.rows) a.rows[(size_t)row * a.rows_stride + s_out] = pos;
        if (a.rows_flat) {
            const int S = a.lo + (a.legal - a.hi) + a.k;
            a.rows_flat[(size_t)row * S + s_out] = (int64_t)pos + (int64_t)row * a.C;
        }
    }
}

// F positions and, in score order, the sorted candidates.
__device__ __forceinline__ void finish_row(const SelectArgs& a, int row, SelectShared& sh) {
    const int tid = threadIdx.x;
    const int nrec = a.legal - a.hi;
    const int S = a.lo + nrec + a.k;
    if (a.rows || a.rows_flat) {
        const int nf = a.lo + nrec;
        for (int f = tid; f < nf; f += kSelThreads) {
            int pos, s_out;
            if (f < a.lo) {
                pos = f;
                s_out = f;
            } else {
                pos = a.hi + (f - a.lo);
                s_out = (a.order == ATTNLAB_ORDER_SCORE) ? f : a.lo + a.k + (f - a.lo);
            }
            if (a.rows) a.rows[(size_t)row * a.rows_stride + s_out] = pos;
            if (a.rows_flat) a.rows_flat[(size_t)row * S + s_out] = (int64_t)pos + (int64_t)row * a.C;
        }
    }
    if (a.order != ATTNLAB_ORDER_SCORE || a.k == 0) return;
    // bitonic sort, descending on (key, ~index): larger score first, then lower index
    int n = 1;
    while (n < a.k) n <<= 1;
    for (int i = a.k + tid; i < n; i += kSelThreads) sh.sortbuf[i] = 0ull;
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
    const int nf = a.lo + nrec;
    for (int j = tid; j < a.k; j += kSelThreads) {
        const uint64_t e = sh.sortbuf[j];
        const int idx = (int)(0xffffffffu - (uint32_t)(e & 0xffffffffu));
        if (a.top_idx) a.top_idx[(size_t)row * a.top_stride + j] = idx;
        if (a.top_val) a.top_val[(size_t)row * a.top_stride + j] = a.scores[(size_t)row * a.score_stride + idx];
        const int pos = a.lo + idx;
        if (a.rows) a.rows[(size_t)row * a.rows_stride + nf + j] = pos;
        if (a.rows_flat) a.rows_flat[(size_t)row * S + nf + j] = (int64_t)pos + (int64_t)row * a.C;
    }
}

// Keys of this thread's segment held in registers (M <= 1024 * KPT).
template <int KPT>
__global__ __launch_bounds__(kSelThreads) void select_reg(SelectArgs a) {
    __shared__ SelectShared sh;
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const float* s = a.scores + (size_t)row * a.score_stride;
    const int seg = tid * KPT;
    const int nvalid = max(0, min(KPT, a.M - seg));
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
    uint32_t krem = 0, T = 0;
    if (a.k > 0) {
        T = radix_threshold(a.k, a.M, [&](auto fn) {
#pragma unroll
            for (int i = 0; i < KPT; ++i)
                if (i < nvalid) fn(key[i]);
        }, sh, krem);
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
        uint32_t slot = egt + min(eeq, krem);
        uint32_t ties = eeq;
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            if (i < nvalid) {
                const uint32_t kk = key[i];
                bool take = kk > T;
                if (kk == T) {
                    take = ties < krem;
                    ++ties;
                }
                if (take) emit(a, row, slot++, seg + i, kk, sh);
            }
        }
    }
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
    uint32_t krem = 0, T = 0;
    if (a.k > 0) {
        T = radix_threshold(a.k, a.M, [&](auto fn) {
            for (int i = 0; i < nvalid; ++i) fn(score_key(s[seg + i]));
        }, sh, krem);
        uint32_t cgt = 0, ceq = 0;
        for (int i = 0; i < nvalid; ++i) {
            const uint32_t kk = score_key(s[seg + i]);
            cgt += kk > T;
            ceq += kk == T;
        }
        uint32_t egt, eeq;
        block_excl_scan2(cgt, ceq, egt, eeq, sh);
        uint32_t slot = egt + min(eeq, krem);
        uint32_t ties = eeq;
        for (int i = 0; i < nvalid; ++i) {
            const uint32_t kk = score_key(s[seg + i]);
            bool take = kk > T;
            if (kk == T) {
                take = ties < krem;
                ++ties;
            }
            if (take) emit(a, row, slot++, seg + i, kk, sh);
        }
    }
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
    SelectArgs a{scores, score_stride, M, k, 0, 0, 0, 1, 0, order, nullptr, 0, nullptr, top_idx, top_val, top_stride};
    return launch_select(a, R, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int attnlab_select_rows(const float* scores, int64_t score_stride, int B, int G, int lo, int hi, int legal,
                                   int k, int C, int order, int32_t* rows, int64_t rows_stride, int64_t* rows_flat,
                                   void* stream) {
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
    if (!rows && !rows_flat) return ATTNLAB_OK;
    SelectArgs a{scores, score_stride, M, k, lo, hi, legal, G, C, order, rows, rows_stride, rows_flat, nullptr, nullptr, 0};
    return launch_select(a, B * G, reinterpret_cast<hipStream_t>(stream));
}
