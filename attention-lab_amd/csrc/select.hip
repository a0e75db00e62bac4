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
// Once the threshold key T and the number of ties to keep are known, every thread owns a contiguous range of indices
// (its segment of the row, or for register-resident rows its word of two LDS bitmaps), and one block-wide exclusive
// scan of (count > T, count == T) gives it the output slot of its first selected element and the rank of its first
// tie: indices come out in ascending order with no sort. The score order (the reference's cat(F, topk) row list)
// sorts the k selected (key, index) pairs once in LDS. Rows up to 32768 scores keep their keys in registers, loaded
// coalesced; longer rows (L = 64K..128K) re-read the row (L2-resident) in every pass.
#include "common.h"
#include "select.h"
#include "select_core.h"
#include "attend_core.h"

namespace attnlab {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;

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
    // select state [R][kSelectStateWords] whose first kHistBins words are the first-digit histogram built by the score
    // kernel (nullable); cleared here after use
    uint32_t* hist;
};

struct SelectShared {
    __attribute__((aligned(16))) uint32_t hist[kHistBins];
    uint32_t wave_tot[kSelWaves][2];
    uint32_t digit, krem, dcount;
    uint64_t sortbuf[kMaxScoreOrderK];
    uint32_t dbase[256];   // score order past 1024 picks: each digit's next slot in a radix pass
};

// Block-wide exclusive scan of two counters for THREADS (<= 1024) threads; tot_a / tot_b receive the block totals.
// The wave totals are scanned by every wave at once: lanes 0..15 hold the first counter's, lanes 16..31 the second's,
// and one row-local DPP scan covers both. Ends synchronised.
template <int THREADS>
__device__ __forceinline__ void block_scan2(uint32_t a, uint32_t b, uint32_t& ea, uint32_t& eb, uint32_t& tot_a,
                                            uint32_t& tot_b, uint32_t (*wave_tot)[2]) {
    constexpr int kWaves = THREADS / 64;
    static_assert(kWaves <= 16, "one row of 16 lanes per counter");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t ia = wave_incl_scan(a), ib = wave_incl_scan(b);
    if (lane == 63) {
        wave_tot[wave][0] = ia;
        wave_tot[wave][1] = ib;
    }
    __syncthreads();
    uint32_t v = 0;
    if (lane < kWaves) v = wave_tot[lane][0];
    else if (lane >= 16 && lane < 16 + kWaves) v = wave_tot[lane - 16][1];
    const uint32_t vi = row16_incl_scan(v);
    const uint32_t ve = vi - v;
    ea = (uint32_t)__builtin_amdgcn_readlane((int)ve, wave) + ia - a;
    eb = (uint32_t)__builtin_amdgcn_readlane((int)ve, 16 + wave) + ib - b;
    tot_a = (uint32_t)__builtin_amdgcn_readlane((int)vi, 15);
    tot_b = (uint32_t)__builtin_amdgcn_readlane((int)vi, 31);
    __syncthreads();
}

// Block-wide exclusive scan of one counter for kSelThreads threads with a single barrier, for a last scan: wave_tot
// is left holding this scan's wave totals, so no other scan may follow it without a barrier first.
__device__ __forceinline__ uint32_t block_excl_scan_once(uint32_t x, uint32_t (*wave_tot)[2]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t inc = wave_incl_scan(x);
    if (lane == 63) wave_tot[wave][0] = inc;
    __syncthreads();
    const uint32_t v = lane < kSelWaves ? wave_tot[lane][0] : 0u;
    const uint32_t vi = row16_incl_scan(v);
    return (uint32_t)__builtin_amdgcn_readlane((int)(vi - v), wave) + inc - x;
}

__device__ __forceinline__ void block_excl_scan2(uint32_t a, uint32_t b, uint32_t& ea, uint32_t& eb, SelectShared& sh) {
    uint32_t ta, tb;
    block_scan2<kSelThreads>(a, b, ea, eb, ta, tb, sh.wave_tot);
}

// The digit D holding the krem-th largest key of a complete histogram (count(digit > D) < krem <= count(digit >= D)),
// found by wave 0 alone, for nbins = 1024 or 2048: lane l sums the l-th chunk of nbins / 64 bins from the
// top (starting at a lane-dependent 16-byte segment, so the lanes spread over the LDS banks), a DPP scan over the
// lanes finds the chunk holding the krem-th largest key, and a second scan over that chunk's bins, one per lane, finds
// the bin. Publishes D, the new krem and the count of bin D; ends with one barrier.
__device__ __forceinline__ void find_digit_wave(SelectShared& sh, const uint32_t* hist, uint32_t krem, int nbins) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const int per = nbins >> 6;                 // 16 or 32 bins per lane
        const int cb = nbins - per * (lane + 1);    // lane 0: the highest chunk
        const int nseg = per >> 2;
        uint32_t sum = 0;
        for (int i = 0; i < nseg; ++i) {
            const uint4 v = *reinterpret_cast<const uint4*>(hist + cb + 4 * ((lane + i) & (nseg - 1)));
            sum += (v.x + v.y) + (v.z + v.w);
        }
        const uint32_t inc = wave_incl_scan(sum);
        const uint64_t m = __ballot(inc >= krem);
        if (m != 0) {
            const int l0 = __ffsll((unsigned long long)m) - 1;
            const uint32_t above = (uint32_t)__builtin_amdgcn_readlane((int)(inc - sum), l0);
            const int top = nbins - per * l0 - 1;    // highest bin of that chunk
            const uint32_t c = lane < per ? hist[top - lane] : 0u;
            const uint32_t inc2 = wave_incl_scan(c) + above;
            const uint64_t m2 = __ballot(lane < per && inc2 >= krem);
            if (m2 != 0 && lane == __ffsll((unsigned long long)m2) - 1) {
                sh.digit = (uint32_t)(top - lane);
                sh.krem = krem - (inc2 - c);
                sh.dcount = c;
            }
        }
    }
    __syncthreads();
}

// Length of the score-order sort: k rounded up to a power of two, at least one 128-element chunk.
__device__ __forceinline__ int sort_len(int k) {
    int n = 128;
    while (n < k) n <<= 1;
    return n;
}

// Score order: fill sortbuf[0, sort_len(k)) with 0, below every staged (key, ~index) pair (~index > 0 for any
// index < 2^32 - 1), so the padding sorts last. Ordered before the emission by the barriers of the block scan that
// follows.
__device__ __forceinline__ void init_sortbuf(const SelectArgs& a, SelectShared& sh) {
    if (a.order != ATTNLAB_ORDER_SCORE) return;
    const int n = sort_len(a.k);
    for (int i = threadIdx.x; i < n; i += kSelThreads) sh.sortbuf[i] = 0ull;
}

// Bitonic sort of buf[0, n), descending, n a power of two >= 128. Every compare-exchange whose partner lies in the same
// 128-element chunk runs in registers: a wave holds a chunk as two elements per lane (c0 + lane, c0 + 64 + lane), so
// stride 64 is within a lane and strides 32..1 are lane shuffles. Only strides >= 128 go through LDS, one barrier
// each; a chunk pass runs every stride of a merge below 128 (and, first, every merge up to 128) with one barrier.
__device__ __forceinline__ void cmpx_reg(uint64_t& x, int i, int stride, int size, int lane) {
    const uint64_t y = __shfl_xor(x, stride);
    const bool lower = (lane & stride) == 0;
    const bool desc = (i & size) == 0;
    // the lower element of a pair keeps the larger value in a descending block
    const bool take_max = lower == desc;
    x = take_max ? (x > y ? x : y) : (x < y ? x : y);
}

__device__ __forceinline__ void chunk_pass(uint64_t* buf, int n, int size_first, int size_last, int stride_first) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int kWaves = kSelThreads / 64;
    for (int c0 = wave * 128; c0 < n; c0 += kWaves * 128) {
        uint64_t x0 = buf[c0 + lane], x1 = buf[c0 + 64 + lane];
        const int i0 = c0 + lane, i1 = c0 + 64 + lane;
        for (int size = size_first; size <= size_last; size <<= 1) {
            int stride = size == size_first ? stride_first : size >> 1;
            if (stride == 64) {
                const bool desc = (i0 & size) == 0;
                if ((x0 < x1) == desc) {
                    const uint64_t t = x0;
                    x0 = x1;
                    x1 = t;
                }
                stride = 32;
            }
            for (; stride > 0; stride >>= 1) {
                cmpx_reg(x0, i0, stride, size, lane);
                cmpx_reg(x1, i1, stride, size, lane);
            }
        }
        buf[c0 + lane] = x0;
        buf[c0 + 64 + lane] = x1;
    }
}

__device__ __forceinline__ void bitonic_sort_desc(uint64_t* buf, int n) {
    const int tid = threadIdx.x;
    chunk_pass(buf, n, 2, 128, 1);   // every merge up to size 128, inside the chunks
    __syncthreads();
    for (int size = 256; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride >= 128; stride >>= 1) {
            for (int i = tid; i < n / 2; i += kSelThreads) {
                const int lo_i = 2 * i - (i & (stride - 1));
                const int hi_i = lo_i + stride;
                const bool desc = (lo_i & size) == 0;
                const uint64_t x = buf[lo_i], y = buf[hi_i];
                if ((x < y) == desc) {
                    buf[lo_i] = y;
                    buf[hi_i] = x;
                }
            }
            __syncthreads();
        }
        chunk_pass(buf, n, size, size, 64);
        __syncthreads();
    }
}

// Score order for up to 1024 staged pairs (one per thread): a stable LSD radix sort on the pair's key, passes of 8
// bits, descending (each digit complemented). The pairs arrive in ascending index order (the emission's slots), so
// stability leaves equal keys in index order, the same order as sorting on (key, ~index). A pass: the lanes of a wave
// holding the same digit find each other with eight ballots (rank among them: the lanes below); each group's leader
// writes its count into a [digit][wave] table; one exclusive scan of the table's 4096 entries in that order (thread t
// owns entries 4t..4t+3, one 8-byte read) gives every (digit, wave) group its first slot; every pair then moves to its
// slot in the other buffer. Two count tables alternate, so the one for the next pass is cleared while this one is read:
// four barriers per pass. A pass whose 8 bits are the same in every key would leave the order as it is and is skipped
// (the bits that differ anywhere are gathered during the first pass). Buffers: sortbuf[0, 1024) and
// sortbuf[1024, 2048); the tables after them. Returns the buffer holding the sorted pairs.
__device__ __forceinline__ const uint64_t* radix_sort_desc_1024(SelectShared& sh, int k) {
    static_assert(sizeof(SelectShared::sortbuf) >= 4096 * sizeof(uint64_t),
                  "two 1024-pair buffers and two count tables of 256 x 16 uint16");
    static_assert(kSelThreads * 4 == 256 * kSelWaves, "four table entries per thread");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = sort_len(k);
    // pairs in sortbuf[1024 * cur, +1024), the pass's count table in sortbuf[2048 + 1024 * cur, +1024) as uint16
    // [256][16]; cur alternates between passes (offsets, not an array of pointers, so the accesses stay LDS ones)
    uint64_t* const base = sh.sortbuf;
    reinterpret_cast<uint32_t*>(base + 2048)[tid] = 0u;   // table 0: 2048 words, two per thread
    reinterpret_cast<uint32_t*>(base + 2048)[tid + kSelThreads] = 0u;
    __syncthreads();
    const bool valid = tid < n;
    const uint64_t lt = (1ull << lane) - 1ull;
    uint32_t differ = 0xffffffffu;   // key bits that differ between some two pairs (all, until the first pass knows)
    int cur = 0;
#pragma unroll
    for (int pass = 0; pass < 4; ++pass) {
        if (pass > 0 && ((differ >> (8 * pass)) & 255u) == 0u) continue;   // uniform digit: a stable no-op
        uint64_t* const src = base + 1024 * cur;
        uint64_t* const dst = base + 1024 * (cur ^ 1);
        uint16_t* const c = reinterpret_cast<uint16_t*>(base + 2048 + 1024 * cur);
        uint32_t* const next = reinterpret_cast<uint32_t*>(base + 2048 + 1024 * (cur ^ 1));
        const uint64_t x = valid ? src[tid] : 0ull;
        const uint32_t key = (uint32_t)(x >> 32);
        const uint32_t dg = 255u - ((key >> (8 * pass)) & 255u);
        // lanes whose digit equals this lane's: per bit, the lanes that agree with it are the ballot of the bit
        // XNOR this lane's bit as an all-ones / zero mask
        const uint64_t act = __ballot(valid);
        uint32_t plo = (uint32_t)act, phi = (uint32_t)(act >> 32);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint32_t bm = (uint32_t)__builtin_amdgcn_sbfe((int)key, 8 * pass + b, 1);   // 0 or ~0
            const uint64_t m = __ballot(bm != 0u);
            plo &= ~((uint32_t)m ^ bm);
            phi &= ~((uint32_t)(m >> 32) ^ bm);
        }
        const uint64_t peers = ((uint64_t)phi << 32) | plo;
        const uint32_t rank = (uint32_t)__popcll(peers & lt);
        const int slot = (int)dg * kSelWaves + wave;
        if (valid && rank == 0) c[slot] = (uint16_t)__popcll(peers);
        next[tid] = 0u;   // the next pass's table, untouched in this one
        next[tid + kSelThreads] = 0u;
        if (pass == 0) {   // OR over the block of key ^ (the first pair's key), a wave's share in wave_tot[.][1]
            uint32_t d = valid ? key ^ (uint32_t)(base[0] >> 32) : 0u;
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) d |= (uint32_t)__shfl_xor((int)d, m, 64);
            if (lane == 0) sh.wave_tot[wave][1] = d;
        }
        __syncthreads();
        if (pass == 0) {
            differ = 0u;
#pragma unroll
            for (int w = 0; w < kSelWaves; ++w) differ |= sh.wave_tot[w][1];
        }
        // exclusive scan of the table in (digit, wave) order: thread t owns entries 4t..4t+3
        uint2* const cw = reinterpret_cast<uint2*>(c);
        const uint2 raw = cw[tid];
        const uint32_t c0 = raw.x & 0xffffu, c1 = raw.x >> 16, c2 = raw.y & 0xffffu, c3 = raw.y >> 16;
        const uint32_t s = c0 + c1 + c2 + c3;
        const uint32_t inc = wave_incl_scan(s);
        if (lane == 63) sh.wave_tot[wave][0] = inc;
        __syncthreads();
        const uint32_t wt = (lane < wave) ? sh.wave_tot[lane][0] : 0u;   // lanes 0..14 of row 0: earlier waves
        const uint32_t before = (uint32_t)__builtin_amdgcn_readlane((int)row16_incl_scan(wt), 15);
        const uint32_t e0 = before + inc - s, e1 = e0 + c0, e2 = e1 + c1, e3 = e2 + c2;
        cw[tid] = make_uint2(e0 | (e1 << 16), e2 | (e3 << 16));
        __syncthreads();
        if (valid) dst[c[slot] + rank] = x;
        cur ^= 1;
        __syncthreads();
    }
    return base + 1024 * cur;
}

// Score order for k <= 1024 staged pairs in slots [0, k) (one per thread), when the keys spread out: one pass into
// 2048 bins that are linear in the key over [kmin, kmax] (bin = (kmax - key) >> s, with s the smallest shift that
// leaves at most 2048 bins, so bin order is descending key order), then each pair's rank inside its bin by comparison
// with the bin's other pairs, larger (key, ~index) first (equal pairs, which only zero padding can form, by their
// place in the bin). Six barriers in all, against four per pass of the radix sort. The top k of a smooth score
// distribution puts a few pairs in a bin; when a bin holds more than kBinSortMax (ties, outliers that stretch the key
// range), nothing has been moved yet and the function returns nullptr for the caller's other sort. Counts in sh.hist;
// bin starts and cursors in sortbuf[2048, 4096) (as uint32); pairs placed by bin in sortbuf[1024, 2048), sorted into
// sortbuf[0, k).
constexpr uint32_t kBinSortMax = 48;
__device__ __forceinline__ const uint64_t* bin_sort_desc_1024(SelectShared& sh, int k) {
    static_assert(kHistBins == 2 * kSelThreads, "two bins per thread");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint64_t* const buf = sh.sortbuf;
    uint32_t* const cnt = sh.hist;
    uint32_t* const start = reinterpret_cast<uint32_t*>(buf + 2048);
    uint32_t* const cur = start + kHistBins;
    uint64_t* const tmp = buf + 1024;
    const bool valid = tid < k;
    const uint64_t x = valid ? buf[tid] : 0ull;
    const uint32_t key = (uint32_t)(x >> 32);
    uint32_t mn = valid ? key : 0xffffffffu, mx = valid ? key : 0u;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        mn = min(mn, (uint32_t)__shfl_xor((int)mn, m, 64));
        mx = max(mx, (uint32_t)__shfl_xor((int)mx, m, 64));
    }
    if (lane == 0) {
        sh.wave_tot[wave][0] = mn;
        sh.wave_tot[wave][1] = mx;
    }
    cnt[tid] = 0u;
    cnt[tid + kSelThreads] = 0u;
    __syncthreads();
    uint32_t kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
    for (int w = 0; w < kSelWaves; ++w) {
        kmin = min(kmin, sh.wave_tot[w][0]);
        kmax = max(kmax, sh.wave_tot[w][1]);
    }
    const uint32_t span = kmax - kmin;   // k >= 1, so kmin <= kmax
    const int shift = span >> 11 ? 32 - __clz((int)span) - 11 : 0;
    const uint32_t bin = (kmax - key) >> shift;   // < 2048
    if (valid) atomicAdd(&cnt[bin], 1u);
    __syncthreads();
    // exclusive scan of the 2048 counts (thread t: bins 2t, 2t + 1) and the largest count
    const uint2 c2 = reinterpret_cast<const uint2*>(cnt)[tid];
    const uint32_t s2 = c2.x + c2.y;
    const uint32_t inc = wave_incl_scan(s2);
    uint32_t big = max(c2.x, c2.y);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) big = max(big, (uint32_t)__shfl_xor((int)big, m, 64));
    __syncthreads();   // every thread has read the minimum and maximum out of wave_tot
    if (lane == 63) sh.wave_tot[wave][0] = inc;
    if (lane == 0) sh.wave_tot[wave][1] = big;
    __syncthreads();
    uint32_t before = 0u, largest = 0u;
#pragma unroll
    for (int w = 0; w < kSelWaves; ++w) {
        before += w < wave ? sh.wave_tot[w][0] : 0u;
        largest = max(largest, sh.wave_tot[w][1]);
    }
    if (largest > kBinSortMax) {
        __syncthreads();   // the other sort reuses wave_tot
        return nullptr;
    }
    const uint32_t e0 = before + inc - s2;
    reinterpret_cast<uint2*>(start)[tid] = make_uint2(e0, e0 + c2.x);
    reinterpret_cast<uint2*>(cur)[tid] = make_uint2(e0, e0 + c2.x);
    __syncthreads();
    uint32_t pos = 0u;
    if (valid) {
        pos = atomicAdd(&cur[bin], 1u);
        tmp[pos] = x;
    }
    __syncthreads();
    if (valid) {
        const uint32_t b0 = start[bin], b1 = cur[bin];
        uint32_t rank = 0u;
        for (uint32_t j = b0; j < b1; ++j) {
            const uint64_t y = tmp[j];
            rank += (y > x) || (y == x && j < pos);
        }
        buf[b0 + rank] = x;
    }
    __syncthreads();
    return buf;
}

// Score order for 1024 < sort_len(k) <= 4096 staged pairs: the same stable LSD radix sort (passes of 8 bits, each
// digit complemented so that ascending digit order is descending score; stability keeps equal keys in index order),
// the pairs taken as up to four sub-blocks of 1024 (sub-block e: pairs 1024 e + t). A pass first counts its digit over
// all pairs (LDS atomics) and scans the counts into each digit's first slot (dbase). Then, sub-block by sub-block in
// order: the lanes of a wave holding the same digit find each other with eight ballots (rank among them: the lanes
// below), each group's leader writes its count into a [digit][wave] table, a scan along each digit's row gives every
// (digit, wave) group its offset among the sub-block's pairs of that digit, every pair moves to dbase + offset + rank,
// and dbase advances by the sub-block's count of each digit. Passes whose 8 bits are the same in every key are
// skipped. Buffers: sortbuf[0, 4096) and sortbuf[4096, 8192); the table in sh.hist. Returns the sorted buffer.
__device__ __forceinline__ const uint64_t* radix_sort_desc_4096(SelectShared& sh, int k) {
    static_assert(sizeof(SelectShared::sortbuf) >= 8192 * sizeof(uint64_t), "two 4096-pair buffers");
    static_assert(sizeof(SelectShared::hist) >= 256 * kSelWaves * sizeof(uint16_t), "the count table in hist");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = sort_len(k);   // 2048 or 4096
    const int E = n >> 10;
    uint64_t* const base = sh.sortbuf;
    uint16_t* const c = reinterpret_cast<uint16_t*>(sh.hist);   // [256][16]
    uint32_t* const cw = sh.hist;
    uint32_t* const db = sh.dbase;
    const uint64_t lt = (1ull << lane) - 1ull;
    // key bits that differ between some two pairs: OR over the pairs of key ^ (the first pair's key)
    {
        const uint32_t k0 = (uint32_t)(base[0] >> 32);
        uint32_t d = 0u;
        for (int e = 0; e < E; ++e) d |= (uint32_t)(base[1024 * e + tid] >> 32) ^ k0;
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) d |= (uint32_t)__shfl_xor((int)d, m, 64);
        if (lane == 0) sh.wave_tot[wave][1] = d;
    }
    __syncthreads();
    uint32_t differ = 0u;
#pragma unroll
    for (int w = 0; w < kSelWaves; ++w) differ |= sh.wave_tot[w][1];
    int cur = 0;
    for (int pass = 0; pass < 4; ++pass) {
        if (((differ >> (8 * pass)) & 255u) == 0u) continue;   // uniform digit: a stable no-op (the same in every wave)
        const uint64_t* const src = base + 4096 * cur;
        uint64_t* const dst = base + 4096 * (cur ^ 1);
        const int sh8 = 32 + 8 * pass;
        // phase 1: the digit's counts over all pairs, then their exclusive scan into db
        __syncthreads();   // the previous pass's last table and db reads are done
        if (tid < 256) db[tid] = 0u;
        cw[tid] = 0u;
        cw[tid + kSelThreads] = 0u;
        __syncthreads();
        for (int e = 0; e < E; ++e)
            atomicAdd(&db[255u - ((uint32_t)(src[1024 * e + tid] >> sh8) & 255u)], 1u);
        __syncthreads();
        uint32_t v = 0u, inc = 0u;
        if (tid < 256) {
            v = db[tid];
            inc = wave_incl_scan(v);
            if (lane == 63) sh.wave_tot[wave][0] = inc;
        }
        __syncthreads();
        if (tid < 256) {
            uint32_t before = 0u;
            for (int w = 0; w < wave; ++w) before += sh.wave_tot[w][0];
            db[tid] = before + inc - v;
        }
        __syncthreads();
        // phase 2: the sub-blocks in order
        for (int e = 0; e < E; ++e) {
            const uint64_t x = src[1024 * e + tid];
            const uint32_t key = (uint32_t)(x >> 32);
            const uint32_t dg = 255u - ((key >> (8 * pass)) & 255u);
            uint32_t plo = 0xffffffffu, phi = 0xffffffffu;
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const uint32_t bm = (uint32_t)__builtin_amdgcn_sbfe((int)key, 8 * pass + b, 1);   // 0 or ~0
                const uint64_t m = __ballot(bm != 0u);
                plo &= ~((uint32_t)m ^ bm);
                phi &= ~((uint32_t)(m >> 32) ^ bm);
            }
            const uint64_t peers = ((uint64_t)phi << 32) | plo;
            const uint32_t rank = (uint32_t)__popcll(peers & lt);
            const int slot = (int)dg * kSelWaves + wave;
            if (rank == 0) c[slot] = (uint16_t)__popcll(peers);
            __syncthreads();
            uint32_t rowtot = 0u;
            if (tid < 256) {   // digit tid: exclusive prefix over the 16 waves' counts, in place
                uint4* rp = reinterpret_cast<uint4*>(c + tid * kSelWaves);
                uint4 r[2] = {rp[0], rp[1]};
                uint32_t* w32 = reinterpret_cast<uint32_t*>(r);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const uint32_t lo = w32[i] & 0xffffu, hi = w32[i] >> 16;
                    w32[i] = rowtot | ((rowtot + lo) << 16);
                    rowtot += lo + hi;
                }
                rp[0] = r[0];
                rp[1] = r[1];
            }
            __syncthreads();
            dst[db[dg] + c[slot] + rank] = x;
            __syncthreads();
            if (tid < 256) db[tid] += rowtot;   // the next sub-block's pairs of each digit follow these
            cw[tid] = 0u;
            cw[tid + kSelThreads] = 0u;
            __syncthreads();
        }
        cur ^= 1;
    }
    return base + 4096 * cur;
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
    // descending on (key, ~index): larger score first, then lower index (sortbuf[0, sort_len(k)) was pre-filled by
    // init_sortbuf before the emission)
    __syncthreads();
    // 128 pairs: the bitonic sort (one chunk pass in registers). 256 to 1024: the bin sort, or where its bins crowd
    // the bitonic sort (256) or the radix sort (512, 1024). 1025 to 4096: the radix sort by sub-blocks; past 4096 the
    // bitonic sort. Single-workgroup top-k on MI355X, score order's cost over position order per launch, 32K keys:
    // k = 1024 3.7 us (radix sort alone 6.0), k = 512 3.3 (radix 4.3), k = 128 2.6 (bitonic; radix 4.0).
    const uint64_t* sorted = nullptr;
    const int n = sort_len(k);
    if (n > 128 && n <= kSelThreads) sorted = bin_sort_desc_1024(sh, k);
    if (sorted == nullptr) {
        sorted = sh.sortbuf;
        if (n > 256 && n <= kSelThreads) sorted = radix_sort_desc_1024(sh, k);
        else if (n > kSelThreads && n <= 4 * kSelThreads) sorted = radix_sort_desc_4096(sh, k);
        else bitonic_sort_desc(sh.sortbuf, n);
    }
    const float* srow = a.scores + (size_t)row * a.score_stride;
    int32_t* ti = a.top_idx ? a.top_idx + (size_t)row * a.top_stride : nullptr;
    float* tv = a.top_val ? a.top_val + (size_t)row * a.top_stride : nullptr;
    for (int j = tid; j < k; j += kSelThreads) {
        const uint64_t e = sorted[j];
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

    // v: the key's score (read only in score order and for top_val)
    __device__ __forceinline__ void put(uint32_t slot, int idx, float v) const {
        if (slot >= k) return;
        if (order == ATTNLAB_ORDER_SCORE) {
            sortbuf[slot] = ((uint64_t)score_key(v) << 32) | (uint64_t)(0xffffffffu - (uint32_t)idx);
            return;
        }
        if (ti) ti[slot] = idx;
        if (tv) tv[slot] = v;
        if (rows) rows[slot] = lo + idx;
        if (flat) flat[slot] = base + lo + idx;
    }

    // The set bits of `word`, ascending, as indices idx0 + bit at slots slot, slot + 1, ...: the scores of up to four
    // of them are loaded before any is used, so a word costs one memory round trip per four keys, not one per key
    // (eight at a time pushed select_resolve to 120 VGPRs and 152 bytes of scratch per lane).
    __device__ __forceinline__ void put_word(uint32_t word, int idx0, uint32_t& slot) const {
        const bool need = order == ATTNLAB_ORDER_SCORE || tv != nullptr;
        while (word) {
            int ix[4];
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                ix[u] = word ? idx0 + (int)(__ffs(word) - 1) : -1;
                word &= word - 1u;   // stays 0 once empty
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = (need && ix[u] >= 0) ? srow[ix[u]] : 0.0f;
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (ix[u] >= 0) put(slot++, ix[u], v[u]);
        }
    }
};

// The lowest n set bits of w (the tie rule: the first n keys equal to the threshold, in index order).
__device__ __forceinline__ uint32_t lowest_bits(uint32_t w, uint32_t n) {
    uint32_t keep = 0u;
    for (; n != 0u && w != 0u; --n) {
        keep |= w & (0u - w);
        w &= w - 1u;
    }
    return keep;
}

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

// Keys in registers (M <= 4096 * CH). Thread t holds keys 4096 c + 4 t + e (c < CH, e < 4), so every load instruction
// of a wave reads 1 KB of the row (a lane-contiguous segment per thread makes each instruction touch 64 lines, and a
// 32K row then takes ~5 us to reach one CU). All global loads are issued before any is used: this thread's two words
// of the first-digit histogram, then the row. The radix passes need no order. Index order comes back through two
// bitmaps in LDS (keys above the threshold, keys equal to it), zeroed before the first barrier: each thread ORs in its
// non-zero 4-bit pieces (a few percent of the keys are selected, so most threads OR nothing), and thread t then owns
// word t (keys 32 t .. 32 t + 31) for the tie rule (the first krem equal keys in index order) and the emission, with
// one block scan.
constexpr int kRegMaxChunks = 8;                        // M <= 32768
constexpr int kRegWords = 4096 * kRegMaxChunks / 32;    // 1024 bitmap words, one per thread
static_assert(kRegWords == kSelThreads, "one bitmap word per thread");

template <int CH>
__global__ __launch_bounds__(kSelThreads) void select_reg(SelectArgs a) {
    static_assert(kHistBins == 2 * kSelThreads, "two histogram words per thread");
    static_assert(CH >= 1 && CH <= kRegMaxChunks, "chunks of 4096 keys");
    constexpr int KPT = 4 * CH;
    __shared__ SelectShared sh;
    __shared__ __attribute__((aligned(16))) uint32_t hist2[2048];
    __shared__ __attribute__((aligned(16))) uint32_t hist3[1024];
    __shared__ uint32_t gtbits[kRegWords];
    __shared__ uint32_t eqbits[kRegWords];
    const int row = xcd_contiguous_block();   // the XCD whose L2 holds the row's scores after the scan
    const int tid = threadIdx.x;
    const float* s = a.scores + (size_t)row * a.score_stride;
    const int M = a.M;
    uint32_t* ghist = a.hist ? a.hist + (size_t)row * kSelectStateWords : nullptr;
    const bool use_hist = ghist && a.k > 0 && a.k < M;
    uint32_t g0 = 0u, g1 = 0u;
    if (use_hist) {
        g0 = ghist[tid];
        g1 = ghist[tid + kSelThreads];
    }
    float v[KPT];
    const bool vec = (reinterpret_cast<uintptr_t>(s) & 15) == 0;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int i0 = 4096 * c + 4 * tid;
        if (vec && i0 + 3 < M) {
            const float4 f = *reinterpret_cast<const float4*>(s + i0);
            v[4 * c] = f.x;
            v[4 * c + 1] = f.y;
            v[4 * c + 2] = f.z;
            v[4 * c + 3] = f.w;
        } else if (i0 < M) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * c + e] = s[min(i0 + e, M - 1)];   // in bounds; past M is masked
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * c + e] = 0.0f;
        }
    }
    uint32_t key[KPT];
    uint32_t valid = 0u;   // bit j: key j lies inside the row
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
        const bool ok = 4096 * (j >> 2) + 4 * tid + (j & 3) < M;
        key[j] = ok ? score_key(v[j]) : 0u;
        valid |= (uint32_t)ok << j;
    }
    // the three digit histograms are zeroed (or, for the first, filled from the state) before the first barrier
    sh.hist[tid] = g0;
    sh.hist[tid + kSelThreads] = g1;
    hist2[tid] = 0u;
    hist2[tid + kSelThreads] = 0u;
    hist3[tid] = 0u;
    gtbits[tid] = 0u;
    eqbits[tid] = 0u;
    if (tid == 0) {   // defaults keep every later index in range even for a state that does not match the scores
        sh.digit = 0u;
        sh.krem = 0u;
        sh.dcount = 0u;
    }
    if (a.k > 0) {
        // MSB-first radix select on the registers: digits of 11, 11 and 10 bits, each histogram searched by one wave
        uint32_t T = 0u, krem = 0xffffffffu;   // k >= M: every key is selected
        __syncthreads();
        if (a.k < M) {
            if (!use_hist) {
#pragma unroll
                for (int j = 0; j < KPT; ++j)
                    if ((valid >> j) & 1u) atomicAdd(&sh.hist[key[j] >> 21], 1u);
                __syncthreads();
            }
            find_digit_wave(sh, sh.hist, (uint32_t)a.k, 2048);
            const uint32_t d1 = sh.digit & 2047u;
            krem = sh.krem;
#pragma unroll
            for (int j = 0; j < KPT; ++j)
                if (((valid >> j) & 1u) && (key[j] >> 21) == d1) atomicAdd(&hist2[(key[j] >> 10) & 2047u], 1u);
            __syncthreads();
            find_digit_wave(sh, hist2, krem, 2048);
            const uint32_t p2 = (d1 << 11) | (sh.digit & 2047u);
            krem = sh.krem;
#pragma unroll
            for (int j = 0; j < KPT; ++j)
                if (((valid >> j) & 1u) && (key[j] >> 10) == p2) atomicAdd(&hist3[key[j] & 1023u], 1u);
            __syncthreads();
            find_digit_wave(sh, hist3, krem, 1024);
            T = (p2 << 10) | (sh.digit & 1023u);
            krem = sh.krem;
        }
        init_sortbuf(a, sh);
        // bitmap words: chunk c of thread t is bits 4 (t % 8) .. + 3 of word 128 c + t / 8
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            uint32_t gt = 0u, eq = 0u;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = 4 * c + e;
                const bool ok = (valid >> j) & 1u;
                gt |= (uint32_t)(ok && key[j] > T) << e;
                eq |= (uint32_t)(ok && key[j] == T) << e;
            }
            const int w = 128 * c + (tid >> 3), sh4 = 4 * (tid & 7);
            if (gt) atomicOr(&gtbits[w], gt << sh4);
            if (eq) atomicOr(&eqbits[w], eq << sh4);
        }
        __syncthreads();
        const bool mine = tid < 128 * CH;
        const uint32_t gw = mine ? gtbits[tid] : 0u, ew = mine ? eqbits[tid] : 0u;
        uint32_t egt, eeq;
        block_excl_scan2(__popc(gw), __popc(ew), egt, eeq, sh);
        uint32_t word = gw | lowest_bits(ew, krem > eeq ? krem - eeq : 0u);
        if (word) {
            uint32_t slot = egt + min(eeq, krem);
            const bool direct = a.order == ATTNLAB_ORDER_POSITION && !a.top_idx && !a.top_val;
            if (direct) {
                // the decode step's row list: candidate m at slot lo + (its rank), as the Emitter would write it
                const int S = a.lo + (a.legal - a.hi) + a.k;
                int32_t* rows = a.rows ? a.rows + (size_t)row * a.rows_stride + a.lo : nullptr;
                int64_t* flat = a.rows_flat ? a.rows_flat + (size_t)row * S + a.lo : nullptr;
                const int64_t base = (int64_t)row * a.C + a.lo;
                while (word) {
                    const int idx = 32 * tid + (int)(__ffs(word) - 1);
                    word &= word - 1;
                    if (slot < (uint32_t)a.k) {
                        if (rows) rows[slot] = a.lo + idx;
                        if (flat) flat[slot] = base + idx;
                    }
                    ++slot;
                }
            } else {
                make_emitter(a, row, sh).put_word(word, 32 * tid, slot);
            }
        }
    }
    if (ghist)  // leave the first-digit histogram zeroed for the next score/select pair
        for (int i = tid; i < kSelectStateWords; i += kSelThreads) ghist[i] = 0u;
    __syncthreads();
    finish_row(a, row, sh);
}

// One row of any length with 1024 threads (rows past 32768 keys without a select state, and the resolve whose
// threshold bin overflowed its candidate list). The row is re-read from global memory (L2-resident after the first
// pass) in every pass, coalesced as in select_reg: thread t reads keys 4096 c + 4 t + e, four chunks' loads in flight
// at a time. Threshold: the first digit's histogram (from the state, or built by a pass), then two passes over the keys
// that share the prefix, each histogram searched by one wave. Emission in windows of 32768 keys through select_reg's
// two LDS bitmaps, one block scan per window, with the counts of the earlier windows carried over.
struct StreamLds {
    uint32_t* hist2;    // 2048 words
    uint32_t* hist3;    // 1024
    uint32_t* gtbits;   // kRegWords
    uint32_t* eqbits;   // kRegWords
};

// fn(c, key[4], valid mask) for every chunk c of 4096 keys this thread touches (keys 4096 c + 4 t + e).
template <typename Fn>
__device__ __forceinline__ void for_each_chunk(const float* s, int M, int c_begin, int c_end, Fn fn) {
    constexpr int kBatch = 4;
    const int tid = threadIdx.x;
    const bool vec = (reinterpret_cast<uintptr_t>(s) & 15) == 0;
    for (int c0 = c_begin; c0 < c_end; c0 += kBatch) {
        float v[4 * kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int i0 = 4096 * (c0 + u) + 4 * tid;
            if (c0 + u < c_end && vec && i0 + 3 < M) {
                const float4 f = *reinterpret_cast<const float4*>(s + i0);
                v[4 * u] = f.x;
                v[4 * u + 1] = f.y;
                v[4 * u + 2] = f.z;
                v[4 * u + 3] = f.w;
            } else if (c0 + u < c_end && i0 < M) {
#pragma unroll
                for (int e = 0; e < 4; ++e) v[4 * u + e] = s[min(i0 + e, M - 1)];   // in bounds; past M is masked
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) v[4 * u + e] = 0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            if (c0 + u >= c_end) break;
            const int i0 = 4096 * (c0 + u) + 4 * tid;
            uint32_t key[4], valid = 0u;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const bool ok = i0 + e < M;
                key[e] = ok ? score_key(v[4 * u + e]) : 0u;
                valid |= (uint32_t)ok << e;
            }
            fn(c0 + u, key, valid);
        }
    }
}

__device__ void select_row_streaming(const SelectArgs& a, int row, SelectShared& sh, const StreamLds& L) {
    const int tid = threadIdx.x;
    const int M = a.M;
    const int nch = (M + 4095) / 4096;
    const float* s = a.scores + (size_t)row * a.score_stride;
    uint32_t* ghist = a.hist ? a.hist + (size_t)row * kSelectStateWords : nullptr;
    const bool use_hist = ghist && a.k > 0 && a.k < M;
    for (int i = tid; i < kHistBins; i += kSelThreads) sh.hist[i] = use_hist ? ghist[i] : 0u;
    for (int i = tid; i < 2048; i += kSelThreads) L.hist2[i] = 0u;
    for (int i = tid; i < 1024; i += kSelThreads) L.hist3[i] = 0u;
    if (tid == 0) {   // defaults keep every later index in range even for a state that does not match the scores
        sh.digit = 0u;
        sh.krem = 0u;
        sh.dcount = 0u;
    }
    __syncthreads();
    if (a.k > 0) {
        uint32_t T = 0u, krem = 0xffffffffu;   // k >= M: every key is selected
        if (a.k < M) {
            if (!use_hist) {
                for_each_chunk(s, M, 0, nch, [&](int, const uint32_t* key, uint32_t valid) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if ((valid >> e) & 1u) atomicAdd(&sh.hist[key[e] >> 21], 1u);
                });
                __syncthreads();
            }
            find_digit_wave(sh, sh.hist, (uint32_t)a.k, 2048);
            const uint32_t d1 = sh.digit & 2047u;
            krem = sh.krem;
            for_each_chunk(s, M, 0, nch, [&](int, const uint32_t* key, uint32_t valid) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (((valid >> e) & 1u) && (key[e] >> 21) == d1) atomicAdd(&L.hist2[(key[e] >> 10) & 2047u], 1u);
            });
            __syncthreads();
            find_digit_wave(sh, L.hist2, krem, 2048);
            const uint32_t p2 = (d1 << 11) | (sh.digit & 2047u);
            krem = sh.krem;
            for_each_chunk(s, M, 0, nch, [&](int, const uint32_t* key, uint32_t valid) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (((valid >> e) & 1u) && (key[e] >> 10) == p2) atomicAdd(&L.hist3[key[e] & 1023u], 1u);
            });
            __syncthreads();
            find_digit_wave(sh, L.hist3, krem, 1024);
            T = (p2 << 10) | (sh.digit & 1023u);
            krem = sh.krem;
        }
        init_sortbuf(a, sh);
        const bool direct = a.order == ATTNLAB_ORDER_POSITION && !a.top_idx && !a.top_val;
        const int S = a.lo + (a.legal - a.hi) + a.k;
        int32_t* rows = a.rows ? a.rows + (size_t)row * a.rows_stride + a.lo : nullptr;
        int64_t* flat = a.rows_flat ? a.rows_flat + (size_t)row * S + a.lo : nullptr;
        const int64_t base = (int64_t)row * a.C + a.lo;
        const Emitter em = make_emitter(a, row, sh);
        uint32_t gt_before = 0u, eq_before = 0u;   // selected-above and tied keys of the earlier windows
        for (int c_w = 0; c_w < nch; c_w += kRegMaxChunks) {
            L.gtbits[tid] = 0u;
            L.eqbits[tid] = 0u;
            __syncthreads();
            for_each_chunk(s, M, c_w, min(nch, c_w + kRegMaxChunks), [&](int c, const uint32_t* key, uint32_t valid) {
                uint32_t gt = 0u, eq = 0u;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool ok = (valid >> e) & 1u;
                    gt |= (uint32_t)(ok && key[e] > T) << e;
                    eq |= (uint32_t)(ok && key[e] == T) << e;
                }
                const int w = 128 * (c - c_w) + (tid >> 3), sh4 = 4 * (tid & 7);
                if (gt) atomicOr(&L.gtbits[w], gt << sh4);
                if (eq) atomicOr(&L.eqbits[w], eq << sh4);
            });
            __syncthreads();
            const uint32_t gw = L.gtbits[tid], ew = L.eqbits[tid];
            uint32_t egt, eeq, tgt, teq;
            block_scan2<kSelThreads>(__popc(gw), __popc(ew), egt, eeq, tgt, teq, sh.wave_tot);
            const uint32_t ties = eq_before + eeq;   // tied keys before this thread's word
            uint32_t word = gw | lowest_bits(ew, krem > ties ? krem - ties : 0u);
            if (word) {
                uint32_t slot = gt_before + egt + min(ties, krem);
                if (direct) {
                    while (word) {
                        const int idx = 4096 * c_w + 32 * tid + (int)(__ffs(word) - 1);
                        word &= word - 1;
                        if (slot < (uint32_t)a.k) {
                            if (rows) rows[slot] = a.lo + idx;
                            if (flat) flat[slot] = base + idx;
                        }
                        ++slot;
                    }
                } else {
                    em.put_word(word, 4096 * c_w + 32 * tid, slot);
                }
            }
            gt_before += tgt;
            eq_before += teq;
        }
    }
    if (ghist)  // leave the first-digit histogram zeroed for the next score/select pair
        for (int i = tid; i < kSelectStateWords; i += kSelThreads) ghist[i] = 0u;
    __syncthreads();
    finish_row(a, row, sh);
}

__global__ __launch_bounds__(kSelThreads) void select_stream(SelectArgs a) {
    __shared__ SelectShared sh;
    __shared__ __attribute__((aligned(16))) uint32_t hist2[2048];
    __shared__ __attribute__((aligned(16))) uint32_t hist3[1024];
    __shared__ uint32_t gtbits[kRegWords];
    __shared__ uint32_t eqbits[kRegWords];
    select_row_streaming(a, xcd_contiguous_block(), sh, StreamLds{hist2, hist3, gtbits, eqbits});
}

static int launch_select(const SelectArgs& a, int R, hipStream_t s) {
    const int chunks = (a.M + 4095) / 4096;
    const dim3 grid(R), block(kSelThreads);
    if (chunks <= 1) hipLaunchKernelGGL(select_reg<1>, grid, block, 0, s, a);
    else if (chunks <= 2) hipLaunchKernelGGL(select_reg<2>, grid, block, 0, s, a);
    else if (chunks <= 4) hipLaunchKernelGGL(select_reg<4>, grid, block, 0, s, a);
    else if (chunks <= kRegMaxChunks) hipLaunchKernelGGL(select_reg<kRegMaxChunks>, grid, block, 0, s, a);
    else hipLaunchKernelGGL(select_stream, grid, block, 0, s, a);
    return check_launch("select");
}

// ---------------------------------------------------------------------------------------------------------------
// Tiled select (first-digit histogram given by the score kernel, or built by select_hist for attnlab_topk_tiled):
//   A select_classify  (rows x tiles of 4096 keys, 256 threads): the threshold's first digit b1 from the row's
//                      super-bins and bins; every key of the tile is classified as "above" (first digit > b1: selected for sure)
//                      or "candidate" (first digit == b1), written as two bitmaps of the row (one bit per key).
//   B select_resolve   (one 1024-thread workgroup per row): compacts the candidate bitmap into an index-ordered list,
//                      gathers the candidates' scores, finds the threshold among them with the remaining two radix
//                      digits, takes the tied keys at the threshold in index order, ORs the selected candidates into
//                      the "above" bitmap in LDS and writes the set bits in index order (plus F), or in score order
//                      after one LDS sort; it then clears the row's histogram. A row with more than CAP candidates
//                      runs the single-workgroup select.
// Every kernel issues its global loads before it uses any of them: each is a few memory round trips long.
// ---------------------------------------------------------------------------------------------------------------
constexpr int kTileKeys = 4096;
constexpr int kTileThreads = 256;
constexpr int kTileKPT = kTileKeys / kTileThreads;   // 16 keys per thread, one contiguous segment (half a bitmap word)
// Candidates per row listed in LDS (in sortbuf): 4096 while rows are at most 64K long (a first-digit bin there holds a
// few thousand keys at most for any smooth distribution), 8192 beyond, where the larger list costs ~2 us of resolve
constexpr int kCandCapShort = 4096, kCandCapLong = 8192;
constexpr int kCandCapLongFromM = 65537;
static_assert(kCandCapLong * sizeof(uint32_t) <= sizeof(SelectShared::sortbuf), "the candidate list lives in sortbuf");
constexpr int kMaxWords = 8192;                       // bitmap words per row held in LDS: M <= 262144
constexpr int kMaxWordsPerThread = kMaxWords / kSelThreads;

struct TiledArgs {
    uint32_t* above;   // [R, W] bit i: key i's first digit > b1
    uint32_t* cand;    // [R, W] bit i: key i's first digit == b1
    int W;             // bitmap words per row = ceil(M / 32)
    int T;             // tiles per row
};

__host__ __device__ inline int64_t tiled_scratch_bytes(int R, int M) {
    return (int64_t)R * 2 * 4 * (((int64_t)M + 31) / 32);
}

// b1 = first digit of the k-th largest key, from the row's select state: one wave scans the 64 super-bins (lane 0 =
// the highest), picks the one holding the k-th key, then scans its 32 bins. Two small loads and two DPP scans, no LDS
// and no barrier, so every wave can run it on its own. Returns 0 when the state holds fewer than k keys.
__device__ __forceinline__ uint32_t first_digit_2level(const uint32_t* st, uint32_t k) {
    static_assert(kSuperBins == 64, "one super-bin per lane");
    const int lane = threadIdx.x & 63;
    const uint32_t v = st[kHistBins + (kSuperBins - 1 - lane)];
    const uint32_t inc = wave_incl_scan(v);
    const uint64_t m = __ballot(inc >= k);
    if (m == 0) return 0u;
    const int l0 = __ffsll((unsigned long long)m) - 1;
    const uint32_t above = (uint32_t)__builtin_amdgcn_readlane((int)(inc - v), l0);
    const int sb = kSuperBins - 1 - l0;
    const uint32_t c = lane < 32 ? st[32 * sb + (31 - lane)] : 0u;
    const uint32_t inc2 = wave_incl_scan(c) + above;
    const uint64_t m2 = __ballot(lane < 32 && inc2 >= k);
    if (m2 == 0) return (uint32_t)(32 * sb);
    return (uint32_t)(32 * sb + 31 - (__ffsll((unsigned long long)m2) - 1));
}

// This thread's 16 scores of the tile as raw floats; positions at or past M are not read.
__device__ __forceinline__ int load_tile_scores(const float* s, int i0, int M, float (&v)[kTileKPT]) {
    const int nvalid = max(0, min(kTileKPT, M - i0));
    if (nvalid == kTileKPT && (reinterpret_cast<uintptr_t>(s + i0) & 15) == 0) {
#pragma unroll
        for (int q = 0; q < kTileKPT / 4; ++q) {
            const float4 f = *reinterpret_cast<const float4*>(s + i0 + 4 * q);
            v[4 * q] = f.x;
            v[4 * q + 1] = f.y;
            v[4 * q + 2] = f.z;
            v[4 * q + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < kTileKPT; ++i) v[i] = i < nvalid ? s[i0 + i] : 0.0f;
    }
    return nvalid;
}

__global__ __launch_bounds__(kTileThreads) void select_classify(SelectArgs a, TiledArgs t) {
    // the tiles of one row go to one XCD, the one that scanned the row and resolves it, so the row's select state
    // and scores are fetched into that XCD's L2 once
    const int lin = xcd_contiguous_block();
    const int row = lin / t.T, tile = lin - row * t.T;
    const int tid = threadIdx.x;
    const float* s = a.scores + (size_t)row * a.score_stride;
    const int i0 = tile * kTileKeys + tid * kTileKPT;
    float v[kTileKPT];
    const int nvalid = load_tile_scores(s, i0, a.M, v);
    const uint32_t b1 = first_digit_2level(a.hist + (size_t)row * kSelectStateWords, (uint32_t)a.k);
    uint32_t abits = 0, cbits = 0;
#pragma unroll
    for (int i = 0; i < kTileKPT; ++i) {
        const uint32_t dg = score_key(v[i]) >> kHistShift;
        if (i < nvalid) {
            abits |= (uint32_t)(dg > b1) << i;
            cbits |= (uint32_t)(dg == b1) << i;
        }
    }
    // two threads per 32-bit word: the even thread's keys are the low half
    const uint32_t an = __shfl_xor(abits, 1, 64), cn = __shfl_xor(cbits, 1, 64);
    const int w = tile * (kTileKeys / 32) + (tid >> 1);
    if ((tid & 1) == 0 && w < t.W) {
        t.above[(size_t)row * t.W + w] = abits | (an << 16);
        t.cand[(size_t)row * t.W + w] = cbits | (cn << 16);
    }
}

// Standalone top-k (no score kernel in front): the first-digit histogram and super-bin counts of every row, over the
// same 4096-key tiles, added into the row's select state.
__global__ __launch_bounds__(kTileThreads) void select_hist(SelectArgs a, TiledArgs t) {
    __shared__ __attribute__((aligned(16))) uint32_t hsh[kHistBins];
    const int lin = xcd_contiguous_block();
    const int row = lin / t.T, tile = lin - row * t.T;
    const int tid = threadIdx.x;
    float v[kTileKPT];
    const int nvalid = load_tile_scores(a.scores + (size_t)row * a.score_stride, tile * kTileKeys + tid * kTileKPT, a.M, v);
    clear_histogram<kTileThreads>(hsh);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kTileKPT; ++i)
        if (i < nvalid) atomicAdd(&hsh[score_key(v[i]) >> kHistShift], 1u);
    flush_histogram<kTileThreads>(hsh, a.hist, row);
}

template <int CAP>
__global__ __launch_bounds__(kSelThreads) void select_resolve(SelectArgs a, TiledArgs t) {
    constexpr int kCandPerThread = CAP / kSelThreads;
    __shared__ SelectShared sh;                 // sortbuf holds the candidate list (as uint32 indices)
    __shared__ __attribute__((aligned(16))) uint32_t hist3[1024];
    __shared__ __attribute__((aligned(16))) uint32_t bits[kMaxWords];
    const int row = xcd_contiguous_block();   // the XCD that classified the row
    const int tid = threadIdx.x;
    const int W = t.W;
    const int wpt = (W + kSelThreads - 1) / kSelThreads;   // <= kMaxWordsPerThread
    const int w0 = tid * wpt;
    uint32_t cb[kMaxWordsPerThread], ab[kMaxWordsPerThread];
#pragma unroll
    for (int j = 0; j < kMaxWordsPerThread; ++j) {
        const bool ok = j < wpt && w0 + j < W;
        cb[j] = ok ? t.cand[(size_t)row * W + w0 + j] : 0u;
        ab[j] = ok ? t.above[(size_t)row * W + w0 + j] : 0u;
    }
    for (int i = tid; i < kHistBins; i += kSelThreads) sh.hist[i] = 0u;
    hist3[tid] = 0u;
    if (tid == 0) {   // defaults keep every later index in range even for a state that does not match the scores
        sh.digit = 0u;
        sh.krem = 0u;
        sh.dcount = 0u;
    }
    uint32_t nc = 0, na = 0;
#pragma unroll
    for (int j = 0; j < kMaxWordsPerThread; ++j) {
        if (j < wpt && w0 + j < W) bits[w0 + j] = ab[j];
        nc += __popc(cb[j]);
        na += __popc(ab[j]);
    }
    uint32_t ec, unused, n, n_above;
    block_scan2<kSelThreads>(nc, na, ec, unused, n, n_above, sh.wave_tot);
    if (n > (uint32_t)CAP) {   // too many keys share the threshold's first digit: single-workgroup select
        // bits[] (the above bitmap) is no longer needed: it holds the streaming select's LDS histograms and bitmaps
        select_row_streaming(a, row, sh, StreamLds{bits, bits + 2048, bits + 3072, bits + 3072 + kRegWords});
        return;
    }
    // candidate list in index order
    uint32_t* list = reinterpret_cast<uint32_t*>(sh.sortbuf);
    uint32_t pos = ec;
#pragma unroll
    for (int j = 0; j < kMaxWordsPerThread; ++j) {
        uint32_t word = cb[j];
        while (word) {
            const uint32_t b = __ffs(word) - 1;
            word &= word - 1;
            if (pos < (uint32_t)CAP) list[pos] = (uint32_t)(w0 + j) * 32u + b;
            ++pos;
        }
    }
    __syncthreads();
    // this thread's candidates: list entries [4 tid, 4 tid + 4), so ties rank in index order across threads
    const float* srow = a.scores + (size_t)row * a.score_stride;
    uint32_t cidx[kCandPerThread], low[kCandPerThread];
    bool cv[kCandPerThread];
#pragma unroll
    for (int i = 0; i < kCandPerThread; ++i) {
        const uint32_t p = (uint32_t)(kCandPerThread * tid + i);
        cv[i] = p < n;
        cidx[i] = cv[i] ? min(list[p], (uint32_t)a.M - 1u) : 0u;
    }
#pragma unroll
    for (int i = 0; i < kCandPerThread; ++i) low[i] = cv[i] ? score_key(srow[cidx[i]]) & 0x1fffffu : 0u;
    // the candidates share the first digit: the threshold is found on the low 21 bits (digits of 11 and 10 bits)
    uint32_t krem = (uint32_t)a.k - n_above;     // candidates to take, 1 <= krem <= n
#pragma unroll
    for (int i = 0; i < kCandPerThread; ++i)
        if (cv[i]) atomicAdd(&sh.hist[low[i] >> 10], 1u);
    __syncthreads();
    find_digit_wave(sh, sh.hist, krem, 2048);
    const uint32_t d2 = sh.digit & 2047u;
    krem = sh.krem;
#pragma unroll
    for (int i = 0; i < kCandPerThread; ++i)
        if (cv[i] && (low[i] >> 10) == d2) atomicAdd(&hist3[low[i] & 1023u], 1u);
    __syncthreads();
    find_digit_wave(sh, hist3, krem, 1024);
    const uint32_t tlow = (d2 << 10) | (sh.digit & 1023u);
    krem = sh.krem;
    if (sh.dcount <= krem) {
        // every key equal to the threshold is taken (the usual case: no tie at the boundary)
#pragma unroll
        for (int i = 0; i < kCandPerThread; ++i)
            if (cv[i] && low[i] >= tlow) atomicOr(&bits[cidx[i] >> 5], 1u << (cidx[i] & 31u));
    } else {
        // equal keys at the threshold: the first krem of them in index order are taken
        uint32_t neq = 0;
#pragma unroll
        for (int i = 0; i < kCandPerThread; ++i) neq += cv[i] && low[i] == tlow;
        uint32_t eeq, unused2, teq, unused_t2;
        block_scan2<kSelThreads>(neq, 0u, eeq, unused2, teq, unused_t2, sh.wave_tot);
#pragma unroll
        for (int i = 0; i < kCandPerThread; ++i) {
            if (!cv[i]) continue;
            const bool eq = low[i] == tlow;
            if (low[i] > tlow || (eq && eeq < krem)) atomicOr(&bits[cidx[i] >> 5], 1u << (cidx[i] & 31u));
            eeq += eq;
        }
    }
    __syncthreads();
    // emission: the set bits of this thread's words, in index order; in score order they are staged as (key, ~index)
    // pairs in sortbuf (the candidate list there was consumed before the last barrier) and finish_row sorts them
    init_sortbuf(a, sh);
    uint32_t sw[kMaxWordsPerThread];
    uint32_t ns = 0;
#pragma unroll
    for (int j = 0; j < kMaxWordsPerThread; ++j) {
        sw[j] = (j < wpt && w0 + j < W) ? bits[w0 + j] : 0u;
        ns += __popc(sw[j]);
    }
    uint32_t slot, unused3, tsel, unused_t3;
    block_scan2<kSelThreads>(ns, 0u, slot, unused3, tsel, unused_t3, sh.wave_tot);
    uint32_t* st = a.hist + (size_t)row * kSelectStateWords;   // leave the histogram zeroed for the next call
    if (a.order == ATTNLAB_ORDER_POSITION && !a.top_idx && !a.top_val) {
        // the decode step's row list: candidates at slots lo.., then F, written directly
        const int nrec = a.legal - a.hi, S = a.lo + nrec + a.k, nf = a.lo + nrec;
        int32_t* rows = a.rows ? a.rows + (size_t)row * a.rows_stride : nullptr;
        int64_t* flat = a.rows_flat ? a.rows_flat + (size_t)row * S : nullptr;
        const int64_t base = (int64_t)row * a.C;
#pragma unroll
        for (int j = 0; j < kMaxWordsPerThread; ++j) {
            uint32_t word = sw[j];
            while (word) {
                const uint32_t b = __ffs(word) - 1;
                word &= word - 1;
                const int idx = (w0 + j) * 32 + (int)b;
                if (slot < (uint32_t)a.k) {
                    if (rows) rows[a.lo + slot] = a.lo + idx;
                    if (flat) flat[a.lo + slot] = base + a.lo + idx;
                }
                ++slot;
            }
        }
        for (int f = tid; f < nf; f += kSelThreads) {
            const int p = f < a.lo ? f : a.hi + (f - a.lo);
            const int s_out = f < a.lo ? f : a.lo + a.k + (f - a.lo);
            if (rows) rows[s_out] = p;
            if (flat) flat[s_out] = base + p;
        }
        for (int i = tid; i < kSelectStateWords; i += kSelThreads) st[i] = 0u;
        return;
    }
    // the words again from the LDS bitmap (a loop that needs no unrolled register copy)
    const Emitter em = make_emitter(a, row, sh);
    for (int j = 0; j < wpt; ++j)
        if (w0 + j < W) em.put_word(bits[w0 + j], (w0 + j) * 32, slot);
    for (int i = tid; i < kSelectStateWords; i += kSelThreads) st[i] = 0u;
    __syncthreads();
    finish_row(a, row, sh);   // F positions; in score order the sort and the outputs
}

// ---------------------------------------------------------------------------------------------------------------
// Compact tiled select, rows of at most kCompactMaxTiles tiles (M <= 32768, the decode step's 32K context):
//   A select_classify_compact  as select_classify, but instead of a candidate bitmap each wave writes its candidates
//                              (first digit == b1) as (index, low 21 key bits) entries, in index order, into a region
//                              of its own (no barrier, no atomic), with (above, candidate) counts beside it.
//   B select_resolve_compact   one round trip loads the row's above bitmap, the region counts and the entries; the two
//                              remaining digits are searched on the entries' low key bits, the chosen candidates are
//                              ORed into the bitmap and the set bits emitted as in select_resolve. No candidate list is
//                              built and no score is gathered. A wave region that overflowed sends the row to the
//                              single-workgroup streaming select.
// ---------------------------------------------------------------------------------------------------------------
constexpr int kCompactMaxTiles = 8;
constexpr int kCompactWaves = kTileThreads / 64;                         // regions per tile
constexpr int kCompactRegions = kCompactMaxTiles * kCompactWaves;        // 32 per row
constexpr int kCompactWaveCap = 128;                                     // entries per region (a wave's 1024 keys)
constexpr int kCompactEntries = kCompactRegions * kCompactWaveCap;       // 4096 per row
constexpr int kCompactPerThread = kCompactEntries / kSelThreads;         // 4 entries per resolve thread
constexpr int kCompactWords = kCompactMaxTiles * kTileKeys / 32;         // 1024 bitmap words: one per resolve thread
static_assert(kCompactPerThread == 4 && kCompactWords == kSelThreads, "resolve layout");
static_assert(kCompactWaveCap % kCompactPerThread == 0, "a thread's entries lie in one region");

struct CompactArgs {
    uint32_t* above;   // [R, W] bit i: key i's first digit > b1
    uint2* counts;     // [R, kCompactRegions] (keys above b1, candidates) of each classify wave
    uint2* entries;    // [R, kCompactRegions, kCompactWaveCap] (candidate index, low 21 bits of its key)
    int W, T;
};

__host__ __device__ inline int64_t align_bytes(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

// Per-row byte layout of the compact scratch: the above bitmap, the counts, the entries (16-byte aligned parts).
__host__ __device__ inline int64_t compact_bitmap_bytes(int M) { return align_bytes(((int64_t)M + 31) / 32 * 4, 16); }
__host__ __device__ inline int64_t compact_row_bytes(int M) {
    return compact_bitmap_bytes(M) + (int64_t)kCompactRegions * 8 + (int64_t)kCompactEntries * 8;
}

__host__ __device__ inline bool compact_fits(int M) { return M <= kCompactMaxTiles * kTileKeys; }

// Scratch of the tiled select (either form) for R rows of M candidates.
__host__ __device__ inline int64_t tiled_region_bytes(int R, int M) {
    return compact_fits(M) ? (int64_t)R * compact_row_bytes(M) : tiled_scratch_bytes(R, M);
}

__global__ __launch_bounds__(kTileThreads) void select_classify_compact(SelectArgs a, CompactArgs t) {
    const int lin = xcd_contiguous_block();
    const int row = lin / t.T, tile = lin - row * t.T;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* s = a.scores + (size_t)row * a.score_stride;
    const int i0 = tile * kTileKeys + tid * kTileKPT;
    float v[kTileKPT];
    const int nvalid = load_tile_scores(s, i0, a.M, v);
    const uint32_t b1 = first_digit_2level(a.hist + (size_t)row * kSelectStateWords, (uint32_t)a.k);
    uint32_t abits = 0, cbits = 0, low[kTileKPT];
#pragma unroll
    for (int i = 0; i < kTileKPT; ++i) {
        const uint32_t key = score_key(v[i]);
        const uint32_t dg = key >> kHistShift;
        low[i] = key & ((1u << kHistShift) - 1u);
        if (i < nvalid) {
            abits |= (uint32_t)(dg > b1) << i;
            cbits |= (uint32_t)(dg == b1) << i;
        }
    }
    // above bitmap: two threads per 32-bit word, the even thread's keys in the low half
    const uint32_t an = __shfl_xor(abits, 1, 64);
    const int w = tile * (kTileKeys / 32) + (tid >> 1);
    if ((tid & 1) == 0 && w < t.W) t.above[(size_t)row * t.W + w] = abits | (an << 16);
    // this wave's candidates, lane after lane (index order), from the packed inclusive scan of (above << 16 | cand)
    // (each field's wave total is at most 1024, so the halves never carry into each other)
    const uint32_t na = (uint32_t)__popc(abits), nc = (uint32_t)__popc(cbits);
    const uint32_t inc = wave_incl_scan((na << 16) | nc);
    const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)inc, 63);
    const int region = tile * kCompactWaves + wave;
    uint2* ent = t.entries + ((size_t)row * kCompactRegions + region) * kCompactWaveCap;
    uint32_t slot = (inc & 0xffffu) - nc;
#pragma unroll
    for (int i = 0; i < kTileKPT; ++i) {   // static indices: low[] stays in registers
        if ((cbits >> i) & 1u) {
            if (slot < (uint32_t)kCompactWaveCap) ent[slot] = make_uint2((uint32_t)(i0 + i), low[i]);
            ++slot;
        }
    }
    if (lane == 0) t.counts[(size_t)row * kCompactRegions + region] = make_uint2(tot >> 16, tot & 0xffffu);
}

// Emission of a selection bitmap held one word per thread (word tid of the row; slot = this thread's first output
// slot), then F and the cleared state. Shared by select_resolve_compact's position and score orders.
__device__ __forceinline__ void emit_word_row(const SelectArgs& a, int row, SelectShared& sh, uint32_t word,
                                              uint32_t slot) {
    const int tid = threadIdx.x;
    uint32_t* st = a.hist + (size_t)row * kSelectStateWords;   // leave the histogram zeroed for the next call
    if (a.order == ATTNLAB_ORDER_POSITION && !a.top_idx && !a.top_val) {
        const int nrec = a.legal - a.hi, S = a.lo + nrec + a.k, nf = a.lo + nrec;
        int32_t* rows = a.rows ? a.rows + (size_t)row * a.rows_stride : nullptr;
        int64_t* flat = a.rows_flat ? a.rows_flat + (size_t)row * S : nullptr;
        const int64_t base = (int64_t)row * a.C;
        while (word) {
            const uint32_t b = __ffs(word) - 1;
            word &= word - 1;
            const int idx = tid * 32 + (int)b;
            if (slot < (uint32_t)a.k) {
                if (rows) rows[a.lo + slot] = a.lo + idx;
                if (flat) flat[a.lo + slot] = base + a.lo + idx;
            }
            ++slot;
        }
        for (int f = tid; f < nf; f += kSelThreads) {
            const int p = f < a.lo ? f : a.hi + (f - a.lo);
            const int s_out = f < a.lo ? f : a.lo + a.k + (f - a.lo);
            if (rows) rows[s_out] = p;
            if (flat) flat[s_out] = base + p;
        }
        for (int i = tid; i < kSelectStateWords; i += kSelThreads) st[i] = 0u;
        return;
    }
    make_emitter(a, row, sh).put_word(word, tid * 32, slot);
    for (int i = tid; i < kSelectStateWords; i += kSelThreads) st[i] = 0u;
    __syncthreads();
    finish_row(a, row, sh);   // F positions; in score order the sort and the outputs
}

__global__ __launch_bounds__(kSelThreads) void select_resolve_compact(SelectArgs a, CompactArgs t) {
    __shared__ SelectShared sh;   // hist: the second digit's histogram; sortbuf: score order's staged pairs
    // the third digit's histogram and the selection bitmap, or the streaming fallback's histograms and bitmaps
    __shared__ __attribute__((aligned(16))) uint32_t lds[2048 + 1024 + 2 * kRegWords];
    __shared__ uint32_t totals[2];   // keys above b1, overflow flag
    uint32_t* hist3 = lds;
    uint32_t* bits = lds + 1024;
    const int row = xcd_contiguous_block();   // the XCD that classified the row
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nreg = kCompactWaves * t.T;
    // one round trip: this thread's bitmap word, its four entries and their region's count (wave 0: every count)
    const int e0 = kCompactPerThread * tid;
    const int reg = e0 / kCompactWaveCap, slot0 = e0 - reg * kCompactWaveCap;
    const uint32_t aw = tid < t.W ? t.above[(size_t)row * t.W + tid] : 0u;
    uint4 p01 = make_uint4(0, 0, 0, 0), p23 = make_uint4(0, 0, 0, 0);
    uint2 rc = make_uint2(0, 0), wc = make_uint2(0, 0);
    if (reg < nreg) {
        const uint4* ep = reinterpret_cast<const uint4*>(t.entries + (size_t)row * kCompactEntries + e0);
        p01 = ep[0];
        p23 = ep[1];
        rc = t.counts[(size_t)row * kCompactRegions + reg];
    }
    if (wave == 0 && lane < nreg) wc = t.counts[(size_t)row * kCompactRegions + lane];
    sh.hist[tid] = 0u;
    sh.hist[tid + kSelThreads] = 0u;
    hist3[tid] = 0u;
    bits[tid] = aw;
    if (wave == 0) {
        uint32_t na = wc.x;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) na += __shfl_xor(na, o, 64);
        const bool over = __ballot(wc.y > (uint32_t)kCompactWaveCap) != 0;
        if (lane == 0) {
            totals[0] = na;
            totals[1] = over;
            sh.digit = 0u;   // defaults keep every later index in range even for a state that does not match the scores
            sh.krem = 0u;
            sh.dcount = 0u;
        }
    }
    __syncthreads();
    if (totals[1]) {   // a wave region overflowed: the single-workgroup select over the row's scores
        select_row_streaming(a, row, sh, StreamLds{lds, lds + 2048, lds + 3072, lds + 3072 + kRegWords});
        return;
    }
    uint32_t krem = (uint32_t)a.k - totals[0];   // candidates to take, 1 <= krem <= candidates
    const uint32_t ex[4] = {p01.x, p01.z, p23.x, p23.z}, ey[4] = {p01.y, p01.w, p23.y, p23.w};
    bool ev[4];
    uint32_t eidx[4], elow[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        ev[j] = reg < nreg && (uint32_t)(slot0 + j) < rc.y;
        eidx[j] = ev[j] ? min(ex[j], (uint32_t)a.M - 1u) : 0u;
        elow[j] = ey[j] & ((1u << kHistShift) - 1u);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (ev[j]) atomicAdd(&sh.hist[elow[j] >> 10], 1u);
    __syncthreads();
    find_digit_wave(sh, sh.hist, krem, 2048);
    const uint32_t d2 = sh.digit & 2047u;
    krem = sh.krem;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (ev[j] && (elow[j] >> 10) == d2) atomicAdd(&hist3[elow[j] & 1023u], 1u);
    __syncthreads();
    find_digit_wave(sh, hist3, krem, 1024);
    const uint32_t tlow = (d2 << 10) | (sh.digit & 1023u);
    krem = sh.krem;
    if (sh.dcount <= krem) {
        // every key equal to the threshold is taken (the usual case: no tie at the boundary)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (ev[j] && elow[j] >= tlow) atomicOr(&bits[eidx[j] >> 5], 1u << (eidx[j] & 31u));
    } else {
        // equal keys at the threshold: the first krem of them in index order. Regions follow the index order (tile
        // after tile, wave after wave), entries inside a region too, and thread t holds entries 4t..4t+3, so a block
        // scan of the tied counts ranks the ties by index.
        uint32_t neq = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) neq += ev[j] && elow[j] == tlow;
        uint32_t eeq, unused, teq, unused_t;
        block_scan2<kSelThreads>(neq, 0u, eeq, unused, teq, unused_t, sh.wave_tot);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (!ev[j]) continue;
            const bool eq = elow[j] == tlow;
            if (elow[j] > tlow || (eq && eeq < krem)) atomicOr(&bits[eidx[j] >> 5], 1u << (eidx[j] & 31u));
            eeq += eq;
        }
    }
    __syncthreads();
    init_sortbuf(a, sh);   // score order: the staged pairs' padding, ordered by the scan's barriers
    const uint32_t sw = tid < t.W ? bits[tid] : 0u;
    uint32_t slot, unused2, tsel, unused_t2;
    block_scan2<kSelThreads>((uint32_t)__popc(sw), 0u, slot, unused2, tsel, unused_t2, sh.wave_tot);
    emit_word_row(a, row, sh, sw, slot);
}

// ---------------------------------------------------------------------------------------------------------------
// List select (the fused decode step, rows of at most kListMaxM candidates): one 1024-thread workgroup per row builds
// the row's selection bitmap from the score kernel's per-workgroup key lists (list_select_bitmap), then emits it as
// select_resolve_compact does (F, position or score order) and clears the row's select state.
// ---------------------------------------------------------------------------------------------------------------
constexpr int kListSlots = 8;   // entries per lane loaded in the first round trip
static_assert(kListWords == kSelThreads, "one selection bitmap word per thread");

struct ListArgs {
    const uint2* entries;   // [R, tiles, cap]
    const uint2* hdr;       // [R, tiles]
    int cap, tiles, nsub, lspl;
    TableRef table;         // where SelectArgs::scores is null: the table the scores are recomputed from
};

template <int MAXSUB>
__global__ __launch_bounds__(kSelThreads) void select_lists(SelectArgs a, ListArgs t) {
    __shared__ SelectShared sh;   // hist: the first digit's bins; sortbuf: candidates, then score order's pairs
    __shared__ __attribute__((aligned(16))) uint32_t lds[2048 + 1024 + 2 * kListWords];
    __shared__ uint2 hdr[kListMaxTiles];
    __shared__ uint32_t sup2[64];
    __shared__ uint32_t misc[4];
    static_assert(kListCandCap * sizeof(uint2) <= sizeof(SelectShared::sortbuf), "candidates live in sortbuf");
    const int row = xcd_contiguous_block();   // the XCD whose score workgroups wrote the row
    ListLds L;
    L.hist = sh.hist;
    L.hist2 = lds;
    L.sup2 = sup2;
    L.hist3 = lds + 2048;
    L.bits = lds + 3072;
    L.ties = lds + 3072 + kListWords;
    L.hdr = hdr;
    L.cand = reinterpret_cast<uint2*>(sh.sortbuf);
    L.misc = misc;
    L.wave_tot = sh.wave_tot;
    ListRow r;
    r.scores = RowScores{a.scores ? a.scores + (size_t)row * a.score_stride : nullptr, t.table, row, a.lo, a.hi};
    r.state = a.hist + (size_t)row * kSelectStateWords;
    r.entries = t.entries + (size_t)row * t.tiles * t.cap;
    r.hdr = t.hdr + (size_t)row * t.tiles;
    r.M = a.M;
    r.k = a.k;
    r.lo = a.lo;
    r.hi = a.hi;
    r.cap = t.cap;
    r.tiles = t.tiles;
    r.nsub = t.nsub;
    r.lspl = t.lspl;
    list_select_bitmap<kSelThreads, kListSlots, MAXSUB>(r, L);
    const uint32_t sw = L.bits[threadIdx.x];
    init_sortbuf(a, sh);   // score order: the staged pairs' padding (the candidates in sortbuf are no longer read)
    emit_word_row(a, row, sh, sw, block_excl_scan_once((uint32_t)__popc(sw), sh.wave_tot));
}

// ---------------------------------------------------------------------------------------------------------------
// Select and attend in one launch (the fused step in position order when no row list leaves the call): workgroup
// (b, g, head group qg, partition p) of the attend's grid first selects its row from the score kernel's key lists
// (list_select_bitmap, eight waves), keeps the positions of its own partition of the row list in LDS, and then its first
// four waves attend them exactly as attend_kernel does (the same pipeline, merges and split-K merge, so the output is
// the same bit for bit). Every workgroup of a row computes the same selection; the last of them to have read the row's
// first-digit bins clears them, and the attend's last partition leaves its arrival counter zero, so the select state is
// zero again after the call. Saves the select's launch, its row-list stores and the attend's staging round trip.
// ---------------------------------------------------------------------------------------------------------------
constexpr int kSAThreads = 512;
constexpr int kSAWaves = kSAThreads / 64;
constexpr int kSASlots = 8;            // list entries per lane in the first round trip
constexpr int kSAMaxRows = 4096;       // positions of one partition held in LDS
// K/V register stages of the fused attend (attend_kernel keeps kStages): the output does not depend on the depth, and
// three measured 0.08-0.14 us per layer faster than four at B = 1, 2, 4, 8 and 16 (two: up to 3 us slower)
constexpr int kSAStages = 3;
constexpr int kSAReadCounter = kSelectStateWords - 1;   // the row's readers of its bins: the last arrival word
static_assert(kListWords == 2 * kSAThreads, "two selection bitmap words per thread");

template <int MAXSUB, int H>
__global__ __launch_bounds__(kSAThreads) void select_attend(SelectArgs sa, ListArgs t, AttendArgs a) {
    __shared__ __attribute__((aligned(16))) uint32_t hist[kHistBins];
    __shared__ __attribute__((aligned(16))) uint32_t lds[2048 + 1024 + 2 * kListWords];
    __shared__ __attribute__((aligned(16))) uint2 cand[kListCandCap];
    __shared__ uint2 hdr[kListMaxTiles];
    __shared__ uint32_t sup2[64];
    __shared__ uint32_t misc[4];
    __shared__ uint32_t wave_tot[kSAWaves][2];
    __shared__ float red_ml[kMergeSlots][H][2];
    __shared__ __attribute__((aligned(16))) float red_acc[kMergeSlots][H][kHeadDim];
    __shared__ uint32_t last_sh;
    int* idx_sh = reinterpret_cast<int*>(cand);   // the partition's positions, once the selection no longer needs cand
    static_assert(kSAMaxRows * sizeof(int) <= sizeof(cand), "the positions fit the candidate array");
    const int lin = xcd_contiguous_block();   // (b, g) on the XCD whose score workgroups wrote its lists
    const int bg = lin / (a.Q * a.P);
    const int rem = lin - bg * a.Q * a.P;
    const int qg = rem / a.P;
    const int p = rem - qg * a.P;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool active = tid < kAttThreads;    // the attending waves
    const int hq = a.h / a.Q, h0 = qg * hq;
    uint32_t qw[H][8];   // loaded first: it arrives while the selection runs
    attend_load_q<H>(a, bg, h0, hq, qw);

    ListLds L;
    L.hist = hist;
    L.hist2 = lds;
    L.sup2 = sup2;
    L.hist3 = lds + 2048;
    L.bits = lds + 3072;
    L.ties = lds + 3072 + kListWords;
    L.hdr = hdr;
    L.cand = cand;
    L.misc = misc;
    L.wave_tot = wave_tot;
    ListRow r;
    r.scores = RowScores{sa.scores ? sa.scores + (size_t)bg * sa.score_stride : nullptr, t.table, bg, sa.lo, sa.hi};
    r.state = sa.hist + (size_t)bg * kSelectStateWords;
    r.entries = t.entries + (size_t)bg * t.tiles * t.cap;
    r.hdr = t.hdr + (size_t)bg * t.tiles;
    r.M = sa.M;
    r.k = sa.k;
    r.lo = sa.lo;
    r.hi = sa.hi;
    r.cap = t.cap;
    r.tiles = t.tiles;
    r.nsub = t.nsub;
    r.lspl = t.lspl;
    list_select_bitmap<kSAThreads, kSASlots, MAXSUB>(r, L);
    // this thread's selected candidates [64 tid, 64 tid + 64) and their first slot among the k picks
    const uint2 wv = reinterpret_cast<const uint2*>(L.bits)[tid];
    uint64_t word = (uint64_t)wv.x | ((uint64_t)wv.y << 32);
    const uint32_t x = (uint32_t)__popcll(word);
    const uint32_t inc = wave_incl_scan(x);
    if (lane == 63) wave_tot[wave][0] = inc;
    __syncthreads();   // also: the candidates (cand) are no longer read, so idx_sh may take their place
    const uint32_t v = lane < kSAWaves ? wave_tot[lane][0] : 0u;
    const uint32_t vi = row16_incl_scan(v);
    const uint32_t slot = (uint32_t)__builtin_amdgcn_readlane((int)(vi - v), wave) + inc - x;
    // the partition's entries of the row list [F sinks | the k picks by position | F recent]
    const int lo = sa.lo, k = sa.k, nrec = sa.legal - sa.hi, nf = lo + nrec;
    const int Sp = (a.S + a.P - 1) / a.P;
    const int s_begin = p * Sp, s_end = min(a.S, s_begin + Sp);
    const int pos0 = lo + 64 * tid;
    // this thread's picks take slots [slot, slot + x) of the k (row-list entries lo + slot ..); those inside the
    // partition, [first, last), go to LDS: the picks before it are dropped, and no lane loops over picks past it
    const int first = max((int)slot, s_begin - lo), last = min((int)slot + (int)x, min(s_end - lo, k));
    if (first < last) {
        for (int j = (int)slot; j < first; ++j) word &= word - 1;
        int* dst = idx_sh + (lo + first - s_begin);
        for (int n = last - first; n > 0; --n) {
            *dst++ = pos0 + (__ffsll((unsigned long long)word) - 1);
            word &= word - 1;
        }
    }
    for (int f = tid; f < nf; f += kSAThreads) {
        const int e = f < lo ? f : lo + k + (f - lo);
        if (e >= s_begin && e < s_end) idx_sh[e - s_begin] = f < lo ? f : sa.hi + (f - lo);
    }
    __syncthreads();
    if (wave == kAttWaves) {
        // every thread has passed the selection's barriers, so this workgroup has read the row's bins: wave kAttWaves,
        // idle while the first four attend, counts it as a reader, and the row's last reader sets the bins, the
        // super-bins and the count back to zero (off the attend's path: its atomic's return is waited for here)
        uint32_t* st = sa.hist + (size_t)bg * kSelectStateWords;
        uint32_t readers = 0u;
        if (lane == 0)
            readers = __hip_atomic_fetch_add(st + kSAReadCounter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((uint32_t)__builtin_amdgcn_readfirstlane((int)readers) == (uint32_t)(a.Q * a.P - 1)) {
            for (int i = lane; i < kHistBins + kSuperBins; i += 64) st[i] = 0u;
            if (lane == 0) st[kSAReadCounter] = 0u;
        }
    }
    float m[H], l[H], acc[H][16];
#pragma unroll
    for (int i = 0; i < H; ++i) {
        m[i] = -INFINITY;
        l[i] = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;
    }
    if (active && s_end > s_begin) {
        const size_t bg_off = (size_t)bg * a.kv_bg_stride;
        const uint16_t* Kb = a.K + bg_off + 8 * (tid & 7);
        const uint16_t* Vb = a.V + bg_off + 8 * (tid & 7);
        attend_chunk<H, kSAStages, false, false>(a, Kb, Vb, s_begin, s_end - s_begin, idx_sh, qw, m, l, acc);
    }
    attend_finish<H>(a, bg, qg, p, hq, h0, m, l, acc, red_ml, red_acc, &last_sh, active);
}

// ---------------------------------------------------------------------------------------------------------------
// Score order past kMaxScoreOrderK, where the k selected pairs no longer fit the LDS sort: the select runs in position
// order into `stage` (candidate indices, ascending), then select_sort_score lists them by descending score with three
// stable LSD radix passes over the order-preserving key (digits of 10, 11 and 11 bits, each complemented so that
// ascending digit order is descending score). Stability keeps equal scores in ascending index order, as the LDS sort
// does. One 1024-thread workgroup per row. A pass counts its digit over the row (LDS histogram; its exclusive scan is
// each digit's first slot), then places the row 1024 elements at a time: a lane's rank among the lanes of its wave
// with the same digit comes from one ballot per digit bit, the earlier waves' counts of that digit from an LDS table,
// the earlier tiles' from a running count. Elements move as (key << 32 | index) through two scratch buffers; the last
// pass writes the outputs and F.
// ---------------------------------------------------------------------------------------------------------------
struct SortScratch {
    int32_t* stage;   // [R, k] the position-order select's candidate indices
    uint64_t* buf0;   // [R, k]
    uint64_t* buf1;   // [R, k]
};

__host__ __device__ inline int64_t sort_scratch_bytes(int R, int k) {
    return align_bytes((int64_t)R * k * 4, 256) + 2 * align_bytes((int64_t)R * k * 8, 256);
}

struct SortShared {
    uint16_t cnt[kSelWaves][kHistBins];   // this tile's count of each digit per wave, zero between tiles
    uint32_t base[kHistBins];             // first slot of each digit in this pass
    uint32_t run[kHistBins];              // elements of each digit placed by the earlier tiles
    uint32_t wave_tot[kSelWaves][2];
};

__global__ __launch_bounds__(kSelThreads) void select_sort_score(SelectArgs a, SortScratch sc) {
    __shared__ SortShared sh;
    const int row = xcd_contiguous_block();
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int k = a.k;
    const float* srow = a.scores + (size_t)row * a.score_stride;
    const int32_t* stage = sc.stage + (size_t)row * k;
    uint64_t* b0 = sc.buf0 + (size_t)row * k;
    uint64_t* b1 = sc.buf1 + (size_t)row * k;
    const int nrec = a.legal - a.hi, nf = a.lo + nrec, S = nf + k;
    int32_t* rows = a.rows ? a.rows + (size_t)row * a.rows_stride : nullptr;
    int64_t* flat = a.rows_flat ? a.rows_flat + (size_t)row * S : nullptr;
    int32_t* ti = a.top_idx ? a.top_idx + (size_t)row * a.top_stride : nullptr;
    float* tv = a.top_val ? a.top_val + (size_t)row * a.top_stride : nullptr;
    const int64_t base = (int64_t)row * a.C;
    for (int i = tid; i < kSelWaves * kHistBins / 2; i += kSelThreads) reinterpret_cast<uint32_t*>(&sh.cnt[0][0])[i] = 0u;
    const uint64_t lt = (1ull << lane) - 1ull;
    for (int pass = 0; pass < 3; ++pass) {
        const int shift = pass == 0 ? 0 : (pass == 1 ? 10 : 21);
        const int nbits = pass == 0 ? 10 : 11;
        const uint32_t dmask = (1u << nbits) - 1u;
        // pass 0: stage (keys gathered) -> b1 -> b0; pass 1: b0 -> b1; pass 2: b1 -> outputs
        const uint64_t* src = pass == 1 ? b0 : b1;
        uint64_t* dst = pass == 0 ? b0 : b1;
        sh.base[tid] = 0u;
        sh.base[tid + kSelThreads] = 0u;
        sh.run[tid] = 0u;
        sh.run[tid + kSelThreads] = 0u;
        __syncthreads();
        for (int e = tid; e < k; e += kSelThreads) {
            uint64_t x;
            if (pass == 0) {
                const uint32_t idx = (uint32_t)min(max(stage[e], 0), a.M - 1);
                x = ((uint64_t)score_key(srow[idx]) << 32) | idx;
                b1[e] = x;
            } else {
                x = src[e];
            }
            atomicAdd(&sh.base[dmask - (((uint32_t)(x >> 32) >> shift) & dmask)], 1u);
        }
        __syncthreads();
        {   // exclusive scan of the digit counts (two bins per thread; the second is 0 past nbins)
            const uint32_t c0 = sh.base[2 * tid], c1 = sh.base[2 * tid + 1];
            uint32_t ex, unused, tot, unused_t;
            block_scan2<kSelThreads>(c0 + c1, 0u, ex, unused, tot, unused_t, sh.wave_tot);
            sh.base[2 * tid] = ex;
            sh.base[2 * tid + 1] = ex + c0;
        }
        __syncthreads();
        for (int t0 = 0; t0 < k; t0 += kSelThreads) {
            const int e = t0 + tid;
            const bool ok = e < k;
            const uint64_t x = ok ? src[e] : 0ull;
            const uint32_t dg = dmask - (((uint32_t)(x >> 32) >> shift) & dmask);
            uint64_t peers = __ballot(ok);
            for (int b = 0; b < nbits; ++b) {
                const bool bit = (dg >> b) & 1u;
                const uint64_t m = __ballot(bit);
                peers &= bit ? m : ~m;
            }
            const bool leader = ok && (peers & lt) == 0;
            const uint32_t n = (uint32_t)__popcll(peers);
            if (leader) sh.cnt[wave][dg] = (uint16_t)n;
            __syncthreads();
            uint32_t off = 0u;
            if (leader) {
                off = sh.base[dg] + sh.run[dg];
                for (int w = 0; w < wave; ++w) off += sh.cnt[w][dg];
            }
            const int src_lane = ok ? __ffsll((unsigned long long)peers) - 1 : lane;
            off = (uint32_t)__shfl((int)off, src_lane, 64);
            const uint32_t slot = off + (uint32_t)__popcll(peers & lt);
            if (ok && slot < (uint32_t)k) {
                if (pass < 2) {
                    dst[slot] = x;
                } else {
                    const int idx = (int)(uint32_t)x;
                    if (ti) ti[slot] = idx;
                    if (tv) tv[slot] = srow[idx];
                    if (rows) rows[nf + slot] = a.lo + idx;
                    if (flat) flat[nf + slot] = base + a.lo + idx;
                }
            }
            __syncthreads();
            if (leader) {
                sh.cnt[wave][dg] = 0;
                atomicAdd(&sh.run[dg], n);
            }
        }
        __syncthreads();
    }
    for (int f = tid; f < nf; f += kSelThreads) {   // F first, ascending (cat(fixed_rows, topk) of decode.py:93)
        const int p = f < a.lo ? f : a.hi + (f - a.lo);
        if (rows) rows[f] = p;
        if (flat) flat[f] = base + p;
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------------------------------
// Bytes of the scratch: the tiled select's region, then (score order past kMaxScoreOrderK) the sort's stage and buffers.
int64_t select_scratch_bytes(int R, int M, int k, int order) {
    int64_t b = align_bytes(tiled_region_bytes(R, M), 256);
    if (staged_score_order(order, k)) b += sort_scratch_bytes(R, k);
    return b;
}

static int launch_tiled(const SelectArgs& a, int R, void* scratch, hipStream_t s, bool build_hist) {
    const int W = (a.M + 31) / 32, T = (a.M + kTileKeys - 1) / kTileKeys;
    if (compact_fits(a.M)) {
        CompactArgs c;
        char* p = static_cast<char*>(scratch);
        c.above = reinterpret_cast<uint32_t*>(p);
        c.counts = reinterpret_cast<uint2*>(p + (size_t)R * compact_bitmap_bytes(a.M));
        c.entries = c.counts + (size_t)R * kCompactRegions;
        c.W = W;
        c.T = T;
        // above is [R, W] (rows W words apart) inside the first R * compact_bitmap_bytes(M) bytes
        if (build_hist) {
            TiledArgs th{c.above, nullptr, W, T};
            hipLaunchKernelGGL(select_hist, dim3(R * T), dim3(kTileThreads), 0, s, a, th);
        }
        hipLaunchKernelGGL(select_classify_compact, dim3(R * T), dim3(kTileThreads), 0, s, a, c);
        hipLaunchKernelGGL(select_resolve_compact, dim3(R), dim3(kSelThreads), 0, s, a, c);
        return check_launch("select_compact");
    }
    TiledArgs t;
    t.above = static_cast<uint32_t*>(scratch);
    t.cand = t.above + (size_t)R * W;
    t.W = W;
    t.T = T;
    if (build_hist) hipLaunchKernelGGL(select_hist, dim3(R * t.T), dim3(kTileThreads), 0, s, a, t);
    hipLaunchKernelGGL(select_classify, dim3(R * t.T), dim3(kTileThreads), 0, s, a, t);
    if (a.M >= kCandCapLongFromM) hipLaunchKernelGGL(select_resolve<kCandCapLong>, dim3(R), dim3(kSelThreads), 0, s, a, t);
    else hipLaunchKernelGGL(select_resolve<kCandCapShort>, dim3(R), dim3(kSelThreads), 0, s, a, t);
    return check_launch("select_tiled");
}

// The selection of R rows with `a` (its outputs and order), run tiled when `tiled`, else one workgroup per row; score
// order past kMaxScoreOrderK goes through the position-order select into the sort's stage and select_sort_score.
static int run_select(const SelectArgs& a, int R, bool tiled, void* scratch, hipStream_t s, bool build_hist) {
    SelectArgs sel = a;
    SortScratch sc{};
    const bool staged = staged_score_order(a.order, a.k);
    if (staged) {
        char* p = static_cast<char*>(scratch) + align_bytes(tiled_region_bytes(R, a.M), 256);
        sc.stage = reinterpret_cast<int32_t*>(p);
        sc.buf0 = reinterpret_cast<uint64_t*>(p + align_bytes((int64_t)R * a.k * 4, 256));
        sc.buf1 = reinterpret_cast<uint64_t*>(p + align_bytes((int64_t)R * a.k * 4, 256) +
                                              align_bytes((int64_t)R * a.k * 8, 256));
        sel.order = ATTNLAB_ORDER_POSITION;
        sel.rows = nullptr;
        sel.rows_flat = nullptr;
        sel.top_idx = sc.stage;
        sel.top_val = nullptr;
        sel.top_stride = a.k;
    }
    const int rc = tiled ? launch_tiled(sel, R, scratch, s, build_hist) : launch_select(sel, R, s);
    if (rc || !staged) return rc;
    hipLaunchKernelGGL(select_sort_score, dim3(R), dim3(kSelThreads), 0, s, a, sc);
    return check_launch("select_sort_score");
}

int select_check(int B, int G, int lo, int hi, int legal, int k, int C, int order, const int32_t* rows,
                 int64_t rows_stride, const float* scores, int64_t score_stride, bool scores_needed) {
    ATTNLAB_REQUIRE(B >= 1 && G >= 1, "B and G must be positive (B=%d G=%d)", B, G);
    ATTNLAB_REQUIRE(0 <= lo && lo <= hi && hi <= legal && legal <= C, "need 0 <= lo <= hi <= legal <= C, got %d %d %d %d",
                    lo, hi, legal, C);
    const int M = hi - lo;
    ATTNLAB_REQUIRE(0 <= k && k <= M, "need 0 <= k <= hi - lo, got k=%d M=%d", k, M);
    ATTNLAB_REQUIRE(order == ATTNLAB_ORDER_POSITION || order == ATTNLAB_ORDER_SCORE, "unknown order %d", order);
    const int S = lo + (legal - hi) + k;
    ATTNLAB_REQUIRE(S >= 1, "empty row list");
    ATTNLAB_REQUIRE(rows == nullptr || rows_stride >= S, "rows_stride=%lld smaller than S=%d", (long long)rows_stride, S);
    ATTNLAB_REQUIRE(k == 0 || !scores_needed || (scores != nullptr && score_stride >= M),
                    "scores must hold M=%d values per row", M);
    return ATTNLAB_OK;
}

int select_lists_impl(const float* scores, int64_t score_stride, int B, int G, int lo, int hi, int legal, int k, int C,
                      int order, int32_t* rows, int64_t rows_stride, int64_t* rows_flat, uint32_t* state,
                      const ScoreLists& lists, FusedGeometry geo, hipStream_t stream, TableRef table) {
    // without stored scores: the table they are recomputed from; position order (score order reads them back)
    const bool recompute = scores == nullptr;
    ATTNLAB_REQUIRE(!recompute || (table.zT != nullptr && table.u != nullptr && table.C % 8 == 0 && hi <= table.C &&
                                   (table.dtype == ATTNLAB_DT_BF16 || table.dtype == ATTNLAB_DT_F32) &&
                                   (reinterpret_cast<uintptr_t>(table.zT) & 15) == 0 &&
                                   order == ATTNLAB_ORDER_POSITION),
                    "the list select without stored scores needs the aligned index table, u and position order");
    int rc = select_check(B, G, lo, hi, legal, k, C, order, rows, rows_stride, scores, score_stride, !recompute);
    if (rc) return rc;
    const int M = hi - lo;
    ATTNLAB_REQUIRE(k > 0 && M <= kListMaxM && geo.nsub >= 1 && geo.nsub <= 8 && geo.tiles >= 1 &&
                        geo.tiles <= kListMaxTiles && (int64_t)geo.tiles * geo.nsub * 512 >= ((hi + 7) & ~7) - (lo & ~7),
                    "the list select needs 0 < k, M <= %d and the score tiling that wrote the lists", kListMaxM);
    ATTNLAB_REQUIRE(!staged_score_order(order, k), "the list select sorts at most %d rows in score order",
                    kMaxScoreOrderK);
    ATTNLAB_REQUIRE(state != nullptr && lists.entries != nullptr && lists.hdr != nullptr && lists.cap >= 1,
                    "the list select needs the select state and the lists");
    SelectArgs a{scores, score_stride, M, k, lo, hi, legal, G, C, order, rows, rows_stride, rows_flat, nullptr, nullptr, 0,
                 state};
    ListArgs t{lists.entries, lists.hdr, lists.cap, geo.tiles, geo.nsub, list_lspl(geo.tiles, kSelWaves, kListSlots, lists.lmin),
               recompute ? table : TableRef{}};
    // the instance for up to four sub-tiles per score workgroup keeps fewer registers live
    if (geo.nsub <= 4) hipLaunchKernelGGL(select_lists<4>, dim3(B * G), dim3(kSelThreads), 0, stream, a, t);
    else hipLaunchKernelGGL(select_lists<8>, dim3(B * G), dim3(kSelThreads), 0, stream, a, t);
    return check_launch("select_lists");
}

bool select_attend_applies(int B, int G, int lo, int hi, int legal, int k, int h, int P) {
    if (k <= 0 || hi - lo > kListMaxM || P < 1 || h < 1) return false;
    const int S = lo + (legal - hi) + k;
    const int Q = attend_head_groups(B * G, h, P);
    const int hq = h / Q;
    return (hq == 1 || hq == 2 || hq == 4) && (S + P - 1) / P <= kSAMaxRows && Q <= kSAReadCounter - kArriveOffset;
}

int select_attend_impl(int B, int G, int lo, int hi, int legal, int k, int C, uint32_t* state, const ScoreLists& lists,
                       FusedGeometry geo, TableRef table, const uint16_t* K, const uint16_t* V, const uint16_t* q, int h,
                       int P, float scale, uint16_t* out, float* part, hipStream_t stream) {
    const int M = hi - lo, S = lo + (legal - hi) + k;
    if (!select_attend_applies(B, G, lo, hi, legal, k, h, P)) return set_error(ATTNLAB_EINVAL, "select_attend: shape");
    ATTNLAB_REQUIRE(state && lists.entries && lists.hdr && table.zT && table.u && K && V && q && out &&
                        (P == 1 || part != nullptr),
                    "select_attend needs the state, the lists, the table, the cache, q, out and (P > 1) partials");
    SelectArgs sa{nullptr, 0, M, k, lo, hi, legal, G, C, ATTNLAB_ORDER_POSITION, nullptr, 0, nullptr, nullptr, nullptr, 0,
                  state};
    ListArgs t{lists.entries, lists.hdr, lists.cap, geo.tiles, geo.nsub,
               list_lspl(geo.tiles, kSAWaves, kSASlots, lists.lmin), table};
    const int Q = attend_head_groups(B * G, h, P);
    AttendArgs a{K, V, (int64_t)C * kHeadDim, kHeadDim, q, nullptr, 0, S, C, h, P, Q, scale * kLog2e, out, 1, part};
    if (P > 1) {
        a.arrive = state + kArriveOffset;
        a.arrive_stride = kSelectStateWords;
    }
    const dim3 grid(B * G * Q * P), block(kSAThreads);
    const int hq = h / Q;
#define SA_LAUNCH(MS)                                                                                     \
    do {                                                                                                  \
        if (hq == 1) hipLaunchKernelGGL((select_attend<MS, 1>), grid, block, 0, stream, sa, t, a);        \
        else if (hq == 2) hipLaunchKernelGGL((select_attend<MS, 2>), grid, block, 0, stream, sa, t, a);   \
        else hipLaunchKernelGGL((select_attend<MS, 4>), grid, block, 0, stream, sa, t, a);                \
    } while (0)
    if (geo.nsub <= 4) SA_LAUNCH(4);
    else SA_LAUNCH(8);
#undef SA_LAUNCH
    return check_launch("select_attend");
}

int select_rows_impl(const float* scores, int64_t score_stride, int B, int G, int lo, int hi, int legal, int k, int C,
                     int order, int32_t* rows, int64_t rows_stride, int64_t* rows_flat, uint32_t* state,
                     void* scratch, int64_t scratch_bytes, hipStream_t stream) {
    int rc = select_check(B, G, lo, hi, legal, k, C, order, rows, rows_stride, scores, score_stride);
    if (rc) return rc;
    ATTNLAB_REQUIRE(scratch_bytes >= 0, "negative scratch_bytes");
    const int M = hi - lo;
    const int R = B * G;
    const bool staged = k > 0 && staged_score_order(order, k);
    ATTNLAB_REQUIRE(!staged || (scratch != nullptr && (reinterpret_cast<uintptr_t>(scratch) & 255) == 0 &&
                                scratch_bytes >= select_scratch_bytes(R, M, k, order)),
                    "score order with k=%d > %d needs a 256-byte aligned scratch of attnlab_select_scratch_bytes = %lld "
                    "bytes", k, kMaxScoreOrderK, (long long)select_scratch_bytes(R, M, k, order));
    if (!rows && !rows_flat && !state) return ATTNLAB_OK;
    SelectArgs a{scores, score_stride, M, k, lo, hi, legal, G, C, order, rows, rows_stride, rows_flat, nullptr, nullptr, 0,
                 state};
    const int W = (M + 31) / 32;
    const bool tiled = state && scratch && k > 0 && W <= kMaxWords &&
                       (reinterpret_cast<uintptr_t>(state) & 15) == 0 && (reinterpret_cast<uintptr_t>(scratch) & 15) == 0 &&
                       scratch_bytes >= align_bytes(tiled_region_bytes(R, M), 256);
    return run_select(a, R, tiled, scratch, stream, false);
}

}  // namespace attnlab

using namespace attnlab;

extern "C" int attnlab_topk(const float* scores, int64_t score_stride, int R, int M, int k, int order, int32_t* top_idx,
                            float* top_val, int64_t top_stride, void* stream) {
    ATTNLAB_REQUIRE(R >= 0 && M >= 0, "R=%d and M=%d must be non-negative", R, M);
    ATTNLAB_REQUIRE(0 <= k && k <= M, "need 0 <= k <= M, got k=%d M=%d", k, M);
    ATTNLAB_REQUIRE(order == ATTNLAB_ORDER_POSITION || order == ATTNLAB_ORDER_SCORE, "unknown order %d", order);
    ATTNLAB_REQUIRE(order != ATTNLAB_ORDER_SCORE || k <= kMaxScoreOrderK,
                    "score order with k=%d > %d needs the scratch of attnlab_topk_tiled", k, kMaxScoreOrderK);
    if (R == 0 || k == 0) return ATTNLAB_OK;
    ATTNLAB_REQUIRE(scores != nullptr && score_stride >= M, "scores must hold M=%d values per row", M);
    ATTNLAB_REQUIRE(top_stride >= k, "top_stride=%lld smaller than k=%d", (long long)top_stride, k);
    SelectArgs a{scores, score_stride, M, k, 0, 0, 0, 1, 0, order, nullptr, 0, nullptr, top_idx, top_val, top_stride,
                 nullptr};
    return launch_select(a, R, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int attnlab_topk_tiled(const float* scores, int64_t score_stride, int R, int M, int k, int order,
                                  int32_t* top_idx, float* top_val, int64_t top_stride, uint32_t* state, void* scratch,
                                  int64_t scratch_bytes, void* stream) {
    ATTNLAB_REQUIRE(R >= 0 && M >= 0, "R=%d and M=%d must be non-negative", R, M);
    ATTNLAB_REQUIRE(0 <= k && k <= M, "need 0 <= k <= M, got k=%d M=%d", k, M);
    ATTNLAB_REQUIRE(order == ATTNLAB_ORDER_POSITION || order == ATTNLAB_ORDER_SCORE, "unknown order %d", order);
    ATTNLAB_REQUIRE(scratch_bytes >= 0, "negative scratch_bytes");
    if (R == 0 || k == 0) return ATTNLAB_OK;
    ATTNLAB_REQUIRE(scores != nullptr && score_stride >= M, "scores must hold M=%d values per row", M);
    ATTNLAB_REQUIRE(top_stride >= k, "top_stride=%lld smaller than k=%d", (long long)top_stride, k);
    ATTNLAB_REQUIRE(state != nullptr && (reinterpret_cast<uintptr_t>(state) & 15) == 0,
                    "state must be a 16-byte aligned [R, %d] buffer", kSelectStateWords);
    const int64_t need = select_scratch_bytes(R, M, k, order);
    ATTNLAB_REQUIRE(scratch != nullptr && (reinterpret_cast<uintptr_t>(scratch) & 255) == 0 && scratch_bytes >= need,
                    "scratch must be 256-byte aligned and hold attnlab_select_scratch_bytes(%d, %d, %d, %d) = %lld bytes",
                    R, M, k, order, (long long)need);
    SelectArgs a{scores, score_stride, M, k, 0, 0, 0, 1, 0, order, nullptr, 0, nullptr, top_idx, top_val, top_stride,
                 state};
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if ((M + 31) / 32 > kMaxWords) {   // rows past 262144 keys: single-workgroup select, which builds its own histograms
        a.hist = nullptr;
        return run_select(a, R, false, scratch, s, false);
    }
    return run_select(a, R, true, scratch, s, true);
}

extern "C" int attnlab_select_rows(const float* scores, int64_t score_stride, int B, int G, int lo, int hi, int legal,
                                   int k, int C, int order, int32_t* rows, int64_t rows_stride, int64_t* rows_flat,
                                   uint32_t* state, void* scratch, int64_t scratch_bytes, void* stream) {
    return select_rows_impl(scores, score_stride, B, G, lo, hi, legal, k, C, order, rows, rows_stride, rows_flat, state,
                            scratch, scratch_bytes, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int attnlab_select_lists(const float* scores, int64_t score_stride, int B, int G, int lo, int hi, int legal,
                                    int k, int C, int order, int32_t* rows, int64_t rows_stride, int64_t* rows_flat,
                                    uint32_t* state, const void* lists, int64_t lists_bytes, const void* zT,
                                    int z_dtype, const float* u, void* stream) {
    int rc = select_check(B, G, lo, hi, legal, k, C, order, rows, rows_stride, scores, score_stride, scores != nullptr);
    if (rc) return rc;
    const FusedGeometry geo = fused_tiling(B * G, lo, hi);
    const ListPlan plan = hi > lo ? list_plan(hi - lo, k, geo) : ListPlan{0, 0};
    ATTNLAB_REQUIRE(plan.cap > 0, "the list select does not apply to B*G=%d, M=%d, k=%d", B * G, hi - lo, k);
    ATTNLAB_REQUIRE(!staged_score_order(order, k), "the list select sorts at most %d rows in score order (k=%d); "
                    "attnlab_select_rows takes larger k", kMaxScoreOrderK, k);
    ATTNLAB_REQUIRE(state != nullptr && (reinterpret_cast<uintptr_t>(state) & 15) == 0,
                    "the list select needs the 16-byte aligned select state");
    ATTNLAB_REQUIRE(lists != nullptr && (reinterpret_cast<uintptr_t>(lists) & 255) == 0 &&
                        lists_bytes >= list_bytes(B * G, geo, plan),
                    "lists must be 256-byte aligned and hold attnlab_list_bytes = %lld bytes",
                    (long long)list_bytes(B * G, geo, plan));
    const TableRef table = scores ? TableRef{} : TableRef{zT, z_dtype, C, u};
    return select_lists_impl(scores, score_stride, B, G, lo, hi, legal, k, C, order, rows, rows_stride, rows_flat,
                             state, list_layout(const_cast<void*>(lists), B * G, geo, plan), geo,
                             reinterpret_cast<hipStream_t>(stream), table);
}

extern "C" int64_t attnlab_select_scratch_bytes(int R, int M, int k, int order) {
    if (R < 0 || M < 0 || k < 0 || k > M) return -1;
    return select_scratch_bytes(R, M, k, order);
}
