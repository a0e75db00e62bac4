// The list select of one row as a device function (select_lists runs it with 1024 threads per row; the code takes
// any multiple of 64 threads up to 1024 that divides the 1024-word bitmap).
//
// The score kernel leaves, per workgroup of a row, a list of its largest keys (every key whose first digit is at least
// that of the workgroup's lmin-th largest, d_L) with a header (d_L, length). list_select_bitmap then
//   1. in one round trip loads the row's first-digit histogram, the headers and the first entries of every list (wave
//      w owns lists w, w + waves, ...); every wave finds b1, the first digit of the k-th largest key, on its own
//      (super-bins in registers, then the chosen super-bin's 32 bins from LDS);
//   2. takes, from each list whose d_L <= b1 and whose length fits its capacity (such a list holds every key of its
//      tile with first digit >= b1), the keys above b1 into the selection bitmap and the keys in bin b1 into a
//      candidate array (one LDS atomic per wave and pass) while counting their second digit. A list that fails either
//      test is replaced by its tile's scores (the columns of the score workgroup: sub-tile s covers
//      (lo & ~7) + (s * tiles + w) * 512 + [0, 512));
//   3. finds the second digit; when its bin holds exactly the keys still to take (the usual case) the selection is
//      complete, else a third digit and the first krem tied keys in index order (a tie bitmap and one block scan).
// A bin b1 holding more than kListCandCap keys is resolved by three radix passes over the row's scores instead. The
// scores of an incomplete list's tile and of a radix-resolved row are the stored ones where the score stage wrote them,
// else recomputed from the index table in the score kernel's exact operation order (rescore8). The result is the
// selection bitmap in LDS (bit i: candidate i is among the top k; ties go to the lower index).
#pragma once

#include "common.h"
#include "select.h"

namespace attnlab {

constexpr int kListCandCap = 8192;                    // keys of bin b1 held in LDS as (index, low 21 key bits)
constexpr int kListWords = kListMaxM / 32;            // selection bitmap words: 1024

// One row of the list select. The score kernel's tiling (nsub sub-tiles of 512 columns per workgroup, tiles
// workgroups) locates an incomplete list's scores.
struct ListRow {
    RowScores scores;         // the row's M candidate scores (stored, or recomputed from the index table)
    const uint32_t* state;    // the row's select state (first-digit bins, then super-bins)
    const uint2* entries;     // the row's lists [tiles, cap]
    const uint2* hdr;         // [tiles] (d_L, length)
    int M, k, lo, hi;
    int cap, tiles, nsub;
    int lspl;                 // log2 of the entries per lane and list loaded in the first round trip
};

// LDS of list_select_bitmap (the caller places the arrays, so that they can share memory with its other phases). Fill
// it field by field in the kernel: an aggregate of LDS addresses given as a constant initializer cannot be emitted.
struct ListLds {
    uint32_t* hist;           // kHistBins: the first digit's bins
    uint32_t* hist2;          // 2048: the second digit over bin b1
    uint32_t* sup2;           // 64: super-bins of hist2
    uint32_t* hist3;          // 1024: the third digit
    uint32_t* bits;           // kListWords: the selection bitmap (the result)
    uint32_t* ties;           // kListWords
    uint2* hdr;               // kListMaxTiles
    uint2* cand;              // kListCandCap
    uint32_t* misc;           // 4: candidate count, then a wave-0 search's digit, keys left, bin count
    uint32_t (*wave_tot)[2];  // one per wave
};

// Entries per lane and list of the first round trip (as a power of two): the largest with every list of a wave covered
// (slots / lists per wave), but no more 64-entry slots than cover 2 lmin entries; slots past cap are not loaded, and a
// longer list's tail is read after the first round trip. A list holds lmin entries plus the rest of the first-digit bin
// of its lmin-th key: for Gaussian scores 1.3 lmin on average and under 2 lmin in 999 of 1000 lists (numpy model of the
// lists at lmin = 64, 105, 177). At 32K the limit halves B=1's first round trip to 128 entries per list (lmin = 64;
// select 6.93 -> 6.56-6.62 us, step 21.0 -> 20.56 us per layer in alternating runs) and trims B=2's from 320 to 256
// (lmin = 105); B=4 and up keep theirs.
inline int list_lspl(int tiles, int waves, int slots, int lmin) {
    const int nlw = (tiles + waves - 1) / waves;
    int l = 0;
    while ((2 << l) <= slots / nlw) ++l;
    while (l > 0 && (64 << (l - 1)) >= 2 * lmin) --l;
    return l;
}

// b1 and the keys above bin b1 for this wave, from the super-bin counts in registers (lane l: super-bin 63 - l) and
// the bins in LDS; no barrier. b1 = 0 and above = 0 when the histogram holds fewer than k keys.
__device__ __forceinline__ uint32_t wave_first_digit(uint32_t sbv, const uint32_t* bins, uint32_t k, uint32_t& above,
                                                     uint32_t& count) {
    const int lane = threadIdx.x & 63;
    const uint32_t inc = wave_incl_scan(sbv);
    const uint64_t m = __ballot(inc >= k);
    above = 0u;
    count = 0u;
    if (m == 0) return 0u;
    const int l0 = __ffsll((unsigned long long)m) - 1;
    const uint32_t a0 = (uint32_t)__builtin_amdgcn_readlane((int)(inc - sbv), l0);
    const int top = kHistBins - 32 * l0 - 1;   // highest bin of that super-bin
    const uint32_t c = lane < 32 ? bins[top - lane] : 0u;
    const uint32_t inc2 = wave_incl_scan(c) + a0;
    const uint64_t m2 = __ballot(lane < 32 && inc2 >= k);
    if (m2 == 0) return 0u;
    const int l1 = __ffsll((unsigned long long)m2) - 1;
    count = (uint32_t)__builtin_amdgcn_readlane((int)c, l1);
    above = (uint32_t)__builtin_amdgcn_readlane((int)inc2, l1) - count;
    return (uint32_t)(top - l1);
}

// The digit D holding the krem-th largest key of a complete histogram of nbins (1024 or 2048) bins, searched by wave
// 0: res[0] = D, res[1] = keys still to take from bin D, res[2] = its count (left unchanged when no bin qualifies).
// Ends with one barrier.
__device__ __forceinline__ void wave0_find_digit(uint32_t* res, const uint32_t* hist, uint32_t krem, int nbins) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const int per = nbins >> 6;
        const int cb = nbins - per * (lane + 1);
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
            const int top = nbins - per * l0 - 1;
            const uint32_t c = lane < per ? hist[top - lane] : 0u;
            const uint32_t inc2 = wave_incl_scan(c) + above;
            const uint64_t m2 = __ballot(lane < per && inc2 >= krem);
            if (m2 != 0 && lane == __ffsll((unsigned long long)m2) - 1) {
                res[0] = (uint32_t)(top - lane);
                res[1] = krem - (inc2 - c);
                res[2] = c;
            }
        }
    }
    __syncthreads();
}

// Block-wide exclusive scan of one counter; `total` receives the block total. Ends synchronised.
template <int THREADS>
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t x, uint32_t& total, uint32_t (*wave_tot)[2]) {
    constexpr int kWaves = THREADS / 64;
    static_assert(kWaves <= 16, "one row of 16 lanes");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t inc = wave_incl_scan(x);
    if (lane == 63) wave_tot[wave][0] = inc;
    __syncthreads();
    const uint32_t v = lane < kWaves ? wave_tot[lane][0] : 0u;
    const uint32_t vi = row16_incl_scan(v);
    total = (uint32_t)__builtin_amdgcn_readlane((int)vi, kWaves - 1);
    const uint32_t ex = (uint32_t)__builtin_amdgcn_readlane((int)(vi - v), wave) + inc - x;
    __syncthreads();
    return ex;
}

// The first krem tied keys in index order join the selection: thread t owns words [t W, t W + W) of both bitmaps.
template <int THREADS>
__device__ __forceinline__ void take_ties(const ListLds& L, uint32_t krem) {
    constexpr int W = kListWords / THREADS;
    const int tid = threadIdx.x;
    uint32_t n = 0;
#pragma unroll
    for (int i = 0; i < W; ++i) n += (uint32_t)__popc(L.ties[tid * W + i]);
    uint32_t total;
    uint32_t rank = block_excl_scan<THREADS>(n, total, L.wave_tot);
#pragma unroll
    for (int i = 0; i < W; ++i) {
        uint32_t tw = L.ties[tid * W + i], take = 0u;
        while (tw && rank < krem) {
            take |= tw & (0u - tw);   // lowest set bit
            tw &= tw - 1u;
            ++rank;
        }
        L.bits[tid * W + i] |= take;
    }
    __syncthreads();
}

// Bin b1 too full for the candidate array: the remaining two digits by passes over the row's scores, then every key
// above the threshold and the first krem keys equal to it. Called by every thread with the same b1 and krem. The three
// passes are one loop (pass 0: second digit of bin b1's keys; pass 1: third digit of prefix p2; pass 2: keys above
// and equal to the threshold T into the two bitmaps), so the score read, possibly a recompute from the table, is
// emitted once.
template <int THREADS>
__device__ __forceinline__ void radix_bitmap(const ListRow& r, const ListLds& L, uint32_t b1, uint32_t krem) {
    const int tid = threadIdx.x;
    uint32_t prefix = b1;   // pass 0: the first digit; pass 1: the first two (p2); pass 2: the threshold key T
#pragma unroll 1
    for (int pass = 0; pass < 3; ++pass) {
        for (int c0 = (r.lo & ~7) + 8 * tid; c0 < r.hi; c0 += 8 * THREADS) {
            float v[8];
            r.scores.group8(c0, v);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int c = c0 + i;
                if (c < r.lo || c >= r.hi) continue;
                const uint32_t key = score_key(v[i]), m = (uint32_t)(c - r.lo);
                if (pass == 0) {
                    if ((key >> kHistShift) == prefix) atomicAdd(&L.hist2[(key >> 10) & 2047u], 1u);
                } else if (pass == 1) {
                    if ((key >> 10) == prefix) atomicAdd(&L.hist3[key & 1023u], 1u);
                } else if (key > prefix) {   // both bitmaps start zeroed (the first round trip cleared them)
                    atomicOr(&L.bits[m >> 5], 1u << (m & 31u));
                } else if (key == prefix) {
                    atomicOr(&L.ties[m >> 5], 1u << (m & 31u));
                }
            }
        }
        __syncthreads();
        if (pass == 0) {
            wave0_find_digit(L.misc + 1, L.hist2, krem, 2048);
            prefix = (b1 << 11) | (L.misc[1] & 2047u);
        } else if (pass == 1) {
            wave0_find_digit(L.misc + 1, L.hist3, krem, 1024);
            prefix = (prefix << 10) | (L.misc[1] & 1023u);
        }
        krem = pass < 2 ? L.misc[2] : krem;
    }
    take_ties<THREADS>(L, krem);
}

// The selection bitmap of one row (in L.bits, complete and synchronised on return). SLOTS: entries per lane loaded
// in the first round trip (the first 64 << r.lspl entries of each of the wave's first SLOTS >> r.lspl lists; later
// entries and lists are read afterwards). MAXSUB (4 or 8): the most sub-tiles per score workgroup this instance reads
// for an incomplete list (r.nsub <= MAXSUB). Called by every thread of the workgroup.
template <int THREADS, int SLOTS, int MAXSUB>
__device__ __forceinline__ void list_select_bitmap(const ListRow& r, const ListLds& L) {
    static_assert(MAXSUB == 4 || MAXSUB == 8, "sub-tiles are read four at a time");
    constexpr int kWaves = THREADS / 64;
    constexpr int W = kListWords / THREADS;
    static_assert(SLOTS % 8 == 0, "slots are taken in passes of 8");
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nt = r.tiles;
    const int spl = 1 << r.lspl;
    // round trip 1: bins, this wave's super-bins, the headers, the lists' first entries
    uint32_t hb[kHistBins / THREADS];
#pragma unroll
    for (int i = 0; i < kHistBins / THREADS; ++i) hb[i] = r.state[tid + THREADS * i];
    const uint32_t sbv = r.state[kHistBins + (kSuperBins - 1 - lane)];
    uint2 hv[(kListMaxTiles + THREADS - 1) / THREADS];
#pragma unroll
    for (int i = 0; i < (kListMaxTiles + THREADS - 1) / THREADS; ++i) {
        const int w = tid + THREADS * i;
        hv[i] = w < nt ? r.hdr[w] : make_uint2(0u, 0u);
    }
    uint2 e[SLOTS];
#pragma unroll
    for (int u = 0; u < SLOTS; ++u) {
        const int w = wave + kWaves * (u >> r.lspl), j = 64 * (u & (spl - 1)) + lane;
        e[u] = w < nt && j < r.cap ? r.entries[(size_t)w * r.cap + j] : make_uint2(0u, 0u);
    }
#pragma unroll
    for (int i = 0; i < kHistBins / THREADS; ++i) L.hist[tid + THREADS * i] = hb[i];
#pragma unroll
    for (int i = 0; i < (kListMaxTiles + THREADS - 1) / THREADS; ++i)
        if (tid + THREADS * i < nt) L.hdr[tid + THREADS * i] = hv[i];
#pragma unroll
    for (int i = 0; i < 2048 / THREADS; ++i) L.hist2[tid + THREADS * i] = 0u;
#pragma unroll
    for (int i = 0; i < 1024 / THREADS; ++i) L.hist3[tid + THREADS * i] = 0u;
#pragma unroll
    for (int i = 0; i < W; ++i) {
        L.bits[tid * W + i] = 0u;
        L.ties[tid * W + i] = 0u;
    }
    if (tid < 64) L.sup2[tid] = 0u;
    if (tid < 4) L.misc[tid] = 0u;   // candidate count; a search's defaults keep later indices in range
    __syncthreads();
    uint32_t above, nb1;
    const uint32_t b1 = wave_first_digit(sbv, L.hist, (uint32_t)r.k, above, nb1);
    uint32_t krem = (uint32_t)r.k - above;
    if (nb1 > (uint32_t)kListCandCap) {   // the same test in every wave
        radix_bitmap<THREADS>(r, L, b1, krem);
        return;
    }
    const uint32_t M = (uint32_t)r.M;
    // keys of one pass (n per lane, ok bits): above b1 into the bitmap, bin b1 counted (second digit) and appended
    auto take = [&](const uint32_t* idx, const uint32_t* key, uint32_t ok, int n) {
        uint32_t cm = 0u;
        for (int i = 0; i < n; ++i) {
            const uint32_t ix = min(idx[i], M - 1u);   // in range for any list contents
            const uint32_t dg = key[i] >> kHistShift;
            const bool v = (ok >> i) & 1u;
            if (v && dg > b1) atomicOr(&L.bits[ix >> 5], 1u << (ix & 31u));
            if (v && dg == b1) {
                cm |= 1u << i;
                const uint32_t d2 = (key[i] >> 10) & 2047u;
                atomicAdd(&L.hist2[d2], 1u);
                atomicAdd(&L.sup2[d2 >> 5], 1u);
            }
        }
        const uint32_t nc = (uint32_t)__popc(cm);
        const uint32_t inc = wave_incl_scan(nc);
        const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)inc, 63);
        if (tot == 0) return;
        uint32_t base = 0u;
        if (lane == 63) base = atomicAdd(&L.misc[0], tot);
        uint32_t off = (uint32_t)__builtin_amdgcn_readlane((int)base, 63) + inc - nc;
        for (int i = 0; i < n; ++i) {
            if ((cm >> i) & 1u) {
                if (off < (uint32_t)kListCandCap)
                    L.cand[off] = make_uint2(min(idx[i], M - 1u), key[i] & ((1u << kHistShift) - 1u));
                ++off;
            }
        }
    };
    // step 2: the slots of the first round trip, then what they did not cover
    {
        uint32_t idx[SLOTS], key[SLOTS];
        uint64_t okw = 0u;
#pragma unroll
        for (int u = 0; u < SLOTS; ++u) {
            const int w = wave + kWaves * (u >> r.lspl), jj = u & (spl - 1);
            const uint2 h = w < nt ? L.hdr[w] : make_uint2(0xffffffffu, 0u);
            const bool complete = h.x <= b1 && h.y <= (uint32_t)r.cap;
            idx[u] = e[u].x;
            key[u] = e[u].y;
            okw |= (uint64_t)(complete && (uint32_t)(64 * jj + lane) < h.y) << u;
        }
#pragma unroll
        for (int u0 = 0; u0 < SLOTS; u0 += 8) take(idx + u0, key + u0, (uint32_t)(okw >> u0) & 0xffu, 8);
    }
    for (int w = wave, i = 0; w < nt; w += kWaves, ++i) {
        const uint2 h = L.hdr[w];
        if (h.x <= b1 && h.y <= (uint32_t)r.cap) {
            const uint2* ep = r.entries + (size_t)w * r.cap;
            // entries past the first round trip (h.y <= cap)
            for (int j0 = i < (SLOTS >> r.lspl) ? 64 * spl : 0; j0 < (int)h.y; j0 += 512) {
                uint32_t idx[8], key[8], ok = 0u;
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const int j = j0 + 64 * u + lane;
                    const uint2 v = j < (int)h.y ? ep[j] : make_uint2(0u, 0u);
                    idx[u] = v.x;
                    key[u] = v.y;
                    ok |= (uint32_t)(j < (int)h.y) << u;
                }
                take(idx, key, ok, 8);
            }
        } else if (!r.scores.srow) {
            // an incomplete list whose scores were not stored: its tile is recomputed by every thread below
        } else {
            // an incomplete list: the tile's stored scores, lane -> 8 consecutive columns of each sub-tile, four
            // sub-tiles' loads issued before the first is used
            const float* srow = r.scores.srow;
            const int cb = (r.lo & ~7) + w * 512 + lane * 8;
#pragma unroll
            for (int sb = 0; sb < MAXSUB; sb += 4) {
                if (sb >= r.nsub) break;
                float v[4][8];
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const int c = cb + (sb + s) * nt * 512 + i;
                        v[s][i] = sb + s < r.nsub && c >= r.lo && c < r.hi ? srow[c - r.lo] : 0.0f;
                    }
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    if (sb + s >= r.nsub) break;
                    uint32_t idx[8], key[8], ok = 0u;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const int c = cb + (sb + s) * nt * 512 + i;
                        key[i] = score_key(v[s][i]);
                        idx[i] = (uint32_t)(c - r.lo);
                        ok |= (uint32_t)(c >= r.lo && c < r.hi) << i;
                    }
                    take(idx, key, ok, 8);
                }
            }
        }
    }
    if (!r.scores.srow) {
        // The tiles of the incomplete lists, recomputed from the index table by the whole workgroup: a wave takes 64
        // groups of 8 columns at a time (group q: list = the (q / (64 nsub))-th incomplete one, sub-tile
        // (q / 64) % nsub, columns 8 (q % 64) .. + 8 of it). Every wave reads the same headers, so the lists agree.
        const uint2 h0 = lane < nt ? L.hdr[lane] : make_uint2(0u, 0u);
        const uint2 h1 = lane + 64 < nt ? L.hdr[lane + 64] : make_uint2(0u, 0u);
        const uint64_t f0 = __ballot(lane < nt && (h0.x > b1 || h0.y > (uint32_t)r.cap));
        const uint64_t f1 = __ballot(lane + 64 < nt && (h1.x > b1 || h1.y > (uint32_t)r.cap));
        const int nf = __popcll(f0) + __popcll(f1);
        const int items = nf * r.nsub * 64;
        for (int q0 = 64 * wave; q0 < items; q0 += 64 * kWaves) {
            const int q = q0 + lane;
            float v[8];
            int c0 = 0;
            if (q < items) {
                int nth = q / (64 * r.nsub);   // the nth incomplete list (its number: the nth set bit of f0, f1)
                uint64_t m = f0;
                int base = 0;
                if (nth >= __popcll(f0)) {
                    nth -= __popcll(f0);
                    m = f1;
                    base = 64;
                }
                for (; nth > 0; --nth) m &= m - 1;
                const int wl = base + __ffsll((unsigned long long)m) - 1;
                const int sb = (q / 64) % r.nsub;
                c0 = (r.lo & ~7) + (sb * nt + wl) * 512 + (q % 64) * 8;
            }
            if (q < items && c0 < r.hi) {
                r.scores.group8(c0, v);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = 0.0f;
            }
            uint32_t idx[8], key[8], ok = 0u;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int c = c0 + i;
                key[i] = score_key(v[i]);
                idx[i] = (uint32_t)(c - r.lo);
                ok |= (uint32_t)(q < items && c >= r.lo && c < r.hi) << i;
            }
            take(idx, key, ok, 8);
        }
    }
    __syncthreads();
    // step 3: the second digit over every key of bin b1, found by every wave on its own as b1 was
    uint32_t above2, n2;
    const uint32_t d2 = wave_first_digit(L.sup2[63 - lane], L.hist2, krem, above2, n2);
    krem -= above2;
    const uint32_t nc = min(L.misc[0], (uint32_t)kListCandCap);
    if (n2 == krem) {
        // bin d2 holds exactly the keys still to take: every candidate whose second digit is d2 or above
        for (uint32_t j = tid; j < nc; j += THREADS) {
            const uint2 c = L.cand[j];
            if ((c.y >> 10) >= d2) atomicOr(&L.bits[c.x >> 5], 1u << (c.x & 31u));
        }
        __syncthreads();
        return;
    }
    for (uint32_t j = tid; j < nc; j += THREADS) {
        const uint2 c = L.cand[j];
        if ((c.y >> 10) == d2) atomicAdd(&L.hist3[c.y & 1023u], 1u);
    }
    __syncthreads();
    wave0_find_digit(L.misc + 1, L.hist3, krem, 1024);
    const uint32_t tlow = (d2 << 10) | (L.misc[1] & 1023u);
    krem = L.misc[2];
    if (L.misc[3] <= krem) {
        // every key equal to the threshold is taken
        for (uint32_t j = tid; j < nc; j += THREADS) {
            const uint2 c = L.cand[j];
            if (c.y >= tlow) atomicOr(&L.bits[c.x >> 5], 1u << (c.x & 31u));
        }
        __syncthreads();
        return;
    }
    for (uint32_t j = tid; j < nc; j += THREADS) {
        const uint2 c = L.cand[j];
        if (c.y > tlow) atomicOr(&L.bits[c.x >> 5], 1u << (c.x & 31u));
        else if (c.y == tlow) atomicOr(&L.ties[c.x >> 5], 1u << (c.x & 31u));
    }
    __syncthreads();
    take_ties<THREADS>(L, krem);
}

}  // namespace attnlab
