// Pieces shared by the score and select kernels: the order-preserving score key and the first radix digit, whose
// per-row histogram the score kernel builds for the select kernel in the fused decode step.
#pragma once

#include "common.h"

namespace attnlab {

constexpr int kHistBits = 11;                 // first digit: sign, exponent and the top two mantissa bits
constexpr int kHistBins = 1 << kHistBits;
constexpr int kHistShift = 32 - kHistBits;
// Per-row select state shared by the score and select kernels: the first-digit histogram (kHistBins words), then
// kSuperBins counts of 32 consecutive bins each (so the threshold's first digit is found from 64 + 32 words instead of
// 2048). Zero before the first call; the select leaves it zero.
constexpr int kSuperBins = kHistBins / 32;
constexpr int kSelectStateWords = kHistBins + kSuperBins;
static_assert(kSelectStateWords == 2112, "ABI: ATTNLAB_SELECT_STATE_WORDS");

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

// The argument checks of attnlab_select_rows (the decode step runs them before its first launch, so a rejected call
// leaves the select state untouched).
int select_check(int B, int G, int lo, int hi, int legal, int k, int C, int order, const int32_t* rows,
                 int64_t rows_stride, const float* scores, int64_t score_stride);

// attnlab_select_rows: `state` [B*G][kSelectStateWords] (nullable) holds the first-digit histograms the score kernel
// built; with it and a scratch of select_scratch_bytes(B*G, M, k, order) the select runs tiled over the chip.
int select_rows_impl(const float* scores, int64_t score_stride, int B, int G, int lo, int hi, int legal, int k, int C,
                     int order, int32_t* rows, int64_t rows_stride, int64_t* rows_flat, uint32_t* state,
                     void* scratch, int64_t scratch_bytes, hipStream_t stream);

// Scratch bytes of the tiled select for R rows of M candidates, plus the score-order sort's buffers when order is
// score order and k exceeds what the LDS sort holds (no zeroing needed).
int64_t select_scratch_bytes(int R, int M, int k, int order);

// attnlab_score_grouped with an optional select-state output: per row, the first-digit histogram of the scores.
int score_grouped_impl(uint16_t* zT, const uint16_t* k_new, const uint16_t* wk, const uint16_t* q_cat,
                       const uint16_t* wq_t, const float* u_in, float* u_out, float* out, int64_t out_stride, int B,
                       int G, int r, int C, int d, int hd, int lo, int hi, int write_col, int vector, uint32_t* hist,
                       hipStream_t stream);

// attnlab_score_grouped_f32: the same score on float32 tables (trained index banks); two launches (prologue, scan).
int score_grouped_f32_impl(float* zT, const float* k_new, const float* wk, const float* q_cat, const float* wq_t,
                           const float* u_in, float* u_out, float* out, int64_t out_stride, int B, int G, int r,
                           int C, int d, int hd, int lo, int hi, int write_col, uint32_t* hist, hipStream_t stream);

}  // namespace attnlab
