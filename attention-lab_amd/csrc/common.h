// Device helpers shared by the gfx950 kernels: 16-bit float unpacking, RNE packing, wave64 cross-lane sums and
// the per-thread error slot of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attnlab.h"

namespace attnlab {

// ---------------------------------------------------------------------------------------------------------------
// 16-bit floats. bf16 is the top half of an fp32, so unpacking is a shift or a mask; a 32-bit word holds the element
// at the lower address in its low half.
// ---------------------------------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 with round-to-nearest-even; NaN stays a (quiet) NaN and infinities stay infinite.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u) {
        const uint16_t top = (uint16_t)(u >> 16);
        return (u & 0x007fffffu) ? (uint16_t)(top | 0x0040u) : top;
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t x) { return (float)__builtin_bit_cast(_Float16, x); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// a.lo*b.lo + a.hi*b.hi + c on packed bf16 pairs (v_dot2_f32_bf16), fp32 accumulate.
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

// ---------------------------------------------------------------------------------------------------------------
// Cross-lane moves. DPP controls: quad_perm [1,0,3,2] = 0xB1 (xor 1), [2,3,0,1] = 0x4E (xor 2),
// row_half_mirror = 0x141 (lane i <-> 7-i inside each group of 8), row_ror:8 = 0x128 (xor 8 inside a row of 16).
// ---------------------------------------------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Sum over each aligned group of 8 lanes; every lane of the group receives the total.
__device__ __forceinline__ float sum8(float x) {
    x += dpp_f32<0xB1>(x);
    x += dpp_f32<0x4E>(x);
    x += dpp_f32<0x141>(x);
    return x;
}

// x shifted across lanes by DPP control CTRL; lanes whose source is outside the row (or whose row is masked off by
// ROW_MASK) read 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_u32_or_zero(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROW_MASK, 0xf, true);
}

// Inclusive prefix sum within each row of 16 lanes (row_shr 1, 2, 4, 8).
__device__ __forceinline__ uint32_t row16_incl_scan(uint32_t x) {
    x += dpp_u32_or_zero<0x111, 0xf>(x);
    x += dpp_u32_or_zero<0x112, 0xf>(x);
    x += dpp_u32_or_zero<0x114, 0xf>(x);
    x += dpp_u32_or_zero<0x118, 0xf>(x);
    return x;
}

// Inclusive prefix sum over the 64 lanes of a wave: the row scans, then row_bcast:15 carries row 0's (row 2's) total
// into row 1 (row 3), and row_bcast:31 carries the lower half's total into rows 2 and 3. Six DPP adds, no LDS.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x) {
    x = row16_incl_scan(x);
    x += dpp_u32_or_zero<0x142, 0xa>(x);
    x += dpp_u32_or_zero<0x143, 0xc>(x);
    return x;
}

__device__ __forceinline__ float shfl_xor_f32(float x, int mask) { return __shfl_xor(x, mask, 64); }

// exp2 on the hardware transcendental unit (v_exp_f32); exp2(-inf) = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Workgroups of a launch are dealt to MI355X's 8 XCDs round robin (workgroup b runs on XCD b % 8), each with its own
// L2. This renumbers them so that XCD x gets the contiguous logical range [x * n / 8, (x + 1) * n / 8) when the grid
// size n is a multiple of 8: kernels that split the same rows the same way then touch a row's data from one XCD.
__device__ __forceinline__ int xcd_contiguous_block() {
    const int b = blockIdx.x, n = gridDim.x;
    return (n & 7) == 0 ? (b & 7) * (n >> 3) + (b >> 3) : b;
}

constexpr float kLog2e = 1.4426950408889634f;

}  // namespace attnlab

// ---------------------------------------------------------------------------------------------------------------
// Host side: the per-thread error message behind attnlab_last_error() and the argument-check macros.
// ---------------------------------------------------------------------------------------------------------------
namespace attnlab {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
}  // namespace attnlab

#define ATTNLAB_REQUIRE(cond, ...)                                  \
    do {                                                            \
        if (!(cond)) return ::attnlab::set_error(ATTNLAB_EINVAL, __VA_ARGS__); \
    } while (0)
