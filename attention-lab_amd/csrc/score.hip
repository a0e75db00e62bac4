// Index score kernels for gfx950.
//
// Grouped (parity) mode, the reference's indexer (src/attention_lab/indexer.py:15-29, metal_score.py:44-246):
// one launch per decode step writes the z column of the newest key, builds u = q_cat . wq_t in fp32 and scans the
// candidate columns of the transposed index table zT [B,G,r,C]. The table is column-contiguous for each j, so a
// lane owns 8 adjacent columns and streams them with one 16-byte load per j (32 loads for r = 32): every wave load
// is a 1 KiB contiguous run of HBM. The loads are issued before u is built, so the prologue (16-32 KiB of weights,
// L2-resident after the first block) hides under the HBM latency instead of adding to it.
//
// Lightning mode (the north_star generalisation; no reference kernel): keys are stored one r-vector per position
// [B,KG,Lk,r] (64 bytes of fp16/bf16 per position), four lanes share a position with 16 bytes each, the per-head
// partial dot products of a quad's four keys are reduced and transposed with two DPP steps, and ReLU and the head
// weights are applied in fp32.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "select.h"

namespace attnlab {

struct ScoreArgs {
    uint16_t* zT;           // [BG, r, C]
    const uint16_t* k_new;  // [BG, d] or null
    const uint16_t* wk;     // [G, r, d]
    const uint16_t* q_cat;  // [BG, hd]
    const uint16_t* wq_t;   // [G, hd, r]
    const float* u_in;      // [BG, r] or null
    float* u_out;           // [BG, r] or null
    float* out;             // row bg at out + bg * out_stride
    int64_t out_stride;
    int G, r, C, d, hd, lo, M, write_col;
    int tiles;              // column tiles per (b, g) row
    uint32_t* hist;         // [BG, kSelectStateWords] select state: first-digit histogram bins first, or null
    ScoreLists lists;       // per-workgroup key lists (entries null: none; score_scan_fused only)
    uint32_t* sink = nullptr;   // score_scan_fused<NSUB, true> (the read probe): one folded word per thread
};

constexpr int kMaxR = 32;
constexpr int kMaxHd = 1024;   // q_cat features (h * d, h <= 8) whose u loads are all issued at once

// u[j] = sum_f q_cat[f] * wq_t[f, j] for one (b, g), reduced into u_sh[0..r). Uses `red` (BLOCK/64 x 32 floats).
template <int BLOCK>
__device__ __forceinline__ void build_u(const ScoreArgs& a, int bg, int g, float* u_sh, float* red) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint16_t* q = a.q_cat + (size_t)bg * a.hd;
    const uint16_t* w = a.wq_t + (size_t)g * a.hd * a.r;
    if (a.r == 32) {
        // thread -> (feature stride BLOCK/4, j slice of 8): one 16-byte load covers 8 consecutive j of one feature.
        // Up to kMaxHd features the loads of all iterations are issued before the first multiply (one memory round
        // trip instead of one per feature row).
        constexpr int kIter = kMaxHd / (BLOCK / 4);
        const int js = tid & 3;
        float acc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
        if (a.hd <= kMaxHd) {
            uint4 wv[kIter];
            float qf[kIter];
#pragma unroll
            for (int it = 0; it < kIter; ++it) {
                const int f = (tid >> 2) + it * (BLOCK / 4);
                wv[it] = make_uint4(0, 0, 0, 0);
                qf[it] = 0.0f;
                if (f < a.hd) {
                    wv[it] = *reinterpret_cast<const uint4*>(w + (size_t)f * 32 + js * 8);
                    qf[it] = bf16_to_f32(q[f]);
                }
            }
#pragma unroll
            for (int it = 0; it < kIter; ++it) {
                acc[0] += qf[it] * bf16_lo(wv[it].x); acc[1] += qf[it] * bf16_hi(wv[it].x);
                acc[2] += qf[it] * bf16_lo(wv[it].y); acc[3] += qf[it] * bf16_hi(wv[it].y);
                acc[4] += qf[it] * bf16_lo(wv[it].z); acc[5] += qf[it] * bf16_hi(wv[it].z);
                acc[6] += qf[it] * bf16_lo(wv[it].w); acc[7] += qf[it] * bf16_hi(wv[it].w);
            }
        } else {
            for (int f = tid >> 2; f < a.hd; f += BLOCK / 4) {
                const float qv = bf16_to_f32(q[f]);
                const uint4 wl = *reinterpret_cast<const uint4*>(w + (size_t)f * 32 + js * 8);
                acc[0] += qv * bf16_lo(wl.x); acc[1] += qv * bf16_hi(wl.x);
                acc[2] += qv * bf16_lo(wl.y); acc[3] += qv * bf16_hi(wl.y);
                acc[4] += qv * bf16_lo(wl.z); acc[5] += qv * bf16_hi(wl.z);
                acc[6] += qv * bf16_lo(wl.w); acc[7] += qv * bf16_hi(wl.w);
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float v = acc[i];
            v += shfl_xor_f32(v, 4);
            v += shfl_xor_f32(v, 8);
            v += shfl_xor_f32(v, 16);
            v += shfl_xor_f32(v, 32);
            acc[i] = v;
        }
        if (lane < 4) {
#pragma unroll
            for (int i = 0; i < 8; ++i) red[wave * 32 + lane * 8 + i] = acc[i];
        }
    } else {
        // general r <= 32: thread -> (j = tid % 32, feature stride BLOCK/32)
        const int j = tid & 31;
        float acc = 0.0f;
        if (j < a.r)
            for (int f = tid >> 5; f < a.hd; f += BLOCK / 32) acc += bf16_to_f32(q[f]) * bf16_to_f32(w[(size_t)f * a.r + j]);
        acc += shfl_xor_f32(acc, 32);
        if (lane < 32) red[wave * 32 + lane] = acc;
    }
    __syncthreads();
    if (tid < 32) {
        float s = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < BLOCK / 64; ++w2) s += red[w2 * 32 + tid];
        u_sh[tid] = (tid < a.r) ? s : 0.0f;
        if (a.u_out && tid < a.r) a.u_out[(size_t)bg * a.r + tid] = s;
    }
}

// z column of the newest key: zT[bg, j, write_col] = bf16_rne(wk[g, j, :] . k_new[bg, :]); 8 lanes per j. For d = 128
// and 16-byte aligned rows each lane reads its 16 elements of wk and k_new with four 16-byte loads.
template <int BLOCK>
__device__ __forceinline__ void write_z(const ScoreArgs& a, int bg, int g) {
    const int tid = threadIdx.x;
    const uint16_t* kn = a.k_new + (size_t)bg * a.d;
    if (a.d == 128 && a.r <= BLOCK / 8 && ((reinterpret_cast<uintptr_t>(a.wk) | reinterpret_cast<uintptr_t>(kn)) & 15) == 0) {
        const int j = tid >> 3, e0 = (tid & 7) * 16;
        uint4 w0 = make_uint4(0u, 0u, 0u, 0u), w1 = w0, k0 = w0, k1 = w0;
        if (j < a.r) {
            const uint16_t* wr = a.wk + ((size_t)g * a.r + j) * 128 + e0;
            w0 = *reinterpret_cast<const uint4*>(wr);
            w1 = *reinterpret_cast<const uint4*>(wr + 8);
            k0 = *reinterpret_cast<const uint4*>(kn + e0);
            k1 = *reinterpret_cast<const uint4*>(kn + e0 + 8);
        }
        const float s = z_dot16(w0, w1, k0, k1);
        if ((tid & 7) == 0 && j < a.r) a.zT[((size_t)bg * a.r + j) * a.C + a.write_col] = f32_to_bf16_rne(s);
        return;
    }
    for (int j0 = 0; j0 < a.r; j0 += BLOCK / 8) {
        const int j = j0 + (tid >> 3);
        float s = 0.0f;
        if (j < a.r) {
            const uint16_t* wr = a.wk + ((size_t)g * a.r + j) * a.d;
            for (int e = tid & 7; e < a.d; e += 8) s += bf16_to_f32(wr[e]) * bf16_to_f32(kn[e]);
        }
        s = sum8(s);
        if ((tid & 7) == 0 && j < a.r) a.zT[((size_t)bg * a.r + j) * a.C + a.write_col] = f32_to_bf16_rne(s);
    }
}

// 8-byte-load scan: thread -> 4 adjacent columns starting at a 4-aligned column, 32 non-temporal 8-byte loads (the
// table is read once per step, so it should not displace reused lines from the caches). A 256-thread block covers 1024
// columns. Four columns per thread keeps the register count low enough for 4+ waves per SIMD; measured on MI355X at
// B=16, L=32K it streams the table faster than 8 columns per thread with 16-byte loads (5.9 vs 5.3 TB/s). Columns of
// the aligned group outside [lo, hi) are loaded (inside the row since C % 4 == 0) but never stored. With u_in the
// block only stages u; otherwise it builds u itself (the single-launch form) while the table loads are in flight.
template <int BLOCK>
__global__ __launch_bounds__(BLOCK) void score_scan_vec(ScoreArgs a) {
    __shared__ float u_sh[32];
    __shared__ float red[(BLOCK / 64) * 32];
    __shared__ __attribute__((aligned(16))) uint32_t hsh[kHistBins];
    const int bg = blockIdx.x / a.tiles;
    const int tile = blockIdx.x - bg * a.tiles;
    const int g = bg % a.G;
    const int tid = threadIdx.x;
    const int lo = a.lo, hi = a.lo + a.M;
    const int c0 = (lo & ~3) + (tile * BLOCK + tid) * 4;
    const bool active = a.M > 0 && c0 < hi;
    const uint16_t* col = a.zT + (size_t)bg * a.r * a.C + c0;

    u32x2_t v[kMaxR];
    if (active) {
#pragma unroll
        for (int j = 0; j < kMaxR; ++j)
            if (j < a.r) v[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(col + (size_t)j * a.C));
    }
    if (a.hist) clear_histogram<BLOCK>(hsh);
    if (a.u_in) {
        if (tid < 32) u_sh[tid] = tid < a.r ? a.u_in[(size_t)bg * a.r + tid] : 0.0f;
    } else {
        build_u<BLOCK>(a, bg, g, u_sh, red);
    }
    if (tile == 0 && a.k_new) write_z<BLOCK>(a, bg, g);
    __syncthreads();

    if (active) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < kMaxR; ++j) {
            if (j < a.r) {
                const float u = u_sh[j];
                acc[0] += u * bf16_lo(v[j].x);
                acc[1] += u * bf16_hi(v[j].x);
                acc[2] += u * bf16_lo(v[j].y);
                acc[3] += u * bf16_hi(v[j].y);
            }
        }
        float* o = a.out + (size_t)bg * a.out_stride - lo;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = c0 + i;
            if (c >= lo && c < hi) {
                o[c] = acc[i];
                if (a.hist) atomicAdd(&hsh[score_key(acc[i]) >> kHistShift], 1u);
            }
        }
    }
    if (a.hist) flush_histogram<BLOCK>(hsh, a.hist, bg);
}

// 16-byte-load scan with the index dimension split over the waves (u given): wave w of a 256-thread block reads j in
// [8w, 8w + 8) of 512 columns, lane -> 8 adjacent columns, so every load instruction reads 1 KiB of one table row and
// each thread issues eight 16-byte loads (128 bytes, the per-thread amount at which MI355X streams fastest). The four
// waves' partial sums meet in LDS; thread t then stores and histograms columns 2t and 2t + 1. Measured on MI355X at
// L = 32K: 47.6 us at B = 16 (6.0 TB/s with the score writes) against 51.1 us for the 8-byte scan, 4.7 against 5.7 us
// at B = 1; splitting j over the 16-lane rows of each wave instead (four table rows per load instruction) ran at a
// third of the speed at B = 1. Needs C % 8 == 0 and a 16-byte aligned table: the loaded groups of 8 columns then never
// leave the row.
template <int BLOCK>
__global__ __launch_bounds__(BLOCK) void score_scan_v16(ScoreArgs a) {
    static_assert(BLOCK == 256, "four waves of eight table rows");
    constexpr int kCols = 512;
    __shared__ float u_sh[32];
    __shared__ __attribute__((aligned(16))) uint32_t hsh[kHistBins];
    __shared__ __attribute__((aligned(16))) float part[4][kCols];
    const int lin = xcd_contiguous_block();   // a row's tiles on one XCD, which also selects from the row
    const int bg = lin / a.tiles;
    const int tile = lin - bg * a.tiles;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lo = a.lo, hi = a.lo + a.M;
    const int cb = (lo & ~7) + tile * kCols;
    const int c0 = cb + lane * 8;
    const bool active = c0 < hi;
    const uint16_t* col = a.zT + (size_t)bg * a.r * a.C + c0;

    u32x4_t v[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
        const int j = 8 * wave + jj;
        v[jj] = (u32x4_t){0u, 0u, 0u, 0u};
        if (active && j < a.r) v[jj] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(col + (size_t)j * a.C));
    }
    if (a.hist) clear_histogram<BLOCK>(hsh);
    if (tid < 32) u_sh[tid] = tid < a.r ? a.u_in[(size_t)bg * a.r + tid] : 0.0f;
    __syncthreads();

    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
        const float u = u_sh[8 * wave + jj];
        acc[0] += u * bf16_lo(v[jj].x);
        acc[1] += u * bf16_hi(v[jj].x);
        acc[2] += u * bf16_lo(v[jj].y);
        acc[3] += u * bf16_hi(v[jj].y);
        acc[4] += u * bf16_lo(v[jj].z);
        acc[5] += u * bf16_hi(v[jj].z);
        acc[6] += u * bf16_lo(v[jj].w);
        acc[7] += u * bf16_hi(v[jj].w);
    }
    float4* pw = reinterpret_cast<float4*>(&part[wave][lane * 8]);
    pw[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    pw[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
    __syncthreads();
    const int cc = 2 * tid;
    const float2 p0 = *reinterpret_cast<const float2*>(&part[0][cc]);
    const float2 p1 = *reinterpret_cast<const float2*>(&part[1][cc]);
    const float2 p2 = *reinterpret_cast<const float2*>(&part[2][cc]);
    const float2 p3 = *reinterpret_cast<const float2*>(&part[3][cc]);
    const float s0 = (p0.x + p1.x) + (p2.x + p3.x), s1 = (p0.y + p1.y) + (p2.y + p3.y);
    float* o = a.out + (size_t)bg * a.out_stride - lo;
    const int c = cb + cc;
    if (c >= lo && c < hi) {
        o[c] = s0;
        if (a.hist) atomicAdd(&hsh[score_key(s0) >> kHistShift], 1u);
    }
    if (c + 1 >= lo && c + 1 < hi) {
        o[c + 1] = s1;
        if (a.hist) atomicAdd(&hsh[score_key(s1) >> kHistShift], 1u);
    }
    if (a.hist) flush_histogram<BLOCK>(hsh, a.hist, bg);
}

// The v16 scan with the prologue folded in (r = 32, q_cat features hd <= 512, 16-byte aligned operands): one launch per
// step instead of two, which saves a kernel boundary (a few microseconds of launch, drain and cache maintenance on
// MI355X, more than the prologue's own work). Wave w needs u[j] only for its own j in [8w, 8w + 8): it reads those 8
// weights of every q_cat feature (one 16-byte load per feature, 8 KB per wave, L2-resident) just before its first
// table loads, and reduces them in registers (DPP within rows of 16 lanes, then readlane) while the table is in
// flight, so u costs no barrier. A workgroup covers NSUB 512-column sub-tiles of its row, `tiles` sub-tiles apart,
// double-buffered (the loads of sub-tile s + 1 are issued before sub-tile s is reduced), which spreads the weight reads
// and the histogram flush over NSUB sub-tiles.
// The workgroup of tile 0 also writes the z column and, when asked, u.
// PROBE (measurement only, attnlab_scan_probe): the same grid, prologue, loads and pipeline, but every loaded word is
// XOR-folded instead of multiplied, and nothing is reduced, counted, listed or stored beyond one word per thread.
template <int NSUB, bool PROBE = false>
__global__ __launch_bounds__(256) void score_scan_fused(ScoreArgs a) {
    constexpr int kCols = 512;
    constexpr int kUIter = 512 / 64;   // q_cat features per lane
    __shared__ __attribute__((aligned(16))) uint32_t hsh[kHistBins];
    __shared__ __attribute__((aligned(16))) float part[4][kCols];
    __shared__ uint32_t lcount[2];   // the key list: entries placed, waves done
    const int lin = xcd_contiguous_block();   // a row's tiles on one XCD, which also selects from the row
    const int bg = lin / a.tiles;
    const int tile = lin - bg * a.tiles;
    const int g = bg % a.G;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lo = a.lo, hi = a.lo + a.M;
    // sub-tile s of workgroup `tile` is the row's 512-column sub-tile s * tiles + tile: at each step the workgroups of a
    // row read one contiguous stretch of every table row, as a grid of one-tile workgroups would
    const int cb0 = (lo & ~7) + tile * kCols;
    const int sstride = a.tiles * kCols;
    const int c_last = (hi - 1) & ~7;   // last 8-column group holding a scanned column (in bounds: C % 8 == 0)
    const uint16_t* zw = a.zT + ((size_t)bg * 32 + 8 * wave) * a.C;

    // Sub-tile s: this lane's 8 columns of the wave's 8 table rows. Groups past the row end re-read the last group
    // (in bounds, results discarded), so every sub-tile issues the same eight loads.
    auto load = [&](int s, u32x4_t (&v)[8]) {
        const int c0 = min(cb0 + s * sstride + lane * 8, c_last);
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
            v[jj] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(zw + (size_t)jj * a.C + c0));
    };
    // u[8 wave + c], c < 8: lane -> features lane + 64 i. The weight loads (L2 hits after the first workgroups) are
    // issued before the table loads: loads retire in issue order, so u can then be built while the table is in flight.
    // Features past hd re-read feature hd - 1 with q = 0 (no branch, so no wait is placed between the loads).
    float u[8];
    // sub-tiles in flight: two ahead at 8 sub-tiles per workgroup (B=16, 32K: 74.5 against 75.2 us per layer in the
    // step, 135 VGPRs and three waves per SIMD), one ahead otherwise (equal or 0.1 us better at 2 and 4)
    constexpr int kDepth = NSUB >= 8 ? 3 : 2;
    u32x4_t vb[kDepth][8];
    // The z column (tile 0) in a grid of at most one workgroup per CU: its loads go out first and its dot products
    // follow u, so that the tile-0 workgroups do not end a memory round trip after the others (B=1, 32K: score 7.45 ->
    // 7.23 us). Larger grids keep it at the end (no gain there; at B=16 the early form cost 0.5 us, and the column spread
    // over the row's workgroups, ceil(32 / tiles) index rows each with the prologue, gained nothing), as do other
    // layouts (write_z).
    const uint16_t* kn = a.k_new ? a.k_new + (size_t)bg * a.d : nullptr;
    const bool z_early = !PROBE && tile == 0 && gridDim.x <= 256 && kn != nullptr && a.d == 128 &&
                         ((reinterpret_cast<uintptr_t>(a.wk) | reinterpret_cast<uintptr_t>(kn)) & 15) == 0;
    {
        const uint16_t* qp = a.q_cat + (size_t)bg * a.hd;
        const uint16_t* wp = a.wq_t + (size_t)g * a.hd * 32 + 8 * wave;
        uint4 zw0, zw1, zk0, zk1;
        if (z_early) {   // thread -> index row tid / 8, dims 16 (tid % 8) .. + 15, as write_z
            const uint16_t* wr = a.wk + ((size_t)g * 32 + (tid >> 3)) * 128 + (tid & 7) * 16;
            zw0 = *reinterpret_cast<const uint4*>(wr);
            zw1 = *reinterpret_cast<const uint4*>(wr + 8);
            zk0 = *reinterpret_cast<const uint4*>(kn + (tid & 7) * 16);
            zk1 = *reinterpret_cast<const uint4*>(kn + (tid & 7) * 16 + 8);
        }
        uint4 wv[kUIter];
        float qf[kUIter];
#pragma unroll
        for (int it = 0; it < kUIter; ++it) {
            const int f = lane + 64 * it;
            const int fc = min(f, a.hd - 1);
            wv[it] = *reinterpret_cast<const uint4*>(wp + (size_t)fc * 32);
            qf[it] = bf16_to_f32(qp[fc]);
            if (f >= a.hd) qf[it] = 0.0f;
        }
        load(0, vb[0]);
        if (kDepth > 2) load(1, vb[1]);
        __builtin_amdgcn_sched_barrier(0);   // keep every load above the first use of a weight
#pragma unroll
        for (int c = 0; c < 8; ++c) u[c] = 0.0f;
#pragma unroll
        for (int it = 0; it < kUIter; ++it) {
            u[0] += qf[it] * bf16_lo(wv[it].x); u[1] += qf[it] * bf16_hi(wv[it].x);
            u[2] += qf[it] * bf16_lo(wv[it].y); u[3] += qf[it] * bf16_hi(wv[it].y);
            u[4] += qf[it] * bf16_lo(wv[it].z); u[5] += qf[it] * bf16_hi(wv[it].z);
            u[6] += qf[it] * bf16_lo(wv[it].w); u[7] += qf[it] * bf16_hi(wv[it].w);
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            float x = sum8(u[c]);
            x += dpp_f32<0x140>(x);   // row_mirror: lane i <-> 15 - i, so the two groups of 8 of each row meet
            const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
            const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
            const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
            const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
            u[c] = (r0 + r1) + (r2 + r3);
        }
        if (z_early) {
            const float z = z_dot16(zw0, zw1, zk0, zk1);
            if ((tid & 7) == 0) a.zT[((size_t)bg * 32 + (tid >> 3)) * a.C + a.write_col] = f32_to_bf16_rne(z);
        }
    }
    if (a.hist) clear_histogram<256>(hsh);
    if (tid < 2) lcount[tid] = 0u;
    __syncthreads();

    if constexpr (PROBE) {
        uint32_t fx = __float_as_uint(u[0]) & 1u;
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
            if (s + kDepth - 1 < NSUB) load(s + kDepth - 1, vb[(s + kDepth - 1) % kDepth]);
            const u32x4_t (&v)[8] = vb[s % kDepth];
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) fx ^= v[jj].x ^ v[jj].y ^ v[jj].z ^ v[jj].w;
        }
        a.sink[(size_t)lin * 256 + tid] = fx;
        return;
    }
    // a.out null (key lists only, the fused step's position order): no score is stored; the list select recomputes
    // the few tiles it needs from the table
    float* o = a.out ? a.out + (size_t)bg * a.out_stride - lo : nullptr;
    uint32_t lkey[2 * NSUB];   // this thread's keys (columns cb0 + s * sstride + 2 tid + e), kept for the list
    uint32_t lvalid = 0u;
#pragma unroll
    for (int s = 0; s < NSUB; ++s) {
        if (s + kDepth - 1 < NSUB) load(s + kDepth - 1, vb[(s + kDepth - 1) % kDepth]);
        const u32x4_t (&v)[8] = vb[s % kDepth];
        float acc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
        // explicit fma chains from zero in row order: rescore8 (the select's recompute) repeats them bit for bit
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            acc[0] = __builtin_fmaf(u[jj], bf16_lo(v[jj].x), acc[0]);
            acc[1] = __builtin_fmaf(u[jj], bf16_hi(v[jj].x), acc[1]);
            acc[2] = __builtin_fmaf(u[jj], bf16_lo(v[jj].y), acc[2]);
            acc[3] = __builtin_fmaf(u[jj], bf16_hi(v[jj].y), acc[3]);
            acc[4] = __builtin_fmaf(u[jj], bf16_lo(v[jj].z), acc[4]);
            acc[5] = __builtin_fmaf(u[jj], bf16_hi(v[jj].z), acc[5]);
            acc[6] = __builtin_fmaf(u[jj], bf16_lo(v[jj].w), acc[6]);
            acc[7] = __builtin_fmaf(u[jj], bf16_hi(v[jj].w), acc[7]);
        }
        float4* pw = reinterpret_cast<float4*>(&part[wave][lane * 8]);
        pw[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
        pw[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
        __syncthreads();
        const int cc = 2 * tid;
        const float2 p0 = *reinterpret_cast<const float2*>(&part[0][cc]);
        const float2 p1 = *reinterpret_cast<const float2*>(&part[1][cc]);
        const float2 p2 = *reinterpret_cast<const float2*>(&part[2][cc]);
        const float2 p3 = *reinterpret_cast<const float2*>(&part[3][cc]);
        const float s0 = (p0.x + p1.x) + (p2.x + p3.x), s1 = (p0.y + p1.y) + (p2.y + p3.y);
        const int c = cb0 + s * sstride + cc;
        lkey[2 * s] = score_key(s0);
        lkey[2 * s + 1] = score_key(s1);
        if (c >= lo && c < hi) {
            if (o) o[c] = s0;
            lvalid |= 1u << (2 * s);
            if (a.hist) atomicAdd(&hsh[lkey[2 * s] >> kHistShift], 1u);
        }
        if (c + 1 >= lo && c + 1 < hi) {
            if (o) o[c + 1] = s1;
            lvalid |= 2u << (2 * s);
            if (a.hist) atomicAdd(&hsh[lkey[2 * s + 1] >> kHistShift], 1u);
        }
        if (s + 1 < NSUB) __syncthreads();   // part is rewritten by the next sub-tile
    }
    if (tile == 0) {
        if (a.k_new && !z_early) write_z<256>(a, bg, g);
        if (a.u_out && lane < 8) {
            float uo = u[0];
#pragma unroll
            for (int c = 1; c < 8; ++c) uo = lane == c ? u[c] : uo;
            a.u_out[(size_t)bg * 32 + 8 * wave + lane] = uo;
        }
    }
    if (a.hist) flush_histogram<256>(hsh, a.hist, bg);
    if (a.lists.entries)
        write_key_list<NSUB>(a.lists, hsh, lcount, lkey, lvalid, (size_t)bg * a.tiles + tile, cb0, sstride, lo);
}

// 2-byte-load scan for tables whose rows are not 16-byte aligned: thread -> 8 adjacent columns from lo, never
// loading at or beyond hi.
template <int BLOCK>
__global__ __launch_bounds__(BLOCK) void score_scan_scalar(ScoreArgs a) {
    __shared__ float u_sh[32];
    __shared__ float red[(BLOCK / 64) * 32];
    __shared__ __attribute__((aligned(16))) uint32_t hsh[kHistBins];
    const int bg = blockIdx.x / a.tiles;
    const int tile = blockIdx.x - bg * a.tiles;
    const int g = bg % a.G;
    const int tid = threadIdx.x;
    const int m0 = (tile * BLOCK + tid) * 8;
    if (a.hist) clear_histogram<BLOCK>(hsh);
    if (a.u_in) {
        if (tid < 32) u_sh[tid] = tid < a.r ? a.u_in[(size_t)bg * a.r + tid] : 0.0f;
    } else {
        build_u<BLOCK>(a, bg, g, u_sh, red);
    }
    if (tile == 0 && a.k_new) write_z<BLOCK>(a, bg, g);
    __syncthreads();
    if (m0 < a.M) {
        const int n = min(8, a.M - m0);
        const uint16_t* col = a.zT + (size_t)bg * a.r * a.C + a.lo + m0;
        float acc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
        for (int j = 0; j < a.r; ++j) {
            const float u = u_sh[j];
            const uint16_t* row = col + (size_t)j * a.C;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (i < n) acc[i] += u * bf16_to_f32(row[i]);
        }
        float* o = a.out + (size_t)bg * a.out_stride + m0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (i < n) {
                o[i] = acc[i];
                if (a.hist) atomicAdd(&hsh[score_key(acc[i]) >> kHistShift], 1u);
            }
        }
    }
    if (a.hist) flush_histogram<BLOCK>(hsh, a.hist, bg);
}

// u and the z column only, one block per (b, g).
__global__ __launch_bounds__(256) void score_prologue(ScoreArgs a) {
    __shared__ float u_sh[32];
    __shared__ float red[4 * 32];
    const int bg = blockIdx.x;
    const int g = bg % a.G;
    build_u<256>(a, bg, g, u_sh, red);
    if (a.k_new) write_z<256>(a, bg, g);
}

// The prologue for r = 32, d = 128, q_cat features hd <= 512 and 16-byte aligned operands, spread over four workgroups
// per (b, g): workgroup `part` computes u[j] and the z entry for j in [8 part, 8 part + 8). One workgroup per (b, g)
// has to stream 41 KB of weights and queries through a single CU, whose outstanding-miss budget, not bandwidth,
// bounds it; a quarter of the weights per CU halves the kernel time.
__global__ __launch_bounds__(256) void score_prologue_split(ScoreArgs a) {
    __shared__ float red[4][8];
    __shared__ float zred[8];
    const int lin = xcd_contiguous_block();   // (b, g) on the XCD that scans its row
    const int bg = lin >> 2, part = lin & 3;
    const int g = bg % a.G;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // u: thread -> features tid and tid + 256 (when below hd), 8 j of this part per feature (one 16-byte load)
    const uint16_t* q = a.q_cat + (size_t)bg * a.hd;
    const uint16_t* w = a.wq_t + (size_t)g * a.hd * 32 + part * 8;
    uint4 wv[2];
    float qf[2];
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int f = tid + it * 256;
        wv[it] = make_uint4(0, 0, 0, 0);
        qf[it] = 0.0f;
        if (f < a.hd) {
            wv[it] = *reinterpret_cast<const uint4*>(w + (size_t)f * 32);
            qf[it] = bf16_to_f32(q[f]);
        }
    }
    // z: thread -> (j = 8 part + tid / 32, elements 4 (tid % 32) .. + 4)
    float zs = 0.0f;
    const int zj = part * 8 + (tid >> 5), ze = (tid & 31) * 4;
    if (a.k_new) {
        const uint16_t* wr = a.wk + ((size_t)g * 32 + zj) * 128 + ze;
        const uint16_t* kn = a.k_new + (size_t)bg * 128 + ze;
        const uint2 w2 = *reinterpret_cast<const uint2*>(wr), k2 = *reinterpret_cast<const uint2*>(kn);
        zs = dot2_bf16(w2.x, k2.x, zs);
        zs = dot2_bf16(w2.y, k2.y, zs);
    }
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        acc[0] += qf[it] * bf16_lo(wv[it].x); acc[1] += qf[it] * bf16_hi(wv[it].x);
        acc[2] += qf[it] * bf16_lo(wv[it].y); acc[3] += qf[it] * bf16_hi(wv[it].y);
        acc[4] += qf[it] * bf16_lo(wv[it].z); acc[5] += qf[it] * bf16_hi(wv[it].z);
        acc[6] += qf[it] * bf16_lo(wv[it].w); acc[7] += qf[it] * bf16_hi(wv[it].w);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float v = acc[i];
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) v += shfl_xor_f32(v, o);
        acc[i] = v;
    }
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) red[wave][i] = acc[i];
    }
    if (a.k_new) {
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) zs += shfl_xor_f32(zs, o);
        if ((tid & 31) == 0) zred[tid >> 5] = zs;
    }
    __syncthreads();
    if (tid < 8) {
        const float u = (red[0][tid] + red[1][tid]) + (red[2][tid] + red[3][tid]);
        a.u_out[(size_t)bg * 32 + part * 8 + tid] = u;
        if (a.k_new)
            a.zT[((size_t)bg * 32 + part * 8 + tid) * a.C + a.write_col] = f32_to_bf16_rne(zred[tid]);
    }
}

// Launch the prologue (u into a.u_out, and the z column when a.k_new is set) over B*G rows.
static void launch_prologue(const ScoreArgs& a, int BG, hipStream_t s) {
    const bool split = a.r == 32 && a.hd <= 512 && a.u_out != nullptr && (a.k_new == nullptr || a.d == 128) &&
                       ((reinterpret_cast<uintptr_t>(a.wq_t) | reinterpret_cast<uintptr_t>(a.wk) |
                         reinterpret_cast<uintptr_t>(a.k_new)) & 15) == 0;
    if (split) hipLaunchKernelGGL(score_prologue_split, dim3(BG * 4), dim3(256), 0, s, a);
    else hipLaunchKernelGGL(score_prologue, dim3(BG), dim3(256), 0, s, a);
}

// ---------------------------------------------------------------------------------------------------------------
// Lightning mode: keys one 32-vector per position, nh index heads, ReLU and per-head weights (see score_lightning).
// ---------------------------------------------------------------------------------------------------------------
struct LightningArgs {
    const uint16_t* keys;  // [BKG, Lk, 32]
    const float* q;        // [BKG, nh, 32]
    const float* w;        // [BKG, nh]
    float* out;
    int64_t out_stride;
    int Lk, nh, lo, M;
    int tiles;             // tiles per row; a tile is 256 * ng keys
    int ng;                // 64-key groups per wave per tile
};

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// a.x * b.x + a.y * b.y + c on packed 16-bit pairs, fp32 accumulate (v_dot2_f32_f16 / v_dot2_f32_bf16)
template <bool F16>
__device__ __forceinline__ float dot2_16(uint32_t a, uint32_t b, float c) {
    if constexpr (F16)
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c, false);
    else
        return dot2_bf16(a, b, c);
}

// (x, y) -> packed 16-bit pair (RNE) and its value back in fp32
template <bool F16>
__device__ __forceinline__ uint32_t pack2_16(float x, float y, float& xr, float& yr) {
    if constexpr (F16) {
        const f16x2_t h = {(_Float16)x, (_Float16)y};
        xr = (float)h.x;
        yr = (float)h.y;
        return __builtin_bit_cast(uint32_t, h);
    } else {
        const uint32_t lo16 = f32_to_bf16_rne(x), hi16 = f32_to_bf16_rne(y);
        xr = bf16_to_f32((uint16_t)lo16);
        yr = bf16_to_f32((uint16_t)hi16);
        return lo16 | (hi16 << 16);
    }
}

__device__ __forceinline__ float relu_f32(float x) { return __int_as_float(max(__float_as_int(x), 0)); }

// Lightning-indexer score, one query per (b, kg) (decode):
//   out[bkg, m] = sum_i w[bkg, i] * act(q[bkg, i, :] . key[bkg, lo + m, :])
// HBM-bound: 64 key bytes in, 4 score bytes out per position. Lane (quad qd, quarter c) reads dims [8c, 8c + 8) of a
// key with one 16-byte load, so each load instruction covers 16 whole keys = 1 KiB contiguous; a wave takes 64 keys
// per group (four loads per lane), three groups in flight, and the four waves of a workgroup read adjacent 4 KiB
// chunks.
// With fp16 keys the fp32 query is held as fp16 head + remainder pairs (q = hi + lo) and multiplied with v_dot2_f32_f16
// (fp32 accumulate); with bf16 keys the keys are widened to fp32. Either way scores keep fp32 accuracy. The quad's partial sums of its 4 keys are reduced and transposed with two
// DPP steps (xor 1, xor 2), after which lane c holds all heads of key c; ReLU and the head weights follow, and the
// wave's 64 scores go out as one 256-byte store.
template <bool F16, int NH, bool RELU>
__global__ __launch_bounds__(256) void score_lightning(LightningArgs a) {
    const int lin = xcd_contiguous_block();
    const int bkg = lin / a.tiles, tile = lin - bkg * a.tiles;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int qd = lane >> 2, c = lane & 3;
    // fp16 keys: q as 16-bit head + remainder pairs for v_dot2_f32_f16 (remainder error ~2^-22 |q|); bf16 keys: q in
    // fp32 and the keys widened (exact), since a bf16 head + remainder keeps only ~17 bits of q
    uint32_t qh[NH][4], ql[NH][4];
    float qf[F16 ? 1 : NH][8];
    float w[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        const int hh = min(h, a.nh - 1);
        const float4* qp = reinterpret_cast<const float4*>(a.q + ((size_t)bkg * a.nh + hh) * 32 + 8 * c);
        const float4 x0 = qp[0], x1 = qp[1];
        const bool on = h < a.nh;
        const float x[8] = {on ? x0.x : 0.0f, on ? x0.y : 0.0f, on ? x0.z : 0.0f, on ? x0.w : 0.0f,
                            on ? x1.x : 0.0f, on ? x1.y : 0.0f, on ? x1.z : 0.0f, on ? x1.w : 0.0f};
        if constexpr (F16) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float xr, yr, d0, d1;
                qh[h][i] = pack2_16<F16>(x[2 * i], x[2 * i + 1], xr, yr);
                ql[h][i] = pack2_16<F16>(x[2 * i] - xr, x[2 * i + 1] - yr, d0, d1);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) qf[h][e] = x[e];
        }
        w[h] = on ? a.w[(size_t)bkg * a.nh + hh] : 0.0f;
    }
    const uint16_t* kb = a.keys + ((size_t)bkg * a.Lk + a.lo) * 32 + 8 * c;
    float* orow = a.out + (size_t)bkg * a.out_stride;
    const int tile_base = tile * 256 * a.ng;
    // group g of this wave: keys tile_base + 64 (4 g + wave) + [0, 64); load jj: key + 16 jj + qd (clamped: past the
    // end a real key is read and its score not stored)
    auto load = [&](int g, u32x4_t (&b)[4]) {
        const int gbase = tile_base + 64 * (4 * g + wave);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int m = min(gbase + 16 * jj + qd, a.M - 1);
            b[jj] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(kb + (size_t)m * 32));
        }
    };
    auto process = [&](int g, const u32x4_t (&b)[4], bool masked) {
        float p[NH][4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const uint32_t kw[4] = {b[jj].x, b[jj].y, b[jj].z, b[jj].w};
            if constexpr (F16) {
#pragma unroll
                for (int h = 0; h < NH; ++h) {
                    float s = 0.0f;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        s = dot2_16<F16>(kw[i], qh[h][i], s);
                        s = dot2_16<F16>(kw[i], ql[h][i], s);
                    }
                    p[h][jj] = s;
                }
            } else {
                float kf[8];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    kf[2 * i] = bf16_lo(kw[i]);
                    kf[2 * i + 1] = bf16_hi(kw[i]);
                }
#pragma unroll
                for (int h = 0; h < NH; ++h) {
                    float s = 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) s += qf[h][e] * kf[e];
                    p[h][jj] = s;
                }
            }
        }
        const bool b0 = (c & 1) != 0, b1 = (c & 2) != 0;
        float score = 0.0f;
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            float r[2];
#pragma unroll
            for (int m2 = 0; m2 < 2; ++m2) {   // xor 1: keep the keys whose bit 0 matches this lane's
                const float keep = b0 ? p[h][2 * m2 + 1] : p[h][2 * m2];
                const float send = b0 ? p[h][2 * m2] : p[h][2 * m2 + 1];
                r[m2] = keep + dpp_f32<0xB1>(send);
            }
            const float keep = b1 ? r[1] : r[0];   // xor 2: keep key c
            const float send = b1 ? r[0] : r[1];
            const float s = keep + dpp_f32<0x4E>(send);
            score += w[h] * (RELU ? relu_f32(s) : s);
        }
        const int m = tile_base + 64 * (4 * g + wave) + 16 * c + qd;
        if (!masked || m < a.M) orow[m] = score;
    };
    auto run = [&](auto masked_tag) {
        constexpr bool kMasked = decltype(masked_tag)::value;
        // three groups in flight; the host picks 1, 2, 5 or 8 groups per tile, for which no load below reaches past
        // the tile's last group (such a load would read keys of the next tile: 1/9 more traffic at 8 groups)
        u32x4_t A[4], B[4], C[4];
        load(0, A);
        if (a.ng == 1) {
            process(0, A, kMasked);
            return;
        }
        load(1, B);
        int g = 0;
        for (; g + 3 <= a.ng; g += 3) {
            load(g + 2, C);
            process(g, A, kMasked);
            load(g + 3, A);
            process(g + 1, B, kMasked);
            load(g + 4, B);
            process(g + 2, C, kMasked);
        }
        if (g < a.ng) process(g, A, kMasked);
        if (g + 1 < a.ng) process(g + 1, B, kMasked);
    };
    if (tile_base + 256 * a.ng > a.M) run(std::true_type{});   // the row's last, partial tile
    else run(std::false_type{});
}

}  // namespace attnlab

using namespace attnlab;

extern "C" int attnlab_scan_probe(const uint16_t* zT, const uint16_t* q_cat, const uint16_t* wq_t, int B, int G,
                                  int C, int hd, int lo, int hi, uint32_t* sink, void* stream) {
    ATTNLAB_REQUIRE(B >= 1 && G >= 1 && 0 <= lo && lo < hi && hi <= C && hd >= 1,
                    "need B, G, hd >= 1 and 0 <= lo < hi <= C");
    ATTNLAB_REQUIRE(zT && q_cat && wq_t && sink, "zT, q_cat, wq_t and sink must be device pointers");
    const FusedGeometry geo = fused_geometry(B * G, C, 32, hd, lo, hi, zT, false);
    ATTNLAB_REQUIRE(geo.nsub > 0 && reinterpret_cast<uintptr_t>(wq_t) % 16 == 0,
                    "the probe needs the one-launch score's layout (C %% 8 == 0, 16-byte aligned zT and wq_t, h*d <= 512)");
    ScoreArgs a{const_cast<uint16_t*>(zT), nullptr, nullptr, q_cat, wq_t, nullptr, nullptr, nullptr, 0, G, 32, C, 128, hd,
                lo, hi - lo, 0, geo.tiles, nullptr, ScoreLists{nullptr, nullptr, 0, 0}};
    a.sink = sink;
    const dim3 grid(B * G * geo.tiles), block(256);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (geo.nsub == 8) hipLaunchKernelGGL((score_scan_fused<8, true>), grid, block, 0, s, a);
    else if (geo.nsub == 4) hipLaunchKernelGGL((score_scan_fused<4, true>), grid, block, 0, s, a);
    else if (geo.nsub == 2) hipLaunchKernelGGL((score_scan_fused<2, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((score_scan_fused<1, true>), grid, block, 0, s, a);
    return check_launch("scan_probe");
}

extern "C" int attnlab_score_grouped(uint16_t* zT, const uint16_t* k_new, const uint16_t* wk, const uint16_t* q_cat,
                                     const uint16_t* wq_t, const float* u_in, float* u_out, float* out,
                                     int64_t out_stride, int B, int G, int r, int C, int d, int hd, int lo, int hi,
                                     int write_col, int vector, uint32_t* hist, void* stream) {
    return score_grouped_impl(zT, k_new, wk, q_cat, wq_t, u_in, u_out, out, out_stride, B, G, r, C, d, hd, lo, hi,
                              write_col, vector, hist, reinterpret_cast<hipStream_t>(stream));
}

FusedGeometry attnlab::fused_geometry(int BG, int C, int r, int hd, int lo, int hi, const void* zT, bool u_given) {
    const bool v16_table = (C % 8 == 0) && (reinterpret_cast<uintptr_t>(zT) % 16 == 0);
    if (u_given || !v16_table || r != 32 || hd > 512 || hi <= lo) return FusedGeometry{0, 0};
    return fused_tiling(BG, lo, hi);
}

int attnlab::score_grouped_impl(uint16_t* zT, const uint16_t* k_new, const uint16_t* wk, const uint16_t* q_cat,
                                const uint16_t* wq_t, const float* u_in, float* u_out, float* out, int64_t out_stride,
                                int B, int G, int r, int C, int d, int hd, int lo, int hi, int write_col, int vector,
                                uint32_t* hist, hipStream_t s, const ScoreLists* lists) {
    ATTNLAB_REQUIRE(B >= 1 && G >= 1, "B and G must be positive (B=%d G=%d)", B, G);
    ATTNLAB_REQUIRE(r >= 1 && r <= kMaxR, "index width r=%d outside [1, %d]", r, kMaxR);
    ATTNLAB_REQUIRE(C >= 1, "C=%d must be positive", C);
    ATTNLAB_REQUIRE(k_new == nullptr || d >= 1, "writing the z column needs d >= 1, got %d", d);
    ATTNLAB_REQUIRE(0 <= lo && lo <= hi && hi <= C, "need 0 <= lo <= hi <= C, got lo=%d hi=%d C=%d", lo, hi, C);
    ATTNLAB_REQUIRE(zT != nullptr, "zT must be a device pointer");
    ATTNLAB_REQUIRE(k_new == nullptr || wk != nullptr, "writing the z column needs wk");
    ATTNLAB_REQUIRE(u_in != nullptr || (q_cat != nullptr && wq_t != nullptr && hd >= 1),
                    "either u_in or (q_cat, wq_t, hd >= 1) is required");
    if (k_new) {
        ATTNLAB_REQUIRE(0 <= write_col && write_col < C, "write_col=%d outside [0, %d)", write_col, C);
        ATTNLAB_REQUIRE(!(lo <= write_col && write_col < hi), "write_col=%d lies inside the scanned range [%d, %d)",
                        write_col, lo, hi);
    }
    const int M = hi - lo;
    ATTNLAB_REQUIRE(M == 0 || (out != nullptr && out_stride >= M) || (out == nullptr && lists != nullptr),
                    "out must hold M=%d scores per row", M);
    ScoreArgs a{zT, k_new, wk, q_cat, wq_t, u_in, u_out, out, out_stride, G, r, C, d, hd, lo, M, write_col, 1, hist,
                ScoreLists{nullptr, nullptr, 0, 0}};
    const bool vec = vector && (C % 4 == 0) && (reinterpret_cast<uintptr_t>(zT) % 8 == 0);
    // the r == 32 prologue reads wq_t with 16-byte loads
    if (r == 32 && u_in == nullptr)
        ATTNLAB_REQUIRE(reinterpret_cast<uintptr_t>(wq_t) % 16 == 0, "wq_t must be 16-byte aligned");
    const int BG = B * G;
    if (M == 0) {
        if (!k_new && !u_out) return ATTNLAB_OK;
        launch_prologue(a, BG, s);
        return check_launch("score_prologue");
    }
    const bool v16_table = vec && (C % 8 == 0) && (reinterpret_cast<uintptr_t>(zT) % 16 == 0);
    const FusedGeometry geo = fused_geometry(BG, C, r, hd, lo, hi, zT, u_in != nullptr);
    if (lists) {
        ATTNLAB_REQUIRE(vec && geo.nsub > 0 && hist != nullptr && lists->entries && lists->hdr &&
                            lists->lmin >= 1 && lists->cap >= 1 && lists->cap <= 512 * geo.nsub,
                        "key lists need the one-launch score (r = 32, h*d <= 512, aligned table) and a select state");
        a.lists = *lists;
    }
    if (vec && geo.nsub > 0) {
        // one launch: u and the z column inside the scan
        a.tiles = geo.tiles;
        const dim3 grid(BG * a.tiles), block(256);
        if (geo.nsub == 8) hipLaunchKernelGGL(score_scan_fused<8>, grid, block, 0, s, a);
        else if (geo.nsub == 4) hipLaunchKernelGGL(score_scan_fused<4>, grid, block, 0, s, a);
        else if (geo.nsub == 2) hipLaunchKernelGGL(score_scan_fused<2>, grid, block, 0, s, a);
        else hipLaunchKernelGGL(score_scan_fused<1>, grid, block, 0, s, a);
        return check_launch("score_scan_fused");
    }
    if (u_in == nullptr && u_out != nullptr) {
        // two launches: u (and the z column) once per (b, g), then a scan that only stages u; the per-block u of the
        // single-launch form costs ~20% of the scan time at B=16, L=32K
        launch_prologue(a, BG, s);
        const int rc = check_launch("score_prologue");
        if (rc) return rc;
        a.u_in = u_out;
        a.k_new = nullptr;
    }
    const bool v16 = v16_table && a.u_in != nullptr;
    if (v16) {
        const int span = ((hi + 7) & ~7) - (lo & ~7);
        a.tiles = (span + 511) / 512;
        hipLaunchKernelGGL(score_scan_v16<256>, dim3(BG * a.tiles), dim3(256), 0, s, a);
    } else if (vec) {
        const int span = ((hi + 3) & ~3) - (lo & ~3);   // columns the threads cover
        a.tiles = (span + 1023) / 1024;
        hipLaunchKernelGGL(score_scan_vec<256>, dim3(BG * a.tiles), dim3(256), 0, s, a);
    } else {
        a.tiles = (M + 2047) / 2048;
        hipLaunchKernelGGL(score_scan_scalar<256>, dim3(BG * a.tiles), dim3(256), 0, s, a);
    }
    return check_launch("score_scan");
}

extern "C" int64_t attnlab_list_bytes(int B, int G, int lo, int hi, int k, int order) {
    if (B < 1 || G < 1 || lo < 0 || hi < lo || k < 0 || k > hi - lo) return -1;
    if (order != ATTNLAB_ORDER_POSITION && order != ATTNLAB_ORDER_SCORE) return -1;
    return staged_score_order(order, k) ? 0 : list_region_bytes((int64_t)B * G, lo, hi, k);
}

extern "C" int attnlab_score_grouped_lists(uint16_t* zT, const uint16_t* k_new, const uint16_t* wk,
                                           const uint16_t* q_cat, const uint16_t* wq_t, float* u_out, float* out,
                                           int64_t out_stride, int B, int G, int r, int C, int d, int hd, int lo,
                                           int hi, int write_col, int k, int order, uint32_t* state, void* lists,
                                           int64_t lists_bytes, void* stream) {
    ATTNLAB_REQUIRE(B >= 1 && G >= 1 && 0 <= lo && lo <= hi && 0 <= k && k <= hi - lo,
                    "need B, G >= 1, 0 <= lo <= hi and 0 <= k <= hi - lo (B=%d G=%d lo=%d hi=%d k=%d)", B, G, lo, hi, k);
    ATTNLAB_REQUIRE(order == ATTNLAB_ORDER_POSITION || order == ATTNLAB_ORDER_SCORE, "unknown order %d", order);
    // refused here, before the state is touched: the list select sorts at most kMaxScoreOrderK picks by score
    ATTNLAB_REQUIRE(!staged_score_order(order, k), "the list select sorts at most %d rows in score order (k=%d); "
                    "attnlab_score_grouped with attnlab_select_rows takes larger k", kMaxScoreOrderK, k);
    const FusedGeometry geo = fused_geometry(B * G, C, r, hd, lo, hi, zT, false);
    const ListPlan plan = list_plan(hi - lo, k, geo);
    ATTNLAB_REQUIRE(plan.cap > 0, "the list select does not apply: it needs the one-launch score (r = 32, h*d <= 512, "
                    "a 16-byte aligned table with C %% 8 == 0), hi - lo <= %d and k small against hi - lo", kListMaxM);
    ATTNLAB_REQUIRE(state != nullptr && (reinterpret_cast<uintptr_t>(state) & 15) == 0,
                    "the key lists need a 16-byte aligned select state");
    ATTNLAB_REQUIRE(lists != nullptr && (reinterpret_cast<uintptr_t>(lists) & 255) == 0 &&
                        lists_bytes >= list_bytes(B * G, geo, plan),
                    "lists must be 256-byte aligned and hold attnlab_list_bytes = %lld bytes",
                    (long long)list_bytes(B * G, geo, plan));
    const ScoreLists ls = list_layout(lists, B * G, geo, plan);
    return score_grouped_impl(zT, k_new, wk, q_cat, wq_t, nullptr, u_out, out, out_stride, B, G, r, C, d, hd, lo, hi,
                              write_col, 1, state, reinterpret_cast<hipStream_t>(stream), &ls);
}

extern "C" int attnlab_score_prologue(uint16_t* zT, const uint16_t* k_new, const uint16_t* wk, const uint16_t* q_cat,
                                      const uint16_t* wq_t, float* u_out, int B, int G, int r, int C, int d, int hd,
                                      int write_col, void* stream) {
    ATTNLAB_REQUIRE(B >= 1 && G >= 1, "B and G must be positive (B=%d G=%d)", B, G);
    ATTNLAB_REQUIRE(r >= 1 && r <= kMaxR, "index width r=%d outside [1, %d]", r, kMaxR);
    ATTNLAB_REQUIRE(q_cat && wq_t && hd >= 1 && u_out, "q_cat, wq_t and u_out are required");
    if (k_new) ATTNLAB_REQUIRE(zT && wk && 0 <= write_col && write_col < C, "write_col=%d outside [0, %d)", write_col, C);
    if (r == 32) ATTNLAB_REQUIRE(reinterpret_cast<uintptr_t>(wq_t) % 16 == 0, "wq_t must be 16-byte aligned");
    ScoreArgs a{zT, k_new, wk, q_cat, wq_t, nullptr, u_out, nullptr, 0, G, r, C, d, hd, 0, 0, write_col, 1};
    launch_prologue(a, B * G, reinterpret_cast<hipStream_t>(stream));
    return check_launch("score_prologue");
}

extern "C" int attnlab_score_lightning(const uint16_t* keys, int key_dtype, const float* q, const float* w, float* out,
                                       int64_t out_stride, int B, int KG, int Lk, int r, int nh, int lo, int hi,
                                       int relu, void* stream) {
    ATTNLAB_REQUIRE(B >= 1 && KG >= 1, "B and KG must be positive (B=%d KG=%d)", B, KG);
    ATTNLAB_REQUIRE(r == 32, "lightning keys must have r == 32, got %d", r);
    ATTNLAB_REQUIRE(nh >= 1 && nh <= 8, "index heads nh=%d outside [1, 8]", nh);
    ATTNLAB_REQUIRE(key_dtype == ATTNLAB_DT_F16 || key_dtype == ATTNLAB_DT_BF16, "key dtype must be fp16 or bf16");
    ATTNLAB_REQUIRE(0 <= lo && lo <= hi && hi <= Lk, "need 0 <= lo <= hi <= Lk, got lo=%d hi=%d Lk=%d", lo, hi, Lk);
    ATTNLAB_REQUIRE(reinterpret_cast<uintptr_t>(keys) % 16 == 0, "keys must be 16-byte aligned");
    const int M = hi - lo;
    if (M == 0) return ATTNLAB_OK;
    ATTNLAB_REQUIRE(out != nullptr && out_stride >= M, "out must hold M=%d scores per row", M);
    ATTNLAB_REQUIRE(q != nullptr && w != nullptr && reinterpret_cast<uintptr_t>(q) % 16 == 0,
                    "q and w are required; q must be 16-byte aligned");
    // 64-key groups per wave and tile: tiles of 256..2048 keys, as large as still gives ~1024 workgroups, and one of
    // 1, 2, 5 or 8 groups (the kernel's three-group pipeline then loads nothing past a tile)
    const int64_t per = (int64_t)M * B * KG / 262144;
    const int ng = per >= 8 ? 8 : per >= 5 ? 5 : per >= 2 ? 2 : 1;
    const int tiles = (M + 256 * ng - 1) / (256 * ng);
    LightningArgs a{keys, q, w, out, out_stride, Lk, nh, lo, M, tiles, ng};
    const dim3 grid(B * KG * tiles);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const bool f16 = key_dtype == ATTNLAB_DT_F16;
#define LAUNCH_LIGHTNING(NHV)                                                                                      \
    do {                                                                                                           \
        if (f16 && relu) hipLaunchKernelGGL((score_lightning<true, NHV, true>), grid, dim3(256), 0, s, a);         \
        else if (f16) hipLaunchKernelGGL((score_lightning<true, NHV, false>), grid, dim3(256), 0, s, a);           \
        else if (relu) hipLaunchKernelGGL((score_lightning<false, NHV, true>), grid, dim3(256), 0, s, a);          \
        else hipLaunchKernelGGL((score_lightning<false, NHV, false>), grid, dim3(256), 0, s, a);                   \
    } while (0)
    if (nh <= 1) LAUNCH_LIGHTNING(1);
    else if (nh <= 2) LAUNCH_LIGHTNING(2);
    else if (nh <= 4) LAUNCH_LIGHTNING(4);
    else LAUNCH_LIGHTNING(8);
#undef LAUNCH_LIGHTNING
    return check_launch("score_lightning");
}
