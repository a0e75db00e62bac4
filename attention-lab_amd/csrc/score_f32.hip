// Grouped-indexer score on float32 index tables: the trained bank's dtype (trained.py:13-18, 78-81: FrozenIndexer keeps
// Wq and Wk in float32, make_trained_state builds a float32 index cache). Same formula as the bf16 path
// (indexer.py:15-29), with no rounding anywhere:
//   zT[b,g,j,write_col] = sum_e wk[g,j,e] * k_new[b,g,e]           (float32, stored unrounded)
//   u[j]                = sum_f q_cat[b,g,f] * wq_t[g,f,j]          (1/sqrt(r) folded into wq_t, as in the reference)
//   out[b,g,m]          = sum_j u[j] * zT[b,g,j,lo+m]               for m in [lo, hi)
// Where the bf16 path's one-launch tiling applies (r = 32, h*d <= 512, 16-byte rows), one launch does it all:
// score_scan_fused_f32 computes u and the z column inside the scan and writes the first-digit histogram and the
// per-workgroup key lists of the list select, exactly as the bf16 kernel does. Otherwise two launches: a prologue
// (u and the z column, one workgroup per (b, g)) and a scan with 16-byte loads (4 columns of one row per load) that
// leaves the first-digit histogram for the tiled select. The table is 4 bytes per element, so the scan moves twice
// the bf16 bytes.
#include "common.h"
#include "select.h"

namespace attnlab {
namespace {

struct ScoreF32Args {
    float* zT;              // [BG, r, C]
    const float* k_new;     // [BG, d] or null
    const float* wk;        // [G, r, d]
    const float* q_cat;     // [BG, hd]
    const float* wq_t;      // [G, hd, r]
    const float* u_in;      // [BG, r] or null
    float* u_out;           // [BG, r]
    float* out;             // row bg at out + bg * out_stride
    int64_t out_stride;
    int G, r, C, d, hd, lo, M, write_col;
    int tiles;
    uint32_t* hist;         // select state [BG, kSelectStateWords] or null
    ScoreLists lists;       // per-workgroup key lists (entries null: none; score_scan_fused_f32 only)
};

typedef float f32x4v_t __attribute__((ext_vector_type(4)));

constexpr int kF32MaxR = 32;
constexpr int kF32Cols = 1024;   // columns per scan workgroup: 256 threads x 4

// z column of the newest key, 256 threads: thread -> (j = tid / 8, e = tid % 8, +8, ...); the 8 partial sums of a j
// are adjacent lanes (shuffle reduce).
__device__ __forceinline__ void write_z_f32(const ScoreF32Args& a, int bg, int g) {
    const int tid = threadIdx.x;
    const int j = tid >> 3, e0 = tid & 7;
    const float* kn = a.k_new + (size_t)bg * a.d;
    float acc = 0.0f;
    if (j < a.r) {
        const float* wr = a.wk + ((size_t)g * a.r + j) * a.d;
        for (int e = e0; e < a.d; e += 8) acc += wr[e] * kn[e];
    }
    acc += __shfl_xor(acc, 1);
    acc += __shfl_xor(acc, 2);
    acc += __shfl_xor(acc, 4);
    if (j < a.r && e0 == 0) a.zT[((size_t)bg * a.r + j) * a.C + a.write_col] = acc;
}

// u (and the z column), one workgroup per (b, g).
// u: with r % 4 == 0 and 16-byte rows, thread -> (columns 4*(tid % 8) .. +3 of u, feature slice tid / 8 of 32): 16
// iterations of one 16-byte weight load at hd = 512; otherwise thread -> (j = tid % 32, slice tid / 32 of 8) with
// 4-byte loads. The slices meet in LDS.
// z: thread -> (j = tid / 8, e = tid % 8, +8, ...); the 8 partial sums of a j are adjacent lanes (shuffle reduce).
__global__ __launch_bounds__(256) void score_prologue_f32(ScoreF32Args a) {
    __shared__ float red[32][kF32MaxR + 1];
    const int bg = blockIdx.x, g = bg % a.G;
    const int tid = threadIdx.x;
    if (a.u_out && !a.u_in) {
        const float* q = a.q_cat + (size_t)bg * a.hd;
        const float* w = a.wq_t + (size_t)g * a.hd * a.r;
        const bool vec = (a.r & 3) == 0 && (reinterpret_cast<uintptr_t>(w) & 15) == 0;
        if (vec) {
            const int jq = tid & 7, sl = tid >> 3;
            float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (4 * jq < a.r) {
#pragma unroll 4
                for (int f = sl; f < a.hd; f += 32) {
                    const float qf = q[f];
                    const float4 wv = *reinterpret_cast<const float4*>(w + (size_t)f * a.r + 4 * jq);
                    acc.x += qf * wv.x;
                    acc.y += qf * wv.y;
                    acc.z += qf * wv.z;
                    acc.w += qf * wv.w;
                }
            }
            red[sl][4 * jq + 0] = acc.x;
            red[sl][4 * jq + 1] = acc.y;
            red[sl][4 * jq + 2] = acc.z;
            red[sl][4 * jq + 3] = acc.w;
            __syncthreads();
            if (tid < a.r) {
                float sum = 0.0f;
#pragma unroll 8
                for (int i = 0; i < 32; ++i) sum += red[i][tid];
                a.u_out[(size_t)bg * a.r + tid] = sum;
            }
        } else {
            const int j = tid & 31, sl = tid >> 5;
            float acc = 0.0f;
            if (j < a.r)
                for (int f = sl; f < a.hd; f += 8) acc += q[f] * w[(size_t)f * a.r + j];
            red[sl][j] = acc;
            __syncthreads();
            if (tid < a.r) {
                float sum = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) sum += red[i][tid];
                a.u_out[(size_t)bg * a.r + tid] = sum;
            }
        }
    }
    if (a.k_new) write_z_f32(a, bg, g);
}

// Scan: thread -> 4 adjacent columns from a 4-aligned column, one 16-byte load per index row j (all r loads issued
// before the first multiply). Columns outside [lo, hi) are loaded where they exist and never stored. VEC needs
// 16-byte rows (C % 4 == 0, aligned table); otherwise each of the 4 columns is a 4-byte load of its own.
template <bool VEC>
__global__ __launch_bounds__(256) void score_scan_f32(ScoreF32Args a) {
    __shared__ float u_sh[kF32MaxR];
    __shared__ __attribute__((aligned(16))) uint32_t hsh[kHistBins];
    const int lin = xcd_contiguous_block();
    const int bg = lin / a.tiles, tile = lin - bg * a.tiles;
    const int tid = threadIdx.x;
    if (tid < kF32MaxR) u_sh[tid] = tid < a.r ? a.u_in[(size_t)bg * a.r + tid] : 0.0f;
    if (a.hist) clear_histogram<256>(hsh);
    __syncthreads();
    const int lo = a.lo, hi = a.lo + a.M;
    const int c0 = (lo & ~3) + (tile * 256 + tid) * 4;
    f32x4v_t v[kF32MaxR];
    if constexpr (VEC) {
        const int cl = min(c0, a.C - 4);   // in bounds (C % 4 == 0): a tail thread re-reads the last group
        const float* col = a.zT + (size_t)bg * a.r * a.C + cl;
#pragma unroll
        for (int jj = 0; jj < kF32MaxR; ++jj)
            if (jj < a.r)
                v[jj] = __builtin_nontemporal_load(reinterpret_cast<const f32x4v_t*>(col + (size_t)jj * a.C));
    } else {
        const float* row = a.zT + (size_t)bg * a.r * a.C;
#pragma unroll
        for (int jj = 0; jj < kF32MaxR; ++jj) {
            if (jj < a.r) {
                const float* rj = row + (size_t)jj * a.C;
#pragma unroll
                for (int i = 0; i < 4; ++i) v[jj][i] = c0 + i < a.C ? rj[c0 + i] : 0.0f;
            }
        }
    }
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
    for (int jj = 0; jj < kF32MaxR; ++jj) {
        if (jj < a.r) {
            const float u = u_sh[jj];
            s0 += u * v[jj].x;
            s1 += u * v[jj].y;
            s2 += u * v[jj].z;
            s3 += u * v[jj].w;
        }
    }
    const float sv[4] = {s0, s1, s2, s3};
    float* o = a.out + (size_t)bg * a.out_stride - lo;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = c0 + i;
        if (c >= lo && c < hi) {
            o[c] = sv[i];
            if (a.hist) atomicAdd(&hsh[score_key(sv[i]) >> kHistShift], 1u);
        }
    }
    if (a.hist) flush_histogram<256>(hsh, a.hist, bg);
}

// One launch per step over a float32 table, with the bf16 one-launch kernel's tiling and outputs (r = 32,
// C % 8 == 0, 16-byte aligned table; for u: h*d <= 512, 16-byte aligned wq_t): u from q_cat and wq_t (or given, read
// from u_in, for a scan in the same summation order), the z column (tile 0), the scan of
// NSUB sub-tiles of 512 columns (sub-tile s of workgroup w is the row's sub-tile s * tiles + w: at each step the row's
// workgroups read one contiguous stretch of every table row), the first-digit histogram and the key lists. Wave w
// reads table rows 8w .. 8w + 7; lane l -> columns 4l .. 4l + 3 and 256 + 4l .. 256 + 4l + 3 of the sub-tile, so each
// of its two 16-byte loads per row is one contiguous kilobyte across the wave (16 loads per sub-tile, double
// buffered); the waves' partial sums meet in LDS and thread t finishes columns 2t and 2t + 1 of the sub-tile.
template <int NSUB>
__global__ __launch_bounds__(256) void score_scan_fused_f32(ScoreF32Args a) {
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
    const int cb0 = (lo & ~7) + tile * kCols;
    const int sstride = a.tiles * kCols;
    const int c_last = (hi - 1) & ~3;   // last 4-column group holding a scanned column (in bounds: C % 8 == 0)
    const float* zw = a.zT + ((size_t)bg * 32 + 8 * wave) * a.C;

    // Sub-tile s: this lane's two 4-column groups of the wave's 8 table rows. Groups past the row end re-read the last
    // group (in bounds, results discarded), so every sub-tile issues the same sixteen loads.
    auto load = [&](int s, f32x4v_t (&v)[16]) {
        const int ca = min(cb0 + s * sstride + lane * 4, c_last);
        const int cb = min(cb0 + s * sstride + 256 + lane * 4, c_last);
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const float* row = zw + (size_t)jj * a.C;
            v[2 * jj] = __builtin_nontemporal_load(reinterpret_cast<const f32x4v_t*>(row + ca));
            v[2 * jj + 1] = __builtin_nontemporal_load(reinterpret_cast<const f32x4v_t*>(row + cb));
        }
    };
    // u[8 wave + c], c < 8: lane -> features lane + 64 i (two 16-byte weight loads each). The weight loads are issued
    // before the table loads, so u is built while the table is in flight. Features past hd re-read feature hd - 1
    // with q = 0 (no branch, so no wait is placed between the loads).
    float u[8];
    f32x4v_t vb[2][16];
    if (a.u_in) {   // u given: the same scan, so the scores match the one-launch form's bit for bit
        const float* up = a.u_in + (size_t)bg * 32 + 8 * wave;
#pragma unroll
        for (int c = 0; c < 8; ++c) u[c] = up[c];
        load(0, vb[0]);
    } else {
        const float* qp = a.q_cat + (size_t)bg * a.hd;
        const float* wp = a.wq_t + (size_t)g * a.hd * 32 + 8 * wave;
        f32x4v_t wv[kUIter][2];
        float qf[kUIter];
#pragma unroll
        for (int it = 0; it < kUIter; ++it) {
            const int f = lane + 64 * it;
            const int fc = min(f, a.hd - 1);
            const f32x4v_t* wr = reinterpret_cast<const f32x4v_t*>(wp + (size_t)fc * 32);
            wv[it][0] = wr[0];
            wv[it][1] = wr[1];
            qf[it] = qp[fc];
            if (f >= a.hd) qf[it] = 0.0f;
        }
        load(0, vb[0]);
        __builtin_amdgcn_sched_barrier(0);   // keep every load above the first use of a weight
#pragma unroll
        for (int c = 0; c < 8; ++c) u[c] = 0.0f;
#pragma unroll
        for (int it = 0; it < kUIter; ++it)
#pragma unroll
            for (int c = 0; c < 8; ++c) u[c] += qf[it] * wv[it][c >> 2][c & 3];
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
    }
    if (a.hist) clear_histogram<256>(hsh);
    if (tid < 2) lcount[tid] = 0u;
    __syncthreads();

    float* o = a.out ? a.out + (size_t)bg * a.out_stride - lo : nullptr;   // null: key lists only
    uint32_t lkey[2 * NSUB];   // this thread's keys (columns cb0 + s * sstride + 2 tid + e), kept for the list
    uint32_t lvalid = 0u;
#pragma unroll
    for (int s = 0; s < NSUB; ++s) {
        if (s + 1 < NSUB) load(s + 1, vb[(s + 1) & 1]);
        const f32x4v_t (&v)[16] = vb[s & 1];
        float acc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
        // explicit fma chains from zero in row order: rescore8 (the select's recompute) repeats them bit for bit
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = __builtin_fmaf(u[jj], v[2 * jj + (i >> 2)][i & 3], acc[i]);
        *reinterpret_cast<float4*>(&part[wave][lane * 4]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
        *reinterpret_cast<float4*>(&part[wave][256 + lane * 4]) = make_float4(acc[4], acc[5], acc[6], acc[7]);
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
        if (a.k_new) write_z_f32(a, bg, g);
        if (a.u_out && !a.u_in && lane < 8) {
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

// Bulk build: zT[bg, j, col0 + t] = wk[g, j, :] . k_pre[bg, t, :] in float32. Block = 4 waves over 64 positions;
// lane = position, wave w owns j = w, w + 4, ...; the 64 key rows and the r weight rows are staged in LDS.
constexpr int kPkPos = 64;
constexpr int kPkPitch = 128 + 4;   // floats per staged row (d <= 128)

struct ProjectF32Args {
    const float* k_pre;
    int64_t k_bg_stride, k_row_stride;
    const float* wk;
    float* zT;
    int G, T, r, d, C, col0, tiles;
    int vec4 = 0;   // zT columns col0 + 4i are 16-byte aligned (16-byte stores)
};

__global__ __launch_bounds__(256) void project_keys_f32(ProjectF32Args a) {
    __shared__ float ks[kPkPos * kPkPitch];
    __shared__ float ws[kF32MaxR * kPkPitch];
    const int bg = blockIdx.x / a.tiles, tile = blockIdx.x - bg * a.tiles;
    const int g = bg % a.G;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = tile * kPkPos;
    for (int i = tid; i < kPkPos * 32; i += 256) {   // 64 rows x 32 float4 (d <= 128)
        const int row = i >> 5, seg = i & 31;
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (t0 + row < a.T && seg * 4 < a.d)
            v = *reinterpret_cast<const float4*>(a.k_pre + (size_t)bg * a.k_bg_stride +
                                                 (size_t)(t0 + row) * a.k_row_stride + seg * 4);
        *reinterpret_cast<float4*>(&ks[row * kPkPitch + seg * 4]) = v;
    }
    for (int i = tid; i < a.r * 32; i += 256) {
        const int j = i >> 5, seg = i & 31;
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (seg * 4 < a.d) v = *reinterpret_cast<const float4*>(a.wk + ((size_t)g * a.r + j) * a.d + seg * 4);
        *reinterpret_cast<float4*>(&ws[j * kPkPitch + seg * 4]) = v;
    }
    __syncthreads();
    const int t = t0 + lane;
    const float* krow = &ks[lane * kPkPitch];
    for (int j = wave; j < a.r; j += 4) {
        const float* wrow = &ws[j * kPkPitch];
        float s = 0.0f;
        for (int e = 0; e < a.d; ++e) s += krow[e] * wrow[e];
        if (t < a.T) a.zT[((size_t)bg * a.r + j) * a.C + a.col0 + t] = s;
    }
}

// Bulk build on the fp32 matrix cores (d % 16 == 0): Z[j, t] = sum_e wk[g, j, e] * k_pre[bg, t, e] as a GEMM with
// v_mfma_f32_16x16x4_f32. A = wk rows (index dims, MT 16-row tiles, staged in LDS), B = key rows (positions), D lane l
// holds Z[4 (l / 16) + i][l % 16]. The reduction dim is permuted so that every lane feeds 4 steps from one 16-byte
// load: at step 4 p + i, lane group q = l / 16 supplies e = 16 p + 4 q + i of both operands (the sum over e is the
// same). A wave covers 64 positions (4 column tiles), a workgroup 256; rows past T are clamped on load and never
// stored. At d = 128 the reduction loop is unrolled at compile time, so that the compiler issues key loads ahead of
// the products (583 -> 545 us at B=16, G=8, T=32K); a version that forces all 32 loads ahead (150 VGPRs, two waves per
// SIMD) gained 1 % more at B=16 and lost 3-8 % at B=1.
constexpr int kPkmPos = 256;
constexpr int kPkmPitch = 128 + 4;   // floats per staged weight row

constexpr int kZPitch = 68;   // floats per staged output row (64 positions + 4)

template <int MT, int PC>   // PC: d / 16 fixed at compile time (every key load issued before the first product), or 0
__global__ __launch_bounds__(256) void project_keys_f32_mfma(ProjectF32Args a) {
    // the weight rows, then the four waves' staged output tiles
    constexpr int kWsFloats = 16 * MT * kPkmPitch > 4 * 16 * kZPitch ? 16 * MT * kPkmPitch : 4 * 16 * kZPitch;
    __shared__ __attribute__((aligned(16))) float ws[kWsFloats];
    const int bg = blockIdx.x / a.tiles, tile = blockIdx.x - bg * a.tiles;
    const int g = bg % a.G;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int segs = a.d >> 2;
    for (int i = tid; i < 16 * MT * segs; i += 256) {
        const int j = i / segs, seg = i - j * segs;
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (j < a.r) v = *reinterpret_cast<const float4*>(a.wk + ((size_t)g * a.r + j) * a.d + seg * 4);
        *reinterpret_cast<float4*>(&ws[j * kPkmPitch + seg * 4]) = v;
    }
    __syncthreads();
    const int q = lane >> 4, c = lane & 15;
    const int t0 = tile * kPkmPos + wave * 64;
    const float* kb = a.k_pre + (size_t)bg * a.k_bg_stride + 4 * q;
    const float* krow[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) krow[nt] = kb + (size_t)min(t0 + 16 * nt + c, a.T - 1) * a.k_row_stride;
    f32x4v_t acc[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = f32x4v_t{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (PC > 0) {
        float4 kv[PC][4];
#pragma unroll
        for (int p = 0; p < PC; ++p)
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) kv[p][nt] = *reinterpret_cast<const float4*>(krow[nt] + 16 * p);
#pragma unroll
        for (int p = 0; p < PC; ++p) {
            float4 wv[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                wv[mt] = *reinterpret_cast<const float4*>(&ws[(16 * mt + c) * kPkmPitch + 16 * p + 4 * q]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const float av = i == 0 ? wv[mt].x : i == 1 ? wv[mt].y : i == 2 ? wv[mt].z : wv[mt].w;
#pragma unroll
                    for (int nt = 0; nt < 4; ++nt) {
                        const float4& k4 = kv[p][nt];
                        const float bv = i == 0 ? k4.x : i == 1 ? k4.y : i == 2 ? k4.z : k4.w;
                        acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[mt][nt], 0, 0, 0);
                    }
                }
            }
        }
    }
    const int P = PC > 0 ? 0 : a.d >> 4;
    for (int p = 0; p < P; ++p) {
        float4 kv[4], wv[MT];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) kv[nt] = *reinterpret_cast<const float4*>(krow[nt] + 16 * p);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
            wv[mt] = *reinterpret_cast<const float4*>(&ws[(16 * mt + c) * kPkmPitch + 16 * p + 4 * q]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const float av = i == 0 ? wv[mt].x : i == 1 ? wv[mt].y : i == 2 ? wv[mt].z : wv[mt].w;
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                    const float bv = i == 0 ? kv[nt].x : i == 1 ? kv[nt].y : i == 2 ? kv[nt].z : kv[nt].w;
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[mt][nt], 0, 0, 0);
                }
            }
        }
    }
    // Output through LDS (the weight rows are no longer read once every wave is past the products): a wave stages
    // each 16-row tile as 16 x 64 floats, then writes every row's 64 positions as 256 contiguous bytes (16 lanes x
    // 16 bytes) instead of 64-byte runs. Row pitch 68 floats: the staging stores of lane groups q and q + 1 fall in
    // different banks.
    __syncthreads();
    float* zs = ws + wave * 16 * kZPitch;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
#pragma unroll
            for (int i = 0; i < 4; ++i) zs[(4 * q + i) * kZPitch + 16 * nt + c] = acc[mt][nt][i];
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int row = 4 * it + (lane >> 4);
            const int j = 16 * mt + row;
            const int tp = t0 + 4 * (lane & 15);
            const float4 v = *reinterpret_cast<const float4*>(&zs[row * kZPitch + 4 * (lane & 15)]);
            if (j < a.r) {
                float* dst = a.zT + ((size_t)bg * a.r + j) * a.C + a.col0 + tp;
                if (a.vec4 && tp + 3 < a.T) {
                    *reinterpret_cast<float4*>(dst) = v;
                } else {
                    if (tp < a.T) dst[0] = v.x;
                    if (tp + 1 < a.T) dst[1] = v.y;
                    if (tp + 2 < a.T) dst[2] = v.z;
                    if (tp + 3 < a.T) dst[3] = v.w;
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
}

}  // namespace

FusedGeometry fused_geometry_f32(int BG, int C, int r, int hd, int lo, int hi, const void* zT, const void* wq_t,
                                 bool u_given) {
    const bool table = C % 8 == 0 && reinterpret_cast<uintptr_t>(zT) % 16 == 0;
    const bool u_ok = u_given || (hd >= 1 && hd <= 512 && reinterpret_cast<uintptr_t>(wq_t) % 16 == 0);
    if (!table || !u_ok || r != 32 || hi <= lo) return FusedGeometry{0, 0};
    return fused_tiling(BG, lo, hi);
}

int score_grouped_f32_impl(float* zT, const float* k_new, const float* wk, const float* q_cat, const float* wq_t,
                           const float* u_in, float* u_out, float* out, int64_t out_stride, int B, int G, int r,
                           int C, int d, int hd, int lo, int hi, int write_col, uint32_t* hist, hipStream_t s,
                           const ScoreLists* lists) {
    ATTNLAB_REQUIRE(B >= 1 && G >= 1, "B and G must be positive (B=%d G=%d)", B, G);
    ATTNLAB_REQUIRE(r >= 1 && r <= kF32MaxR, "index width r=%d outside [1, %d]", r, kF32MaxR);
    ATTNLAB_REQUIRE(0 <= lo && lo <= hi && hi <= C, "need 0 <= lo <= hi <= C, got lo=%d hi=%d C=%d", lo, hi, C);
    const int M = hi - lo;
    if (M > 0 || k_new) {   // a u-only call (no column, no candidate) never touches the table
        ATTNLAB_REQUIRE(zT != nullptr && reinterpret_cast<uintptr_t>(zT) % 4 == 0, "zT must be a float32 table");
    }
    if (k_new) {
        ATTNLAB_REQUIRE(wk && d >= 1 && 0 <= write_col && write_col < C && (write_col < lo || write_col >= hi),
                        "write_col=%d must lie in [0, C) and outside [lo, hi)", write_col);
    }
    const bool need_u = !u_in && u_out;   // the prologue projects the query whenever u_out is given without u_in
    if (need_u) ATTNLAB_REQUIRE(q_cat && wq_t && hd >= 1, "computing u needs q_cat, wq_t and hd >= 1");
    if (M > 0) {
        ATTNLAB_REQUIRE((out != nullptr && out_stride >= M) || (out == nullptr && lists != nullptr),
                        "out must hold M=%d scores per row", M);
        ATTNLAB_REQUIRE(u_in || u_out, "give u_in, or q_cat, wq_t and a u_out buffer for the prologue");
    }
    const int BG = B * G;
    ScoreF32Args a{zT, k_new, wk, q_cat, wq_t, u_in, u_out, out, out_stride, G, r, C, d, hd, lo, M, write_col, 0, hist,
                   ScoreLists{nullptr, nullptr, 0, 0}};
    // one launch (u or u given, z column, scan, histogram, key lists) wherever its tiling applies
    const FusedGeometry geo = M > 0 ? fused_geometry_f32(BG, C, r, hd, lo, hi, zT, wq_t, u_in != nullptr)
                                    : FusedGeometry{0, 0};
    if (lists) {
        ATTNLAB_REQUIRE(geo.nsub > 0 && hist != nullptr && lists->entries && lists->hdr && lists->lmin >= 1 &&
                            lists->cap >= 1 && lists->cap <= 512 * geo.nsub,
                        "key lists need the one-launch score (r = 32, h*d <= 512, aligned table) and a select state");
        a.lists = *lists;
    }
    if (geo.nsub > 0) {
        a.tiles = geo.tiles;
        const dim3 grid(BG * a.tiles), block(256);
        if (geo.nsub == 8) hipLaunchKernelGGL(score_scan_fused_f32<8>, grid, block, 0, s, a);
        else if (geo.nsub == 4) hipLaunchKernelGGL(score_scan_fused_f32<4>, grid, block, 0, s, a);
        else if (geo.nsub == 2) hipLaunchKernelGGL(score_scan_fused_f32<2>, grid, block, 0, s, a);
        else hipLaunchKernelGGL(score_scan_fused_f32<1>, grid, block, 0, s, a);
        return check_launch("score_scan_fused_f32");
    }
    if (need_u || k_new) {
        ScoreF32Args p = a;
        if (!need_u) p.u_out = nullptr;
        hipLaunchKernelGGL(score_prologue_f32, dim3(BG), dim3(256), 0, s, p);
        const int rc = check_launch("score_prologue_f32");
        if (rc) return rc;
    }
    if (M == 0) return ATTNLAB_OK;
    a.u_in = u_in ? u_in : u_out;
    const int span = ((hi + 3) & ~3) - (lo & ~3);
    a.tiles = (span + kF32Cols - 1) / kF32Cols;
    if (C % 4 == 0 && reinterpret_cast<uintptr_t>(zT) % 16 == 0)
        hipLaunchKernelGGL(score_scan_f32<true>, dim3(BG * a.tiles), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(score_scan_f32<false>, dim3(BG * a.tiles), dim3(256), 0, s, a);
    return check_launch("score_scan_f32");
}

}  // namespace attnlab

using namespace attnlab;

extern "C" int attnlab_score_grouped_f32(float* zT, const float* k_new, const float* wk, const float* q_cat,
                                         const float* wq_t, const float* u_in, float* u_out, float* out,
                                         int64_t out_stride, int B, int G, int r, int C, int d, int hd, int lo, int hi,
                                         int write_col, uint32_t* state, void* stream) {
    return score_grouped_f32_impl(zT, k_new, wk, q_cat, wq_t, u_in, u_out, out, out_stride, B, G, r, C, d, hd, lo, hi,
                                  write_col, state, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int attnlab_project_keys_f32(const float* k_pre, int64_t k_bg_stride, int64_t k_row_stride, const float* wk,
                                        float* zT, int B, int G, int T, int r, int d, int C, int col0, void* stream) {
    ATTNLAB_REQUIRE(B >= 1 && G >= 1 && T >= 0, "B=%d G=%d T=%d out of range", B, G, T);
    ATTNLAB_REQUIRE(r >= 1 && r <= kF32MaxR, "index width r=%d outside [1, %d]", r, kF32MaxR);
    ATTNLAB_REQUIRE(d >= 4 && d <= 128 && d % 4 == 0, "head_dim d=%d must be a multiple of 4 in [4, 128]", d);
    ATTNLAB_REQUIRE(0 <= col0 && col0 + T <= C, "columns [%d, %d) outside the table of C=%d", col0, col0 + T, C);
    ATTNLAB_REQUIRE(k_pre && wk && zT, "k_pre, wk and zT must be device pointers");
    ATTNLAB_REQUIRE(k_row_stride % 4 == 0 && k_bg_stride % 4 == 0 && reinterpret_cast<uintptr_t>(k_pre) % 16 == 0 &&
                        reinterpret_cast<uintptr_t>(wk) % 16 == 0,
                    "k_pre rows and wk must be 16-byte aligned");
    if (T == 0) return ATTNLAB_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (d % 16 == 0) {
        ProjectF32Args a{k_pre, k_bg_stride, k_row_stride, wk, zT, G, T, r, d, C, col0, (T + kPkmPos - 1) / kPkmPos};
        a.vec4 = C % 4 == 0 && col0 % 4 == 0 && reinterpret_cast<uintptr_t>(zT) % 16 == 0;
        const dim3 grid(B * G * a.tiles), block(256);
        if (r <= 16) {
            if (d == 128) hipLaunchKernelGGL((project_keys_f32_mfma<1, 8>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((project_keys_f32_mfma<1, 0>), grid, block, 0, s, a);
        } else {
            if (d == 128) hipLaunchKernelGGL((project_keys_f32_mfma<2, 8>), grid, block, 0, s, a);
            else hipLaunchKernelGGL((project_keys_f32_mfma<2, 0>), grid, block, 0, s, a);
        }
        return check_launch("project_keys_f32_mfma");
    }
    ProjectF32Args a{k_pre, k_bg_stride, k_row_stride, wk, zT, G, T, r, d, C, col0, (T + kPkPos - 1) / kPkPos};
    hipLaunchKernelGGL(project_keys_f32, dim3(B * G * a.tiles), dim3(256), 0, s, a);
    return check_launch("project_keys_f32");
}
