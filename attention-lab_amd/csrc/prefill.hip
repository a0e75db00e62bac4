// Prefill contractions on the matrix cores of gfx950: the bulk index-table build (project_keys, below) and the batched
// lightning-indexer score, T queries of one (b, kg) against its keys,
//   out[b,kg,t,m-lo] = sum_i w[b,kg,t,i] * act(q[b,kg,t,i,:] . key[b,kg,m,:])   m in [lo, hi), m <= q_pos0 + t if causal
// It is the T-query form of attnlab_score_lightning (one query per (b, kg), HBM-bound, no MFMA). With T queries the
// contraction over r = 32 is a real GEMM, [T*nh, 32] x [32, M], so it runs on v_mfma_f32_16x16x32_{f16,bf16}; the
// head reduction, ReLU and weights are applied to the accumulators in registers and only the fp32 scores leave the
// CU. The fp32 queries are split into a 16-bit head and a 16-bit remainder (q = hi + lo) and both are multiplied, so
// the result keeps fp32 accuracy (the remainder's rounding error is about 2^-22 of |q|).
//
// The kernel writes T*M*4 bytes and reads the keys once per 64-query tile (from L2 after the first), so at any T above
// a few dozen it is bound by the score writes to HBM, not by the matrix cores: one 16x16x32 MFMA pair makes 16 x 16
// dot products = 1 KB of scores at nh = 4 for 32 Kflop, which at 8 TB/s of writes asks for a quarter of the MFMA peak.
// A workgroup stages its keys in LDS before its first MFMA, so its main loop issues stores and no global loads: on this
// part loads and stores share one in-order completion counter, and a wait for a key load issued after a score store
// would also wait for that store to reach memory.
#include <cfloat>
#include <type_traits>

#include "common.h"

namespace attnlab {
namespace {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint16_t u16x8_t __attribute__((ext_vector_type(8)));

struct LightningBatchArgs {
    const uint16_t* keys;   // [BKG, Lk, 32] fp16 or bf16
    const float* q;         // [BKG, T, nh, 32]
    const float* w;         // [BKG, T, nh]
    float* out;             // row (bkg, t) at out + (bkg * T + t) * out_stride; column m - lo
    int64_t out_stride;     // multiple of 4
    int Lk, T, lo, hi;
    int q_pos0;             // causal: query t reads keys m <= q_pos0 + t; negative: no causal bound
    int relu;
    int qtiles, ktiles;
};

constexpr int kQTile = 64;     // queries per workgroup: 16 per wave
constexpr int kKBlock = 64;    // keys per step of a wave: four 16-column MFMA tiles
constexpr int kKTile = 512;    // keys per workgroup, staged in LDS (32 KB)

// LDS slot (16-byte units) of chunk kq (elements 8 kq .. 8 kq + 7) of key j of the workgroup's range: four keys share a
// 256-byte row and the row's 16 slots are permuted by the row number, so the 16 lanes of one MFMA B read (keys
// j0 + 4 n + c, n < 16, of a 64-key block, one chunk) land in 16 different slots, i.e. on all 64 banks once.
__device__ __forceinline__ int key_slot(int j, int kq) {
    return (j >> 2) * 16 + ((((j & 3) << 2) | kq) ^ ((j >> 2) & 15));
}

// 8 consecutive fp32 -> (head, remainder) 16-bit vectors, both rounded to nearest even.
template <bool F16>
__device__ __forceinline__ void split8(const float4& x0, const float4& x1,
                                       std::conditional_t<F16, f16x8_t, bf16x8_t>& hi,
                                       std::conditional_t<F16, f16x8_t, bf16x8_t>& lo) {
    const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    if constexpr (F16) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            hi[e] = (_Float16)x[e];
            lo[e] = (_Float16)(x[e] - (float)hi[e]);
        }
    } else {
        u16x8_t h, l;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            h[e] = f32_to_bf16_rne(x[e]);
            l[e] = f32_to_bf16_rne(x[e] - bf16_to_f32(h[e]));
        }
        hi = __builtin_bit_cast(bf16x8_t, h);
        lo = __builtin_bit_cast(bf16x8_t, l);
    }
}

// max(x, 0) as one integer max: negative numbers and -0.0 have the sign bit set, so they compare below 0.
__device__ __forceinline__ float relu(float x) { return __int_as_float(max(__float_as_int(x), 0)); }

template <bool F16>
__device__ __forceinline__ f32x4_t mfma16x16x32(const std::conditional_t<F16, f16x8_t, bf16x8_t>& a,
                                                const std::conditional_t<F16, f16x8_t, bf16x8_t>& b, f32x4_t c) {
    if constexpr (F16) return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    else return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Workgroup = 64 queries x 512 keys of one (b, kg); wave w owns queries [16 w, 16 w + 16) of the tile and walks the
// keys 64 at a time. MFMA operands (lane l, n = l & 15, K elements 8 (l >> 4) .. + 7):
//   A row n    = (query n / nh, head n % nh) of one row group of 16 / nh queries; the wave has nh such groups
//   B column n = key m0 + 4 n + c for the c-th of four tiles, so after the four tiles a lane holds 4 adjacent keys
//   D          lane l holds rows 4 (l >> 4) + i, i < 4, of column n
// so every lane ends with whole heads of 4 / nh queries (nh = 8: half the heads, the other half in lane l ^ 16) and
// writes them as one 16-byte store of 4 adjacent scores per query. The workgroup's keys (those its last visible query
// reads, rounded up to whole blocks; past the table: its last key, results not stored) are staged in LDS first.
template <bool F16, int NH, bool RELU>
__global__ __launch_bounds__(256) void lightning_batched(LightningBatchArgs a) {
    using vec8 = std::conditional_t<F16, f16x8_t, bf16x8_t>;
    constexpr int QG = 16 / NH;             // queries per row group
    constexpr int NG = NH;                  // row groups per wave (16 queries)
    constexpr int QPL = NH >= 4 ? 1 : 4 / NH;   // queries per lane per row group
    constexpr int HPL = NH >= 4 ? 4 : NH;       // heads per lane per query
    __shared__ u32x4_t ksh[kKTile * 4];
    const int lin = xcd_contiguous_block();   // a (b, kg)'s tiles on one XCD: its keys stay in that L2
    const int kt = lin % a.ktiles;
    const int rest = lin / a.ktiles;
    const int qt = rest % a.qtiles;
    const int bkg = rest / a.qtiles;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t_wave = qt * kQTile + wave * 16;
    const int m_begin = a.lo + kt * kKTile;
    const bool causal = a.q_pos0 >= 0;
    int m_wg = min(a.hi, m_begin + kKTile);   // keys read by the workgroup's last visible query
    if (causal) m_wg = min(m_wg, a.q_pos0 + min(qt * kQTile + kQTile - 1, a.T - 1) + 1);
    if (m_begin >= m_wg) return;   // the whole workgroup: nothing of it is visible (before the barrier)

    const int n = lane & 15, kq = lane >> 4;
    vec8 ahi[NG], alo[NG];
    float wv[NG][4];
    const float* qb = a.q + (size_t)bkg * a.T * NH * 32;
    const float* wb = a.w + (size_t)bkg * a.T * NH;
    float4 qraw[NG][2];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const int t = min(t_wave + g * QG + n / NH, a.T - 1);   // rows past T compute on the last query, not stored
        const float4* src = reinterpret_cast<const float4*>(qb + ((size_t)t * NH + n % NH) * 32 + 8 * kq);
        qraw[g][0] = src[0];
        qraw[g][1] = src[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rr = 4 * kq + i;
            const int tt = min(t_wave + g * QG + rr / NH, a.T - 1);
            wv[g][i] = wb[(size_t)tt * NH + rr % NH];
        }
    }
    // keys [m_begin, m_begin + nst) into LDS: all loads issued, then the stores (eight 16-byte chunks per thread)
    {
        const int nst = min(kKTile, (m_wg - m_begin + kKBlock - 1) / kKBlock * kKBlock);
        const uint16_t* kb = a.keys + (size_t)bkg * a.Lk * 32;
        u32x4_t kv[kKTile * 4 / 256];
#pragma unroll
        for (int i = 0; i < kKTile * 4 / 256; ++i) {
            const int e = (int)threadIdx.x + 256 * i;
            const int m = min(m_begin + min(e >> 2, nst - 1), a.Lk - 1);
            kv[i] = *reinterpret_cast<const u32x4_t*>(kb + (size_t)m * 32 + 8 * (e & 3));
        }
#pragma unroll
        for (int i = 0; i < kKTile * 4 / 256; ++i) {
            const int e = (int)threadIdx.x + 256 * i;
            ksh[key_slot(e >> 2, e & 3)] = kv[i];
        }
    }
#pragma unroll
    for (int g = 0; g < NG; ++g) split8<F16>(qraw[g][0], qraw[g][1], ahi[g], alo[g]);
    __syncthreads();
    int m_end = min(a.hi, m_begin + kKTile);
    if (causal) m_end = min(m_end, a.q_pos0 + min(t_wave + 15, a.T - 1) + 1);
    if (t_wave >= a.T || m_begin >= m_end) return;   // this wave: nothing visible (no barrier below)

    // B tiles of the block at key offset j0 (a multiple of 64) from LDS: key j0 + 4 n + c, chunk kq, at slot
    // 4 j0 + 16 n + ((4 c + kq) ^ n)
    int boff[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) boff[c] = 16 * n + (((c << 2) | kq) ^ n);
    auto read_keys = [&](int m0, vec8 (&b)[4]) {
        const u32x4_t* kp = ksh + 4 * (m0 - m_begin);
#pragma unroll
        for (int c = 0; c < 4; ++c) b[c] = __builtin_bit_cast(vec8, kp[boff[c]]);
    };
    float* ob = a.out + (size_t)bkg * a.T * a.out_stride - a.lo;
    // Scores of row group g against the four key tiles in b: v[p][c] = score of the lane's p-th query and key
    // m0 + 4 n + c (nh = 8: the sum over both lane halves' heads, in both lanes).
    auto scores = [&](int g, const vec8 (&b)[4], f32x4_t (&v)[QPL]) {
        f32x4_t acc[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            acc[c] = mfma16x16x32<F16>(ahi[g], b[c], f32x4_t{0.0f, 0.0f, 0.0f, 0.0f});
            acc[c] = mfma16x16x32<F16>(alo[g], b[c], acc[c]);
        }
#pragma unroll
        for (int p = 0; p < QPL; ++p) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                float x = 0.0f;
#pragma unroll
                for (int i = p * HPL; i < p * HPL + HPL; ++i) x += wv[g][i] * (RELU ? relu(acc[c][i]) : acc[c][i]);
                if constexpr (NH == 8) x += shfl_xor_f32(x, 16);
                v[p][c] = x;
            }
        }
    };
    // nh = 8: the two lanes holding a query's halves store two scores each, so every lane stores
    const int half = NH == 8 ? 2 * (kq & 1) : 0;

    // Interior blocks (every key visible to every query of the wave): unconditional stores. Then at most a couple of
    // boundary blocks (the causal diagonal, the row end, queries past T) with per-score masks.
    int m_int = m_begin;
    if (t_wave + 15 < a.T) {
        int lim = min(a.hi, m_begin + kKTile);
        if (causal) lim = min(lim, a.q_pos0 + t_wave + 1);
        m_int = m_begin + max(0, (lim - m_begin) / kKBlock) * kKBlock;
    }
    // row pointers of the lane's queries for the interior blocks, which exist only when all 16 queries are below T
    float* rowp[NG][QPL];
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int p = 0; p < QPL; ++p)
            rowp[g][p] = ob + (size_t)min(t_wave + g * QG + (4 * kq) / NH + p, a.T - 1) * a.out_stride + 4 * n + half;
    int m0 = m_begin;
    for (; m0 < m_int; m0 += kKBlock) {
        vec8 b[4];
        read_keys(m0, b);
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            f32x4_t v[QPL];
            scores(g, b, v);
#pragma unroll
            for (int p = 0; p < QPL; ++p) {
                float* dst = rowp[g][p] + m0;
                if constexpr (NH == 8) {
                    const f32x2_t h2 = half ? f32x2_t{v[p][2], v[p][3]} : f32x2_t{v[p][0], v[p][1]};
                    __builtin_nontemporal_store(h2, reinterpret_cast<f32x2_t*>(dst));
                } else {
                    __builtin_nontemporal_store(v[p], reinterpret_cast<f32x4_t*>(dst));
                }
            }
        }
    }
    for (; m0 < m_end; m0 += kKBlock) {
        vec8 b[4];
        read_keys(m0, b);
        const int mk = m0 + 4 * n;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            f32x4_t v[QPL];
            scores(g, b, v);
#pragma unroll
            for (int p = 0; p < QPL; ++p) {
                const int t = t_wave + g * QG + (4 * kq) / NH + p;
                if (t >= a.T) continue;
                const int limit = causal ? min(a.hi, a.q_pos0 + t + 1) : a.hi;
                float* dst = ob + (size_t)t * a.out_stride + mk;
#pragma unroll
                for (int c = half; c < (NH == 8 ? half + 2 : 4); ++c)
                    if (mk + c < limit) dst[c] = v[p][c];
            }
        }
    }
}


// ---------------------------------------------------------------------------------------------------------------
// Bulk index-table build (prefill): zT[bg, j, col0 + t] = bf16_rne(wk[g, j, :] . k_pre[bg, t, :]) for t < T.
// Two kernels: project_keys_mfma (d a multiple of 32) and project_keys_lds for other head dims.
//
// project_keys_lds: block = 4 waves over 64 positions; lane = position, wave w owns j = w, w + 4, ...; the 64 key rows
// are staged in LDS (row pitch 136 halves, so lanes reading their own row hit distinct banks) and wk rows are LDS
// broadcasts. Stores of one j are 64 consecutive columns (128 bytes).
// ---------------------------------------------------------------------------------------------------------------
struct ProjectArgs {
    const uint16_t* k_pre;  // row t of bg at k_pre + bg * k_bg_stride + t * k_row_stride
    int64_t k_bg_stride, k_row_stride;
    const uint16_t* wk;     // [G, r, d]
    uint16_t* zT;           // [BG, r, C]
    int G, T, r, d, C, col0, tiles;
    int vec;                // zT columns col0 + 4i are 8-byte aligned (8-byte stores)
};

constexpr int kProjMaxR = 32;
constexpr int kProjPos = 64;
constexpr int kProjPitch = 136;  // halves per staged key row (128 + 8 padding)

__global__ __launch_bounds__(256) void project_keys_lds(ProjectArgs a) {
    __shared__ uint16_t ks[kProjPos * kProjPitch];
    __shared__ uint16_t ws[kProjMaxR * 128];
    const int bg = blockIdx.x / a.tiles;
    const int tile = blockIdx.x - bg * a.tiles;
    const int g = bg % a.G;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = tile * kProjPos;
    // stage 64 key rows (d <= 128 halves each) with 16-byte loads: 16 lanes per row
    for (int i = tid; i < kProjPos * 16; i += 256) {
        const int row = i >> 4, seg = i & 15;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (t0 + row < a.T && seg * 8 < a.d)
            v = *reinterpret_cast<const uint4*>(a.k_pre + (size_t)bg * a.k_bg_stride + (size_t)(t0 + row) * a.k_row_stride + seg * 8);
        *reinterpret_cast<uint4*>(&ks[row * kProjPitch + seg * 8]) = v;
    }
    for (int i = tid; i < a.r * 16; i += 256) {
        const int j = i >> 4, seg = i & 15;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (seg * 8 < a.d) v = *reinterpret_cast<const uint4*>(a.wk + ((size_t)g * a.r + j) * a.d + seg * 8);
        *reinterpret_cast<uint4*>(&ws[j * 128 + seg * 8]) = v;
    }
    __syncthreads();
    const int t = t0 + lane;
    const uint32_t* krow = reinterpret_cast<const uint32_t*>(&ks[lane * kProjPitch]);
    for (int j = wave; j < a.r; j += 4) {
        const uint32_t* wrow = reinterpret_cast<const uint32_t*>(&ws[j * 128]);
        float s = 0.0f;
        for (int e2 = 0; e2 < a.d / 2; ++e2) {
            const uint32_t kw = krow[e2], ww = wrow[e2];
            s += bf16_lo(kw) * bf16_lo(ww);
            s += bf16_hi(kw) * bf16_hi(ww);
        }
        if (t < a.T) a.zT[((size_t)bg * a.r + j) * a.C + a.col0 + t] = f32_to_bf16_rne(s);
    }
}

// project_keys_mfma: the GEMM zT[bg, :, cols] = wk[g] (r x d) . k_pre[bg]^T (d x 64) per wave, on
// v_mfma_f32_16x16x32_bf16 (fp32 accumulate, one RNE to bf16 at the end). A rows are index dims j (two 16-row tiles
// cover r <= 32); B column n of the c-th of four 16-column tiles is position t0 + 4 n + c, so each lane ends with 4
// adjacent columns of 8 index dims and writes each dim's 4 columns as one 8-byte store. The wave's 64 key rows are all
// loaded before the first MFMA. Workgroup = 4 waves = 256 positions of one (b, g); wk[g] is staged in LDS once per
// workgroup (each wave reading its own 8 KB copy from L2 took 15 % of the kernel's time at B=16, T=32K).
template <int KD>   // d / 32
__global__ __launch_bounds__(256) void project_keys_mfma(ProjectArgs a) {
    const int bg = blockIdx.x / a.tiles;
    const int tile = blockIdx.x - bg * a.tiles;
    const int g = bg % a.G;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, kq = lane >> 4;
    const int t0 = tile * 256 + wave * 64;
    // wk[g] staged once per workgroup: row j (32 of them, zero past r) as 4 KD 16-byte chunks, rows 4 KD + 1 chunks
    // apart so that the 16 rows a read instruction touches fall in different banks
    constexpr int kW = 4 * KD, kWPitch = 4 * KD + 1;
    __shared__ u32x4_t wsh[32 * kWPitch];
    for (int e = threadIdx.x; e < 32 * kW; e += 256) {
        const int j = e / kW, ch = e - j * kW;
        u32x4_t w = u32x4_t{0u, 0u, 0u, 0u};
        if (j < a.r) w = *reinterpret_cast<const u32x4_t*>(a.wk + ((size_t)g * a.r + j) * a.d + 8 * ch);
        wsh[j * kWPitch + ch] = w;
    }
    const uint16_t* kb = a.k_pre + (size_t)bg * a.k_bg_stride + 8 * kq;
    bf16x8_t kv[4][KD];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int t = min(t0 + 4 * n + c, a.T - 1);   // columns past T compute on row T - 1, not stored
#pragma unroll
        for (int kc = 0; kc < KD; ++kc)
            kv[c][kc] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(kb + (size_t)t * a.k_row_stride + 32 * kc));
    }
    __syncthreads();
    if (t0 >= a.T) return;   // whole wave, after the workgroup's only barrier
    bf16x8_t wv[2][KD];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int kc = 0; kc < KD; ++kc) wv[rt][kc] = __builtin_bit_cast(bf16x8_t, wsh[(16 * rt + n) * kWPitch + 4 * kc + kq]);
    f32x4_t acc[2][4];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[rt][c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kc = 0; kc < KD; ++kc)
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
                acc[rt][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wv[rt][kc], kv[c][kc], acc[rt][c], 0, 0, 0);
    // lane: rows j = 16 rt + 4 kq + i, columns t0 + 4 n + c
    const int tc = t0 + 4 * n;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = 16 * rt + 4 * kq + i;
            if (j >= a.r) continue;
            uint16_t h[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) h[c] = f32_to_bf16_rne(acc[rt][c][i]);
            uint16_t* dst = a.zT + ((size_t)bg * a.r + j) * a.C + a.col0 + tc;
            if (a.vec && tc + 3 < a.T) {
                *reinterpret_cast<u32x2_t*>(dst) = u32x2_t{(uint32_t)h[0] | ((uint32_t)h[1] << 16),
                                                            (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (tc + c < a.T) dst[c] = h[c];
            }
        }
    }
}


// ---------------------------------------------------------------------------------------------------------------
// Causal prefill attention on the matrix cores: T queries at consecutive positions q_pos0 + t of one KV group,
// every query head of the group, against the cache rows j <= q_pos0 + t, j < legal (the legality rule of
// reference.py:41-48, the full read of full.py:17-44 for a prefill chunk):
//   out[bg, i, t, :] = sum_j softmax_j(scale * q[bg, i, t] . K[bg, j]) V[bg, j]
// A workgroup owns 128 (query, head) rows: 128 / h consecutive positions with all h heads of the group, so each K/V
// block is read once for every head. Per block of 64 keys:
//   S^T = K Q^T    v_mfma_f32_32x32x16_bf16, A = 32 keys x 16 dims (LDS, row-major), B = Q^T (registers); lane l's
//                  column is its own query row, so the softmax state of a row lives in lanes n and n + 32
//   P^T           online softmax in the log2 domain on the accumulators; the C layout of S^T is already the B
//                  layout P^T needs for the next product (keys 8 (i/4) + 4 (l/32) + i%4 of row l%32)
//   O^T += V^T P^T A = 32 dims x 16 keys from V^T in LDS (staged transposed, two keys per 32-bit word), B = P^T
// O^T keeps each row's 128 outputs in the lanes of that row, so rescaling needs no exchange. The next block's K/V
// is loaded into registers while the current one is computed.
// ---------------------------------------------------------------------------------------------------------------
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2v_t __attribute__((ext_vector_type(2)));

struct PrefillAttendArgs {
    const uint16_t* q;      // [BG, h, T, 128]
    const uint16_t* K;      // row j of bg at K + bg * kv_bg_stride + j * kv_row_stride
    const uint16_t* V;
    int64_t kv_bg_stride;
    int kv_row_stride;
    uint16_t* out;          // [BG, h, T, 128]
    int h, T, q_pos0, legal;
    int qtiles;             // ceil(T / (128 / h))
    float scale_log2;
    // key split (a grid too small to fill the chip): workgroup (bg, qt, sp) reads the keys [sp kspan, (sp + 1) kspan)
    // of its tile and writes its rows' (m, l, o) to part [BG, h, T, splits, 132] instead of out; splits == 1: none
    int splits = 1, kspan = 0;
    float* part = nullptr;
};
constexpr int kPaPart = 132;   // m, l, two unused words (16-byte aligned rows), the 128 unnormalised outputs
constexpr int kPrefillMaxSplits = 16;

constexpr int kPaRows = 128;          // (query, head) rows per workgroup: 4 waves x 32
constexpr int kPaKeys = 64;           // keys per block
constexpr int kPaKPitch = 128 + 8;    // bf16 per K row in LDS (272 bytes: 16-byte aligned rows)
constexpr int kPaVPitch = 64 + 4;     // bf16 per V^T row in LDS (136 bytes)

// V^T in LDS: row d (a head dim) holds the block's 64 keys as 16 groups of 4 (8 bytes); group g of row d sits at slot
// g ^ ((d >> 4) & 7). The staging store of a wave writes 16 rows 8 apart, which without the permutation land on 4 of
// the 32 banks (8-way conflicts); with it they cover all 32. The MFMA reads (32 consecutive rows, one group) keep one
// permutation per 16 rows and stay conflict-free.
__device__ __forceinline__ int vt_at(int d, int key) {
    return d * kPaVPitch + ((((key >> 2) ^ (d >> 4)) & 15) << 2) + (key & 3);
}
constexpr float kPaLazy = 8.0f;       // rescale O only when the running max grows by more than 2^8

// two fp32 -> packed bf16 pair, round to nearest even (gfx950 converts in hardware: v_cvt_pk_bf16_f32)
typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float x, float y) {
    const bf16x2v_t v = {(__bf16)x, (__bf16)y};
    return __builtin_bit_cast(uint32_t, v);
}

// two workgroups per CU: the register budget then fits without AGPRs (230 VGPRs), and one workgroup's softmax
// hides the other's matrix-core latency (1.2-1.3x over one workgroup per CU)
template <bool SPLIT>   // SPLIT: a.splits > 1, partials to a.part (the one-pass instance keeps no split logic)
__global__ __launch_bounds__(256, 2) void prefill_attend(PrefillAttendArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t ks[kPaKeys * kPaKPitch];
    __shared__ __attribute__((aligned(16))) uint16_t vt[128 * kPaVPitch];
    const int lin = xcd_contiguous_block();
    // the query tiles of a (b, g) in reverse: the later tiles read more keys, so they are dispatched first and the
    // short ones fill in behind them; the key splits of a tile are adjacent
    const int nsp = SPLIT ? a.splits : 1;
    const int per_bg = a.qtiles * nsp;
    const int bg = lin / per_bg, rem = lin - bg * per_bg;
    const int qt = a.qtiles - 1 - rem / nsp, sp = rem - (rem / nsp) * nsp;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 31, g = lane >> 5;
    const int BQ = kPaRows / a.h;
    const int t0 = qt * BQ;
    const int R = 32 * wave + n;                 // this lane's row: query t0 + R / h, head R % h
    const int t = t0 + R / a.h, head = R % a.h;
    const int tc = min(t, a.T - 1);
    const int pos = a.q_pos0 + tc;
    bf16x8_t qb[8];                              // B operand of S^T: row R, dims 16 kk + 8 g .. + 7
    {
        const uint16_t* qr = a.q + (((size_t)bg * a.h + head) * a.T + tc) * 128 + 8 * g;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) qb[kk] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(qr + 16 * kk));
    }
    // keys of the workgroup: its tile's visible keys, or this split's share of them
    const int kend_tile = min(a.legal, a.q_pos0 + min(t0 + BQ, a.T));
    const int kb0 = SPLIT ? sp * a.kspan : 0;
    const int kend = SPLIT ? min(kend_tile, kb0 + a.kspan) : kend_tile;
    const int wave_first = a.q_pos0 + min(t0 + (32 * wave) / a.h, a.T - 1);
    const int kend_wave = min(a.legal, a.q_pos0 + min(t0 + (32 * wave + 31) / a.h, a.T - 1) + 1);

    const uint16_t* Kb = a.K + (size_t)bg * a.kv_bg_stride;
    const uint16_t* Vb = a.V + (size_t)bg * a.kv_bg_stride;
    // staging: K chunk c = tid + 256 u -> key c / 16, 16 bytes at dim 8 (c % 16); V unit w = tid + 256 u -> dims
    // 8 (w % 16) .. + 7 of keys 2 (w / 16) and 2 (w / 16) + 1 (16 lanes read one key's 256 bytes)
    u32x4_t kr[4], vr[2][2];
    auto gload = [&](int kb) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int c = tid + 256 * u;
            const int key = min(kb + (c >> 4), kend - 1);
            kr[u] = *reinterpret_cast<const u32x4_t*>(Kb + (size_t)key * a.kv_row_stride + 8 * (c & 15));
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int w = tid + 256 * u;
            const int k0 = min(kb + 2 * (w >> 4), kend - 1), k1 = min(kb + 2 * (w >> 4) + 1, kend - 1);
            vr[u][0] = *reinterpret_cast<const u32x4_t*>(Vb + (size_t)k0 * a.kv_row_stride + 8 * (w & 15));
            vr[u][1] = *reinterpret_cast<const u32x4_t*>(Vb + (size_t)k1 * a.kv_row_stride + 8 * (w & 15));
        }
    };
    auto lds_store = [&]() {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int c = tid + 256 * u;
            *reinterpret_cast<u32x4_t*>(&ks[(c >> 4) * kPaKPitch + 8 * (c & 15)]) = kr[u];
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int w = tid + 256 * u;
            const int kp = w >> 4, d0 = 8 * (w & 15);
            const uint32_t x[4] = {vr[u][0].x, vr[u][0].y, vr[u][0].z, vr[u][0].w};
            const uint32_t y[4] = {vr[u][1].x, vr[u][1].y, vr[u][1].z, vr[u][1].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {   // dims d0 + 2e, d0 + 2e + 1: (key 2kp, key 2kp + 1) pairs
                *reinterpret_cast<uint32_t*>(&vt[vt_at(d0 + 2 * e, 2 * kp)]) = (x[e] & 0xffffu) | (y[e] << 16);
                *reinterpret_cast<uint32_t*>(&vt[vt_at(d0 + 2 * e + 1, 2 * kp)]) = (x[e] >> 16) | (y[e] & 0xffff0000u);
            }
        }
    };

    float m_run = -INFINITY, l_run = 0.0f;
    // the scale (log2 domain), made positive: a negative scale flips the sign of q instead (exact in bf16), and a zero
    // scale becomes the smallest normal float, which gives the same weights (every exponent below fp32's resolution)
    // while a masked key's -inf * scale stays -inf instead of NaN
    const float sc = a.scale_log2 == 0.0f ? FLT_MIN : fabsf(a.scale_log2);
    if (a.scale_log2 < 0.0f) {
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
            qb[kk] = __builtin_bit_cast(bf16x8_t, __builtin_bit_cast(u32x4_t, qb[kk]) ^ 0x80008000u);
    }
    f32x16_t o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] = 0.0f;

    if (kb0 < kend) gload(kb0);
    for (int kb = kb0; kb < kend; kb += kPaKeys) {
        if (kb != kb0) __syncthreads();   // the previous block's LDS reads are done
        lds_store();
        __syncthreads();
        if (kb + kPaKeys < kend) gload(kb + kPaKeys);
        if (kb >= kend_wave) continue;   // every row of this wave ends before the block (no barrier skipped: the
                                         // loop's barriers are at its top)
        f32x16_t s[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int i = 0; i < 16; ++i) s[kt][i] = 0.0f;
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                const bf16x8_t ka = __builtin_bit_cast(
                    bf16x8_t, *reinterpret_cast<const u32x4_t*>(&ks[(32 * kt + n) * kPaKPitch + 16 * kk + 8 * g]));
                s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qb[kk], s[kt], 0, 0, 0);
            }
        }
        // this lane's scores: row R, keys kb + 32 kt + 8 (i / 4) + 4 g + i % 4. The scale is positive here (a negative
        // one flipped the query's sign), so the block's largest scaled score comes from the raw scores and the scale
        // costs one multiply per row here and rides in the exponent's FMA below.
        const bool full = kb + kPaKeys - 1 <= wave_first && kb + kPaKeys <= a.legal;   // no key of the block masked
        float bm = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float v = s[kt][i];
                if (!full) {
                    const int key = kb + 32 * kt + 8 * (i >> 2) + 4 * g + (i & 3);
                    if (key > pos || key >= a.legal) v = -INFINITY;
                }
                s[kt][i] = v;
                bm = fmaxf(bm, v);
            }
        bm = fmaxf(bm, shfl_xor_f32(bm, 32)) * sc;
        if (bm > m_run + kPaLazy) {   // also the first block of the row (m_run = -inf)
            const float al = fast_exp2(m_run - bm);   // exp2(-inf) = 0
            l_run *= al;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[dt][i] *= al;
            m_run = bm;
        }
        // P^T (bf16) as the B operand of O^T += V^T P^T, one per 16-key step ks: tile ks / 2, accumulators
        // 8 (ks % 2) .. + 7, i.e. keys 16 (ks % 2) + 4 g + {0..3, 8..11} of the tile. p = exp2(scale * s - m): one
        // FMA and the exponential.
        bf16x8_t pb[4];
        const float nm = -m_run;
#pragma unroll
        for (int ks2 = 0; ks2 < 4; ++ks2) {
            uint32_t w4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float x0 = s[ks2 >> 1][8 * (ks2 & 1) + 2 * e], x1 = s[ks2 >> 1][8 * (ks2 & 1) + 2 * e + 1];
                const float p0 = m_run == -INFINITY ? 0.0f : fast_exp2(fmaf(x0, sc, nm));
                const float p1 = m_run == -INFINITY ? 0.0f : fast_exp2(fmaf(x1, sc, nm));
                l_run += p0 + p1;
                w4[e] = pack_bf16x2(p0, p1);
            }
            pb[ks2] = __builtin_bit_cast(bf16x8_t, u32x4_t{w4[0], w4[1], w4[2], w4[3]});
        }
#pragma unroll
        for (int ks2 = 0; ks2 < 4; ++ks2) {
            const int key0 = 32 * (ks2 >> 1) + 16 * (ks2 & 1) + 4 * g;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const u32x2v_t lo4 = *reinterpret_cast<const u32x2v_t*>(&vt[vt_at(32 * dt + n, key0)]);
                const u32x2v_t hi4 = *reinterpret_cast<const u32x2v_t*>(&vt[vt_at(32 * dt + n, key0 + 8)]);
                const bf16x8_t va = __builtin_bit_cast(bf16x8_t, u32x4_t{lo4.x, lo4.y, hi4.x, hi4.y});
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[ks2], o[dt], 0, 0, 0);
            }
        }
    }
    const float l_tot = l_run + shfl_xor_f32(l_run, 32);
    if (t >= a.T) return;
    if constexpr (SPLIT) {   // this split's partial: m (log2 domain, scaled), l and the unnormalised outputs
        float* pp = a.part + ((((size_t)bg * a.h + head) * a.T + t) * a.splits + sp) * kPaPart;
        if (g == 0) {
            pp[0] = m_run;
            pp[1] = l_tot;
        }
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4)
                *reinterpret_cast<float4*>(pp + 4 + 32 * dt + 8 * i4 + 4 * g) =
                    make_float4(o[dt][4 * i4], o[dt][4 * i4 + 1], o[dt][4 * i4 + 2], o[dt][4 * i4 + 3]);
        return;
    }
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    uint16_t* orow = a.out + (((size_t)bg * a.h + head) * a.T + t) * 128;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {   // dims 32 dt + 8 i4 + 4 g + 0..3
            const f32x16_t& od = o[dt];
            *reinterpret_cast<u32x2v_t*>(orow + 32 * dt + 8 * i4 + 4 * g) =
                u32x2v_t{pack_bf16x2(od[4 * i4] * inv, od[4 * i4 + 1] * inv),
                         pack_bf16x2(od[4 * i4 + 2] * inv, od[4 * i4 + 3] * inv)};
        }
}

// The key splits' partials of every (b, g, head, query) row merged into out: thread -> (row, four dims); the partials
// are read in split order with one rescale to their largest m (the arithmetic of the non-split kernel's
// normalisation: out = o * (1 / l), zero where no key is visible).
__global__ __launch_bounds__(256) void prefill_combine(PrefillAttendArgs a, int64_t rows) {
    const int64_t item = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (item >= rows * 32) return;
    const int64_t row = item >> 5;
    const int d4 = 4 * (int)(item & 31);
    const float* pp = a.part + row * a.splits * kPaPart;
    float mx = -INFINITY;
    for (int sp = 0; sp < a.splits; ++sp) mx = fmaxf(mx, pp[sp * kPaPart]);
    float l = 0.0f;
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int sp = 0; sp < a.splits; ++sp) {
        const float m = pp[sp * kPaPart];
        const float w = m == -INFINITY ? 0.0f : fast_exp2(m - mx);
        const float4 v = *reinterpret_cast<const float4*>(pp + sp * kPaPart + 4 + d4);
        l += w * pp[sp * kPaPart + 1];
        o.x += w * v.x;
        o.y += w * v.y;
        o.z += w * v.z;
        o.w += w * v.w;
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    *reinterpret_cast<uint2*>(a.out + row * 128 + d4) =
        make_uint2(pack_bf16x2(o.x * inv, o.y * inv), pack_bf16x2(o.z * inv, o.w * inv));
}

}  // namespace
}  // namespace attnlab

using namespace attnlab;

extern "C" int attnlab_project_keys(const uint16_t* k_pre, int64_t k_bg_stride, int64_t k_row_stride, const uint16_t* wk,
                                    uint16_t* zT, int B, int G, int T, int r, int d, int C, int col0, void* stream) {
    ATTNLAB_REQUIRE(B >= 1 && G >= 1 && T >= 0, "B=%d G=%d T=%d out of range", B, G, T);
    ATTNLAB_REQUIRE(r >= 1 && r <= kProjMaxR, "index width r=%d outside [1, %d]", r, kProjMaxR);
    ATTNLAB_REQUIRE(d >= 2 && d <= 128 && d % 8 == 0, "head_dim d=%d must be a multiple of 8 in [8, 128]", d);
    ATTNLAB_REQUIRE(0 <= col0 && col0 + T <= C, "columns [%d, %d) outside the table of C=%d", col0, col0 + T, C);
    ATTNLAB_REQUIRE(k_pre && wk && zT, "k_pre, wk and zT must be device pointers");
    ATTNLAB_REQUIRE(k_row_stride % 8 == 0 && k_bg_stride % 8 == 0 && reinterpret_cast<uintptr_t>(k_pre) % 16 == 0 &&
                        reinterpret_cast<uintptr_t>(wk) % 16 == 0,
                    "k_pre rows and wk must be 16-byte aligned");
    if (T == 0) return ATTNLAB_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    ProjectArgs a{k_pre, k_bg_stride, k_row_stride, wk, zT, G, T, r, d, C, col0, 0,
                  C % 4 == 0 && col0 % 4 == 0 && reinterpret_cast<uintptr_t>(zT) % 8 == 0};
    if (d % 32 == 0) {
        a.tiles = (T + 255) / 256;
        const dim3 grid(B * G * a.tiles), block(256);
        if (d == 32) hipLaunchKernelGGL(project_keys_mfma<1>, grid, block, 0, s, a);
        else if (d == 64) hipLaunchKernelGGL(project_keys_mfma<2>, grid, block, 0, s, a);
        else if (d == 96) hipLaunchKernelGGL(project_keys_mfma<3>, grid, block, 0, s, a);
        else hipLaunchKernelGGL(project_keys_mfma<4>, grid, block, 0, s, a);
        return check_launch("project_keys_mfma");
    }
    a.tiles = (T + kProjPos - 1) / kProjPos;
    hipLaunchKernelGGL(project_keys_lds, dim3(B * G * a.tiles), dim3(256), 0, s, a);
    return check_launch("project_keys_lds");
}


extern "C" int attnlab_score_lightning_batched(const uint16_t* keys, int key_dtype, const float* q, const float* w,
                                               float* out, int64_t out_stride, int B, int KG, int Lk, int r, int nh,
                                               int T, int lo, int hi, int q_pos0, int relu, void* stream) {
    ATTNLAB_REQUIRE(B >= 1 && KG >= 1 && T >= 0, "B, KG must be positive and T >= 0 (B=%d KG=%d T=%d)", B, KG, T);
    ATTNLAB_REQUIRE(r == 32, "lightning keys must have r == 32, got %d", r);
    ATTNLAB_REQUIRE(nh == 1 || nh == 2 || nh == 4 || nh == 8, "index heads nh=%d must be 1, 2, 4 or 8", nh);
    ATTNLAB_REQUIRE(key_dtype == ATTNLAB_DT_F16 || key_dtype == ATTNLAB_DT_BF16, "key dtype must be fp16 or bf16");
    ATTNLAB_REQUIRE(0 <= lo && lo <= hi && hi <= Lk, "need 0 <= lo <= hi <= Lk, got lo=%d hi=%d Lk=%d", lo, hi, Lk);
    const int M = hi - lo;
    if (M == 0 || T == 0) return ATTNLAB_OK;
    ATTNLAB_REQUIRE(keys && q && w && out, "keys, q, w and out are required");
    ATTNLAB_REQUIRE(reinterpret_cast<uintptr_t>(keys) % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0,
                    "keys and q must be 16-byte aligned");
    ATTNLAB_REQUIRE(reinterpret_cast<uintptr_t>(out) % 16 == 0 && out_stride % 4 == 0 && out_stride >= M,
                    "out must be 16-byte aligned with a row stride that is a multiple of 4 and >= M=%d (got %lld)", M,
                    (long long)out_stride);
    LightningBatchArgs a{keys, q, w, out, out_stride, Lk, T, lo, hi, q_pos0 < 0 ? -1 : q_pos0, relu ? 1 : 0,
                         (T + kQTile - 1) / kQTile, (M + kKTile - 1) / kKTile};
    const int64_t blocks = (int64_t)B * KG * a.qtiles * a.ktiles;
    ATTNLAB_REQUIRE(blocks < (int64_t)1 << 31, "grid of %lld workgroups is too large", (long long)blocks);
    const dim3 grid((unsigned)blocks), block(256);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const bool f16 = key_dtype == ATTNLAB_DT_F16;
#define LAUNCH_LB(NHV)                                                                                        \
    do {                                                                                                      \
        if (f16 && relu) hipLaunchKernelGGL((lightning_batched<true, NHV, true>), grid, block, 0, s, a);       \
        else if (f16) hipLaunchKernelGGL((lightning_batched<true, NHV, false>), grid, block, 0, s, a);         \
        else if (relu) hipLaunchKernelGGL((lightning_batched<false, NHV, true>), grid, block, 0, s, a);        \
        else hipLaunchKernelGGL((lightning_batched<false, NHV, false>), grid, block, 0, s, a);                 \
    } while (0)
    if (nh == 1) LAUNCH_LB(1);
    else if (nh == 2) LAUNCH_LB(2);
    else if (nh == 4) LAUNCH_LB(4);
    else LAUNCH_LB(8);
#undef LAUNCH_LB
    return check_launch("lightning_batched");
}

namespace {

int prefill_attend_impl(const uint16_t* q, const uint16_t* K, const uint16_t* V, int64_t kv_bg_stride, int kv_row_stride,
                        uint16_t* out, int B, int G, int h, int T, int d, int q_pos0, int legal, int C, float scale,
                        int splits, float* part, int64_t part_bytes, void* stream) {
    ATTNLAB_REQUIRE(B >= 1 && G >= 1 && T >= 0, "B, G must be positive and T >= 0 (B=%d G=%d T=%d)", B, G, T);
    ATTNLAB_REQUIRE(d == 128, "head_dim must be 128, got %d", d);
    ATTNLAB_REQUIRE(h == 1 || h == 2 || h == 4 || h == 8 || h == 16, "query heads per group h=%d must divide 128 "
                    "(1, 2, 4, 8 or 16)", h);
    ATTNLAB_REQUIRE(q_pos0 >= 0 && 0 < legal && legal <= C, "need q_pos0 >= 0 and 0 < legal <= C (q_pos0=%d "
                    "legal=%d C=%d)", q_pos0, legal, C);
    ATTNLAB_REQUIRE(1 <= splits && splits <= kPrefillMaxSplits, "key splits %d outside [1, %d]", splits,
                    kPrefillMaxSplits);
    if (T == 0) return ATTNLAB_OK;
    ATTNLAB_REQUIRE(q && K && V && out, "q, K, V and out are required");
    ATTNLAB_REQUIRE(kv_row_stride >= 128 && kv_row_stride % 8 == 0 && kv_bg_stride % 8 == 0 &&
                        ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(K) |
                          reinterpret_cast<uintptr_t>(V) | reinterpret_cast<uintptr_t>(out)) & 15) == 0,
                    "q, K, V, out and the K/V rows must be 16-byte aligned");
    const int64_t need = attnlab_prefill_part_bytes(B, G, h, T, splits);
    ATTNLAB_REQUIRE(splits == 1 || (part != nullptr && (reinterpret_cast<uintptr_t>(part) & 15) == 0 && part_bytes >= need),
                    "%d key splits need a 16-byte aligned part buffer of attnlab_prefill_part_bytes = %lld bytes",
                    splits, (long long)need);
    PrefillAttendArgs a{q, K, V, kv_bg_stride, kv_row_stride, out, h, T, q_pos0, legal, 0, scale * kLog2e};
    const int BQ = kPaRows / h;
    a.qtiles = (T + BQ - 1) / BQ;
    if (splits > 1) {
        // every split a whole number of 64-key blocks of the longest tile's visible keys
        const int kmax = min(legal, q_pos0 + T);
        a.splits = splits;
        a.kspan = ((kmax + splits - 1) / splits + kPaKeys - 1) / kPaKeys * kPaKeys;
        a.part = part;
    }
    const int64_t blocks = (int64_t)B * G * a.qtiles * a.splits;
    ATTNLAB_REQUIRE(blocks < (int64_t)1 << 31, "grid of %lld workgroups is too large", (long long)blocks);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (splits > 1) {
        hipLaunchKernelGGL(prefill_attend<true>, dim3((unsigned)blocks), dim3(256), 0, s, a);
        const int64_t rows = (int64_t)B * G * h * T;
        hipLaunchKernelGGL(prefill_combine, dim3((unsigned)((rows * 32 + 255) / 256)), dim3(256), 0, s, a, rows);
    } else {
        hipLaunchKernelGGL(prefill_attend<false>, dim3((unsigned)blocks), dim3(256), 0, s, a);
    }
    return check_launch("prefill_attend");
}

}  // namespace

extern "C" int64_t attnlab_prefill_part_bytes(int B, int G, int h, int T, int splits) {
    if (B < 1 || G < 1 || h < 1 || T < 0 || splits < 1) return -1;
    return splits > 1 ? (int64_t)B * G * h * T * splits * kPaPart * 4 : 0;
}

extern "C" int attnlab_prefill_attend(const uint16_t* q, const uint16_t* K, const uint16_t* V, int64_t kv_bg_stride,
                                      int kv_row_stride, uint16_t* out, int B, int G, int h, int T, int d,
                                      int q_pos0, int legal, int C, float scale, void* stream) {
    return prefill_attend_impl(q, K, V, kv_bg_stride, kv_row_stride, out, B, G, h, T, d, q_pos0, legal, C, scale, 1,
                               nullptr, 0, stream);
}

extern "C" int attnlab_prefill_attend_split(const uint16_t* q, const uint16_t* K, const uint16_t* V,
                                            int64_t kv_bg_stride, int kv_row_stride, uint16_t* out, int B, int G,
                                            int h, int T, int d, int q_pos0, int legal, int C, float scale, int splits,
                                            float* part, int64_t part_bytes, void* stream) {
    return prefill_attend_impl(q, K, V, kv_bg_stride, kv_row_stride, out, B, G, h, T, d, q_pos0, legal, C, scale,
                               splits, part, part_bytes, stream);
}
