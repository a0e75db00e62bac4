// Grouped-indexer score on float32 index tables: the trained bank's dtype (trained.py:13-18, 78-81: FrozenIndexer keeps
// Wq and Wk in float32, make_trained_state builds a float32 index cache). Same formula as the bf16 path
// (indexer.py:15-29), with no rounding anywhere:
//   zT[b,g,j,write_col] = sum_e wk[g,j,e] * k_new[b,g,e]           (float32, stored unrounded)
//   u[j]                = sum_f q_cat[b,g,f] * wq_t[g,f,j]          (1/sqrt(r) folded into wq_t, as in the reference)
//   out[b,g,m]          = sum_j u[j] * zT[b,g,j,lo+m]               for m in [lo, hi)
// Two launches: a prologue (u and the z column, one workgroup per (b, g)) and a scan that reads the table with
// 16-byte loads (4 columns of one row per load) and leaves the first-digit histogram for the tiled select, as the
// bf16 scan does. The table is 4 bytes per element, so the scan moves twice the bf16 bytes.
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
};

typedef float f32x4v_t __attribute__((ext_vector_type(4)));

constexpr int kF32MaxR = 32;
constexpr int kF32Cols = 1024;   // columns per scan workgroup: 256 threads x 4

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
    if (a.k_new) {
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
// stored.
constexpr int kPkmPos = 256;
constexpr int kPkmPitch = 128 + 4;   // floats per staged weight row

template <int MT>
__global__ __launch_bounds__(256) void project_keys_f32_mfma(ProjectF32Args a) {
    __shared__ __attribute__((aligned(16))) float ws[16 * MT * kPkmPitch];
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
    const int P = a.d >> 4;
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
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            const int t = t0 + 16 * nt + c;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = 16 * mt + 4 * q + i;
                if (j < a.r && t < a.T) a.zT[((size_t)bg * a.r + j) * a.C + a.col0 + t] = acc[mt][nt][i];
            }
        }
    }
}

}  // namespace

int score_grouped_f32_impl(float* zT, const float* k_new, const float* wk, const float* q_cat, const float* wq_t,
                           const float* u_in, float* u_out, float* out, int64_t out_stride, int B, int G, int r,
                           int C, int d, int hd, int lo, int hi, int write_col, uint32_t* hist, hipStream_t s) {
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
        ATTNLAB_REQUIRE(out != nullptr && out_stride >= M, "out must hold M=%d scores per row", M);
        ATTNLAB_REQUIRE(u_in || u_out, "give u_in, or q_cat, wq_t and a u_out buffer for the prologue");
    }
    const int BG = B * G;
    ScoreF32Args a{zT, k_new, wk, q_cat, wq_t, u_in, u_out, out, out_stride, G, r, C, d, hd, lo, M, write_col, 0, hist};
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
        if (r <= 16)
            hipLaunchKernelGGL(project_keys_f32_mfma<1>, dim3(B * G * a.tiles), dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL(project_keys_f32_mfma<2>, dim3(B * G * a.tiles), dim3(256), 0, s, a);
        return check_launch("project_keys_f32_mfma");
    }
    ProjectF32Args a{k_pre, k_bg_stride, k_row_stride, wk, zT, G, T, r, d, C, col0, (T + kPkPos - 1) / kPkPos};
    hipLaunchKernelGGL(project_keys_f32, dim3(B * G * a.tiles), dim3(256), 0, s, a);
    return check_launch("project_keys_f32");
}
