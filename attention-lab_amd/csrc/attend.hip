// Decode attention for gfx950: the gather-free sparse read (D) and the dense control read (A) share one kernel.
//
// Reference semantics: MetalAttend (metal_attend.py:46-169) and gathered_decode_step_kernel / full_attention
// (decode.py:131-142, full.py:17-34): out[b,g,i] = softmax(scale * q_i . K[rows]) @ V[rows] for the h query heads of
// KV group g, rows read by original position straight from the cache.
//
// Layout per workgroup (256 threads = 4 waves) of one (b, g, partition): 8 lanes share a position; lane `sub` owns
// dims [8*sub, 8*sub+8) and [64+8*sub, 64+8*sub+8), so one 16-byte load per lane and half-row covers 128 contiguous
// bytes (one cache line) and a wave reads 8 positions per load instruction. Each wave walks its groups of 8 positions
// through kStages rotating register stages: while one group is computed, the K/V rows of the next kStages - 1 groups
// are in flight. (Staging the rows through LDS with global_load_lds instead caps a CU at about 10 GB/s on MI355X, less
// than half of what plain 16-byte loads reach on the same random rows.) q . k is a
// bf16 dot2 (v_dot2_f32_bf16, fp32 accumulate) finished by a 3-step DPP sum over the 8 lanes; every head of the group
// reuses the same K and V registers (GQA sharing). Online softmax runs in the log2 domain with a lazy rescale: the
// running max is raised only when a block max exceeds it by more than 2^8, so the 16*h accumulator rescale is rare.
// Slot pairs are merged with DPP (lane ^ 8), then the remaining 16 slots through LDS by (head, dim) columns.
// With P > 1 partitions every block writes its (m, l, acc) partial and a
// second small kernel merges them; the kernel boundary is what makes the partials of other XCDs' L2s visible, which
// is far cheaper on this part than a device-scope fence per block.
#include "attend_core.h"

namespace attnlab {

template <int H, int D, bool DENSE, bool PAGED = false>
__global__ __launch_bounds__(kAttThreads) void attend_kernel(AttendArgs a) {
    static_assert(!(DENSE && PAGED), "the paged read lists its positions (rows, or [0, S) when rows is null)");
    constexpr int kChunk = 4096;   // row-list entries whose positions are staged in LDS at a time (one chunk for k <= 4096)
    __shared__ __attribute__((aligned(16))) int idx_sh[DENSE ? 4 : kChunk];
    __shared__ float red_ml[kMergeSlots][H][2];
    __shared__ __attribute__((aligned(16))) float red_acc[kMergeSlots][H][kHeadDim];
    __shared__ uint32_t last_sh;
    const int lin = xcd_contiguous_block();   // (b, g) on the XCD that wrote its row list
    const int bg = lin / (a.Q * a.P);
    const int rem = lin - bg * a.Q * a.P;
    const int qg = rem / a.P;
    const int p = rem - qg * a.P;
    const int tid = threadIdx.x;
    const int sub = tid & 7;
    const int hq = a.h / a.Q;   // heads of this workgroup
    const int h0 = qg * hq;
    uint32_t qw[H][8];
    attend_load_q<H>(a, bg, h0, hq, qw);

    const int Sp = (a.S + a.P - 1) / a.P;
    const int s_begin = p * Sp;
    const int s_end = min(a.S, s_begin + Sp);
    const size_t bg_off = PAGED ? 0 : (size_t)bg * a.kv_bg_stride;   // a paged row index already names its (b, g)
    const uint16_t* Kb = a.K + bg_off + 8 * sub;
    const uint16_t* Vb = a.V + bg_off + 8 * sub;
    const int32_t* rl = (DENSE || a.rows == nullptr) ? nullptr : a.rows + (size_t)bg * a.rows_stride;

    float m[H], l[H], acc[H][16];
#pragma unroll
    for (int i = 0; i < H; ++i) {
        m[i] = -INFINITY;
        l[i] = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;
    }

    const int chunk = DENSE ? max(s_end - s_begin, 1) : kChunk;
    for (int c0 = s_begin; c0 < s_end; c0 += chunk) {
        const int clen = min(chunk, s_end - c0);
        if (!DENSE) {
            if (c0 != s_begin) __syncthreads();   // every wave is done with the previous chunk's positions
            if (PAGED && rl == nullptr) {
                for (int i = tid; i < clen; i += kAttThreads) idx_sh[i] = c0 + i;
            } else {
                const int32_t* src = rl + c0;
                if ((reinterpret_cast<uintptr_t>(src) & 15) == 0) {   // 16-byte loads where the chunk is aligned
                    const int nv = clen >> 2;
                    for (int i = tid; i < nv; i += kAttThreads)
                        reinterpret_cast<int4*>(idx_sh)[i] = reinterpret_cast<const int4*>(src)[i];
                    for (int i = 4 * nv + tid; i < clen; i += kAttThreads) idx_sh[i] = src[i];
                } else {
                    for (int i = tid; i < clen; i += kAttThreads) idx_sh[i] = src[i];
                }
            }
            if (PAGED) {
                // the staged positions become pool rows (-1: outside [0, C) or an unmapped page, never read); the
                // 16-byte staging wrote each thread's four entries, the translation reads every 256th, hence the barrier
                __syncthreads();
                const int b = bg / a.G, g = bg - b * a.G;
                const int32_t* bt = a.block_table + (size_t)b * a.bt_stride;
                const int pmask = (1 << a.page_shift) - 1;
                for (int i = tid; i < clen; i += kAttThreads) {
                    const int pos = idx_sh[i];
                    int prow = -1;
                    if ((unsigned)pos < (unsigned)a.C) {
                        const int page = bt[pos >> a.page_shift];
                        if ((unsigned)page < (unsigned)a.num_pages)
                            prow = ((page * a.G + g) << a.page_shift) + (pos & pmask);
                    }
                    idx_sh[i] = prow;
                }
            }
            __syncthreads();
        }
        attend_chunk<H, D, DENSE, PAGED>(a, Kb, Vb, c0, clen, idx_sh, qw, m, l, acc);
    }
    attend_finish<H>(a, bg, qg, p, hq, h0, m, l, acc, red_ml, red_acc, &last_sh, true);
}

// Merge the P partials of every (b, g): thread -> (head, dim). Partials are read eight at a time, all loads of a group
// issued before any is used, with an online rescale between groups.
__global__ __launch_bounds__(1024) void attend_combine(AttendArgs a) {
    constexpr int kGroup = 8;
    const int bg = xcd_contiguous_block();   // the XCD whose attend workgroups wrote these partials
    const int h = a.h;
    const float* pb = a.part + (size_t)bg * a.P * h * (kHeadDim + 2);
    for (int idx = threadIdx.x; idx < h * kHeadDim; idx += blockDim.x) {
        const int i = idx / kHeadDim, dim = idx - i * kHeadDim;
        float ms = -INFINITY, ls = 0.0f, as = 0.0f;
        for (int q0 = 0; q0 < a.P; q0 += kGroup) {
            float mv[kGroup], lv[kGroup], av[kGroup];
#pragma unroll
            for (int u = 0; u < kGroup; ++u) {
                mv[u] = -INFINITY;
                lv[u] = av[u] = 0.0f;
                if (q0 + u < a.P) {
                    const float* pp = pb + ((size_t)(q0 + u) * h + i) * (kHeadDim + 2);
                    mv[u] = pp[0];
                    lv[u] = pp[1];
                    av[u] = pp[2 + dim];
                }
            }
            float mn = ms;
#pragma unroll
            for (int u = 0; u < kGroup; ++u) mn = fmaxf(mn, mv[u]);
            const float w0 = (ms == -INFINITY) ? 0.0f : fast_exp2(ms - mn);
            ls *= w0;
            as *= w0;
#pragma unroll
            for (int u = 0; u < kGroup; ++u) {
                const float w = (mv[u] == -INFINITY) ? 0.0f : fast_exp2(mv[u] - mn);
                ls += w * lv[u];
                as += w * av[u];
            }
            ms = mn;
        }
        store_out(a, ((size_t)bg * h + i) * kHeadDim + dim, as / ls);
    }
}

// Head groups per (b, g): split the h heads over 2, 4, ... workgroups while the grid is below one workgroup per CU.
// Workgroups of one (b, g) read the same rows at the same time on the same XCD, so the second read of a row comes from
// L2 (or the Infinity Cache) and HBM traffic stays one read per row; with P = 1 this replaces the split-K merge.
int attend_head_groups(int BG, int h, int P) {
    constexpr int kFillBlocks = 256;
    int Q = 1;
    while (h % (2 * Q) == 0 && (int64_t)BG * Q * P < kFillBlocks) Q *= 2;
    return Q;
}

template <bool DENSE, bool PAGED = false>
static int launch_attend(const AttendArgs& a, int BG, hipStream_t s) {
    const dim3 grid(BG * a.Q * a.P), block(kAttThreads);
    const int hq = a.h / a.Q;
    if (hq <= 1) hipLaunchKernelGGL((attend_kernel<1, kStages, DENSE, PAGED>), grid, block, 0, s, a);
    else if (hq <= 2) hipLaunchKernelGGL((attend_kernel<2, kStages, DENSE, PAGED>), grid, block, 0, s, a);
    else if (hq <= 4) hipLaunchKernelGGL((attend_kernel<4, kStages, DENSE, PAGED>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((attend_kernel<8, kStages, DENSE, PAGED>), grid, block, 0, s, a);
    if (a.P > 1 && a.arrive == nullptr) hipLaunchKernelGGL(attend_combine, dim3(BG), dim3(a.h * kHeadDim), 0, s, a);
    return check_launch(PAGED ? "attend_paged" : (DENSE ? "dense_decode" : "attend"));
}

static int check_common(const uint16_t* K, const uint16_t* V, int64_t kv_bg_stride, int kv_row_stride,
                        const uint16_t* q, int B, int G, int h, int C, int P, void* out, float* part) {
    ATTNLAB_REQUIRE(B >= 1 && G >= 1 && C >= 1, "B=%d G=%d C=%d must be positive", B, G, C);
    ATTNLAB_REQUIRE(1 <= h && h <= 8, "h=%d outside [1, 8]", h);
    ATTNLAB_REQUIRE(1 <= P && P <= 256, "partitions P=%d outside [1, 256]", P);
    ATTNLAB_REQUIRE(K && V && q && out, "K, V, q and out must be device pointers");
    ATTNLAB_REQUIRE(kv_row_stride >= kHeadDim && kv_row_stride % 8 == 0, "kv_row_stride=%d must be >= 128 and a multiple of 8",
                    kv_row_stride);
    ATTNLAB_REQUIRE(kv_bg_stride >= (int64_t)C * kv_row_stride, "kv_bg_stride too small for C=%d", C);
    ATTNLAB_REQUIRE(reinterpret_cast<uintptr_t>(K) % 16 == 0 && reinterpret_cast<uintptr_t>(V) % 16 == 0 &&
                        reinterpret_cast<uintptr_t>(q) % 16 == 0,
                    "K, V and q must be 16-byte aligned");
    ATTNLAB_REQUIRE(P == 1 || part != nullptr, "P > 1 needs the partial buffer");
    return ATTNLAB_OK;
}

}  // namespace attnlab

using namespace attnlab;

int attnlab::attend_impl(const uint16_t* K, const uint16_t* V, int64_t kv_bg_stride, int kv_row_stride,
                         const uint16_t* q, const int32_t* rows, int64_t rows_stride, int B, int G, int h, int S, int C,
                         int P, float scale, void* out, int out_bf16, float* part, uint32_t* arrive,
                         int64_t arrive_stride, hipStream_t stream) {
    const int rc = check_common(K, V, kv_bg_stride, kv_row_stride, q, B, G, h, C, P, out, part);
    if (rc) return rc;
    ATTNLAB_REQUIRE(S >= 1, "at least one row must be selected (S=%d)", S);
    ATTNLAB_REQUIRE(rows != nullptr && rows_stride >= S, "rows must hold S=%d positions per (b, g)", S);
    AttendArgs a{K, V, kv_bg_stride, kv_row_stride, q, rows, rows_stride, S, C, h, P, attend_head_groups(B * G, h, P),
                 scale * kLog2e, out, out_bf16, part};
    if (P > 1 && arrive != nullptr) {
        ATTNLAB_REQUIRE(a.Q <= kArriveWords && arrive_stride >= a.Q, "arrival counters too small for %d head groups",
                        a.Q);
        a.arrive = arrive;
        a.arrive_stride = arrive_stride;
    }
    return launch_attend<false>(a, B * G, stream);
}

extern "C" int attnlab_attend(const uint16_t* K, const uint16_t* V, int64_t kv_bg_stride, int kv_row_stride,
                              const uint16_t* q, const int32_t* rows, int64_t rows_stride, int B, int G, int h, int S,
                              int C, int P, float scale, void* out, int out_bf16, float* part, void* stream) {
    return attend_impl(K, V, kv_bg_stride, kv_row_stride, q, rows, rows_stride, B, G, h, S, C, P, scale, out, out_bf16,
                       part, nullptr, 0, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int attnlab_dense_decode(const uint16_t* K, const uint16_t* V, int64_t kv_bg_stride, int kv_row_stride,
                                    const uint16_t* q, int B, int G, int h, int L, int C, int P, float scale, void* out,
                                    int out_bf16, float* part, void* stream) {
    const int rc = check_common(K, V, kv_bg_stride, kv_row_stride, q, B, G, h, C, P, out, part);
    if (rc) return rc;
    ATTNLAB_REQUIRE(1 <= L && L <= C, "valid length L=%d outside [1, C=%d]", L, C);
    AttendArgs a{K, V, kv_bg_stride, kv_row_stride, q, nullptr, 0, L, C, h, P, attend_head_groups(B * G, h, P),
                 scale * kLog2e, out, out_bf16, part};
    return launch_attend<true>(a, B * G, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int attnlab_attend_paged(const uint16_t* K_pages, const uint16_t* V_pages, int num_pages, int page_size,
                                    const int32_t* block_table, int64_t bt_stride, int max_pages, const uint16_t* q,
                                    const int32_t* rows, int64_t rows_stride, int B, int G, int h, int S, int P,
                                    float scale, void* out, int out_bf16, float* part, void* stream) {
    ATTNLAB_REQUIRE(page_size >= 1 && page_size <= (1 << 16) && (page_size & (page_size - 1)) == 0,
                    "page_size=%d must be a power of two in [1, 65536]", page_size);
    ATTNLAB_REQUIRE(num_pages >= 1 && max_pages >= 1, "num_pages=%d and max_pages=%d must be positive", num_pages,
                    max_pages);
    ATTNLAB_REQUIRE((int64_t)max_pages * page_size <= INT32_MAX, "max_pages * page_size exceeds 2^31 positions");
    const int C = max_pages * page_size;   // logical capacity of one sequence
    const int rc = check_common(K_pages, V_pages, (int64_t)C * kHeadDim, kHeadDim, q, B, G, h, C, P, out, part);
    if (rc) return rc;
    ATTNLAB_REQUIRE((int64_t)num_pages * G * page_size <= INT32_MAX, "the pool of %d pages x %d groups x %d rows "
                    "exceeds 2^31 rows", num_pages, G, page_size);
    ATTNLAB_REQUIRE(block_table != nullptr && bt_stride >= max_pages, "block_table must hold max_pages=%d entries per "
                    "sequence", max_pages);
    ATTNLAB_REQUIRE(S >= 1, "at least one row must be selected (S=%d)", S);
    ATTNLAB_REQUIRE(rows == nullptr ? S <= C : rows_stride >= S, "rows must hold S=%d positions per (b, g) (or be "
                    "null with S <= max_pages * page_size)", S);
    AttendArgs a{K_pages, V_pages, 0, kHeadDim, q, rows, rows_stride, S, C, h, P, attend_head_groups(B * G, h, P),
                 scale * kLog2e, out, out_bf16, part};
    a.block_table = block_table;
    a.bt_stride = bt_stride;
    a.G = G;
    a.num_pages = num_pages;
    while ((1 << a.page_shift) < page_size) ++a.page_shift;
    return launch_attend<false, true>(a, B * G, reinterpret_cast<hipStream_t>(stream));
}
