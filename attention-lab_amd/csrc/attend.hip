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
#include "common.h"
#include "select.h"

namespace attnlab {

constexpr int kHeadDim = 128;
constexpr int kAttThreads = 256;
constexpr int kAttWaves = kAttThreads / 64;
constexpr float kLazyRescale = 8.0f;     // log2-domain slack of the running max
constexpr int kStages = 4;               // K/V groups per wave in registers: D - 1 in flight while one is computed
constexpr int kMergeSlots = 4 * kAttWaves;  // slots left after the in-register pair merge (4 per wave)

struct AttendArgs {
    const uint16_t* K;
    const uint16_t* V;
    int64_t kv_bg_stride;
    int kv_row_stride;
    const uint16_t* q;  // [BG, h, 128]
    const int32_t* rows;
    int64_t rows_stride;
    int S;  // positions per (b, g): the row list length, or L for the dense read
    int C;  // capacity: listed positions outside [0, C) are skipped, never read
    int h, P;
    int Q;  // head groups: workgroup (b, g, qg, p) attends heads [qg h/Q, (qg + 1) h/Q) over partition p
    float scale_log2;
    void* out;
    int out_bf16;
    float* part;  // [BG, P, h, 130]: m, l, acc[128]
    // paged layout (attend_kernel<..., PAGED = true>): K and V are pools of pages [pages, G, page, 128]; position p of
    // (b, g) lives in row (block_table[b][p >> page_shift] * G + g) * page + (p & (page - 1)) of the pool. rows may be
    // null there: the positions are then [0, S).
    const int32_t* block_table = nullptr;
    int64_t bt_stride = 0;
    int G = 1, page_shift = 0, num_pages = 0;
    // in-kernel split-K merge (P > 1): arrival counters, one per (b, g, head group) at arrive[bg * arrive_stride + qg],
    // zero on entry and left zero; the partition workgroup that arrives last merges the P partials. Null: the combine
    // kernel merges them.
    uint32_t* arrive = nullptr;
    int64_t arrive_stride = 0;
};

__device__ __forceinline__ void merge_state(float& m, float& l, float& m2, float& l2, float& w1, float& w2) {
    const float mn = fmaxf(m, m2);
    w1 = (m == -INFINITY) ? 0.0f : fast_exp2(m - mn);
    w2 = (m2 == -INFINITY) ? 0.0f : fast_exp2(m2 - mn);
    l = w1 * l + w2 * l2;
    m = mn;
}

// A partial's words for the in-kernel merge, written and read at system scope (past the L2 of the writing XCD).
__device__ __forceinline__ void store_coherent(float* p, float v) {
    __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ float load_coherent(const float* p) {
    return __uint_as_float(__hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_SYSTEM));
}

__device__ __forceinline__ void store_out(const AttendArgs& a, size_t idx, float v) {
    if (a.out_bf16) reinterpret_cast<uint16_t*>(a.out)[idx] = f32_to_bf16_rne(v);
    else reinterpret_cast<float*>(a.out)[idx] = v;
}

// One pipeline stage of a wave: this lane's 16-byte words of the K and V rows of its slot's position.
struct KVStage {
    u32x4_t k0, k1, v0, v1;
    bool ok;   // the entry exists and its position is inside [0, C)
};

template <int H, int D, bool DENSE, bool PAGED = false>
__global__ __launch_bounds__(kAttThreads) void attend_kernel(AttendArgs a) {
    static_assert(!(DENSE && PAGED), "the paged read lists its positions (rows, or [0, S) when rows is null)");
    constexpr int kChunk = 4096;   // row-list entries whose positions are staged in LDS at a time (one chunk for k <= 4096)
    __shared__ __attribute__((aligned(16))) int idx_sh[DENSE ? 4 : kChunk];
    __shared__ float red_ml[kMergeSlots][H][2];
    __shared__ __attribute__((aligned(16))) float red_acc[kMergeSlots][H][kHeadDim];
    const int lin = xcd_contiguous_block();   // (b, g) on the XCD that wrote its row list
    const int bg = lin / (a.Q * a.P);
    const int rem = lin - bg * a.Q * a.P;
    const int qg = rem / a.P;
    const int p = rem - qg * a.P;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int slot = lane >> 3;
    const int sub = lane & 7;
    const int h = a.h;          // heads of the KV group (the row stride of q, out and part)
    const int hq = h / a.Q;     // heads of this workgroup
    const int h0 = qg * hq;

    uint32_t qw[H][8];
#pragma unroll
    for (int i = 0; i < H; ++i) {
        uint4 x0 = make_uint4(0, 0, 0, 0), x1 = make_uint4(0, 0, 0, 0);
        if (i < hq) {
            const uint16_t* qp = a.q + ((size_t)bg * h + h0 + i) * kHeadDim + 8 * sub;
            x0 = *reinterpret_cast<const uint4*>(qp);
            x1 = *reinterpret_cast<const uint4*>(qp + 64);
        }
        qw[i][0] = x0.x; qw[i][1] = x0.y; qw[i][2] = x0.z; qw[i][3] = x0.w;
        qw[i][4] = x1.x; qw[i][5] = x1.y; qw[i][6] = x1.z; qw[i][7] = x1.w;
    }

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
        // The chunk's entries form groups of 8 (one per slot of a wave); wave w takes groups w, w + kAttWaves, ...
        const int ng = (clen + 7) / 8;
        const int my_ng = ng > wave ? (ng - wave + kAttWaves - 1) / kAttWaves : 0;
        // Group j of this wave -> a register stage: four 16-byte loads per lane (K lo, K hi, V lo, V hi of its slot's
        // row). Entries past the chunk (also whole groups past the wave's last) or outside [0, C) load row 0, which is
        // in bounds, and are masked in compute. No branch: every path issues the same loads, so the compiler's wait
        // before a stage is used counts exactly the 4 (D - 1) loads issued after it.
        auto issue = [&](int j, KVStage& s) {
            const int e = (wave + kAttWaves * j) * 8 + slot;
            int pos = DENSE ? c0 + e : idx_sh[min(e, clen - 1)];
            const bool ok = e < clen && (DENSE || (PAGED ? pos >= 0 : (unsigned)pos < (unsigned)a.C));
            pos = ok ? pos : 0;
            const size_t off = (size_t)pos * a.kv_row_stride;
            s.k0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(Kb + off));
            s.k1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(Kb + off + 64));
            s.v0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(Vb + off));
            s.v1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(Vb + off + 64));
            s.ok = ok;
        };
        auto compute = [&](const KVStage& s) {
            float sc[H];
#pragma unroll
            for (int i = 0; i < H; ++i) {
                float d = 0.0f;
                d = dot2_bf16(qw[i][0], s.k0.x, d);
                d = dot2_bf16(qw[i][1], s.k0.y, d);
                d = dot2_bf16(qw[i][2], s.k0.z, d);
                d = dot2_bf16(qw[i][3], s.k0.w, d);
                d = dot2_bf16(qw[i][4], s.k1.x, d);
                d = dot2_bf16(qw[i][5], s.k1.y, d);
                d = dot2_bf16(qw[i][6], s.k1.z, d);
                d = dot2_bf16(qw[i][7], s.k1.w, d);
                d = sum8(d);
                sc[i] = s.ok ? d * a.scale_log2 : -INFINITY;
                if (sc[i] > m[i] + kLazyRescale) {
                    const float al = fast_exp2(m[i] - sc[i]);
                    l[i] *= al;
#pragma unroll
                    for (int q = 0; q < 16; ++q) acc[i][q] *= al;
                    m[i] = sc[i];
                }
            }
            float vf[16];
            // a masked entry loaded row 0 in its place: its V words are zeroed so that a non-finite row 0 (a padded
            // slot of a gathered subset, say) cannot turn its zero weight into NaN
            const uint32_t vm = s.ok ? 0xffffffffu : 0u;
            const uint32_t vw[8] = {s.v0.x & vm, s.v0.y & vm, s.v0.z & vm, s.v0.w & vm,
                                    s.v1.x & vm, s.v1.y & vm, s.v1.z & vm, s.v1.w & vm};
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                vf[2 * w] = bf16_lo(vw[w]);
                vf[2 * w + 1] = bf16_hi(vw[w]);
            }
#pragma unroll
            for (int i = 0; i < H; ++i) {
                const float pr = s.ok ? fast_exp2(sc[i] - m[i]) : 0.0f;
                l[i] += pr;
#pragma unroll
                for (int q = 0; q < 16; ++q) acc[i][q] += pr * vf[q];
            }
        };
        // D register stages rotate: while group j is computed, groups j + 1 .. j + D - 1 are in flight. The main loop
        // runs whole blocks of D groups, unrolled so that every stage index is a constant (the stages stay in
        // registers) and with its only exit at the block's end, so the wait before each stage's use stays exact.
        // The last < D groups are already in flight when it ends; the tail only computes them.
        if (my_ng > 0) {
            KVStage st[D];
#pragma unroll
            for (int u = 0; u < D - 1; ++u) issue(u, st[u]);
            int j = 0;
            for (; j + D <= my_ng; j += D) {
#pragma unroll
                for (int u = 0; u < D; ++u) {
                    issue(j + u + D - 1, st[(u + D - 1) % D]);
                    compute(st[u]);
                }
            }
#pragma unroll
            for (int u = 0; u < D - 1; ++u)
                if (j + u < my_ng) compute(st[u]);
        }
    }

    // Merge the 32 slots of the block: slots 2s and 2s + 1 (lane ^ 8, DPP row_ror:8) in registers, then the 16
    // merged slots through LDS, where every thread reduces whole (head, dim) columns. The register-only merge over
    // lane ^ 16 and lane ^ 32 that this replaces took about 2 us per workgroup on MI355X.
#pragma unroll
    for (int i = 0; i < H; ++i) {
        float m2 = dpp_f32<0x128>(m[i]), l2 = dpp_f32<0x128>(l[i]);
        float w1, w2;
        merge_state(m[i], l[i], m2, l2, w1, w2);
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = w1 * acc[i][e] + w2 * dpp_f32<0x128>(acc[i][e]);
    }
    const int rs = wave * 4 + (lane >> 4);   // merged slot: one per 16-lane row
    if ((lane & 15) < 8) {
#pragma unroll
        for (int i = 0; i < H; ++i) {
            if (sub == 0) {
                red_ml[rs][i][0] = m[i];
                red_ml[rs][i][1] = l[i];
            }
            float4* r0 = reinterpret_cast<float4*>(&red_acc[rs][i][8 * sub]);
            float4* r1 = reinterpret_cast<float4*>(&red_acc[rs][i][64 + 8 * sub]);
            r0[0] = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
            r0[1] = make_float4(acc[i][4], acc[i][5], acc[i][6], acc[i][7]);
            r1[0] = make_float4(acc[i][8], acc[i][9], acc[i][10], acc[i][11]);
            r1[1] = make_float4(acc[i][12], acc[i][13], acc[i][14], acc[i][15]);
        }
    }
    __syncthreads();
    // this thread's (head, dim) items: idx = tid + kAttThreads * t (hq * 128 <= 1024 items)
    constexpr int kItems = (H * kHeadDim + kAttThreads - 1) / kAttThreads;
    float own_m[kItems], own_l[kItems], own_a[kItems];
    const bool merge_here = a.P > 1 && a.arrive != nullptr;
#pragma unroll
    for (int t = 0; t < kItems; ++t) {
        const int idx = tid + kAttThreads * t;
        if (idx >= hq * kHeadDim) break;
        const int i = idx / kHeadDim, dim = idx - i * kHeadDim;
        float ms = -INFINITY;
#pragma unroll
        for (int w = 0; w < kMergeSlots; ++w) ms = fmaxf(ms, red_ml[w][i][0]);
        float ls = 0.0f, as = 0.0f;
#pragma unroll
        for (int w = 0; w < kMergeSlots; ++w) {
            const float mw = red_ml[w][i][0];
            const float ww = (mw == -INFINITY) ? 0.0f : fast_exp2(mw - ms);
            ls += ww * red_ml[w][i][1];
            as += ww * red_acc[w][i][dim];
        }
        own_m[t] = ms;
        own_l[t] = ls;
        own_a[t] = as;
        if (a.P == 1) {
            store_out(a, ((size_t)bg * h + h0 + i) * kHeadDim + dim, as / ls);
        } else {
            float* pp = a.part + (((size_t)bg * a.P + p) * h + h0 + i) * (kHeadDim + 2);
            if (merge_here) {
                // system scope: written through to memory, so the merging workgroup reads them on any XCD
                if (dim == 0) {
                    store_coherent(pp, ms);
                    store_coherent(pp + 1, ls);
                }
                store_coherent(pp + 2 + dim, as);
            } else {
                if (dim == 0) {
                    pp[0] = ms;
                    pp[1] = ls;
                }
                pp[2 + dim] = as;
            }
        }
    }
    if (!merge_here) return;
    // Arrival: every partial store of this workgroup has completed before its counter increment (the wait and the
    // barrier); the workgroup that sees P - 1 earlier arrivals therefore finds every other partial in memory.
    __shared__ uint32_t last_sh;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    uint32_t* counter = a.arrive + (size_t)bg * a.arrive_stride + qg;
    if (tid == 0)
        last_sh = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(a.P - 1);
    __syncthreads();
    if (!last_sh) return;
    // The last arrival merges the P partials of its heads in partition order, eight at a time with an online rescale:
    // the arithmetic of attend_combine, so the output is the same bit for bit. Its own partial comes from registers.
#pragma unroll
    for (int t = 0; t < kItems; ++t) {
        const int idx = tid + kAttThreads * t;
        if (idx >= hq * kHeadDim) break;
        const int i = idx / kHeadDim, dim = idx - i * kHeadDim;
        const float* pb = a.part + ((size_t)bg * a.P * h + h0 + i) * (kHeadDim + 2);
        float ms = -INFINITY, ls = 0.0f, as = 0.0f;
        for (int q0 = 0; q0 < a.P; q0 += 8) {
            float mv[8], lv[8], av[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                mv[u] = -INFINITY;
                lv[u] = av[u] = 0.0f;
                const int pq = q0 + u;
                if (pq == p) {
                    mv[u] = own_m[t];
                    lv[u] = own_l[t];
                    av[u] = own_a[t];
                } else if (pq < a.P) {
                    const float* pp = pb + (size_t)pq * h * (kHeadDim + 2);
                    mv[u] = load_coherent(pp);
                    lv[u] = load_coherent(pp + 1);
                    av[u] = load_coherent(pp + 2 + dim);
                }
            }
            float mn = ms;
#pragma unroll
            for (int u = 0; u < 8; ++u) mn = fmaxf(mn, mv[u]);
            const float w0 = (ms == -INFINITY) ? 0.0f : fast_exp2(ms - mn);
            ls *= w0;
            as *= w0;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float w = (mv[u] == -INFINITY) ? 0.0f : fast_exp2(mv[u] - mn);
                ls += w * lv[u];
                as += w * av[u];
            }
            ms = mn;
        }
        store_out(a, ((size_t)bg * h + h0 + i) * kHeadDim + dim, as / ls);
    }
    if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);   // leave it zero
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
static int head_groups(int BG, int h, int P) {
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
    AttendArgs a{K, V, kv_bg_stride, kv_row_stride, q, rows, rows_stride, S, C, h, P, head_groups(B * G, h, P),
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
    AttendArgs a{K, V, kv_bg_stride, kv_row_stride, q, nullptr, 0, L, C, h, P, head_groups(B * G, h, P),
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
    AttendArgs a{K_pages, V_pages, 0, kHeadDim, q, rows, rows_stride, S, C, h, P, head_groups(B * G, h, P),
                 scale * kLog2e, out, out_bf16, part};
    a.block_table = block_table;
    a.bt_stride = bt_stride;
    a.G = G;
    a.num_pages = num_pages;
    while ((1 << a.page_shift) < page_size) ++a.page_shift;
    return launch_attend<false, true>(a, B * G, reinterpret_cast<hipStream_t>(stream));
}
