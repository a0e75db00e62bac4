// The gather-free attend's per-workgroup phases (shared by attend_kernel and the fused select + attend of the decode
// step): q for the workgroup's heads, the D-stage K/V pipeline over one chunk of staged positions, and the slot,
// workgroup and split-K merges with the outputs. The attending threads are the workgroup's first four waves; in a
// larger workgroup the other waves pass `active = false` to attend_finish and only keep its barriers.
#pragma once

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

// The workgroup's q: lane `sub` of a position holds dims [8 sub, 8 sub + 8) and [64 + 8 sub, 64 + 8 sub + 8) of each
// of its hq heads (h0 ..), zero for the heads past hq.
template <int H>
__device__ __forceinline__ void attend_load_q(const AttendArgs& a, int bg, int h0, int hq, uint32_t (&qw)[H][8]) {
    const int sub = threadIdx.x & 7;
#pragma unroll
    for (int i = 0; i < H; ++i) {
        uint4 x0 = make_uint4(0, 0, 0, 0), x1 = make_uint4(0, 0, 0, 0);
        if (i < hq) {
            const uint16_t* qp = a.q + ((size_t)bg * a.h + h0 + i) * kHeadDim + 8 * sub;
            x0 = *reinterpret_cast<const uint4*>(qp);
            x1 = *reinterpret_cast<const uint4*>(qp + 64);
        }
        qw[i][0] = x0.x; qw[i][1] = x0.y; qw[i][2] = x0.z; qw[i][3] = x0.w;
        qw[i][4] = x1.x; qw[i][5] = x1.y; qw[i][6] = x1.z; qw[i][7] = x1.w;
    }
}

// One chunk of clen positions (idx_sh[0, clen), staged; or c0 + e for the dense read) through waves 0..3's pipeline,
// accumulated into the thread's online-softmax state. Kb / Vb: the (b, g) cache base plus the lane's 8 sub dims.
template <int H, int D, bool DENSE, bool PAGED>
__device__ __forceinline__ void attend_chunk(const AttendArgs& a, const uint16_t* Kb, const uint16_t* Vb, int c0,
                                             int clen, const int* idx_sh, const uint32_t (&qw)[H][8], float (&m)[H],
                                             float (&l)[H], float (&acc)[H][16]) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slot = lane >> 3;
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

// The workgroup's merges: the 32 slots of the four attending waves, then its output (P = 1) or its split-K partial, and
// with the arrival counters the in-kernel merge of the P partials by the last partition to arrive. Called by every
// thread of the workgroup; `active`: the thread belongs to the four attending waves.
template <int H>
__device__ __forceinline__ void attend_finish(const AttendArgs& a, int bg, int qg, int p, int hq, int h0, float (&m)[H],
                                              float (&l)[H], float (&acc)[H][16], float (*red_ml)[H][2],
                                              float (*red_acc)[H][kHeadDim], uint32_t* last_sh, bool active) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sub = lane & 7;
    const int h = a.h;
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
    if (active && (lane & 15) < 8) {
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
        if (!active || idx >= hq * kHeadDim) break;
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
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    uint32_t* counter = a.arrive + (size_t)bg * a.arrive_stride + qg;
    if (tid == 0)
        *last_sh = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(a.P - 1);
    __syncthreads();
    if (!*last_sh) return;
    // The last arrival merges the P partials of its heads in partition order, eight at a time with an online rescale:
    // the arithmetic of attend_combine, so the output is the same bit for bit. Its own partial comes from registers.
#pragma unroll
    for (int t = 0; t < kItems; ++t) {
        const int idx = tid + kAttThreads * t;
        if (!active || idx >= hq * kHeadDim) break;
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

}  // namespace attnlab
