// One layer's sparse decode read as a single C-ABI call: score (z column + u + candidate scan + first-digit
// histogram) -> select (top-k + F merge) -> gather-free attend (+ split-K merge), launched in order on the caller's
// stream with the intermediate scores, select scratch and row list in a caller-provided workspace. Counterpart of
// sparse_decode_step_kernel (decode.py:145-163).
#include <algorithm>

#include "common.h"
#include "select.h"

namespace {

constexpr int64_t kAlign = 256;

inline int64_t align_up(int64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

struct Layout {
    int64_t scores, rows, u, sel, part, total;
    int64_t score_stride;
};

// Workspace layout: scores [BG, round_up(M, 4)] fp32 | rows [BG, S] int32 | u [BG, 32] fp32 | select scratch: either
// the tiled select's bitmaps and candidate entries (and for k past the LDS sort the score-order sort's buffers, sized
// for score order so either order fits) or the score kernel's per-workgroup key lists, whichever is larger, since a
// step uses one of them | partials [BG, P, h, 130] fp32. Nothing here needs to start at zero. The select state
// (first-digit histograms, which must start at zero) lives in its own buffer: a region inside this shape-dependent
// layout would overlap other data of a differently shaped earlier call.
Layout layout_of(int B, int G, int h, int lo, int hi, int legal, int k, int P) {
    Layout L{};
    const int64_t BG = (int64_t)B * G;
    const int64_t M = hi - lo;
    const int64_t S = lo + (legal - hi) + k;
    L.score_stride = (M + 3) / 4 * 4;
    L.scores = 0;
    L.rows = align_up(k > 0 ? BG * L.score_stride * 4 : 0);
    L.u = L.rows + align_up(BG * S * 4);
    L.sel = L.u + align_up(k > 0 ? BG * 32 * 4 : 0);
    const int64_t sel = k > 0 ? attnlab::select_scratch_bytes((int)BG, (int)M, k, ATTNLAB_ORDER_SCORE) : 0;
    L.part = L.sel + align_up(std::max(sel, attnlab::list_region_bytes(BG, lo, hi, k)));
    L.total = L.part + align_up(P > 1 ? BG * P * h * 130 * 4 : 0);
    return L;
}

}  // namespace

extern "C" int64_t attnlab_sparse_decode_workspace(int B, int G, int h, int lo, int hi, int legal, int k, int P) {
    if (B < 1 || G < 1 || h < 1 || lo < 0 || hi < lo || legal < hi || k < 0 || P < 1) return -1;
    return layout_of(B, G, h, lo, hi, legal, k, P).total;
}

namespace {

// The launches of one step after the argument checks; score(ws_u, scores, stride, state, lists) runs the score stage
// for the index table's dtype. `geo` is the one-launch score's tiling when the score stage runs it (bf16 or float32
// tables), else nsub == 0; with it, and where list_plan applies, the score kernel also writes per-workgroup key lists
// and the list select replaces the tiled select.
template <typename Score>
int sparse_decode_step_impl(const uint16_t* q_main, const uint16_t* K, const uint16_t* V, bool has_k_new, int B,
                            int G, int h, int C, int lo, int hi, int legal, int k, float scale, int order, int P,
                            uint32_t* state, void* workspace, int64_t workspace_bytes, int32_t* rows_out,
                            int64_t* rows_flat, uint16_t* out, void* stream, attnlab::FusedGeometry geo,
                            const void* zT, int z_dtype, Score score) {
    using namespace attnlab;
    ATTNLAB_REQUIRE(B >= 1 && G >= 1 && h >= 1 && h <= 8, "B=%d G=%d h=%d out of range", B, G, h);
    ATTNLAB_REQUIRE(0 <= lo && lo <= hi && hi <= legal && legal <= C, "need 0 <= lo <= hi <= legal <= C, got %d %d %d %d",
                    lo, hi, legal, C);
    ATTNLAB_REQUIRE(0 <= k && k <= hi - lo, "need 0 <= k <= hi - lo, got k=%d M=%d", k, hi - lo);
    ATTNLAB_REQUIRE(1 <= P && P <= 64, "partitions P=%d outside [1, 64]", P);
    const Layout L = layout_of(B, G, h, lo, hi, legal, k, P);
    ATTNLAB_REQUIRE(workspace != nullptr && workspace_bytes >= L.total, "workspace of %lld bytes needed, got %lld",
                    (long long)L.total, (long long)workspace_bytes);
    ATTNLAB_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % kAlign == 0, "workspace must be 256-byte aligned");
    // the attend's own checks, here so that the one-launch select and attend cannot refuse the call after the score
    ATTNLAB_REQUIRE(q_main && K && V && out, "q_main, K, V and out must be device pointers");
    ATTNLAB_REQUIRE(reinterpret_cast<uintptr_t>(K) % 16 == 0 && reinterpret_cast<uintptr_t>(V) % 16 == 0 &&
                        reinterpret_cast<uintptr_t>(q_main) % 16 == 0,
                    "K, V and q_main must be 16-byte aligned");
    // every check of the select before the first launch: the score kernel adds into the select state, which only the
    // select clears, so a call rejected after the score launch would leave it dirty for the next call
    {
        const int rc0 = select_check(B, G, lo, hi, legal, k, C, order, rows_out, lo + (legal - hi) + k,
                                     reinterpret_cast<const float*>(workspace), L.score_stride);
        if (rc0) return rc0;
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    char* ws = static_cast<char*>(workspace);
    if (k == 0) state = nullptr;
    // no row list leaves the call: its order shows only in the attend's summation order, so take the faster select
    if (!rows_out && !rows_flat) order = ATTNLAB_ORDER_POSITION;
    float* scores = reinterpret_cast<float*>(ws + L.scores);
    int32_t* rows = rows_out ? rows_out : reinterpret_cast<int32_t*>(ws + L.rows);
    float* part = P > 1 ? reinterpret_cast<float*>(ws + L.part) : nullptr;
    const int S = lo + (legal - hi) + k;
    const int d = 128;
    // the list select (it needs the select state, and sorts at most kMaxScoreOrderK picks by score): lists in the
    // select scratch region; otherwise the tiled select, whose scratch (sized for score order) holds the radix sort's
    // buffers
    const ListPlan plan = k > 0 && state && !staged_score_order(order, k) ? list_plan(hi - lo, k, geo) : ListPlan{0, 0};
    const ScoreLists lists = plan.cap > 0 ? list_layout(ws + L.sel, B * G, geo, plan) : ScoreLists{};
    // Stored scores are read only by the tiled select and by score order (which reads the picks' scores back to sort
    // them); the list select in position order recomputes the rare tile it needs from the table and u, so the score
    // kernel then writes key lists only.
    const bool store_scores = plan.cap == 0 || order == ATTNLAB_ORDER_SCORE;
    float* u_ws = reinterpret_cast<float*>(ws + L.u);
    int rc;
    if (k > 0) {
        // u goes to the workspace (the score kernels that build it in-kernel also store it there)
        rc = score(u_ws, store_scores ? scores : nullptr, L.score_stride, lo, hi, state, plan.cap > 0 ? &lists : nullptr,
                   s);
    } else if (has_k_new) {
        // no candidate is read this step, but the newest key still gets its index column (empty scan range)
        rc = score(nullptr, nullptr, 0, lo, lo, nullptr, nullptr, s);
    } else {
        rc = ATTNLAB_OK;
    }
    if (rc) return rc;
    // no row list leaves the call: select and attend in one launch, the row list kept in LDS (the same output bits)
    if (plan.cap > 0 && !rows_out && !rows_flat && select_attend_applies(B, G, lo, hi, legal, k, h, P))
        return select_attend_impl(B, G, lo, hi, legal, k, C, state, lists, geo, TableRef{zT, z_dtype, C, u_ws}, K, V,
                                  q_main, h, P, scale, out, part, s);
    if (plan.cap > 0)
        rc = select_lists_impl(store_scores ? scores : nullptr, L.score_stride, B, G, lo, hi, legal, k, C, order, rows,
                               S, rows_flat, state, lists, geo, s, TableRef{zT, z_dtype, C, u_ws});
    else
        rc = select_rows_impl(scores, L.score_stride, B, G, lo, hi, legal, k, C, order, rows, S, rows_flat, state,
                              k > 0 ? ws + L.sel : nullptr, L.part - L.sel, s);
    if (rc) return rc;
    // with the select state (k > 0) the attend merges its split-K partials itself, counting arrivals in the state's
    // counter words (the select has just zeroed them); without it the combine kernel merges them
    return attend_impl(K, V, (int64_t)C * d, d, q_main, rows, S, B, G, h, S, C, P, scale, out, 1, part,
                       state ? state + kArriveOffset : nullptr, kSelectStateWords, s);
}

}  // namespace

extern "C" int attnlab_sparse_decode_step(const uint16_t* q_main, const uint16_t* q_cat, const uint16_t* K,
                                          const uint16_t* V, uint16_t* zT, const uint16_t* wq_t, const uint16_t* wk,
                                          const uint16_t* k_new, int B, int G, int h, int r, int C, int lo, int hi,
                                          int legal, int k, int write_col, float scale, int order, int P,
                                          uint32_t* state, void* workspace, int64_t workspace_bytes,
                                          int32_t* rows_out, int64_t* rows_flat, uint16_t* out, void* stream) {
    return sparse_decode_step_impl(
        q_main, K, V, k_new != nullptr, B, G, h, C, lo, hi, legal, k, scale, order, P, state, workspace,
        workspace_bytes, rows_out, rows_flat, out, stream,
        attnlab::fused_geometry(B * G, C, r, h * 128, lo, hi, zT, false), zT, ATTNLAB_DT_BF16,
        [&](float* u_ws, float* scores, int64_t stride, int slo, int shi, uint32_t* st, const attnlab::ScoreLists* ls,
            hipStream_t s) {
            return attnlab::score_grouped_impl(zT, k_new, wk, q_cat, wq_t, nullptr, u_ws, scores, stride, B, G, r, C,
                                               128, h * 128, slo, shi, write_col, 1, st, s, ls);
        });
}

extern "C" int attnlab_sparse_decode_step_f32(const uint16_t* q_main, const float* q_cat, const uint16_t* K,
                                              const uint16_t* V, float* zT, const float* wq_t, const float* wk,
                                              const float* k_new, int B, int G, int h, int r, int C, int lo, int hi,
                                              int legal, int k, int write_col, float scale, int order, int P,
                                              uint32_t* state, void* workspace, int64_t workspace_bytes,
                                              int32_t* rows_out, int64_t* rows_flat, uint16_t* out, void* stream) {
    return sparse_decode_step_impl(
        q_main, K, V, k_new != nullptr, B, G, h, C, lo, hi, legal, k, scale, order, P, state, workspace,
        workspace_bytes, rows_out, rows_flat, out, stream,
        attnlab::fused_geometry_f32(B * G, C, r, h * 128, lo, hi, zT, wq_t, false), zT, ATTNLAB_DT_F32,
        [&](float* u_ws, float* scores, int64_t stride, int slo, int shi, uint32_t* st, const attnlab::ScoreLists* ls,
            hipStream_t s) {
            return attnlab::score_grouped_f32_impl(zT, k_new, wk, q_cat, wq_t, nullptr, u_ws, scores, stride, B, G, r,
                                                   C, 128, h * 128, slo, shi, write_col, st, s, ls);
        });
}

// ---------------------------------------------------------------------------------------------------------------
// attnlab_sparse_decode_step_noalloc: the bf16 step with its select state and workspace in a file-scope device array
// instead of caller buffers, for callers that cannot allocate. The array's device address comes from
// hipGetSymbolAddress once per device (the array's name is only a host-side stand-in); every call on a device shares
// that device's copy, so calls that overlap on one device race. Layout: the select state of up to kNoAllocRows rows at
// the start (it must read zero at the start of a call: it is cleared by a fill kernel on a device's first call and
// after any failed call, and every completed call leaves the rows it used zeroed), then the step's workspace.
// ---------------------------------------------------------------------------------------------------------------
#include <mutex>

namespace {

constexpr int64_t kNoAllocBytes = 32ll << 20;   // 32 MiB per device, held until the process ends
constexpr int kNoAllocRows = 256;                // B * G rows of select state
constexpr int64_t kNoAllocStateBytes = (int64_t)kNoAllocRows * ATTNLAB_SELECT_STATE_WORDS * 4;
constexpr int kNoAllocMaxDevices = 64;
static_assert(kNoAllocStateBytes % kAlign == 0, "the workspace after the state stays 256-byte aligned");

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

struct NoAllocDevice {
    char* ptr = nullptr;   // device address of `scratch` on this device
    bool state_dirty = true;
};
std::mutex g_noalloc_mu;
NoAllocDevice g_noalloc[kNoAllocMaxDevices];

__global__ __launch_bounds__(256) void noalloc_clear_state(uint4* p, int64_t n16) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

}  // namespace

extern "C" int attnlab_sparse_decode_step_noalloc(const uint16_t* q_main, const uint16_t* q_cat, const uint16_t* K,
                                                  const uint16_t* V, uint16_t* zT, const uint16_t* wq_t,
                                                  const uint16_t* wk, const uint16_t* k_new, int B, int G, int h, int r,
                                                  int C, int lo, int hi, int legal, int k, int write_col, float scale,
                                                  int order, int P, int32_t* rows_out, int64_t* rows_flat,
                                                  uint16_t* out, void* stream) {
    using namespace attnlab;
    ATTNLAB_REQUIRE(B >= 1 && G >= 1 && (int64_t)B * G <= kNoAllocRows, "B*G=%lld rows exceed the %d of the no-allocation "
                    "entry point", (long long)B * G, kNoAllocRows);
    const int64_t ws = attnlab_sparse_decode_workspace(B, G, h, lo, hi, legal, k, P);
    ATTNLAB_REQUIRE(ws >= 0, "invalid sizes B=%d G=%d h=%d lo=%d hi=%d legal=%d k=%d P=%d", B, G, h, lo, hi, legal, k, P);
    ATTNLAB_REQUIRE(kNoAllocStateBytes + ws <= kNoAllocBytes, "this step needs %lld bytes of workspace; the no-allocation "
                    "entry point holds %lld", (long long)ws, (long long)(kNoAllocBytes - kNoAllocStateBytes));
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(ATTNLAB_ERUNTIME, "hipGetDevice: %s", hipGetErrorString(e));
    ATTNLAB_REQUIRE(dev >= 0 && dev < kNoAllocMaxDevices, "device %d outside the %d the library tracks", dev,
                    kNoAllocMaxDevices);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    char* base;
    {
        std::lock_guard<std::mutex> lock(g_noalloc_mu);
        NoAllocDevice& d = g_noalloc[dev];
        if (d.ptr == nullptr) {
            void* p = nullptr;
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || p == nullptr)
                return set_error(ATTNLAB_ERUNTIME, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
            d.ptr = static_cast<char*>(p);
        }
        if (d.state_dirty) {
            hipLaunchKernelGGL(noalloc_clear_state, dim3(512), dim3(256), 0, s, reinterpret_cast<uint4*>(d.ptr),
                               kNoAllocStateBytes / 16);
            const int rc = check_launch("noalloc_clear_state");
            if (rc) return rc;
            d.state_dirty = false;
        }
        base = d.ptr;
    }
    const int rc = attnlab_sparse_decode_step(q_main, q_cat, K, V, zT, wq_t, wk, k_new, B, G, h, r, C, lo, hi, legal, k,
                                              write_col, scale, order, P, reinterpret_cast<uint32_t*>(base),
                                              base + kNoAllocStateBytes, kNoAllocBytes - kNoAllocStateBytes, rows_out,
                                              rows_flat, out, stream);
    if (rc != ATTNLAB_OK) {   // a launch may have run before the failure: clear the state before the next call
        std::lock_guard<std::mutex> lock(g_noalloc_mu);
        g_noalloc[dev].state_dirty = true;
    }
    return rc;
}
