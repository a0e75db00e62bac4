// Measurement only: the read ceiling of the gather-free attend. attnlab_gather_probe reads exactly the K/V rows the
// attend kernel reads, in the same grid (one workgroup of 4 waves per (b, g, head group, partition), XCD-contiguous
// numbering), the same lane layout (8 lanes per position, one 16-byte non-temporal load per lane and half-row) and the
// same pipeline depth (while one group of 8 positions is folded, the next three are in flight), but does no arithmetic
// beyond XOR-folding the loaded words into one register per thread; each thread stores that word, so no load can be
// dropped. Its time against the attend's over the same row lists separates the cost of reading the rows from the cost of
// the softmax, the merge and the prologue. No reference counterpart.
#include "common.h"

namespace attnlab {
namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeWaves = kProbeThreads / 64;
constexpr int kProbeChunk = 4096;
constexpr int kProbeStages = 4;

struct ProbeArgs {
    const uint16_t* K;
    const uint16_t* V;
    int64_t kv_bg_stride;
    int kv_row_stride;
    const int32_t* rows;
    int64_t rows_stride;
    int S, C, Q, P;
    uint32_t* sink;   // [grid, 256]
};

__global__ __launch_bounds__(kProbeThreads) void gather_probe(ProbeArgs a) {
    __shared__ __attribute__((aligned(16))) int idx_sh[kProbeChunk];
    const int lin = xcd_contiguous_block();
    const int bg = lin / (a.Q * a.P);
    const int p = (lin - bg * a.Q * a.P) % a.P;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int slot = lane >> 3, sub = lane & 7;
    const int Sp = (a.S + a.P - 1) / a.P;
    const int s_begin = p * Sp, s_end = min(a.S, s_begin + Sp);
    const uint16_t* Kb = a.K + (size_t)bg * a.kv_bg_stride + 8 * sub;
    const uint16_t* Vb = a.V + (size_t)bg * a.kv_bg_stride + 8 * sub;
    const int32_t* rl = a.rows + (size_t)bg * a.rows_stride;
    uint32_t fold = 0u;
    for (int c0 = s_begin; c0 < s_end; c0 += kProbeChunk) {
        const int clen = min(kProbeChunk, s_end - c0);
        if (c0 != s_begin) __syncthreads();
        for (int i = tid; i < clen; i += kProbeThreads) idx_sh[i] = rl[c0 + i];
        __syncthreads();
        const int ng = (clen + 7) / 8;
        const int my_ng = ng > wave ? (ng - wave + kProbeWaves - 1) / kProbeWaves : 0;
        auto issue = [&](int j, u32x4_t (&st)[4]) {
            const int e = (wave + kProbeWaves * j) * 8 + slot;
            int pos = idx_sh[min(e, clen - 1)];
            pos = (e < clen && (unsigned)pos < (unsigned)a.C) ? pos : 0;
            const size_t off = (size_t)pos * a.kv_row_stride;
            st[0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(Kb + off));
            st[1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(Kb + off + 64));
            st[2] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(Vb + off));
            st[3] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(Vb + off + 64));
        };
        auto consume = [&](const u32x4_t (&st)[4]) {
#pragma unroll
            for (int w = 0; w < 4; ++w) fold ^= st[w].x ^ st[w].y ^ st[w].z ^ st[w].w;
        };
        if (my_ng > 0) {
            u32x4_t st[kProbeStages][4];
#pragma unroll
            for (int u = 0; u < kProbeStages - 1; ++u) issue(u, st[u]);
            int j = 0;
            for (; j + kProbeStages <= my_ng; j += kProbeStages) {
#pragma unroll
                for (int u = 0; u < kProbeStages; ++u) {
                    issue(j + u + kProbeStages - 1, st[(u + kProbeStages - 1) % kProbeStages]);
                    consume(st[u]);
                }
            }
#pragma unroll
            for (int u = 0; u < kProbeStages - 1; ++u)
                if (j + u < my_ng) consume(st[u]);
        }
    }
    a.sink[(size_t)lin * kProbeThreads + tid] = fold;
}

}  // namespace
}  // namespace attnlab

using namespace attnlab;

extern "C" int attnlab_gather_probe(const uint16_t* K, const uint16_t* V, int64_t kv_bg_stride, int kv_row_stride,
                                    const int32_t* rows, int64_t rows_stride, int B, int G, int S, int C, int Q, int P,
                                    uint32_t* sink, void* stream) {
    ATTNLAB_REQUIRE(B >= 1 && G >= 1 && S >= 1 && C >= 1, "B=%d G=%d S=%d C=%d must be positive", B, G, S, C);
    ATTNLAB_REQUIRE(Q >= 1 && Q <= 8 && P >= 1 && P <= 256, "Q=%d outside [1, 8] or P=%d outside [1, 256]", Q, P);
    ATTNLAB_REQUIRE(K && V && rows && sink, "K, V, rows and sink must be device pointers");
    ATTNLAB_REQUIRE(kv_row_stride >= 128 && kv_row_stride % 8 == 0 && kv_bg_stride >= (int64_t)C * kv_row_stride,
                    "kv strides too small for C=%d", C);
    ATTNLAB_REQUIRE(reinterpret_cast<uintptr_t>(K) % 16 == 0 && reinterpret_cast<uintptr_t>(V) % 16 == 0,
                    "K and V must be 16-byte aligned");
    ATTNLAB_REQUIRE(rows_stride >= S, "rows must hold S=%d positions per (b, g)", S);
    ProbeArgs a{K, V, kv_bg_stride, kv_row_stride, rows, rows_stride, S, C, Q, P, sink};
    hipLaunchKernelGGL(gather_probe, dim3(B * G * Q * P), dim3(kProbeThreads), 0, reinterpret_cast<hipStream_t>(stream), a);
    return check_launch("gather_probe");
}
