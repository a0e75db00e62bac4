// Decode attention for gfx950: the gather-free sparse read (D) and the dense control read (A) share one kernel.
//
// Reference semantics: MetalAttend (metal_attend.py:46-169) and gathered_decode_step_kernel / full_attention
// (decode.py:131-142, full.py:17-34): out[b,g,i] = softmax(scale * q_i . K[rows]) @ V[rows] for the h query heads of
// KV group g, rows read by original position straight from the cache.
//
// Layout per workgroup (256 threads = 4 waves) of one (b, g, partition): 8 lanes share a position; lane `sub` owns
// dims [8*sub, 8*sub+8) and [64+8*sub, 64+8*sub+8), so one 16-byte load per lane and half-row covers 128 contiguous
// bytes (one cache line) and a wave reads 8 positions per load instruction. The 32 position slots of the block walk
// the partition with stride 32, R positions per iteration, all R K/V loads issued before any arithmetic. q . k is a
// bf16 dot2 (v_dot2_f32_bf16, fp32 accumulate) finished by a 3-step DPP sum over the 8 lanes; every head of the group
// reuses the same K and V registers (GQA sharing). Online softmax runs in the log2 domain with a lazy rescale: the
// running max is raised only when a block max exceeds it by more than 2^8, so the 16*h accumulator rescale is rare.
// Slots are merged with DPP/shuffles and LDS. With P > 1 partitions every block writes its (m, l, acc) partial and a
// second small kernel merges them; the kernel boundary is what makes the partials of other XCDs' L2s visible, which
// is far cheaper on this part than a device-scope fence per block.
#include "common.h"

namespace attnlab {

constexpr int kHeadDim = 128;
constexpr int kAttThreads = 256;
constexpr int kSlots = kAttThreads / 8;  // positions in flight per block per step
constexpr float kLazyRescale = 8.0f;     // log2-domain slack of the running max

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
    float scale_log2;
    void* out;
    int out_bf16;
    float* part;  // [BG, P, h, 130]: m, l, acc[128]
};

__device__ __forceinline__ void merge_state(float& m, float& l, float& m2, float& l2, float& w1, float& w2) {
    const float mn = fmaxf(m, m2);
    w1 = (m == -INFINITY) ? 0.0f : fast_exp2(m - mn);
    w2 = (m2 == -INFINITY) ? 0.0f : fast_exp2(m2 - mn);
    l = w1 * l + w2 * l2;
    m = mn;
}

__device__ __forceinline__ void store_out(const AttendArgs& a, size_t idx, float v) {
    if (a.out_bf16) reinterpret_cast<uint16_t*>(a.out)[idx] = f32_to_bf16_rne(v);
    else reinterpret_cast<float*>(a.out)[idx] = v;
}

template <int H, int R, bool DENSE>
__global__ __launch_bounds__(kAttThreads) void attend_kernel(AttendArgs a) {
    __shared__ float red_ml[4][H][2];
    __shared__ float red_acc[4][H][kHeadDim];
    const int bg = blockIdx.x / a.P;
    const int p = blockIdx.x - bg * a.P;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int slot = (wave << 3) | (lane >> 3);
    const int sub = lane & 7;
    const int h = a.h;

    uint32_t qw[H][8];
#pragma unroll
    for (int i = 0; i < H; ++i) {
        uint4 x0 = make_uint4(0, 0, 0, 0), x1 = make_uint4(0, 0, 0, 0);
        if (i < h) {
            const uint16_t* qp = a.q + ((size_t)bg * h + i) * kHeadDim + 8 * sub;
            x0 = *reinterpret_cast<const uint4*>(qp);
            x1 = *reinterpret_cast<const uint4*>(qp + 64);
        }
        qw[i][0] = x0.x; qw[i][1] = x0.y; qw[i][2] = x0.z; qw[i][3] = x0.w;
        qw[i][4] = x1.x; qw[i][5] = x1.y; qw[i][6] = x1.z; qw[i][7] = x1.w;
    }

    const int Sp = (a.S + a.P - 1) / a.P;
    const int s_begin = p * Sp;
    const int s_end = min(a.S, s_begin + Sp);
    const uint16_t* Kb = a.K + (size_t)bg * a.kv_bg_stride + 8 * sub;
    const uint16_t* Vb = a.V + (size_t)bg * a.kv_bg_stride + 8 * sub;
    const int32_t* rl = DENSE ? nullptr : a.rows + (size_t)bg * a.rows_stride;

    float m[H], l[H], acc[H][16];
#pragma unroll
    for (int i = 0; i < H; ++i) {
        m[i] = -INFINITY;
        l[i] = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;
    }

    for (int s0 = s_begin + slot; s0 < s_end; s0 += kSlots * R) {
        bool ok[R];
        uint4 k0[R], k1[R], v0[R], v1[R];
#pragma unroll
        for (int t = 0; t < R; ++t) {
            const int s = s0 + kSlots * t;
            bool okt = s < s_end;
            int pos = 0;
            if (okt) {
                pos = DENSE ? s : rl[s];
                if (!DENSE) okt = (unsigned)pos < (unsigned)a.C;
            }
            ok[t] = okt;
            k0[t] = k1[t] = v0[t] = v1[t] = make_uint4(0, 0, 0, 0);
            if (okt) {
                const size_t off = (size_t)pos * a.kv_row_stride;
                k0[t] = *reinterpret_cast<const uint4*>(Kb + off);
                k1[t] = *reinterpret_cast<const uint4*>(Kb + off + 64);
                v0[t] = *reinterpret_cast<const uint4*>(Vb + off);
                v1[t] = *reinterpret_cast<const uint4*>(Vb + off + 64);
            }
        }
        float sc[R][H];
#pragma unroll
        for (int t = 0; t < R; ++t) {
#pragma unroll
            for (int i = 0; i < H; ++i) {
                float d = 0.0f;
                d = dot2_bf16(qw[i][0], k0[t].x, d);
                d = dot2_bf16(qw[i][1], k0[t].y, d);
                d = dot2_bf16(qw[i][2], k0[t].z, d);
                d = dot2_bf16(qw[i][3], k0[t].w, d);
                d = dot2_bf16(qw[i][4], k1[t].x, d);
                d = dot2_bf16(qw[i][5], k1[t].y, d);
                d = dot2_bf16(qw[i][6], k1[t].z, d);
                d = dot2_bf16(qw[i][7], k1[t].w, d);
                d = sum8(d);
                sc[t][i] = ok[t] ? d * a.scale_log2 : -INFINITY;
            }
        }
#pragma unroll
        for (int i = 0; i < H; ++i) {
            float mb = sc[0][i];
#pragma unroll
            for (int t = 1; t < R; ++t) mb = fmaxf(mb, sc[t][i]);
            if (mb > m[i] + kLazyRescale) {
                const float al = fast_exp2(m[i] - mb);
                l[i] *= al;
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][e] *= al;
                m[i] = mb;
            }
        }
#pragma unroll
        for (int t = 0; t < R; ++t) {
            float vf[16];
            const uint32_t vw[8] = {v0[t].x, v0[t].y, v0[t].z, v0[t].w, v1[t].x, v1[t].y, v1[t].z, v1[t].w};
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                vf[2 * w] = bf16_lo(vw[w]);
                vf[2 * w + 1] = bf16_hi(vw[w]);
            }
#pragma unroll
            for (int i = 0; i < H; ++i) {
                const float pr = ok[t] ? fast_exp2(sc[t][i] - m[i]) : 0.0f;
                l[i] += pr;
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][e] += pr * vf[e];
            }
        }
    }

    // merge the 8 slots of the wave (lanes with equal `sub`): xor 8 (DPP row_ror:8), xor 16, xor 32
#pragma unroll
    for (int i = 0; i < H; ++i) {
#pragma unroll
        for (int step = 0; step < 3; ++step) {
            float m2, l2;
            if (step == 0) { m2 = dpp_f32<0x128>(m[i]); l2 = dpp_f32<0x128>(l[i]); }
            else { m2 = shfl_xor_f32(m[i], step == 1 ? 16 : 32); l2 = shfl_xor_f32(l[i], step == 1 ? 16 : 32); }
            float w1, w2;
            merge_state(m[i], l[i], m2, l2, w1, w2);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float o = (step == 0) ? dpp_f32<0x128>(acc[i][e]) : shfl_xor_f32(acc[i][e], step == 1 ? 16 : 32);
                acc[i][e] = w1 * acc[i][e] + w2 * o;
            }
        }
    }
    if (lane < 8) {
#pragma unroll
        for (int i = 0; i < H; ++i) {
            if (lane == 0) {
                red_ml[wave][i][0] = m[i];
                red_ml[wave][i][1] = l[i];
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                red_acc[wave][i][8 * sub + e] = acc[i][e];
                red_acc[wave][i][64 + 8 * sub + e] = acc[i][8 + e];
            }
        }
    }
    __syncthreads();

    // merge the 4 waves: thread -> (head, dim) pairs
    for (int idx = tid; idx < h * kHeadDim; idx += kAttThreads) {
        const int i = idx / kHeadDim, dim = idx - i * kHeadDim;
        float ms = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) ms = fmaxf(ms, red_ml[w][i][0]);
        float ls = 0.0f, as = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float mw = red_ml[w][i][0];
            const float ww = (mw == -INFINITY) ? 0.0f : fast_exp2(mw - ms);
            ls += ww * red_ml[w][i][1];
            as += ww * red_acc[w][i][dim];
        }
        if (a.P == 1) {
            store_out(a, ((size_t)bg * h + i) * kHeadDim + dim, as / ls);
        } else {
            float* pp = a.part + (((size_t)bg * a.P + p) * h + i) * (kHeadDim + 2);
            if (dim == 0) {
                pp[0] = ms;
                pp[1] = ls;
            }
            pp[2 + dim] = as;
        }
    }
}

// Merge the P partials of every (b, g): thread -> (head, dim).
__global__ __launch_bounds__(1024) void attend_combine(AttendArgs a) {
    const int bg = blockIdx.x;
    const int h = a.h;
    const float* pb = a.part + (size_t)bg * a.P * h * (kHeadDim + 2);
    for (int idx = threadIdx.x; idx < h * kHeadDim; idx += blockDim.x) {
        const int i = idx / kHeadDim, dim = idx - i * kHeadDim;
        float ms = -INFINITY;
        for (int q = 0; q < a.P; ++q) ms = fmaxf(ms, pb[((size_t)q * h + i) * (kHeadDim + 2)]);
        float ls = 0.0f, as = 0.0f;
        for (int q = 0; q < a.P; ++q) {
            const float* pp = pb + ((size_t)q * h + i) * (kHeadDim + 2);
            const float mw = pp[0];
            const float ww = (mw == -INFINITY) ? 0.0f : fast_exp2(mw - ms);
            ls += ww * pp[1];
            as += ww * pp[2 + dim];
        }
        store_out(a, ((size_t)bg * h + i) * kHeadDim + dim, as / ls);
    }
}

template <bool DENSE>
static int launch_attend(const AttendArgs& a, int BG, hipStream_t s) {
    const dim3 grid(BG * a.P), block(kAttThreads);
    if (a.h <= 1) hipLaunchKernelGGL((attend_kernel<1, 4, DENSE>), grid, block, 0, s, a);
    else if (a.h <= 2) hipLaunchKernelGGL((attend_kernel<2, 4, DENSE>), grid, block, 0, s, a);
    else if (a.h <= 4) hipLaunchKernelGGL((attend_kernel<4, 4, DENSE>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((attend_kernel<8, 2, DENSE>), grid, block, 0, s, a);
    if (a.P > 1) hipLaunchKernelGGL(attend_combine, dim3(BG), dim3(a.h * kHeadDim), 0, s, a);
    return check_launch(DENSE ? "dense_decode" : "attend");
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

extern "C" int attnlab_attend(const uint16_t* K, const uint16_t* V, int64_t kv_bg_stride, int kv_row_stride,
                              const uint16_t* q, const int32_t* rows, int64_t rows_stride, int B, int G, int h, int S,
                              int C, int P, float scale, void* out, int out_bf16, float* part, void* stream) {
    const int rc = check_common(K, V, kv_bg_stride, kv_row_stride, q, B, G, h, C, P, out, part);
    if (rc) return rc;
    ATTNLAB_REQUIRE(S >= 1, "at least one row must be selected (S=%d)", S);
    ATTNLAB_REQUIRE(rows != nullptr && rows_stride >= S, "rows must hold S=%d positions per (b, g)", S);
    AttendArgs a{K, V, kv_bg_stride, kv_row_stride, q, rows, rows_stride, S, C, h, P, scale * kLog2e, out, out_bf16, part};
    return launch_attend<false>(a, B * G, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int attnlab_dense_decode(const uint16_t* K, const uint16_t* V, int64_t kv_bg_stride, int kv_row_stride,
                                    const uint16_t* q, int B, int G, int h, int L, int C, int P, float scale, void* out,
                                    int out_bf16, float* part, void* stream) {
    const int rc = check_common(K, V, kv_bg_stride, kv_row_stride, q, B, G, h, C, P, out, part);
    if (rc) return rc;
    ATTNLAB_REQUIRE(1 <= L && L <= C, "valid length L=%d outside [1, C=%d]", L, C);
    AttendArgs a{K, V, kv_bg_stride, kv_row_stride, q, nullptr, 0, L, C, h, P, scale * kLog2e, out, out_bf16, part};
    return launch_attend<true>(a, B * G, reinterpret_cast<hipStream_t>(stream));
}
