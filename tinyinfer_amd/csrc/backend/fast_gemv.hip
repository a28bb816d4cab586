// Projections of the fast arithmetic for a decode step of one sequence
// (B = 1): FP32 GEMV on the vector ALU, one wavefront per output (or per
// RoPE pair), over weights stored row-major [out][in] so that a wavefront's
// loads of one output's weights are one contiguous run. At B = 1 the
// matrix-core tiles of fast_gemm.hip compute 16 rows to use one and give
// each work-group a 16-column block (36 to 96 work-groups for these shapes,
// one long MFMA chain per wavefront); here every projection spreads over
// 480 to 1,536 single-wavefront work-groups, and each wavefront issues all
// its loads at once (down projection 3.0 vs 5.4 us, measured in isolation).
//
// Lane l takes the float4s l, l + 64, ... of the inner dimension; the
// products are summed per lane, then over the 64 lanes in a fixed order
// (DPP within 16-lane rows, then the four rows), so a result depends on
// nothing but the row. RMSNorm of the input (the q|k|v and gate/up
// projections) is computed in the same pass from the residual stream
// itself: the sum of squares over the lanes, then
// (sum_k x[k] g[k] W[n][k]) / sqrt(sum_k x[k]^2 / K + eps). The reference
// evaluates the same quantities in its sequential order
// (llama_runner.cpp:10-16, :30-36, :97); the results are held to its logits
// within 1e-3.
#include "kernels.h"
#include "lanes.h"
#include "layout.h"

// The fast mode's own summation order: multiply-adds may be fused.
#pragma clang fp contract(fast)

namespace mphip {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kRopeDim = 64;

__device__ __forceinline__ float wave_sum(float v) { return rows_sum(row_sum(v)); }
__device__ __forceinline__ float dot4(f4 a, f4 b) { return (a.x * b.x + a.y * b.y) + (a.z * b.z + a.w * b.w); }

// This lane's float4s of row 0 of a quad-layout matrix of width K (float4
// index k4 sits at k4 * 256 floats) and of a plain vector; zero past K.
template <int K>
struct Lanes {
    static constexpr int kIt = (K / 4 + 63) / 64;
    f4 v[kIt];
    __device__ __forceinline__ void quad_row0(const float* x, int lane) {
#pragma unroll
        for (int i = 0; i < kIt; ++i) {
            const int k4 = lane + 64 * i;
            v[i] = k4 < K / 4 ? *reinterpret_cast<const f4*>(x + (size_t)k4 * 256) : f4{0.f, 0.f, 0.f, 0.f};
        }
    }
    __device__ __forceinline__ void plain(const float* p, int lane, bool stream) {
#pragma unroll
        for (int i = 0; i < kIt; ++i) {
            const int k4 = lane + 64 * i;
            const f4* q = reinterpret_cast<const f4*>(p) + k4;
            v[i] = k4 < K / 4 ? (stream ? __builtin_nontemporal_load(q) : *q) : f4{0.f, 0.f, 0.f, 0.f};
        }
    }
};

// q|k|v with RMSNorm, RoPE and the K/V append: work-group p computes the
// pair (d, d + 32) of one 64-wide head (q heads, then k, then v; the v
// pairs are not rotated) for the step's one row.
template <int K>
__global__ __launch_bounds__(64) void gemv_rope_kernel(GemvArgs a) {
    const int lane = threadIdx.x;
    const int pair = blockIdx.x;
    const int head = pair / (kRopeDim / 2), d = pair % (kRopeDim / 2);
    const int n0 = head * kRopeDim + d, n1 = n0 + kRopeDim / 2;
    Lanes<K> x, g, w0, w1;
    x.quad_row0(a.x, lane);
    g.plain(a.norm, lane, false);
    w0.plain(a.w + (size_t)n0 * K, lane, true);
    w1.plain(a.w + (size_t)n1 * K, lane, true);
    // The row's position, page and rotation, loaded with the operands.
    const int pos = a.meta.row_pos[0];
    const int block = a.row_block[0];
    const float cs = a.row_rope[d], sn = a.row_rope[kRopeDim / 2 + d];
    float ss = 0.f, d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int i = 0; i < Lanes<K>::kIt; ++i) {
        const f4 xg = x.v[i] * g.v[i];
        ss += dot4(x.v[i], x.v[i]);
        d0 += dot4(xg, w0.v[i]);
        d1 += dot4(xg, w1.v[i]);
    }
    ss = wave_sum(ss);
    d0 = wave_sum(d0);
    d1 = wave_sum(d1);
    if (lane != 0) return;
    const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
    const float y0 = d0 * inv, y1 = d1 * inv;
    const int hidden = a.heads * kRopeDim, kvw = a.kv.kv_width;
    const bool rotate = n0 < hidden + kvw;
    const float r0 = rotate ? y0 * cs - y1 * sn : y0;
    const float r1 = rotate ? y1 * cs + y0 * sn : y1;
    if (n0 < hidden) {
        a.out[quad_index(0, n0, a.columns)] = r0;
        a.out[quad_index(0, n1, a.columns)] = r1;
        return;
    }
    const int bt = a.kv.block_tokens, slot = pos % bt;
    const size_t base = kv_page_base(block, a.layer, a.kv.layers, bt, kvw);
    if (rotate) {
        const int kvh = (n0 - hidden) / kRopeDim;
        a.kv.keys[base + key_offset(slot, kvh, d, bt, kRopeDim)] = r0;
        a.kv.keys[base + key_offset(slot, kvh, d + kRopeDim / 2, bt, kRopeDim)] = r1;
    } else {
        const int kvh = (n0 - hidden - kvw) / kRopeDim;
        a.kv.values[base + value_offset(slot, kvh, d, bt, kRopeDim)] = r0;
        a.kv.values[base + value_offset(slot, kvh, d + kRopeDim / 2, bt, kRopeDim)] = r1;
    }
}

// out[0][n] += sum_k x[0][k] W[n][k] (the O and down projections with the
// residual add): one work-group per output n.
template <int K>
__global__ __launch_bounds__(64) void gemv_residual_kernel(GemvArgs a) {
    const int lane = threadIdx.x, n = blockIdx.x;
    Lanes<K> x, w;
    x.quad_row0(a.x, lane);
    w.plain(a.w + (size_t)n * K, lane, true);
    float* o = a.out + quad_index(0, n, a.columns);
    const float old = *o;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < Lanes<K>::kIt; ++i) s += dot4(x.v[i], w.v[i]);
    s = wave_sum(s);
    if (lane == 0) *o = old + s;
}

// out[0][n] = SwiGLU of the gate and up projections of RMSNorm(x): one
// work-group per output n (gate row n and up row n).
template <int K>
__global__ __launch_bounds__(64) void gemv_swiglu_kernel(GemvArgs a) {
    const int lane = threadIdx.x, n = blockIdx.x;
    Lanes<K> x, g, wg, wu;
    x.quad_row0(a.x, lane);
    g.plain(a.norm, lane, false);
    wg.plain(a.w + (size_t)n * K, lane, true);
    wu.plain(a.w2 + (size_t)n * K, lane, true);
    float ss = 0.f, dg = 0.f, du = 0.f;
#pragma unroll
    for (int i = 0; i < Lanes<K>::kIt; ++i) {
        const f4 xg = x.v[i] * g.v[i];
        ss += dot4(x.v[i], x.v[i]);
        dg += dot4(xg, wg.v[i]);
        du += dot4(xg, wu.v[i]);
    }
    ss = wave_sum(ss);
    dg = wave_sum(dg);
    du = wave_sum(du);
    if (lane != 0) return;
    const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
    const float gt = dg * inv, up = du * inv;
    a.out[quad_index(0, n, a.columns)] = (gt / (1.0f + __expf(-gt))) * up;
}

}  // namespace

bool gemv_fits(int hidden, int intermediate, int heads, int kv_heads) {
    return hidden == 576 && intermediate == 1536 && hidden / heads == kRopeDim && kv_heads >= 1;
}

hipError_t launch_gemv(hipStream_t s, Epilogue epilogue, const GemvArgs& a) {
    if (a.inner == 576 && epilogue == kRope) {
        if (a.columns != a.heads * kRopeDim + 2 * a.kv.kv_width || a.columns % kRopeDim) return hipErrorInvalidValue;
        gemv_rope_kernel<576><<<a.columns / 2, 64, 0, s>>>(a);
    } else if (a.inner == 576 && epilogue == kSwiglu) {
        gemv_swiglu_kernel<576><<<a.columns, 64, 0, s>>>(a);
    } else if (a.inner == 576 && epilogue == kResidual) {
        gemv_residual_kernel<576><<<a.columns, 64, 0, s>>>(a);
    } else if (a.inner == 1536 && epilogue == kResidual) {
        gemv_residual_kernel<1536><<<a.columns, 64, 0, s>>>(a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mphip
