// Projections of the fast arithmetic for a decode step of up to four
// sequences: FP32 GEMV on the vector ALU, one wavefront per output (or per
// RoPE pair), over weights stored row-major [out][in] so that a wavefront's
// loads of one output's weights are one contiguous run. At such batches the
// matrix-core tiles of fast_gemm.hip compute 16 rows to use one to four and
// give each work-group a 16-column block (36 to 96 work-groups for these
// shapes, one long MFMA chain per wavefront); here every projection spreads
// over 480 to 1,536 single-wavefront work-groups, and each wavefront issues
// all its loads at once (down projection 3.0 vs 5.4 us at B = 1, measured in
// isolation). Whole decode steps measured faster up to four sequences
// (0.82 vs 1.01 ms at B = 1, 0.99 vs 1.05 at B = 4) and slower from six
// (1.12 vs 1.07 ms at B = 6, 1.25 vs 1.07 at B = 8), where each
// wavefront's loads of every row's activations outweigh the tiles' waste.
//
// Lane l takes the float4s l, l + 64, ... of the inner dimension; the
// products are summed per lane, then over the 64 lanes in a fixed order
// (DPP within 16-lane rows, then the four rows), each row on its own, so a
// row's result depends on nothing but the row. RMSNorm of the input (the
// q|k|v and gate/up projections) is computed in the same pass from the
// residual stream itself: the sum of squares over the lanes, then
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

// This lane's float4s of row r (< 64) of a quad-layout matrix of width K
// (float4 k4 of row r sits at k4 * 256 + 4r floats) and of a plain vector;
// zero past K. Every load is unconditional (a lane past K re-reads the
// last float4 and drops it), so that all of them are issued before the
// first wait.
template <int K>
struct Lanes {
    static constexpr int kIt = (K / 4 + 63) / 64;
    f4 v[kIt];
    __device__ __forceinline__ static f4 keep(f4 v, int k4) { return k4 < K / 4 ? v : f4{0.f, 0.f, 0.f, 0.f}; }
    __device__ __forceinline__ void quad_row(const float* x, int r, int lane) {
#pragma unroll
        for (int i = 0; i < kIt; ++i) {
            const int k4 = lane + 64 * i;
            v[i] = *reinterpret_cast<const f4*>(x + (size_t)min(k4, K / 4 - 1) * 256 + 4 * r);
        }
#pragma unroll
        for (int i = 0; i < kIt; ++i) v[i] = keep(v[i], lane + 64 * i);
    }
    __device__ __forceinline__ void plain(const float* p, int lane, bool stream) {
#pragma unroll
        for (int i = 0; i < kIt; ++i) {
            const f4* q = reinterpret_cast<const f4*>(p) + min(lane + 64 * i, K / 4 - 1);
            v[i] = stream ? __builtin_nontemporal_load(q) : *q;
        }
#pragma unroll
        for (int i = 0; i < kIt; ++i) v[i] = keep(v[i], lane + 64 * i);
    }
};

// q|k|v with RMSNorm, RoPE and the K/V append: work-group p computes the
// pair (d, d + 32) of one 64-wide head (q heads, then k, then v; the v
// pairs are not rotated) for each of the step's R rows (lane r stores row
// r's results).
template <int K, int R>
__global__ __launch_bounds__(64) void gemv_rope_kernel(GemvArgs a) {
    const int lane = threadIdx.x & 63;
    const int pair = blockIdx.x;
    const int head = pair / (kRopeDim / 2), d = pair % (kRopeDim / 2);
    const int n0 = head * kRopeDim + d, n1 = n0 + kRopeDim / 2;
    Lanes<K> x[R], g, w0, w1;
#pragma unroll
    for (int r = 0; r < R; ++r) x[r].quad_row(a.x, r, lane);
    g.plain(a.norm, lane, false);
    w0.plain(a.w + (size_t)n0 * K, lane, true);
    w1.plain(a.w + (size_t)n1 * K, lane, true);
    // The rows' positions, pages and rotations, loaded with the operands.
    int pos[R], block[R];
    float cs[R], sn[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        pos[r] = a.meta.row_pos[r];
        block[r] = a.row_block[r];
        cs[r] = a.row_rope[(size_t)r * kRopeDim + d];
        sn[r] = a.row_rope[(size_t)r * kRopeDim + kRopeDim / 2 + d];
    }
    float y0 = 0.f, y1 = 0.f, c = 0.f, sv = 0.f;
    int p = 0, b = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float ss = 0.f, d0 = 0.f, d1 = 0.f;
#pragma unroll
        for (int i = 0; i < Lanes<K>::kIt; ++i) {
            const f4 xg = x[r].v[i] * g.v[i];
            ss += dot4(x[r].v[i], x[r].v[i]);
            d0 += dot4(xg, w0.v[i]);
            d1 += dot4(xg, w1.v[i]);
        }
        ss = wave_sum(ss);
        d0 = wave_sum(d0);
        d1 = wave_sum(d1);
        const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
        if (lane == r) {
            y0 = d0 * inv;
            y1 = d1 * inv;
            c = cs[r];
            sv = sn[r];
            p = pos[r];
            b = block[r];
        }
    }
    if (lane >= R) return;
    const int hidden = a.heads * kRopeDim, kvw = a.kv.kv_width;
    const bool rotate = n0 < hidden + kvw;
    const float r0 = rotate ? y0 * c - y1 * sv : y0;
    const float r1 = rotate ? y1 * c + y0 * sv : y1;
    if (n0 < hidden) {
        a.out[quad_index(lane, n0, a.columns)] = r0;
        a.out[quad_index(lane, n1, a.columns)] = r1;
        return;
    }
    const int bt = a.kv.block_tokens, slot = p % bt;
    const size_t base = kv_page_base(b, a.layer, a.kv.layers, bt, kvw);
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

// out[r][n] += sum_k x[r][k] W[n][k] (the O and down projections with the
// residual add): one work-group per output n, lane r stores row r.
template <int K, int R>
__global__ __launch_bounds__(64) void gemv_residual_kernel(GemvArgs a) {
    const int lane = threadIdx.x & 63, n = blockIdx.x;
    Lanes<K> x[R], w;
#pragma unroll
    for (int r = 0; r < R; ++r) x[r].quad_row(a.x, r, lane);
    w.plain(a.w + (size_t)n * K, lane, true);
    float* o = a.out + quad_index(lane < R ? lane : 0, n, a.columns);
    const float old = *o;
    float y = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < Lanes<K>::kIt; ++i) s += dot4(x[r].v[i], w.v[i]);
        s = wave_sum(s);
        if (lane == r) y = s;
    }
    if (lane < R) *o = old + y;
}

// out[r][n] = SwiGLU of the gate and up projections of RMSNorm(x[r]): one
// work-group per output n (gate row n and up row n), lane r stores row r.
template <int K, int R>
__global__ __launch_bounds__(64) void gemv_swiglu_kernel(GemvArgs a) {
    const int lane = threadIdx.x & 63, n = blockIdx.x;
    Lanes<K> x[R], g, wg, wu;
#pragma unroll
    for (int r = 0; r < R; ++r) x[r].quad_row(a.x, r, lane);
    g.plain(a.norm, lane, false);
    wg.plain(a.w + (size_t)n * K, lane, true);
    wu.plain(a.w2 + (size_t)n * K, lane, true);
    float gt = 0.f, up = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float ss = 0.f, dg = 0.f, du = 0.f;
#pragma unroll
        for (int i = 0; i < Lanes<K>::kIt; ++i) {
            const f4 xg = x[r].v[i] * g.v[i];
            ss += dot4(x[r].v[i], x[r].v[i]);
            dg += dot4(xg, wg.v[i]);
            du += dot4(xg, wu.v[i]);
        }
        ss = wave_sum(ss);
        dg = wave_sum(dg);
        du = wave_sum(du);
        const float inv = 1.0f / sqrtf(ss / (float)K + a.eps);
        if (lane == r) {
            gt = dg * inv;
            up = du * inv;
        }
    }
    if (lane < R) a.out[quad_index(lane, n, a.columns)] = (gt / (1.0f + __expf(-gt))) * up;
}

template <int R>
hipError_t launch_rows(hipStream_t s, Epilogue epilogue, const GemvArgs& a) {
    if (a.inner == 576 && epilogue == kRope) {
        if (a.columns != a.heads * kRopeDim + 2 * a.kv.kv_width || a.columns % kRopeDim) return hipErrorInvalidValue;
        gemv_rope_kernel<576, R><<<a.columns / 2, 64, 0, s>>>(a);
    } else if (a.inner == 576 && epilogue == kSwiglu) {
        gemv_swiglu_kernel<576, R><<<a.columns, 64, 0, s>>>(a);
    } else if (a.inner == 576 && epilogue == kResidual) {
        gemv_residual_kernel<576, R><<<a.columns, 64, 0, s>>>(a);
    } else if (a.inner == 1536 && epilogue == kResidual) {
        gemv_residual_kernel<1536, R><<<a.columns, 64, 0, s>>>(a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

bool gemv_fits(int hidden, int intermediate, int heads, int kv_heads) {
    return hidden == 576 && intermediate == 1536 && hidden / heads == kRopeDim && kv_heads >= 1;
}

hipError_t launch_gemv(hipStream_t s, Epilogue epilogue, const GemvArgs& a) {
    switch (a.rows) {
    case 1: return launch_rows<1>(s, epilogue, a);
    case 2: return launch_rows<2>(s, epilogue, a);
    case 3: return launch_rows<3>(s, epilogue, a);
    case 4: return launch_rows<4>(s, epilogue, a);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace mphip
