// Projections of the fast arithmetic mode on FP32 matrix cores
// (v_mfma_f32_16x16x4f32): out[r][n] = epilogue(sum_k a[r][k] * w[n][k]) in
// the matrix cores' summation order, not the reference's sequential one
// (the reference's result is matched to 1e-3 relative on the logits and
// its greedy tokens are checked, instead of bit for bit).
//
// Operand layout of one 16x16x4 MFMA (measured on gfx950): lane l supplies
// A[l%16][l/16] and B[l/16][l%16]; result register i of lane l is
// D[4*(l/16)+i][l%16]. Each lane loads a float4 of 4 consecutive k for its
// row (A) and its column (B); MFMA j of a 16-k step takes component j of
// both, so the four lane groups l/16 cover k, k+4, k+8, k+12 of the step.
//
// A work-group of four wavefronts computes 16 rows x 16 columns: the
// wavefronts take the 16-k steps of K in turn (step s to wavefront s % 4)
// and sum their 16x16 partials through LDS in wavefront order. Activations
// are in the row-tile quad layout (layout.h), projection weights [n][k].
// Work-groups are laid out so that those sharing a column block (one per
// 16-row block) are dispatched to the same XCD and share its L2 for the
// weights: work-group b runs on XCD b % 8, and the 8-strided sequence of one
// XCD walks the row blocks of a column block first.
//
// Epilogues: store; residual (x += result) writing, for the next RMSNorm,
// the sum of squares of the updated x over the block's 16 columns; SwiGLU
// (gate and up accumulated side by side); LM head (per row and block, the
// first maximum and a non-finite flag, logits row-major on request).
// RMSNorm on the input (NORM): a[r][k] = x[r][k] * g[k], and the result is
// scaled by 1/sqrt(sum_k x[r][k]^2 / K + eps), the sum assembled from the
// producer's per-block partials.
#include "kernels.h"
#include "layout.h"

namespace mphip {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kXcds = 8;

__device__ __forceinline__ f4 ld4(const float* p) { return *reinterpret_cast<const f4*>(p); }

template <int EPI, bool NORM, bool GATHER>
__global__ __launch_bounds__(kWaves * 64) void fast_gemm_kernel(FastGemmArgs a) {
    constexpr int M = EPI == kSwiglu ? 2 : 1;
    __shared__ f4 part_s[kWaves - 1][M][64];
    __shared__ float inv_s[16];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Work-group -> (row block, column block), XCD-grouped.
    const int nrb = (a.rows + 15) >> 4;
    const int ncb = a.columns >> 4;
    const int b = blockIdx.x;
    const int g = b / kXcds, xcd = b % kXcds;
    const int rb = g % nrb;
    const int cb = (g / nrb) * kXcds + xcd;
    if (cb >= ncb) return;
    const int K = a.inner, Q = K >> 2, steps = K >> 4;
    // A: row rb*16 + l%16 (gathered), quads 4s + l/16.
    const int row_a = min(rb * 16 + (lane & 15), a.rows - 1);
    const int xrow = GATHER ? a.row_map[row_a] : row_a;
    const float* xa = a.x + ((size_t)(xrow >> 6) * Q * 64 + (xrow & 63)) * 4 + (size_t)(lane >> 4) * 256;
    // B: column cb*16 + l%16, k 16s + 4(l/16).
    const size_t wcol = (size_t)(cb * 16 + (lane & 15)) * K + (size_t)(lane >> 4) * 4;
    const float* wb = a.w + wcol;
    const float* wb2 = M == 2 ? a.w2 + wcol : nullptr;
    const float* gn = NORM ? a.norm + (lane >> 4) * 4 : nullptr;
    if (NORM && threadIdx.x < 16) {
        // 1/sqrt(mean square + eps) of the block's rows from the producer's partials.
        const int r = min(rb * 16 + (int)threadIdx.x, a.rows - 1);
        const int pr = GATHER ? a.row_map[r] : r;
        float ss = 0.0f;
        for (int p = 0; p < a.ssq_parts; ++p) ss += a.ssq_in[(size_t)p * a.ssq_stride + pr];
        inv_s[threadIdx.x] = 1.0f / sqrtf(ss / (float)K + a.eps);
    }

    f4 acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = f4{0.f, 0.f, 0.f, 0.f};
    // Two steps in flight: this wavefront's next step loads while one multiplies.
    auto load = [&](int s, f4& av, f4 (&bv)[M]) {
        av = ld4(xa + (size_t)s * 1024);  // 4 quads of 64 rows x 4 floats
        if (NORM) av = av * ld4(gn + (size_t)s * 16);
        bv[0] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(wb + (size_t)s * 16));
        if (M == 2) bv[M - 1] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(wb2 + (size_t)s * 16));
    };
    auto mma = [&](const f4& av, const f4 (&bv)[M]) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.x, bv[m].x, acc[m], 0, 0, 0);
            acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.y, bv[m].y, acc[m], 0, 0, 0);
            acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.z, bv[m].z, acc[m], 0, 0, 0);
            acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(av.w, bv[m].w, acc[m], 0, 0, 0);
        }
    };
    int s = wave;
    if (s < steps) {
        f4 a0, a1, b0[M], b1[M];
        load(s, a0, b0);
        for (;;) {
            const int s1 = s + kWaves;
            if (s1 < steps) load(s1, a1, b1);
            mma(a0, b0);
            if (s1 >= steps) break;
            const int s2 = s1 + kWaves;
            if (s2 < steps) load(s2, a0, b0);
            mma(a1, b1);
            if (s2 >= steps) break;
            s = s2;
        }
    }
    // Partials of wavefronts 1..3 to LDS; wavefront 0 adds them in order.
    if (wave > 0)
#pragma unroll
        for (int m = 0; m < M; ++m) part_s[wave - 1][m][lane] = acc[m];
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < kWaves - 1; ++w)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[m] += part_s[w][m][lane];

    // Lane l, register i: row rb*16 + 4(l/16) + i, column cb*16 + l%16.
    const int col = cb * 16 + (lane & 15);
    const int N = a.columns;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int rl = 4 * (lane >> 4) + i;
        const int row = rb * 16 + rl;
        const bool live = row < a.rows;
        float v[M];
#pragma unroll
        for (int m = 0; m < M; ++m) v[m] = NORM ? acc[m][i] * inv_s[rl] : acc[m][i];
        if (EPI == kStore) {
            if (live) a.out[quad_index(row, col, N)] = v[0];
        } else if (EPI == kResidual) {
            float nx = 0.0f;
            if (live) {
                float* o = a.out + quad_index(row, col, N);
                nx = *o + v[0];
                *o = nx;
            }
            // The row's 16 columns sit in the 16 lanes of this lane's group.
            float sq = nx * nx;
            sq += __shfl_xor(sq, 1);
            sq += __shfl_xor(sq, 2);
            sq += __shfl_xor(sq, 4);
            sq += __shfl_xor(sq, 8);
            if (live && (lane & 15) == 0) a.ssq_out[(size_t)cb * a.ssq_stride + row] = sq;
        } else if (EPI == kSwiglu) {
            const float gt = v[0];
            if (live) a.out[quad_index(row, col, N)] = (gt / (1.0f + __expf(-gt))) * v[M - 1];
        } else {  // kHead
            const float x = v[0];
            const bool finite = __builtin_isfinite(x);
            if (live && a.logits) a.logits[(size_t)row * N + col] = x;
            // First maximum of the row's 16 columns (finite values only).
            float bv = finite ? x : -__builtin_inff();
            int bi = finite ? col : -1;
            int bad = finite ? 0 : 1;
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) {
                const float ov = __shfl_xor(bv, o);
                const int oi = __shfl_xor(bi, o);
                bad |= __shfl_xor(bad, o);
                if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) {
                    bv = ov;
                    bi = oi;
                }
            }
            if (live && (lane & 15) == 0) {
                const size_t at = (size_t)row * a.groups + cb;
                a.best_value[at] = bv;
                a.best_index[at] = bi;
                a.bad[at] = bad;
            }
        }
    }
}

// x rows' per-16-column sums of squares (the partials a NORM projection
// reads), for x written by something other than a residual projection.
__global__ __launch_bounds__(256) void fast_ssq_kernel(const float* __restrict__ x, int rows, int width,
                                                       float* __restrict__ ssq, int stride) {
    const int parts = width >> 4;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * parts) return;
    const int r = i % rows, p = i / rows;
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        const float v = x[quad_index(r, p * 16 + c, width)];
        s += v * v;
    }
    ssq[(size_t)p * stride + r] = s;
}

template <int EPI, bool NORM, bool GATHER>
hipError_t launch_fast(hipStream_t s, const FastGemmArgs& a) {
    const int nrb = (a.rows + 15) / 16;
    const int ncb = a.columns / 16;
    const int per_xcd = (ncb + kXcds - 1) / kXcds;  // column blocks per XCD
    const int blocks = per_xcd * nrb * kXcds;
    fast_gemm_kernel<EPI, NORM, GATHER><<<blocks, kWaves * 64, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace

bool fast_gemm_fits(const FastGemmArgs& a) {
    return a.rows > 0 && a.inner > 0 && a.inner % 16 == 0 && a.columns > 0 && a.columns % 16 == 0;
}

hipError_t launch_fast_gemm(hipStream_t s, Epilogue epilogue, const FastGemmArgs& a) {
    if (!fast_gemm_fits(a)) return hipErrorInvalidValue;
    const bool norm = a.norm != nullptr;
    switch (epilogue) {
    case kStore: return norm ? launch_fast<kStore, true, false>(s, a) : launch_fast<kStore, false, false>(s, a);
    case kResidual: return launch_fast<kResidual, false, false>(s, a);
    case kSwiglu: return norm ? launch_fast<kSwiglu, true, false>(s, a) : launch_fast<kSwiglu, false, false>(s, a);
    case kHead: return launch_fast<kHead, true, true>(s, a);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_fast_ssq(hipStream_t s, const float* x, int rows, int width, float* ssq, int stride) {
    if (rows <= 0) return hipSuccess;
    const int total = rows * (width / 16);
    fast_ssq_kernel<<<(total + 255) / 256, 256, 0, s>>>(x, rows, width, ssq, stride);
    return hipGetLastError();
}

}  // namespace mphip
