// Projections of the MiniPrefix forward with the reference CPU path's
// arithmetic: out[r][n] = sum_k x[r][k] * w[k][n] with k in increasing order
// from 0.0f, multiply and add rounded separately (src/backend/cpu/
// matmul_kernel.cpp:101-109 and :289-354; this file is compiled with
// -ffp-contract=off).
//
// Every output is one lane's serial chain, so the parallelism is the number
// of outputs. Lane = row: a wavefront's 64 lanes are the 64 rows of one row
// tile and the wavefront owns C output columns, giving C chains per lane.
// The activation tile reaches each lane as one float4 (4 consecutive k) per
// LDS read; the column's weights (stored transposed, [n][k]) are read as an
// LDS broadcast. A work-group of NW wavefronts covers NW*C consecutive
// columns; k advances in 64-wide chunks that the wavefronts copy straight
// from global memory into an NS-stage LDS ring (global_load_lds, no register
// staging), NS-2 chunks ahead of the arithmetic. Each stage is a separate LDS
// object so that the compiler's own LDS-DMA wait tracking tells stages
// apart; the cross-wavefront hand-off is an explicit vmcnt wait plus a bare
// s_barrier. Prefill and the LM head use this kernel with C > 1.
//
// Decode (one row tile) has too few outputs for C > 1, and with C = 1 the
// LDS copy of the weights costs as much LDS bandwidth as x. There
// gemm_column_kernel runs instead: one column per wavefront, the column's
// weights held in VGPRs (each 16-lane row of the wavefront holds the same
// 16 floats per register) and handed to all 64 lanes by a DPP row broadcast
// folded into v_mul_f32, while x streams from global memory through a
// register ring.
#include "dpp.h"
#include "exact_math.h"
#include "kernels.h"
#include "layout.h"

namespace mphip {
namespace {

constexpr int kChunk = 64;            // k per stage
constexpr int kQuads = kChunk / 4;    // float4 quads of k per stage

template <int C, int NW, int EPI>
struct Shape {
    static constexpr int kThreads = NW * 64;
    static constexpr int kMats = EPI == kSwiglu ? 2 : 1;
    static constexpr int kCols = NW * C;                    // columns per work-group
    static constexpr int kX4 = 64 * kQuads;                 // x float4 per stage (16 KB)
    static constexpr int kWaveW4 = C * kMats * kQuads;      // one wavefront's weights per stage
    static constexpr int kW4 = NW * kWaveW4;
    static constexpr int kXDma = 16 / NW;                   // 1 KB copies per wavefront per stage
    static constexpr int kWDma = (kWaveW4 + 63) / 64;
    static constexpr int kDma = kXDma + kWDma;
    static_assert(16 % NW == 0, "x stage split");
};

template <int X4, int W4>
struct Stage {
    float4 x[X4];  // [q][row]
    float4 w[W4];  // [wave][column][matrix][q]
};

typedef __attribute__((address_space(3))) void* LdsPtr;

// Each lane copies 16 bytes from `src` to lds_base + 16*lane.
__device__ __forceinline__ void dma16(const float4* src, float4* lds_base) {
    __builtin_amdgcn_global_load_lds((const void*)src, (LdsPtr)lds_base, 16, 0, 0);
}

// s_waitcnt vmcnt(N) with every other counter left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xf << 8) | ((N >> 4) << 14));
}

// Barrier without a memory fence: LDS-DMA completion is established by the
// explicit vmcnt waits, and LDS reads complete before their values are used.
__device__ __forceinline__ void bare_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// FULL: inner % 64 == 0 and columns % kCols == 0 (no clamping anywhere).
template <int C, int NW, int EPI, int NS, bool FULL>
__global__ __launch_bounds__(NW * 64) void gemm_rows_kernel(GemmArgs a) {
    using S = Shape<C, NW, EPI>;
    constexpr int M = S::kMats;
    constexpr int D = S::kDma;
    static_assert(NS >= 3 && NS <= 6, "stage count");
    static_assert((NS - 2) * D < 64, "vmcnt range");
    using St = Stage<S::kX4, S::kW4>;
    __shared__ St st0, st1, st2, st3, st4, st5;
    auto stage = [&](int s) -> St& {
        switch (s) {
        case 0: return st0;
        case 1: return st1;
        case 2: return st2;
        case 3: return st3;
        case 4: return st4;
        default: return st5;
        }
    };
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = blockIdx.y;
    const int n0 = blockIdx.x * S::kCols;
    const int col0 = n0 + wave * C;
    const int K = a.inner, N = a.columns;
    const int kq_total = K >> 2;
    const float4* xsrc = reinterpret_cast<const float4*>(a.x) + (size_t)tile * kq_total * 64;
    const float4* w4 = reinterpret_cast<const float4*>(a.w);
    const float4* u4 = reinterpret_cast<const float4*>(a.w2);
    const int chunks = (K + kChunk - 1) / kChunk;

    // Copies chunk c into stage `st`: this wavefront's share of the x tile
    // and its own columns' weights.
    auto issue = [&](int c, St& st) {
        const int q0 = c * kQuads;
#pragma unroll
        for (int j = 0; j < S::kXDma; ++j) {
            const int q = wave * S::kXDma + j;
            const bool in = FULL || q0 + q < kq_total;
            dma16(xsrc + (in ? (size_t)(q0 + q) * 64 + lane : 0), st.x + q * 64);
        }
#pragma unroll
        for (int j = 0; j < S::kWDma; ++j) {
            const int e = j * 64 + lane;  // (column, matrix, q) within the wavefront
            if (S::kWaveW4 % 64 == 0 || e < S::kWaveW4) {
                const int cm = e / kQuads, q = e % kQuads;
                const int c_ = cm / M, m = cm % M;
                const int n = col0 + c_;
                const bool in = FULL || (n < N && q0 + q < kq_total);
                const float4* src = (M == 2 && m) ? u4 : w4;
                dma16(src + (in ? (size_t)n * kq_total + q0 + q : 0), st.w + wave * S::kWaveW4 + j * 64);
            }
        }
    };
    // Waits until at most `later` chunks' copies of this wavefront are in flight.
    auto wait_chunks = [&](int later) {
        switch (later) {
        case 0: wait_vm<0>(); break;
        case 1: wait_vm<D>(); break;
        case 2: wait_vm<(2 * D < 64 ? 2 * D : 63)>(); break;
        case 3: wait_vm<(3 * D < 64 ? 3 * D : 63)>(); break;
        default: wait_vm<((NS - 2) * D)>(); break;
        }
    };

    float acc[M][C];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int c = 0; c < C; ++c) acc[m][c] = 0.0f;

    // One quad: 4 steps of every chain of this lane, k in order.
    auto step4 = [&](const float4& xv, const float4 (&wv)[M][C]) {
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int m = 0; m < M; ++m) {
                float t = acc[m][c];
                t = t + xv.x * wv[m][c].x;
                t = t + xv.y * wv[m][c].y;
                t = t + xv.z * wv[m][c].z;
                t = t + xv.w * wv[m][c].w;
                acc[m][c] = t;
            }
    };
    auto read_quad = [&](const St& st, int q, float4& xv, float4 (&wv)[M][C]) {
        xv = st.x[q * 64 + lane];
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int m = 0; m < M; ++m) wv[m][c] = st.w[wave * S::kWaveW4 + (c * M + m) * kQuads + q];
    };
    // With one chain per lane (decode) a wavefront has no other work to hide
    // LDS latency behind, so a chunk's reads run kDepth quads ahead of its
    // arithmetic; with C chains per lane a quad's own reads are enough.
    constexpr int kDepth = 4;
    auto compute = [&](const St& st, int nq) {
        if (C == 1 && (FULL || nq == kQuads)) {
            float4 xv[kDepth];
            float4 wv[kDepth][M][C];
#pragma unroll
            for (int q = 0; q < kDepth; ++q) read_quad(st, q, xv[q], wv[q]);
#pragma unroll
            for (int q = 0; q < kQuads; ++q) {
                const int d = q % kDepth;
                const float4 x = xv[d];
                float4 w[M][C];
#pragma unroll
                for (int m = 0; m < M; ++m)
#pragma unroll
                    for (int c = 0; c < C; ++c) w[m][c] = wv[d][m][c];
                if (q + kDepth < kQuads) read_quad(st, q + kDepth, xv[d], wv[d]);
                step4(x, w);
            }
        } else {
#pragma unroll 2
            for (int q = 0; q < nq; ++q) {
                float4 x;
                float4 w[M][C];
                read_quad(st, q, x, w);
                step4(x, w);
            }
        }
    };

    // Prologue: chunks 0..NS-2 in flight, then chunk 0 complete everywhere.
#pragma unroll
    for (int s = 0; s < NS - 1; ++s)
        if (s < chunks) issue(s, stage(s));
    wait_chunks(min(NS - 2, chunks - 1));
    bare_barrier();
    for (int c0 = 0; c0 < chunks; c0 += NS) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int c = c0 + s;
            if (c >= chunks) break;
            compute(stage(s), min(kQuads, kq_total - c * kQuads));
            if (c + 1 < chunks) {
                // Chunk c+1 complete in every wavefront; then stage (s-1)
                // (last read by chunk c-1) takes chunk c+NS-1.
                wait_chunks(min(c + NS - 2, chunks - 1) - (c + 1));
                bare_barrier();
                if (c + NS - 1 < chunks) issue(c + NS - 1, stage((s + NS - 1) % NS));
            }
        }
    }

    // Epilogue: lane = row of the tile, columns n0 + wave*C + c.
    const int row = tile * 64 + lane;
    const bool row_ok = row < a.rows;
    if (EPI == kHead) {
        // First maximum over this lane's columns (std::max_element keeps the
        // earliest of equal values), then over the work-group's wavefronts
        // in column order; one partial per (row, work-group).
        __shared__ float red_v[NW][64];
        __shared__ int32_t red_i[NW][64];
        __shared__ int32_t red_bad[NW][64];
        float best = 0.0f;
        int32_t best_i = -1, bad = 0;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const int n = n0 + wave * C + c;
            if (!FULL && n >= N) break;
            const float v = acc[0][c];
            if (!isfinite(v)) bad = 1;
            if (best_i < 0 || best < v) {
                best = v;
                best_i = n;
            }
            if (a.out && row_ok) a.out[(size_t)row * N + n] = v;
        }
        red_v[wave][lane] = best;
        red_i[wave][lane] = best_i;
        red_bad[wave][lane] = bad;
        __syncthreads();
        if (wave == 0 && row_ok) {
            for (int w = 1; w < NW; ++w) {
                const int32_t i = red_i[w][lane];
                if (i >= 0 && (best_i < 0 || best < red_v[w][lane])) {
                    best = red_v[w][lane];
                    best_i = i;
                }
                bad |= red_bad[w][lane];
            }
            const size_t p = (size_t)row * a.groups + blockIdx.x;
            a.best_value[p] = best;
            a.best_index[p] = best_i;
            a.bad[p] = bad;
        }
        return;
    }
    if (!row_ok) return;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int n = n0 + wave * C + c;
        if (!FULL && n >= N) break;
        float* o = a.out + quad_index(row, n, N);
        if (EPI == kStore) {
            *o = acc[0][c];
        } else if (EPI == kResidual) {
            *o = *o + acc[0][c];
        } else if (EPI == kSwiglu) {
            const float g = acc[0][c];
            *o = (g / (1.0f + ref_expf(-g))) * acc[S::kMats - 1][c];
        }
    }
}

// Combines the per-work-group partials of each row in work-group (= column)
// order: largest value, earliest index among equal values.
__global__ __launch_bounds__(256) void head_argmax_kernel(const float* __restrict__ best_value,
                                                          const int32_t* __restrict__ best_index,
                                                          const int32_t* __restrict__ bad, int groups,
                                                          int32_t* __restrict__ argmax,
                                                          int32_t* __restrict__ nonfinite) {
    __shared__ float sv[256];
    __shared__ int32_t si[256];
    __shared__ int32_t sb[256];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float* v = best_value + (size_t)row * groups;
    const int32_t* ix = best_index + (size_t)row * groups;
    const int32_t* bd = bad + (size_t)row * groups;
    float best = 0.0f;
    int32_t best_i = -1, any_bad = 0;
    for (int g = tid; g < groups; g += 256) {
        const int32_t i = ix[g];
        any_bad |= bd[g];
        if (i >= 0 && (best_i < 0 || best < v[g])) {  // g ascending within the thread
            best = v[g];
            best_i = i;
        }
    }
    sv[tid] = best;
    si[tid] = best_i;
    sb[tid] = any_bad;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (tid < s) {
            const float ov = sv[tid + s];
            const int32_t oi = si[tid + s];
            const int32_t ci = si[tid];
            if (oi >= 0 && (ci < 0 || sv[tid] < ov || (sv[tid] == ov && oi < ci))) {
                sv[tid] = ov;
                si[tid] = oi;
            }
            sb[tid] |= sb[tid + s];
        }
        __syncthreads();
    }
    if (tid == 0) {
        argmax[row] = si[0];
        nonfinite[row] = sb[0];
    }
}

template <int C, int NW, int EPI, int NS>
hipError_t launch_shape(hipStream_t s, const GemmArgs& a) {
    using S = Shape<C, NW, EPI>;
    const dim3 grid((a.columns + S::kCols - 1) / S::kCols, (a.rows + 63) / 64);
    const bool full = a.inner % kChunk == 0 && a.columns % S::kCols == 0;
    if (full)
        gemm_rows_kernel<C, NW, EPI, NS, true><<<grid, S::kThreads, 0, s>>>(a);
    else
        gemm_rows_kernel<C, NW, EPI, NS, false><<<grid, S::kThreads, 0, s>>>(a);
    return hipGetLastError();
}


// ---------------------------------------------------------------------------
// Decode projections: one output column per wavefront.

constexpr int kColRing = 8;    // x quads in flight per wavefront
constexpr int kColBlocks = 8;  // 64-k weight blocks held per wavefront

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Quad q of a quad-layout row tile (lane = row) through a buffer resource.
__device__ __forceinline__ f4v load_x_global(__amdgpu_buffer_rsrc_t rsrc, int lane_bytes, int q) {
    return __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(rsrc, lane_bytes, q * 1024, 0));
}

// out[r][n] for the 64 rows r of tile blockIdx.y (lane = row) and column
// n = blockIdx.x*NW + wave; M = 2 runs the gate (w) and up (w2) chains side
// by side for the SwiGLU epilogue. k advances in quads (4 k) and 64-k blocks
// of 16 quads: lane l holds w[n][64J + 4(l%16) .. +3] of block J in one f4v,
// so quad i of block J multiplies by lane i's four floats. The products of
// quad q+1 are formed between the four dependent adds of quad q. Requires
// inner % 64 == 0; rows past a.rows read the tile's padding and are not
// stored.
//
// The weights sit in a ring of D blocks. With RELOAD the slot of block J
// takes block J + D once J is spent; without it the host guarantees
// inner <= 64*D, so the whole column is fetched before the first product.
// That is the faster form where it fits: s_waitcnt retires loads in issue
// order, so a weight block fetched from HBM during the loop stalls every x
// ring wait behind it, while fetched up front it costs one round trip per
// launch.
// With NORM the kernel first forms the RMSNorm of its row tile
// (llama_runner.cpp:10-16, rows.hip's rms_kernel arithmetic): the
// wavefronts load the raw tile into registers, wavefront 0 runs the 64
// sum-of-squares chains (its own quads from registers, the others' squares
// through LDS), and every wavefront writes its share of the tile as
// (x*scale)*w into LDS, from where the products read x. Requires !RELOAD and
// inner <= 64*D (the tile fits the work-group's LDS).
constexpr int kNormBlocks = 9;  // inner <= 576 for the folded RMSNorm

// RMSNorm of a 64-row tile (llama_runner.cpp:10-16, rows.hip's rms_kernel
// arithmetic) into tile_s ([quad][row]; NW spare quads take the writes of
// quads past the tile), for the products to read x from LDS. Wavefront w
// holds quads [w*S, (w+1)*S) of the raw tile in registers; wavefront 0 sums
// its own quads' squares at once while the others write their squares into
// the tile's slots, then continues with adds only over those, and every
// wavefront writes its quads, normalized, into the same slots. Ends with a
// barrier.
template <int NW>
__device__ __forceinline__ void norm_tile(const GemmArgs& a, __amdgpu_buffer_rsrc_t xrs, int xoff, int lane, int wave,
                                          int kq, f4v* tile_s, float* scale_s, float4* norm_s) {
    constexpr int kShare = kNormBlocks * 16 / NW;  // quads per wavefront at most
    static_assert(kNormBlocks * 16 % NW == 0, "tile split");
    const int S = kq / NW, q0 = wave * S;  // kq is a multiple of 16 and NW divides 16
    f4v v[kShare];
#pragma unroll
    for (int i = 0; i < kShare; ++i) v[i] = load_x_global(xrs, xoff, min(q0 + i, kq - 1));
    if ((int)threadIdx.x < kq) norm_s[threadIdx.x] = reinterpret_cast<const float4*>(a.norm)[threadIdx.x];
    // Sum of squares in column order (llama_runner.cpp:10-16).
    float sum = 0.0f;
    if (wave == 0) {
        // The squares of the next quad are formed between the four adds
        // of the pending one; pp starts as four zero squares, whose adds
        // leave sum at +0.0f.
        float pp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < kShare; ++i) {
            if (i < S) {
                sum = sum + pp[0];
                pp[0] = v[i].x * v[i].x;
                __builtin_amdgcn_sched_barrier(0);
                sum = sum + pp[1];
                pp[1] = v[i].y * v[i].y;
                __builtin_amdgcn_sched_barrier(0);
                sum = sum + pp[2];
                pp[2] = v[i].z * v[i].z;
                __builtin_amdgcn_sched_barrier(0);
                sum = sum + pp[3];
                pp[3] = v[i].w * v[i].w;
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        sum = sum + pp[0];
        sum = sum + pp[1];
        sum = sum + pp[2];
        sum = sum + pp[3];
    } else {
#pragma unroll
        for (int i = 0; i < kShare; ++i) {
            const int slot = i < S ? q0 + i : kNormBlocks * 16 + wave;
            tile_s[slot * 64 + lane] = v[i] * v[i];
        }
    }
    __syncthreads();
    if (wave == 0) {
        // Squares of quads S..kq-1, eight read while eight are added.
        auto add_sq = [&](const f4v& q) {
            sum = sum + q.x;
            sum = sum + q.y;
            sum = sum + q.z;
            sum = sum + q.w;
        };
        const int n = kq - S;
        const f4v* t4 = tile_s + S * 64 + lane;
        int q = 0;
        if (n >= 8) {
            f4v u0[8], u1[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) u0[j] = t4[j * 64];
            for (; q + 16 <= n; q += 16) {
#pragma unroll
                for (int j = 0; j < 8; ++j) u1[j] = t4[(q + 8 + j) * 64];
#pragma unroll
                for (int j = 0; j < 8; ++j) add_sq(u0[j]);
#pragma unroll
                for (int j = 0; j < 8; ++j) u0[j] = t4[min(q + 16 + j, n - 1) * 64];
#pragma unroll
                for (int j = 0; j < 8; ++j) add_sq(u1[j]);
            }
            if (q + 8 <= n) {
#pragma unroll
                for (int j = 0; j < 8; ++j) add_sq(u0[j]);
                q += 8;
            }
        }
        for (; q < n; ++q) add_sq(t4[q * 64]);
        scale_s[lane] = 1.0f / sqrtf(sum / (float)a.inner + a.eps);
    }
    __syncthreads();
    const float scale = scale_s[lane];
#pragma unroll
    for (int i = 0; i < kShare; ++i) {
        const float4 g = norm_s[min(q0 + i, kq - 1)];
        const int slot = i < S ? q0 + i : kNormBlocks * 16 + wave;
        tile_s[slot * 64 + lane] =
            f4v{v[i].x * scale * g.x, v[i].y * scale * g.y, v[i].z * scale * g.z, v[i].w * scale * g.w};
    }
    __syncthreads();
}

// UP (M = 2, whole column held): the second matrix's weights (up) also go
// through a per-wavefront LDS ring of two 64-k blocks, written from the
// registers one block ahead by lanes 0-15 and read back at one address four
// quads ahead, so its products are plain v_mul_f32; the first (gate) keeps
// the DPP broadcast. The ring is the wavefront's own: no barrier.
template <int M, int NW, int EPI, int D = kColBlocks, bool RELOAD = true, bool NORM = false, bool UP = false>
__global__ __launch_bounds__(NW * 64) void gemm_column_kernel(GemmArgs a) {
    constexpr int RX = kColRing;
    static_assert((D * 16) % RX == 0, "ring slots repeat every D blocks");
    static_assert(!NORM || (!RELOAD && D == kNormBlocks), "folded RMSNorm holds the whole tile");
    static_assert(!UP || (M == 2 && !RELOAD), "the up ring is filled from the held column");
    // [quad][row]; NW spare quads take the writes of quads past the tile
    __shared__ f4v tile_s[NORM ? (kNormBlocks * 16 + NW) * 64 : 1];
    __shared__ float scale_s[NORM ? 64 : 1];
    __shared__ float4 norm_s[NORM ? kNormBlocks * 16 : 1];  // RMSNorm weights by quad
    __shared__ f4v up_s[UP ? NW * 32 : 1];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tile = blockIdx.y;
    const int N = a.columns;
    const int col = blockIdx.x * NW + wave;
    const int n = min(col, N - 1);
    const int kq = a.inner >> 2, KB = a.inner >> 6;
    const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(a.x + (size_t)tile * kq * 256, (uint32_t)kq * 1024u);
    const int xoff = lane * 16;
    const f4v* ws[2];
    ws[0] = reinterpret_cast<const f4v*>(a.w) + (size_t)n * kq + (lane & 15);
    ws[1] = reinterpret_cast<const f4v*>(M == 2 ? a.w2 : a.w) + (size_t)n * kq + (lane & 15);
    auto load_x = [&](int q) {
        if (NORM) return tile_s[min(q, kq - 1) * 64 + lane];
        return __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff, min(q, kq - 1) * 1024, 0));
    };

    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;
    f4v wr[D][M];
    f4v xr[RX];
    // Weights are read once per step: non-temporal loads.
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
        for (int m = 0; m < M; ++m) wr[d][m] = __builtin_nontemporal_load(&ws[m][min(d, KB - 1) * 16]);
    if (NORM) norm_tile<NW>(a, xrs, xoff, lane, wave, kq, tile_s, scale_s, norm_s);
#pragma unroll
    for (int i = 0; i < RX; ++i) xr[i] = load_x(i);
    // UP: ring quads 0-15 hold block J (even J) or 16-31 (odd J); uq holds
    // the up weights of quads q+1 .. q+4 (slot (q+1) % 4 is used next).
    f4v* const ur = up_s + (UP ? wave * 32 : 0);
    f4v uq[4];
    if (UP) {
        if (lane < 16) {
            ur[lane] = wr[0][M - 1];
            ur[16 + lane] = wr[D > 1 ? 1 : 0][M - 1];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) uq[k] = ur[k];
    }
    float pn[M][4];  // products of the next quad
    {
        const f4v xv = xr[0];
        xr[0] = load_x(RX);
#pragma unroll
        for (int m = 0; m < M; ++m) {
            if (UP && m == 1) {
                pn[m][0] = uq[0].x * xv.x;
                pn[m][1] = uq[0].y * xv.y;
                pn[m][2] = uq[0].z * xv.z;
                pn[m][3] = uq[0].w * xv.w;
            } else {
                pn[m][0] = mul_bcast<0>(wr[0][m].x, xv.x);
                pn[m][1] = mul_bcast<0>(wr[0][m].y, xv.y);
                pn[m][2] = mul_bcast<0>(wr[0][m].z, xv.z);
                pn[m][3] = mul_bcast<0>(wr[0][m].w, xv.w);
            }
        }
        if (UP) uq[0] = ur[4];
    }
    for (int J0 = 0; J0 < KB; J0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int J = J0 + d;
            if (J >= KB) break;
            // UP: block J+1 goes into the ring slot block J-1 has left.
            if (UP && d >= 1 && lane < 16 && J + 1 < KB) ur[((J + 1) & 1) * 16 + lane] = wr[d + 1 < D ? d + 1 : d][M - 1];
            const int jb = (J & 1) * 16;
            // Quad i of block J: add its products in k order while forming
            // those of the next quad (lane i+1 of this block, or lane 0 of
            // the next block held in wr[(d+1)%D]; for UP's second matrix the
            // ring quad read four quads ago).
#define MP_COLUMN_MUL(i, m, c) \
    ((UP && (m) == 1) ? uv.c * xv.c : mul_bcast<((i) + 1) & 15>(wr[dn][m].c, xv.c))
#define MP_COLUMN_QUAD(i)                                                               \
    {                                                                                   \
        const int slot = (d * 16 + (i) + 1) % RX;                                       \
        const int dn = (i) == 15 ? (d + 1) % D : d;                                     \
        const f4v xv = xr[slot];                                                        \
        xr[slot] = load_x(J * 16 + (i) + 1 + RX);                                       \
        const f4v uv = uq[((i) + 1) % 4];                                               \
        for (int m = 0; m < M; ++m) {                                                   \
            float t = acc[m];                                                           \
            t = t + pn[m][0];                                                           \
            pn[m][0] = MP_COLUMN_MUL(i, m, x);                                           \
            __builtin_amdgcn_sched_barrier(0);                                          \
            t = t + pn[m][1];                                                           \
            pn[m][1] = MP_COLUMN_MUL(i, m, y);                                           \
            __builtin_amdgcn_sched_barrier(0);                                          \
            t = t + pn[m][2];                                                           \
            pn[m][2] = MP_COLUMN_MUL(i, m, z);                                           \
            __builtin_amdgcn_sched_barrier(0);                                          \
            t = t + pn[m][3];                                                           \
            pn[m][3] = MP_COLUMN_MUL(i, m, w);                                           \
            __builtin_amdgcn_sched_barrier(0);                                          \
            acc[m] = t;                                                                 \
        }                                                                               \
        if (UP) uq[((i) + 1) % 4] = ur[(jb + (i) + 5) & 31];                            \
    }
            MP_COLUMN_QUAD(0) MP_COLUMN_QUAD(1) MP_COLUMN_QUAD(2) MP_COLUMN_QUAD(3)
            MP_COLUMN_QUAD(4) MP_COLUMN_QUAD(5) MP_COLUMN_QUAD(6) MP_COLUMN_QUAD(7)
            MP_COLUMN_QUAD(8) MP_COLUMN_QUAD(9) MP_COLUMN_QUAD(10) MP_COLUMN_QUAD(11)
            MP_COLUMN_QUAD(12) MP_COLUMN_QUAD(13) MP_COLUMN_QUAD(14)
            // Block J's weights are spent; the slot takes block J + D.
            if (RELOAD) {
#pragma unroll
                for (int m = 0; m < M; ++m) wr[d][m] = ws[m][min(J + D, KB - 1) * 16];
            }
            MP_COLUMN_QUAD(15)
#undef MP_COLUMN_QUAD
#undef MP_COLUMN_MUL
        }
    }

    const int row = tile * 64 + lane;
    if (row >= a.rows || col >= N) return;
    float* o = a.out + quad_index(row, n, N);
    if (EPI == kStore) {
        *o = acc[0];
    } else if (EPI == kResidual) {
        *o = *o + acc[0];
    } else if (EPI == kSwiglu) {
        const float g = acc[0];
        *o = (g / (1.0f + ref_expf(-g))) * acc[M - 1];
    }
}


template <int M, int NW, int EPI, int D, bool RELOAD, bool NORM = false, bool UP = false>
hipError_t launch_column(hipStream_t s, const GemmArgs& a) {
    const dim3 grid((a.columns + NW - 1) / NW, (a.rows + 63) / 64);
    gemm_column_kernel<M, NW, EPI, D, RELOAD, NORM, UP><<<grid, NW * 64, 0, s>>>(a);
    return hipGetLastError();
}

// One row tile, M = 1 (QKV with the folded RMSNorm, O, down): the same
// chains as gemm_column_kernel, k in order from 0, but the weight column is
// staged in LDS (QMAX quads at most) and reaches the lanes through broadcast
// reads (every lane reads the same 16 bytes), so each product is a plain
// v_mul_f32 rather than a DPP row broadcast. Each wavefront writes and reads
// only its own column: LDS orders a wavefront's accesses, no barrier. With
// NORM, x is the RMSNorm of the tile formed by norm_tile in LDS (inner <=
// 576; with four wavefronts the tile and the columns just fit the 160 KB).
constexpr int kColWeightAhead = 4;  // weight quads read ahead from LDS

template <int NW, int EPI, int QMAX, bool NORM = false>
__global__ __launch_bounds__(NW * 64) void gemm_column_lds_kernel(GemmArgs a) {
    constexpr int RX = kColRing, RW = kColWeightAhead;
    static_assert(!NORM || QMAX == kNormBlocks * 16, "the folded RMSNorm holds the whole tile");
    __shared__ f4v tile_s[NORM ? (kNormBlocks * 16 + NW) * 64 : 1];
    __shared__ float scale_s[NORM ? 64 : 1];
    __shared__ float4 norm_s[NORM ? kNormBlocks * 16 : 1];
    static_assert(16 % RX == 0 || RX % 16 == 0, "x ring slots repeat every 16 quads");
    static_assert(16 % RW == 0, "weight ring slots repeat every 16 quads");
    // RW + 1 spare quads per column take the reads past its end (the last
    // step reads quad kq + RW, whose products are never added).
    __shared__ f4v wl_s[NW][QMAX + RW + 1];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tile = blockIdx.y;
    const int N = a.columns;
    const int col = blockIdx.x * NW + wave;
    const int n = min(col, N - 1);
    const int kq = a.inner >> 2;
    const __amdgpu_buffer_rsrc_t xrs = buffer_rsrc(a.x + (size_t)tile * kq * 256, (uint32_t)kq * 1024u);
    const int xoff = lane * 16;
    auto load_x = [&](int q) {
        if (NORM) return tile_s[min(q, kq - 1) * 64 + lane];
        return load_x_global(xrs, xoff, min(q, kq - 1));
    };
    // The column, all loads in flight with the first x quads (or the raw
    // tile of the folded RMSNorm).
    constexpr int WJ = (QMAX + 63) / 64;
    const f4v* wsrc = reinterpret_cast<const f4v*>(a.w) + (size_t)n * kq;
    f4v wt[WJ];
#pragma unroll
    for (int j = 0; j < WJ; ++j) wt[j] = __builtin_nontemporal_load(&wsrc[min(j * 64 + lane, kq - 1)]);
    if (NORM) norm_tile<NW>(a, xrs, xoff, lane, wave, kq, tile_s, scale_s, norm_s);
    f4v xr[RX];
#pragma unroll
    for (int i = 0; i < RX; ++i) xr[i] = load_x(i);
    f4v* const wl = wl_s[wave];
#pragma unroll
    for (int j = 0; j < WJ; ++j)
        if (j * 64 + lane < kq) wl[j * 64 + lane] = wt[j];
    f4v wq[RW];
#pragma unroll
    for (int i = 0; i < RW; ++i) wq[i] = wl[i];

    float acc = 0.0f;
    float pn[4];  // products of the next quad
    {
        const f4v xv = xr[0], wv = wq[0];
        xr[0] = load_x(RX);
        wq[0] = wl[RW];
        pn[0] = wv.x * xv.x;
        pn[1] = wv.y * xv.y;
        pn[2] = wv.z * xv.z;
        pn[3] = wv.w * xv.w;
    }
    for (int q0 = 0; q0 < kq; q0 += 16) {
        const f4v* const wlq = wl + q0 + 1 + RW;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            // Add quad q0+i's products in k order while forming quad q0+i+1's.
            const int sx = (i + 1) % RX, sw = (i + 1) % RW;
            const f4v xv = xr[sx], wv = wq[sw];
            xr[sx] = load_x(q0 + i + 1 + RX);
            wq[sw] = wlq[i];
            float t = acc;
            t = t + pn[0];
            pn[0] = wv.x * xv.x;
            __builtin_amdgcn_sched_barrier(0);
            t = t + pn[1];
            pn[1] = wv.y * xv.y;
            __builtin_amdgcn_sched_barrier(0);
            t = t + pn[2];
            pn[2] = wv.z * xv.z;
            __builtin_amdgcn_sched_barrier(0);
            t = t + pn[3];
            pn[3] = wv.w * xv.w;
            __builtin_amdgcn_sched_barrier(0);
            acc = t;
        }
    }

    const int row = tile * 64 + lane;
    if (row >= a.rows || col >= N) return;
    float* o = a.out + quad_index(row, n, N);
    if (EPI == kStore) *o = acc;
    else *o = *o + acc;
}

template <int NW, int EPI, int QMAX, bool NORM = false>
hipError_t launch_column_lds(hipStream_t s, const GemmArgs& a) {
    const dim3 grid((a.columns + NW - 1) / NW, (a.rows + 63) / 64);
    gemm_column_lds_kernel<NW, EPI, QMAX, NORM><<<grid, NW * 64, 0, s>>>(a);
    return hipGetLastError();
}

// A weight column of up to 24 64-k blocks (inner <= 1536) is held whole;
// longer ones stream through a kColBlocks ring.
template <int EPI>
hipError_t launch_column_one(hipStream_t s, const GemmArgs& a) {
    const int blocks = a.inner / 64;
    if (blocks <= 9) return launch_column_lds<4, EPI, 9 * 16>(s, a);
    if (blocks <= 24) return launch_column_lds<4, EPI, 24 * 16>(s, a);
    return launch_column<1, 4, EPI, kColBlocks, true>(s, a);
}

}  // namespace

int head_groups(int columns) { return (columns + kHeadColumns - 1) / kHeadColumns; }

bool gemm_normed_fits(Epilogue epilogue, const GemmArgs& a) {
    return a.rows > 0 && a.rows <= 64 && a.columns > 0 && a.inner > 0 && a.inner % 64 == 0 &&
           a.inner <= 64 * kNormBlocks && a.norm && (epilogue == kStore || epilogue == kSwiglu);
}

hipError_t launch_gemm_normed(hipStream_t s, Epilogue epilogue, const GemmArgs& a) {
    if (!gemm_normed_fits(epilogue, a)) return hipErrorInvalidValue;
    // The LDS tile allows one work-group per CU: four wavefronts for one
    // matrix, eight for gate and up.
    if (epilogue == kStore) return launch_column_lds<4, kStore, kNormBlocks * 16, true>(s, a);
    // Six wavefronts where they split the tile evenly (inner a multiple of
    // 96): one work-group per CU at 1,536 columns, fewer waves on its LDS.
    if ((a.inner / 4) % 6 == 0) return launch_column<2, 6, kSwiglu, kNormBlocks, false, true, true>(s, a);
    return launch_column<2, 8, kSwiglu, kNormBlocks, false, true, true>(s, a);
}

hipError_t launch_gemm(hipStream_t s, Epilogue epilogue, const GemmArgs& a) {
    if (a.rows <= 0 || a.columns <= 0) return hipSuccess;
    if (a.inner <= 0 || a.inner % 4 || a.columns % 4) return hipErrorInvalidValue;
    // One row tile (decode): one column per wavefront with register-held
    // weights. More rows: C = 4 columns per wavefront through LDS.
    const bool many = a.rows > 64;
    if (!many && a.inner % 64 == 0) {
        switch (epilogue) {
        case kStore: return launch_column_one<kStore>(s, a);
        case kResidual: return launch_column_one<kResidual>(s, a);
        case kSwiglu:
            return a.inner <= 9 * 64 ? launch_column<2, 2, kSwiglu, 9, false>(s, a)
                                     : launch_column<2, 2, kSwiglu, kColBlocks, true>(s, a);
        default: break;
        }
    }
    switch (epilogue) {
    case kStore: return many ? launch_shape<4, 4, kStore, 5>(s, a) : launch_shape<1, 4, kStore, 6>(s, a);
    case kResidual: return many ? launch_shape<4, 4, kResidual, 5>(s, a) : launch_shape<1, 4, kResidual, 6>(s, a);
    case kSwiglu: return many ? launch_shape<4, 4, kSwiglu, 5>(s, a) : launch_shape<1, 4, kSwiglu, 6>(s, a);
    case kHead: {
        using S = Shape<kHeadColumns / 8, 8, kHead>;
        static_assert(S::kCols == kHeadColumns, "head work-group width");
        return launch_shape<kHeadColumns / 8, 8, kHead, 4>(s, a);
    }
    }
    return hipErrorInvalidValue;
}

hipError_t launch_head_argmax(hipStream_t s, const GemmArgs& a, int32_t* argmax, int32_t* nonfinite) {
    if (a.rows <= 0) return hipSuccess;
    head_argmax_kernel<<<a.rows, 256, 0, s>>>(a.best_value, a.best_index, a.bad, a.groups, argmax, nonfinite);
    return hipGetLastError();
}

}  // namespace mphip
