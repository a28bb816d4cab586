// gfx950 kernels of the MiniPrefix FP32 forward.
//
// Every reduction that the reference CPU path performs sequentially
// (miniprefix/src/backend/cpu/llama_runner.cpp:10-104, projections in
// src/backend/cpu/matmul_kernel.cpp:101-109) runs in ONE lane in the same
// order, with multiply and add rounded separately (this file is compiled
// with -ffp-contract=off). Parallelism comes from independent outputs:
// columns x rows for projections, tokens for scores, (head, dim) for the
// PV sums. Tiles are staged through LDS so HBM reads stay coalesced.
#include "kernels.h"
#include "exact_math.h"

namespace mphip {
namespace {

constexpr int kWave = 64;

// Blocks are dispatched round-robin over the 8 XCDs of an MI355X. Give each
// XCD a contiguous range of tiles so neighbouring column tiles (which share
// 128-byte lines) land in the same L2.
__device__ __forceinline__ int xcd_tile(int block, int tiles) {
    const int q = tiles / 8, rem = tiles % 8;
    const int xcd = block % 8, i = block / 8;
    return xcd * q + (xcd < rem ? xcd : rem) + i;
}

// Zeroes a loaded value without a select on the load itself: selects of a
// load are turned into exec-masked branches by the backend, which then
// drains every outstanding load at the branch. The mask is all ones or 0.
__device__ __forceinline__ float keep_if(float v, uint32_t mask) {
    return __uint_as_float(__float_as_uint(v) & mask);
}
__device__ __forceinline__ float4 keep_if(float4 v, uint32_t mask) {
    return make_float4(keep_if(v.x, mask), keep_if(v.y, mask), keep_if(v.z, mask), keep_if(v.w, mask));
}
__device__ __forceinline__ uint32_t mask_of(bool in) { return in ? 0xffffffffu : 0u; }

__global__ void embed_kernel(const float* __restrict__ embedding, const int32_t* __restrict__ tokens,
                             float* __restrict__ x, int hidden) {
    const int r = blockIdx.x;
    const float* src = embedding + (size_t)tokens[r] * hidden;
    float* dst = x + (size_t)r * hidden;
    for (int i = threadIdx.x; i < hidden; i += blockDim.x) dst[i] = src[i];
}

// Sequential float sum of n values (n a multiple of 4, 16-byte aligned) in
// the calling lane, in index order, starting from `sum`. Two blocks of
// sixteen ping-pong: one is read while the other is added.
__device__ __forceinline__ void sum_block(const float4 (&a)[4], float& sum) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        sum = sum + a[j].x;
        sum = sum + a[j].y;
        sum = sum + a[j].z;
        sum = sum + a[j].w;
    }
}

__device__ __forceinline__ float sequential_sum(const float* v, int n, float sum = 0.0f) {
    const float4* v4 = reinterpret_cast<const float4*>(v);
    const int n4 = n / 4;
    int i = 0;
    if (n4 >= 4) {
        float4 a[4], b[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) a[j] = v4[j];
        for (; i + 8 <= n4; i += 8) {
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = v4[i + 4 + j];
            sum_block(a, sum);
            const int in = min(i + 8, n4 - 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) a[j] = v4[in + j];
            sum_block(b, sum);
        }
        if (i + 4 <= n4) {  // `a` holds the block at i
            sum_block(a, sum);
            i += 4;
        }
    }
    for (; i < n4; ++i) {
        const float4 a = v4[i];
        sum = sum + a.x;
        sum = sum + a.y;
        sum = sum + a.z;
        sum = sum + a.w;
    }
    return sum;
}

// One wave per row. Squares are formed in parallel (each is a single
// rounding), the sum runs sequentially in lane 0 like llama_runner.cpp:12.
__global__ __launch_bounds__(64) void rms_kernel(const float* __restrict__ x, int ldx,
                                                 const int32_t* __restrict__ row_map,
                                                 const float* __restrict__ weight,
                                                 float* __restrict__ out, int ldo, int width,
                                                 float eps) {
    extern __shared__ float4 rms_lds4[];
    float* squares = reinterpret_cast<float*>(rms_lds4);
    __shared__ float scale_shared;
    const int r = blockIdx.x;
    const float* xr = x + (size_t)(row_map ? row_map[r] : r) * ldx;
    const int padded = (width + 3) & ~3;
    for (int i = threadIdx.x; i < padded; i += kWave) {
        const float v = i < width ? xr[i] : 0.0f;
        squares[i] = v * v;
    }
    __syncthreads();
    // Zero padding leaves the non-negative running sum unchanged.
    if (threadIdx.x == 0) scale_shared = 1.0f / sqrtf(sequential_sum(squares, padded) / (float)width + eps);
    __syncthreads();
    const float scale = scale_shared;
    float* o = out + (size_t)r * ldo;
    for (int i = threadIdx.x; i < width; i += kWave) o[i] = xr[i] * scale * weight[i];
}

template <int EPI>
__device__ __forceinline__ void store_result(float* out, float acc, float acc2) {
    if (EPI == kStore) {
        *out = acc;
    } else if (EPI == kResidual) {
        *out = *out + acc;
    } else {
        const float g = acc;
        *out = (g / (1.0f + ref_expf(-g))) * acc2;
    }
}

// acc += x[k]*w[k] for k = 0..n-1 in order (and acc2 with u when DUAL),
// multiply and add rounded separately. x, w and u live in LDS; w and u are
// strided by STRIDE floats (0: by `runtime_stride`). Two 16-step register
// blocks ping-pong: one is read from LDS while the other is summed, with no
// register copies between them.
template <bool DUAL>
struct ChainBlock {
    float4 x[4];
    float w[16];
    float u[DUAL ? 16 : 1];
};

template <bool DUAL>
__device__ __forceinline__ void chain_load(ChainBlock<DUAL>& b, const float* x, const float* w,
                                           const float* u, int k, int stride) {
#pragma unroll
    for (int j = 0; j < 4; ++j) b.x[j] = reinterpret_cast<const float4*>(x + k)[j];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        b.w[j] = w[(k + j) * stride];
        if (DUAL) b.u[j] = u[(k + j) * stride];
    }
}

template <bool DUAL>
__device__ __forceinline__ void chain_sum(const ChainBlock<DUAL>& b, float& acc, float& acc2) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        acc = acc + b.x[j].x * b.w[4 * j + 0];
        acc = acc + b.x[j].y * b.w[4 * j + 1];
        acc = acc + b.x[j].z * b.w[4 * j + 2];
        acc = acc + b.x[j].w * b.w[4 * j + 3];
        if (DUAL) {
            acc2 = acc2 + b.x[j].x * b.u[4 * j + 0];
            acc2 = acc2 + b.x[j].y * b.u[4 * j + 1];
            acc2 = acc2 + b.x[j].z * b.u[4 * j + 2];
            acc2 = acc2 + b.x[j].w * b.u[4 * j + 3];
        }
    }
}

template <bool DUAL, int STRIDE>
__device__ __forceinline__ void chain_dot(const float* x, const float* w, const float* u, int n,
                                          float& acc, float& acc2, int runtime_stride = 0) {
    const int stride = STRIDE ? STRIDE : runtime_stride;
    int k = 0;
    if (n >= 16) {
        ChainBlock<DUAL> a, b;
        chain_load(a, x, w, u, 0, stride);
        for (; k + 32 <= n; k += 32) {
            chain_load(b, x, w, u, k + 16, stride);
            chain_sum(a, acc, acc2);
            // Next `a`; on the last pass any aligned in-range block is read and
            // left unused.
            chain_load(a, x, w, u, min(k + 32, (n - 16) & ~3), stride);
            chain_sum(b, acc, acc2);
        }
        if (k + 16 <= n) {  // `a` holds the block at k
            chain_sum(a, acc, acc2);
            k += 16;
        }
    }
    for (; k < n; ++k) {
        acc = acc + x[k] * w[k * stride];
        if (DUAL) acc2 = acc2 + x[k] * u[k * stride];
    }
}

// Few rows (decode of one to four sequences): 16 columns per work-group so
// that even a 576-column projection spreads over 36 CUs. All four waves
// stage a K-chunk of the 16-column weight slab (and of x) into LDS; the
// next chunk's loads are issued before the current chunk is summed. Lanes
// (row, column) of wave 0 walk k in order.
constexpr int kSmallColumns = 16;
constexpr int kSmallRows = 4;
constexpr int kSmallChunk = 384;
constexpr int kSmallWLoads = kSmallChunk * kSmallColumns / 256;  // per thread per matrix
constexpr int kSmallXLoads = kSmallRows * kSmallChunk / 256;

template <int EPI>
__global__ __launch_bounds__(256) void gemm_small_kernel(const float* __restrict__ x, int ldx,
                                                         int rows, int inner,
                                                         const float* __restrict__ w,
                                                         const float* __restrict__ w2,
                                                         int columns, int ldw, float* out, int ldo,
                                                         int tiles) {
    constexpr bool kDual = EPI == kSwiglu;
    __shared__ float xs[kSmallRows * kSmallChunk];
    __shared__ float ws[kSmallChunk * kSmallColumns];
    __shared__ float ws2[kDual ? kSmallChunk * kSmallColumns : 1];
    const int tid = threadIdx.x;
    const int n0 = xcd_tile(blockIdx.x, tiles) * kSmallColumns;
    const int r = tid / kSmallColumns, c = tid % kSmallColumns;
    const int n = n0 + c;
    float wreg[kSmallWLoads], ureg[kDual ? kSmallWLoads : 1], xreg[kSmallXLoads];
    // Issue: raw loads from clamped in-range addresses (masked on commit).
    auto issue = [&](int k0) {
        const int kc = min(kSmallChunk, inner - k0);
#pragma unroll
        for (int j = 0; j < kSmallWLoads; ++j) {
            const int e = tid + j * 256;
            const int kk = e / kSmallColumns, cc = e % kSmallColumns;
            const bool in = kk < kc && n0 + cc < columns;
            const size_t off = in ? (size_t)(k0 + kk) * ldw + n0 + cc : 0;
            wreg[j] = w[off];
            if (kDual) ureg[j] = w2[off];
        }
#pragma unroll
        for (int j = 0; j < kSmallXLoads; ++j) {
            const int e = tid + j * 256;
            const int rr = e / kSmallChunk, kk = e % kSmallChunk;
            const bool in = rr < rows && kk < kc;
            xreg[j] = x[in ? (size_t)rr * ldx + k0 + kk : 0];
        }
    };
    auto commit = [&](int k0) {
        const int kc = min(kSmallChunk, inner - k0);
#pragma unroll
        for (int j = 0; j < kSmallWLoads; ++j) {
            const int e = tid + j * 256;
            const int kk = e / kSmallColumns, cc = e % kSmallColumns;
            const uint32_t m = mask_of(kk < kc && n0 + cc < columns);
            ws[e] = keep_if(wreg[j], m);
            if (kDual) ws2[e] = keep_if(ureg[j], m);
        }
#pragma unroll
        for (int j = 0; j < kSmallXLoads; ++j) {
            const int e = tid + j * 256;
            const int rr = e / kSmallChunk, kk = e % kSmallChunk;
            xs[e] = keep_if(xreg[j], mask_of(rr < rows && kk < kc));
        }
    };
    float acc = 0.0f, acc2 = 0.0f;
    issue(0);
    for (int k0 = 0; k0 < inner; k0 += kSmallChunk) {
        const int kc = min(kSmallChunk, inner - k0);
        commit(k0);
        if (k0 + kSmallChunk < inner) issue(k0 + kSmallChunk);
        __syncthreads();
        if (r < rows)
            chain_dot<kDual, kSmallColumns>(xs + r * kSmallChunk, ws + c, ws2 + (kDual ? c : 0), kc,
                                            acc, acc2);
        __syncthreads();
    }
    if (r < rows && n < columns) store_result<EPI>(out + (size_t)r * ldo + n, acc, acc2);
}

// Many rows (batched decode, prefill chunks): 64 columns x 4 rows per
// 256-thread work-group, one output chain per lane (lane = column,
// wave = row), so even a 576-column projection of 64 rows spans 144 CUs.
// K-chunks of the weight tile are shared by the 4 waves through LDS; the
// global loads of the next kRing chunks stay in flight in a register ring
// so the short per-chunk compute does not wait on memory.
constexpr int kWideThreads = 256;
constexpr int kWideColumns = 64;
constexpr int kWideRows = kWideThreads / 64;
constexpr int kRing = 4;

template <int EPI, bool FULL>
__global__ __launch_bounds__(kWideThreads) void gemm_wide_kernel(const float* __restrict__ x, int ldx,
                                                         int rows, int inner,
                                                         const float* __restrict__ w,
                                                         const float* __restrict__ w2,
                                                         int columns, int ldw, float* out, int ldo,
                                                         int column_tiles) {
    constexpr int kDual = EPI == kSwiglu ? 2 : 1;
    constexpr int kChunk = EPI == kSwiglu ? 32 : 64;          // k rows per chunk
    constexpr int kPerThread = kChunk * kWideColumns / kWideThreads;  // weight floats per thread
    constexpr int kXThreads = kWideRows * kChunk / 4;         // threads staging x (float4 each)
    __shared__ float ws[2][kDual][kChunk * kWideColumns];
    __shared__ float4 xs4[2][kXThreads];
    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int column_tile = xcd_tile(blockIdx.x, column_tiles);
    const int n0 = column_tile * kWideColumns, r0 = blockIdx.y * kWideRows;
    const int n = n0 + lane, row = r0 + wave;
    const int lr = tid / (kChunk / 4), lk = (tid % (kChunk / 4)) * 4;
    float wring[kRing][kDual][kPerThread];
    float4 xring[kRing];
    // Thread element j of a chunk is weight row (tid/64 + rows_per_pass*j),
    // column tid%64 of the tile; offsets are 32-bit from the matrix base.
    constexpr int kRowsPerPass = kWideThreads / kWideColumns;
    const uint32_t thread_off = (uint32_t)(tid / kWideColumns) * (uint32_t)ldw + (uint32_t)(n0 + tid % kWideColumns);
    auto fetch = [&](int k0, float (&wreg)[kDual][kPerThread], float4& xreg) {
#pragma unroll
        for (int m = 0; m < kDual; ++m) {
            const float* src = m == 0 ? w : w2;
#pragma unroll
            for (int j = 0; j < kPerThread; ++j) {
                if (FULL) {
                    wreg[m][j] = src[thread_off + (uint32_t)(k0 + kRowsPerPass * j) * (uint32_t)ldw];
                } else {
                    const int e = tid + j * kWideThreads;
                    const int kk = e / kWideColumns, cc = e % kWideColumns;
                    const bool in = (k0 + kk < inner) && (n0 + cc < columns);
                    // Raw load from an in-range address; masked when stashed, so
                    // the ring's loads stay in flight.
                    wreg[m][j] = src[in ? (size_t)(k0 + kk) * ldw + n0 + cc : 0];
                }
            }
        }
        if (tid < kXThreads) {
            const int gr = r0 + lr;
            if (FULL) {
                xreg = *reinterpret_cast<const float4*>(x + (size_t)(gr < rows ? gr : 0) * ldx + k0 + lk);
            } else {
                float v[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const bool in = gr < rows && k0 + lk + j < inner;
                    v[j] = x[in ? (size_t)gr * ldx + k0 + lk + j : 0];
                }
                xreg = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    };
    float acc = 0.0f, acc2 = 0.0f;
    const int chunks = (inner + kChunk - 1) / kChunk;
#pragma unroll
    for (int j = 0; j < kRing; ++j)
        if (j < chunks) fetch(j * kChunk, wring[j], xring[j]);
    for (int c0 = 0; c0 < chunks; c0 += kRing) {
#pragma unroll
        for (int j = 0; j < kRing; ++j) {
            const int chunk = c0 + j;
            if (chunk >= chunks) break;
            const int buffer = chunk & 1;
            const int k0 = chunk * kChunk;
#pragma unroll
            for (int m = 0; m < kDual; ++m)
#pragma unroll
                for (int e = 0; e < kPerThread; ++e) {
                    const int el = tid + e * kWideThreads;
                    if (FULL) {
                        ws[buffer][m][el] = wring[j][m][e];
                    } else {
                        const int kk = el / kWideColumns, cc = el % kWideColumns;
                        ws[buffer][m][el] = keep_if(wring[j][m][e], mask_of(k0 + kk < inner && n0 + cc < columns));
                    }
                }
            if (tid < kXThreads) {
                const int gr = r0 + lr;
                const float4 xv = xring[j];
                if (FULL)
                    xs4[buffer][tid] = gr < rows ? xv : make_float4(0.f, 0.f, 0.f, 0.f);
                else
                    xs4[buffer][tid] = make_float4(keep_if(xv.x, mask_of(gr < rows && k0 + lk + 0 < inner)),
                                                   keep_if(xv.y, mask_of(gr < rows && k0 + lk + 1 < inner)),
                                                   keep_if(xv.z, mask_of(gr < rows && k0 + lk + 2 < inner)),
                                                   keep_if(xv.w, mask_of(gr < rows && k0 + lk + 3 < inner)));
            }
            if (chunk + kRing < chunks) fetch((chunk + kRing) * kChunk, wring[j], xring[j]);
            __syncthreads();
            const int kc = min(kChunk, inner - chunk * kChunk);
            const float* xr = reinterpret_cast<const float*>(xs4[buffer]) + wave * kChunk;
            const float* wk = ws[buffer][0] + lane;
            const float* uk = ws[buffer][kDual - 1] + lane;
            chain_dot<EPI == kSwiglu, kWideColumns>(xr, wk, uk, kc, acc, acc2);
        }
    }
    if (row < rows && n < columns) store_result<EPI>(out + (size_t)row * ldo + n, acc, acc2);
}

__device__ __forceinline__ size_t pool_offset(const int32_t* table, int token, int layer,
                                              int layers, int block_tokens, int kv_width) {
    return (((size_t)table[token / block_tokens] * layers + layer) * block_tokens +
            token % block_tokens) * (size_t)kv_width;
}

// llama_runner.cpp:17-22 and :81-83. cos/sin come from the host table of
// float(pos)/powf(theta, 2d/dim), so the rotation is bit-identical.
__global__ void rope_append_kernel(float* __restrict__ qkv, int ldqkv, int heads, int kv_heads,
                                   int dim, const float* __restrict__ cos_table,
                                   const float* __restrict__ sin_table, RowMeta meta, PagedKv kv,
                                   int layer) {
    const int r = blockIdx.x;
    const int pos = meta.row_pos[r];
    const int32_t* table = kv.tables + (size_t)meta.seq_slot[meta.row_seq[r]] * kv.table_stride;
    const int half = dim / 2;
    const float* cs_row = cos_table + (size_t)pos * half;
    const float* sn_row = sin_table + (size_t)pos * half;
    float* q = qkv + (size_t)r * ldqkv;
    float* k = q + heads * dim;
    const float* v = k + kv_heads * dim;
    const size_t off = pool_offset(table, pos, layer, kv.layers, kv.block_tokens, kv.kv_width);
    for (int p = threadIdx.x; p < heads * half; p += blockDim.x) {
        const int h = p / half, d = p % half;
        const int i = h * dim + d, j = i + half;
        const float a = q[i], b = q[j], cs = cs_row[d], sn = sn_row[d];
        q[i] = a * cs - b * sn;
        q[j] = b * cs + a * sn;
    }
    for (int p = threadIdx.x; p < kv_heads * half; p += blockDim.x) {
        const int h = p / half, d = p % half;
        const int i = h * dim + d, j = i + half;
        const float a = k[i], b = k[j], cs = cs_row[d], sn = sn_row[d];
        kv.keys[off + i] = a * cs - b * sn;
        kv.keys[off + j] = b * cs + a * sn;
    }
    for (int i = threadIdx.x; i < kv.kv_width; i += blockDim.x) kv.values[off + i] = v[i];
}

// Block-wide float max of one value per thread (max is exact and
// order-free, so a tree is fine here).
__device__ __forceinline__ float block_max(float v, float* shared) {
    for (int o = kWave / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    __syncthreads();
    if (lane == 0) shared[wave] = v;
    __syncthreads();
    float m = shared[0];
    for (int i = 1; i < (int)(blockDim.x / kWave); ++i) m = fmaxf(m, shared[i]);
    return m;
}

constexpr int kAttentionThreads = 256;
constexpr int kMaxGroup = 8;
constexpr int kMaxDim = 256;
constexpr int kLdsTable = 2048;

// One work-group per (row, kv head): the group's query heads share every K
// and V byte. Reference order per (row, head) (llama_runner.cpp:86-92):
//   s_t = (sum_d q_d k_td, sequential d) / sqrt(dim)
//   m   = max_t s_t
//   e_t = expf(s_t - m);  den = sum_t e_t, sequential t
//   out_d = sum_t (e_t/den) * v_td, sequential t
// Scores are parallel over t; the denominator runs in one lane per head and
// each (head, d) output chain in one lane, streaming V page by page with the
// next page's loads already in flight. BT is the page size (0: runtime).
struct AttentionRow {
    const float* q;
    const int32_t* table;
    int length;
    float* out;
};

struct AttentionGeometry {
    int layer, layers, block_tokens, kv_width, group, dim, kh;
};

template <int BT>
__device__ void attention_row(const AttentionRow& row, const float* __restrict__ keys,
                              const float* __restrict__ values, const AttentionGeometry& g,
                              float* scores_global) {
    __shared__ float qs[kMaxGroup * kMaxDim];
    __shared__ float lds_scores[kAttentionLdsScores];
    __shared__ int32_t lds_table[kLdsTable];
    __shared__ float reduce[kAttentionThreads / kWave];
    __shared__ float den_shared[kMaxGroup];
    __shared__ float max_shared[kMaxGroup];
    const int tid = threadIdx.x;
    const int bt = BT ? BT : g.block_tokens;
    const int length = row.length, group = g.group, dim = g.dim;
    const int pages = (length + bt - 1) / bt;
    // Score rows padded to a multiple of 16; the padding holds zeros, which
    // leave the sequential sums unchanged (x + 0 == x for the non-negative
    // running sums here).
    const int stride = (length + 15) & ~15;
    float* scores = group * stride <= kAttentionLdsScores ? lds_scores : scores_global;
    const int32_t* table = row.table;
    if (pages <= kLdsTable) {
        for (int i = tid; i < pages; i += kAttentionThreads) lds_table[i] = row.table[i];
        table = lds_table;
    }
    for (int i = tid; i < group * dim; i += kAttentionThreads) qs[i] = row.q[i];
    __syncthreads();
    const size_t layer_stride = (size_t)bt * g.kv_width;
    auto token_offset = [&](int t) -> size_t {
        const int page = t / bt, slot = t - page * bt;
        return ((size_t)table[page] * g.layers + g.layer) * layer_stride + (size_t)slot * g.kv_width +
               (size_t)g.kh * dim;
    };
    // Scores: one token per thread, `group` sequential dot products.
    float local_max[kMaxGroup];
    for (int h = 0; h < group; ++h) local_max[h] = -INFINITY;
    const float root = sqrtf((float)dim);
    for (int t = tid; t < length; t += kAttentionThreads) {
        const float* k = keys + token_offset(t);
        float s[kMaxGroup];
        for (int h = 0; h < group; ++h) s[h] = 0.0f;
        for (int d0 = 0; d0 < dim; d0 += 16) {
            float4 kv4[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                kv4[j] = d0 + 4 * j < dim ? *reinterpret_cast<const float4*>(k + d0 + 4 * j)
                                          : make_float4(0.f, 0.f, 0.f, 0.f);
            for (int h = 0; h < group; ++h) {
                const float* qh = qs + h * dim + d0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (d0 + 4 * j >= dim) break;
                    s[h] = s[h] + qh[4 * j + 0] * kv4[j].x;
                    s[h] = s[h] + qh[4 * j + 1] * kv4[j].y;
                    s[h] = s[h] + qh[4 * j + 2] * kv4[j].z;
                    s[h] = s[h] + qh[4 * j + 3] * kv4[j].w;
                }
            }
        }
        for (int h = 0; h < group; ++h) {
            const float score = s[h] / root;
            scores[h * stride + t] = score;
            local_max[h] = local_max[h] < score ? score : local_max[h];
        }
    }
    for (int h = 0; h < group; ++h) {
        const float m = block_max(local_max[h], reduce);
        if (tid == 0) max_shared[h] = m;
    }
    __syncthreads();
    for (int h = 0; h < group; ++h) {
        const float m = max_shared[h];
        for (int t = tid; t < stride; t += kAttentionThreads)
            scores[h * stride + t] = t < length ? ref_expf(scores[h * stride + t] - m) : 0.0f;
    }
    __syncthreads();
    if (tid < group) den_shared[tid] = sequential_sum(scores + tid * stride, stride);
    __syncthreads();
    for (int h = 0; h < group; ++h) {
        const float den = den_shared[h];
        for (int t = tid; t < length; t += kAttentionThreads)
            scores[h * stride + t] = scores[h * stride + t] / den;
    }
    __syncthreads();
    // PV chains: thread -> (head, d).
    for (int chain = tid; chain < group * dim; chain += kAttentionThreads) {
        const int h = chain / dim, d = chain % dim;
        const float* p = scores + h * stride;
        const float* vbase = values + (size_t)g.kh * dim + d;
        float total = 0.0f;
        if (BT) {
            // Page-structured stream: a page's BT loads are independent; the
            // next page is loaded while this one is summed.
            float bufa[BT ? BT : 1], bufb[BT ? BT : 1];
            auto load_page = [&](int page, float* buf) {
                if (page >= pages) return;
                const float* src = vbase + ((size_t)table[page] * g.layers + g.layer) * layer_stride;
                const int valid = min(BT, length - page * BT);
#pragma unroll
                for (int j = 0; j < BT; ++j) buf[j] = j < valid ? src[(size_t)j * g.kv_width] : 0.0f;
            };
            auto sum_page = [&](int page, const float* buf) {
                if (page >= pages) return;
                const float4* p4 = reinterpret_cast<const float4*>(p + page * BT);
                const int valid = min(BT, length - page * BT);
#pragma unroll
                for (int j4 = 0; j4 < BT / 4; ++j4) {
                    const float4 pv = p4[j4];
                    if (4 * j4 + 0 < valid) total = total + pv.x * buf[4 * j4 + 0];
                    if (4 * j4 + 1 < valid) total = total + pv.y * buf[4 * j4 + 1];
                    if (4 * j4 + 2 < valid) total = total + pv.z * buf[4 * j4 + 2];
                    if (4 * j4 + 3 < valid) total = total + pv.w * buf[4 * j4 + 3];
                }
            };
            load_page(0, bufa);
            load_page(1, bufb);
            for (int page = 0; page < pages; page += 2) {
                sum_page(page, bufa);
                load_page(page + 2, bufa);
                sum_page(page + 1, bufb);
                load_page(page + 3, bufb);
            }
        } else {
            for (int t = 0; t < length; ++t) total = total + p[t] * vbase[token_offset(t) - (size_t)g.kh * dim];
        }
        row.out[h * dim + d] = total;
    }
    __syncthreads();
}

template <int BT>
__global__ __launch_bounds__(kAttentionThreads) void attention_single_kernel(
    const float* __restrict__ q, const float* __restrict__ keys, const float* __restrict__ values,
    const int32_t* __restrict__ table, int length, int layer, int layers, int block_tokens,
    int heads, int kv_heads, int dim, float* __restrict__ out, float* scratch) {
    const int kh = blockIdx.y;
    const int group = heads / kv_heads;
    AttentionRow row;
    row.q = q + (size_t)kh * group * dim;
    row.table = table;
    row.length = length;
    row.out = out + (size_t)kh * group * dim;
    float* scores_global =
        scratch ? scratch + (size_t)kh * group * (size_t)((length + 15) & ~15) : nullptr;
    const AttentionGeometry g{layer, layers, block_tokens, kv_heads * dim, group, dim, kh};
    attention_row<BT>(row, keys, values, g, scores_global);
}

// ---------------------------------------------------------------------------
// Forward attention as three kernels over ROW BLOCKS. A row block is up to
// kRowBlock consecutive rows (positions) of one sequence; decode rows are
// blocks of one. Each block reads every K and V byte of its sequence once,
// while every (row, head) keeps its own reference-order chains
// (llama_runner.cpp:86-92):
//   scores  : grid (block, kv head, 256-token chunk), thread = token;
//             s = (sum_d q_d k_td, sequential d) / sqrt(dim) for each causal
//             (row, head), plus per-chunk maxima.
//   softmax : grid (row, head): max of chunk maxima, e = expf(s - m),
//             sequential denominator, p = e / den (in place).
//   pv      : grid (block, kv head): V pages streamed through an LDS double
//             buffer by all waves while each (row, head, d) chain sums its
//             causal prefix in token order.
// Score rows are `stride` floats (max length padded to 16, padding zero).
constexpr int kScoreChunk = 256;
constexpr int kMaxRowHeads = 48;       // rows x query heads of one block
constexpr int kPvBatchFloats = 8192;   // one V batch buffer (32 KB)
constexpr int kPvMaxBatchTokens = 128;
constexpr int kPvMaxChains = 12;       // (row, head, d) chains per thread
constexpr int kPvThreads = 256;

__device__ __forceinline__ float wave_max(float v) {
    for (int o = kWave / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

template <int BT, int DIM>
__global__ __launch_bounds__(kScoreChunk) void attn_scores_kernel(
    const float* __restrict__ qkv, int ldq, int heads, int kv_heads, int dim, RowMeta meta,
    PagedKv kv, int layer, const int2* __restrict__ blocks, float* __restrict__ scores, int stride,
    float* __restrict__ chunk_max, int chunks) {
    __shared__ float4 qs4[kPvMaxChains * kPvThreads / 4];
    __shared__ float partial[kScoreChunk / kWave][kMaxRowHeads];
    const int2 blk = blocks[blockIdx.x];
    const int r0 = blk.x, nr = blk.y, kh = blockIdx.y, chunk = blockIdx.z;
    const int pos0 = meta.row_pos[r0];
    const int last_length = pos0 + nr;
    if (chunk * kScoreChunk >= last_length) return;
    if (DIM) dim = DIM;
    const int group = heads / kv_heads, tid = threadIdx.x;
    const int rh = nr * group;
    const int bt = BT ? BT : kv.block_tokens;
    const int32_t* table = kv.tables + (size_t)meta.seq_slot[meta.row_seq[r0]] * kv.table_stride;
    // q of the block's (row, head) pairs, row-major: rh x dim.
    float* qs = reinterpret_cast<float*>(qs4);
    for (int i = tid; i < rh * dim; i += kScoreChunk) {
        const int r = i / (group * dim), rest = i - r * group * dim;
        qs[i] = qkv[(size_t)(r0 + r) * ldq + (size_t)kh * group * dim + rest];
    }
    __syncthreads();
    const int t = chunk * kScoreChunk + tid;
    const bool live = t < last_length;
    const int tc = live ? t : 0;
    const int page = tc / bt, slot = tc - page * bt;
    const float4* k4p = reinterpret_cast<const float4*>(
        kv.keys + (((size_t)table[page] * kv.layers + layer) * bt + slot) * kv.kv_width + (size_t)kh * dim);
    // Row r (relative to the block) sees token t when t <= pos0 + r.
    const int ifirst = (t - pos0 > 0 ? t - pos0 : 0) * group;
    const float root = sqrtf((float)dim);
    const int wave = tid / kWave, lane = tid % kWave;
    float4 kreg[DIM ? DIM / 4 : 1];
    if (DIM) {
#pragma unroll
        for (int j = 0; j < DIM / 4; ++j) kreg[j] = k4p[j];
    }
    for (int i = 0; i < rh; ++i) {
        const float4* q4 = qs4 + i * (dim / 4);
        float acc = 0.0f;
        if (DIM) {
#pragma unroll
            for (int j = 0; j < DIM / 4; ++j) {
                const float4 q = q4[j];
                acc = acc + q.x * kreg[j].x;
                acc = acc + q.y * kreg[j].y;
                acc = acc + q.z * kreg[j].z;
                acc = acc + q.w * kreg[j].w;
            }
        } else {
            for (int j = 0; j < dim / 4; ++j) {
                const float4 q = q4[j], k = k4p[j];
                acc = acc + q.x * k.x;
                acc = acc + q.y * k.y;
                acc = acc + q.z * k.z;
                acc = acc + q.w * k.w;
            }
        }
        const bool keep = live && i >= ifirst;
        const float score = acc / root;
        if (keep) {
            const int r = i / group, h = i - r * group;
            scores[((size_t)(r0 + r) * heads + kh * group + h) * stride + t] = score;
        }
        const float m = wave_max(keep ? score : -INFINITY);
        if (lane == 0) partial[wave][i] = m;
    }
    __syncthreads();
    if (tid < rh) {
        float m = partial[0][tid];
        for (int w = 1; w < kScoreChunk / kWave; ++w) m = fmaxf(m, partial[w][tid]);
        const int r = tid / group, h = tid - r * group;
        chunk_max[((size_t)(r0 + r) * heads + kh * group + h) * chunks + chunk] = m;
    }
}

constexpr int kSoftmaxThreads = 256;
constexpr int kSoftmaxStage = 4096;

__global__ __launch_bounds__(kSoftmaxThreads) void attn_softmax_kernel(
    float* __restrict__ scores, int stride, const float* __restrict__ chunk_max, int chunks,
    RowMeta meta, int heads) {
    __shared__ float stage[kSoftmaxStage];
    __shared__ float reduce[kSoftmaxThreads / kWave];
    __shared__ float den_shared;
    const int r = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int length = meta.row_pos[r] + 1;
    float* row = scores + ((size_t)r * heads + h) * stride;
    const float* cm = chunk_max + ((size_t)r * heads + h) * chunks;
    const int used = (length + kScoreChunk - 1) / kScoreChunk;
    float local = -INFINITY;
    for (int c = tid; c < used; c += kSoftmaxThreads) local = local < cm[c] ? cm[c] : local;
    const float m = block_max(local, reduce);
    // The row's own padded length; e = expf(s - m) staged through LDS, the
    // denominator summed in token order in one lane per staged block.
    const int row_stride = (length + 15) & ~15;
    float den = 0.0f;
    for (int c0 = 0; c0 < row_stride; c0 += kSoftmaxStage) {
        const int n = min(kSoftmaxStage, row_stride - c0);
        for (int i = tid; i < n; i += kSoftmaxThreads) {
            const int t = c0 + i;
            const float e = t < length ? ref_expf(row[t] - m) : 0.0f;
            stage[i] = e;
            if (row_stride > kSoftmaxStage) row[t] = e;
        }
        __syncthreads();
        if (tid == 0) den = sequential_sum(stage, n, den);
        __syncthreads();
    }
    if (tid == 0) den_shared = den;
    __syncthreads();
    den = den_shared;
    if (row_stride <= kSoftmaxStage) {
        for (int t = tid; t < row_stride; t += kSoftmaxThreads) row[t] = t < length ? stage[t] / den : 0.0f;
    } else {
        for (int t = tid; t < row_stride; t += kSoftmaxThreads) row[t] = t < length ? row[t] / den : 0.0f;
    }
}

template <int BT, int DIM>
__global__ __launch_bounds__(kPvThreads) void attn_pv_kernel(
    const float* __restrict__ probs, int stride, int heads, int kv_heads, int dim, RowMeta meta,
    PagedKv kv, int layer, const int2* __restrict__ blocks, float* __restrict__ out, int ldo) {
    __shared__ float4 vbuf4[2][kPvBatchFloats / 4];
    __shared__ float4 pbuf4[2][kMaxRowHeads * kPvMaxBatchTokens / 4];
    __shared__ int32_t lds_table[kLdsTable];
    __shared__ float totals[kPvMaxChains * kPvThreads];  // chain i of thread tid at i*256+tid
    if (DIM) dim = DIM;
    const int2 blk = blocks[blockIdx.x];
    const int r0 = blk.x, nr = blk.y, kh = blockIdx.y, tid = threadIdx.x;
    const int group = heads / kv_heads, rh = nr * group;
    const int bt = BT ? BT : kv.block_tokens;
    const int pos0 = meta.row_pos[r0];
    const int last_length = pos0 + nr;
    const int pages = (last_length + bt - 1) / bt;
    const int32_t* table = kv.tables + (size_t)meta.seq_slot[meta.row_seq[r0]] * kv.table_stride;
    // Page table in LDS (at most kLdsTable pages, checked by the host), so V
    // addresses never wait on a global load.
    for (int i = tid; i < pages; i += kPvThreads) lds_table[i] = table[i];
    __syncthreads();
    int batch_pages = kPvBatchFloats / (bt * dim);
    if (batch_pages * bt > kPvMaxBatchTokens) batch_pages = kPvMaxBatchTokens / bt;
    const int batch_tokens = batch_pages * bt;
    const int batches = (pages + batch_pages - 1) / batch_pages;
    const int vec_per_token = dim / 4;
    const int vec_per_batch = batch_tokens * vec_per_token;
    const int pvec_per_row = batch_tokens / 4;
    constexpr int kLoads = kPvBatchFloats / 4 / kPvThreads;                        // 8
    constexpr int kPLoads = kMaxRowHeads * kPvMaxBatchTokens / 4 / kPvThreads;     // 6
    float4 vreg[kLoads], preg[kPLoads];
    // Fast layout (16-token pages, head_dim 64): thread element j is page
    // batch*8 + j, slot tid/16, float4 tid%16, from a wave-uniform page base.
    constexpr bool kFast = BT == 16 && DIM == 64;
    const uint32_t fast_off = (uint32_t)(tid / 16) * (uint32_t)kv.kv_width + 4u * (uint32_t)(tid % 16);
    auto fetch = [&](int batch) {
        const int t0 = batch * batch_tokens;
        if (kFast) {
#pragma unroll
            for (int j = 0; j < kLoads; ++j) {
                const int page = min(t0 / 16 + j, pages - 1);
                const int block = __builtin_amdgcn_readfirstlane(lds_table[page]);
                const float* base = kv.values + (((size_t)block * kv.layers + layer) * 16) * kv.kv_width +
                                    (size_t)kh * 64;
                vreg[j] = *reinterpret_cast<const float4*>(base + fast_off);
            }
        } else {
#pragma unroll
            for (int j = 0; j < kLoads; ++j) {
                const int e = tid + j * kPvThreads;
                const int tok = e / vec_per_token, d4 = e - tok * vec_per_token;
                const int t = t0 + tok;
                const bool in = e < vec_per_batch && t < last_length;
                const int tc = in ? t : 0;
                const int page = tc / bt, slot = tc - page * bt;
                vreg[j] = *reinterpret_cast<const float4*>(
                    kv.values + (((size_t)lds_table[page] * kv.layers + layer) * bt + slot) * kv.kv_width +
                    (size_t)kh * dim + 4 * (in ? d4 : 0));
            }
        }
#pragma unroll
        for (int j = 0; j < kPLoads; ++j) {
            const int e = tid + j * kPvThreads;
            const int i = e / pvec_per_row, i4 = e - i * pvec_per_row;  // (row, head), token quad
            const int r = i / group, h = i - r * group;
            const bool in = i < rh && t0 + 4 * i4 < stride;
            preg[j] = *reinterpret_cast<const float4*>(
                probs + (in ? ((size_t)(r0 + r) * heads + kh * group + h) * stride + t0 + 4 * i4 : 0));
        }
    };
    // Masks are applied here, after every load of the batch is in flight.
    auto stash = [&](int batch, int buffer) {
        const int t0 = batch * batch_tokens;
        const bool whole = kFast && t0 + batch_tokens <= last_length;
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int e = tid + j * kPvThreads;
            if (whole) {
                vbuf4[buffer][e] = vreg[j];
            } else {
                const int tok = e / vec_per_token;
                vbuf4[buffer][e] = keep_if(vreg[j], mask_of(e < vec_per_batch && t0 + tok < last_length));
            }
        }
#pragma unroll
        for (int j = 0; j < kPLoads; ++j) {
            const int e = tid + j * kPvThreads;
            const int i = e / pvec_per_row, i4 = e - i * pvec_per_row;
            pbuf4[buffer][e] = keep_if(preg[j], mask_of(i < rh && t0 + 4 * i4 < stride));
        }
    };
    const int chains = rh * dim;
    for (int i = 0; i < kPvMaxChains; ++i) totals[i * kPvThreads + tid] = 0.0f;
    fetch(0);
    stash(0, 0);
    __syncthreads();
    for (int b = 0; b < batches; ++b) {
        const int buffer = b & 1;
        const int t0 = b * batch_tokens;
        if (b + 1 < batches) fetch(b + 1);
        const float* vb = reinterpret_cast<const float*>(vbuf4[buffer]);
        const float* pb = reinterpret_cast<const float*>(pbuf4[buffer]);
        for (int i = 0; i < kPvMaxChains; ++i) {
            const int chain = tid + i * kPvThreads;
            if (chain >= chains) break;
            const int rhi = chain / dim, d = chain - rhi * dim;
            const int r = rhi / group;
            // Causal: row r attends tokens [0, pos0 + r].
            const int n = min(batch_tokens, pos0 + r + 1 - t0);
            if (n <= 0) continue;
            float acc = totals[i * kPvThreads + tid];
            float unused = 0.0f;
            chain_dot<false, DIM>(pb + rhi * batch_tokens, vb + d, nullptr, n, acc, unused, dim);
            totals[i * kPvThreads + tid] = acc;
        }
        if (b + 1 < batches) stash(b + 1, buffer ^ 1);
        __syncthreads();
    }
    for (int i = 0; i < kPvMaxChains; ++i) {
        const int chain = tid + i * kPvThreads;
        if (chain >= chains) break;
        const int rhi = chain / dim, d = chain - rhi * dim;
        const int r = rhi / group, h = rhi - r * group;
        out[(size_t)(r0 + r) * ldo + ((size_t)kh * group + h) * dim + d] = totals[i * kPvThreads + tid];
    }
}

// std::max_element semantics: the smallest index among the maxima.
__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ logits,
                                                     int vocabulary, int32_t* __restrict__ argmax,
                                                     int32_t* __restrict__ nonfinite) {
    __shared__ float best_v[1024 / kWave];
    __shared__ int best_i[1024 / kWave];
    const float* row = logits + (size_t)blockIdx.x * vocabulary;
    float bv = -INFINITY;
    int bi = -1;
    bool bad = false;
    for (int i = threadIdx.x; i < vocabulary; i += blockDim.x) {
        const float v = row[i];
        if (!isfinite(v)) bad = true;
        if (bi < 0 || v > bv) {
            bv = v;
            bi = i;
        }
    }
    for (int o = kWave / 2; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) {
            bv = ov;
            bi = oi;
        }
    }
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (lane == 0) {
        best_v[wave] = bv;
        best_i[wave] = bi;
    }
    __shared__ int any_bad;
    if (threadIdx.x == 0) any_bad = 0;
    __syncthreads();
    if (bad) any_bad = 1;
    __syncthreads();
    if (threadIdx.x == 0) nonfinite[blockIdx.x] = any_bad;
    if (threadIdx.x == 0) {
        float v = best_v[0];
        int idx = best_i[0];
        for (int w = 1; w < (int)(blockDim.x / kWave); ++w) {
            const float ov = best_v[w];
            const int oi = best_i[w];
            if (oi >= 0 && (idx < 0 || ov > v || (ov == v && oi < idx))) {
                v = ov;
                idx = oi;
            }
        }
        argmax[blockIdx.x] = idx;
    }
}

__global__ void copy_region_kernel(float* keys, float* values, uint64_t destination,
                                   uint64_t source, uint64_t pitch, uint64_t width) {
    float* pool = blockIdx.y == 0 ? keys : values;
    const uint64_t row = blockIdx.x;
    float* dst = pool + destination + row * pitch;
    const float* src = pool + source + row * pitch;
    for (uint64_t i = threadIdx.x; i < width; i += blockDim.x) dst[i] = src[i];
}

__global__ void transpose_kernel(const float* __restrict__ src, float* __restrict__ dst, int rows,
                                 int cols) {
    __shared__ float tile[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    for (int i = threadIdx.y; i < 32; i += blockDim.y) {
        const int r = r0 + i, c = c0 + threadIdx.x;
        if (r < rows && c < cols) tile[i][threadIdx.x] = src[(size_t)r * cols + c];
    }
    __syncthreads();
    for (int i = threadIdx.y; i < 32; i += blockDim.y) {
        const int c = c0 + i, r = r0 + threadIdx.x;
        if (r < rows && c < cols) dst[(size_t)c * rows + r] = tile[threadIdx.x][i];
    }
}

}  // namespace

hipError_t launch_embed(hipStream_t s, const float* embedding, const int32_t* tokens, float* x,
                        int rows, int hidden) {
    if (rows <= 0) return hipSuccess;
    embed_kernel<<<rows, 256, 0, s>>>(embedding, tokens, x, hidden);
    return hipGetLastError();
}

hipError_t launch_rms(hipStream_t s, const float* x, int ldx, const int32_t* row_map,
                      const float* weight, float* out, int ldo, int rows, int width, float eps) {
    if (rows <= 0) return hipSuccess;
    const size_t lds = sizeof(float) * (size_t)((width + 3) & ~3);
    rms_kernel<<<rows, kWave, lds, s>>>(x, ldx, row_map, weight, out, ldo, width, eps);
    return hipGetLastError();
}

hipError_t launch_gemm(hipStream_t s, Epilogue epilogue, const float* x, int ldx, int rows,
                       int inner, const float* w, const float* w2, int columns, int ldw,
                       float* out, int ldo) {
    if (rows <= 0 || columns <= 0) return hipSuccess;
    if (rows <= kSmallRows) {
        const int tiles = (columns + kSmallColumns - 1) / kSmallColumns;
        switch (epilogue) {
        case kStore: gemm_small_kernel<kStore><<<tiles, 256, 0, s>>>(x, ldx, rows, inner, w, w2, columns, ldw, out, ldo, tiles); break;
        case kResidual: gemm_small_kernel<kResidual><<<tiles, 256, 0, s>>>(x, ldx, rows, inner, w, w2, columns, ldw, out, ldo, tiles); break;
        case kSwiglu: gemm_small_kernel<kSwiglu><<<tiles, 256, 0, s>>>(x, ldx, rows, inner, w, w2, columns, ldw, out, ldo, tiles); break;
        }
    } else {
        const int tiles = (columns + kWideColumns - 1) / kWideColumns;
        const dim3 grid(tiles, (rows + kWideRows - 1) / kWideRows);
        const bool full = inner % 64 == 0 && columns % kWideColumns == 0 && ldx % 4 == 0 &&
                          (size_t)inner * ldw < (1ull << 32);
#define MP_WIDE(E, F) gemm_wide_kernel<E, F><<<grid, kWideThreads, 0, s>>>(x, ldx, rows, inner, w, w2, columns, ldw, out, ldo, tiles)
        if (full) {
            switch (epilogue) {
            case kStore: MP_WIDE(kStore, true); break;
            case kResidual: MP_WIDE(kResidual, true); break;
            case kSwiglu: MP_WIDE(kSwiglu, true); break;
            }
        } else {
            switch (epilogue) {
            case kStore: MP_WIDE(kStore, false); break;
            case kResidual: MP_WIDE(kResidual, false); break;
            case kSwiglu: MP_WIDE(kSwiglu, false); break;
            }
        }
#undef MP_WIDE
    }
    return hipGetLastError();
}

hipError_t launch_rope_append(hipStream_t s, float* qkv, int ldqkv, int rows, int heads,
                              int kv_heads, int dim, const float* cos_table,
                              const float* sin_table, const RowMeta& meta, const PagedKv& kv,
                              int layer) {
    if (rows <= 0) return hipSuccess;
    rope_append_kernel<<<rows, 256, 0, s>>>(qkv, ldqkv, heads, kv_heads, dim, cos_table, sin_table,
                                            meta, kv, layer);
    return hipGetLastError();
}

int attention_row_block(int heads, int kv_heads, int dim) {
    const int group = heads / kv_heads;
    int rows = kMaxRowHeads / group;
    if (rows * group * dim > kPvMaxChains * kPvThreads) rows = kPvMaxChains * kPvThreads / (group * dim);
    return rows < 16 ? rows : 16;
}

hipError_t launch_attention(hipStream_t s, const float* qkv, int ldq, int rows, int heads,
                            int kv_heads, int dim, const RowMeta& meta, const PagedKv& kv,
                            int layer, float* out, int ldo, const AttentionScratch& scratch) {
    if (rows <= 0) return hipSuccess;
    const int group = heads / kv_heads;
    if (group > kMaxGroup || dim > kMaxDim || dim % 4 || group * dim > kPvMaxChains * kPvThreads ||
        kv.block_tokens * dim > kPvBatchFloats)
        return hipErrorInvalidValue;
    const dim3 sgrid(scratch.blocks, kv_heads, scratch.chunks);
    if (kv.block_tokens == 16 && dim == 64)
        attn_scores_kernel<16, 64><<<sgrid, kScoreChunk, 0, s>>>(qkv, ldq, heads, kv_heads, dim, meta, kv, layer, scratch.row_blocks, scratch.scores, scratch.stride, scratch.chunk_max, scratch.chunks);
    else
        attn_scores_kernel<0, 0><<<sgrid, kScoreChunk, 0, s>>>(qkv, ldq, heads, kv_heads, dim, meta, kv, layer, scratch.row_blocks, scratch.scores, scratch.stride, scratch.chunk_max, scratch.chunks);
    attn_softmax_kernel<<<dim3(rows, heads), kSoftmaxThreads, 0, s>>>(scratch.scores, scratch.stride, scratch.chunk_max, scratch.chunks, meta, heads);
    const dim3 pgrid(scratch.blocks, kv_heads);
    if (kv.block_tokens == 16 && dim == 64)
        attn_pv_kernel<16, 64><<<pgrid, kPvThreads, 0, s>>>(scratch.scores, scratch.stride, heads, kv_heads, dim, meta, kv, layer, scratch.row_blocks, out, ldo);
    else
        attn_pv_kernel<0, 0><<<pgrid, kPvThreads, 0, s>>>(scratch.scores, scratch.stride, heads, kv_heads, dim, meta, kv, layer, scratch.row_blocks, out, ldo);
    return hipGetLastError();
}

hipError_t launch_attention_single(hipStream_t s, const float* q, const float* keys,
                                   const float* values, const int32_t* table, int length,
                                   int layer, int layers, int block_tokens, int heads,
                                   int kv_heads, int dim, float* out, float* scratch) {
    if (heads / kv_heads > kMaxGroup || dim > kMaxDim || dim % 4) return hipErrorInvalidValue;
    const dim3 grid(1, kv_heads);
    if (block_tokens == 16)
        attention_single_kernel<16><<<grid, kAttentionThreads, 0, s>>>(q, keys, values, table, length, layer, layers, block_tokens, heads, kv_heads, dim, out, scratch);
    else
        attention_single_kernel<0><<<grid, kAttentionThreads, 0, s>>>(q, keys, values, table, length, layer, layers, block_tokens, heads, kv_heads, dim, out, scratch);
    return hipGetLastError();
}

hipError_t launch_argmax(hipStream_t s, const float* logits, int rows, int vocabulary,
                         int32_t* argmax, int32_t* nonfinite) {
    if (rows <= 0) return hipSuccess;
    argmax_kernel<<<rows, 1024, 0, s>>>(logits, vocabulary, argmax, nonfinite);
    return hipGetLastError();
}

hipError_t launch_copy_region(hipStream_t s, float* keys, float* values, uint64_t destination,
                              uint64_t source, uint64_t pitch, uint64_t width, uint64_t rows) {
    if (!rows || !width) return hipSuccess;
    copy_region_kernel<<<dim3((unsigned)rows, 2), 256, 0, s>>>(keys, values, destination, source,
                                                               pitch, width);
    return hipGetLastError();
}

hipError_t launch_transpose(hipStream_t s, const float* src, float* dst, int rows, int cols) {
    transpose_kernel<<<dim3((cols + 31) / 32, (rows + 31) / 32), dim3(32, 8), 0, s>>>(src, dst, rows,
                                                                                     cols);
    return hipGetLastError();
}

}  // namespace mphip
