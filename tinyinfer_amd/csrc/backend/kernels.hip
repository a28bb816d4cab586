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

__global__ void embed_kernel(const float* __restrict__ embedding, const int32_t* __restrict__ tokens,
                             float* __restrict__ x, int hidden) {
    const int r = blockIdx.x;
    const float* src = embedding + (size_t)tokens[r] * hidden;
    float* dst = x + (size_t)r * hidden;
    for (int i = threadIdx.x; i < hidden; i += blockDim.x) dst[i] = src[i];
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
    for (int i = threadIdx.x; i < width; i += kWave) {
        const float v = xr[i];
        squares[i] = v * v;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float sum = 0;
        int d = 0;
        for (; d + 4 <= width; d += 4) {
            const float4 v = *reinterpret_cast<const float4*>(squares + d);
            sum = sum + v.x;
            sum = sum + v.y;
            sum = sum + v.z;
            sum = sum + v.w;
        }
        for (; d < width; ++d) sum = sum + squares[d];
        scale_shared = 1.0f / sqrtf(sum / (float)width + eps);
    }
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

// Few rows (decode of one to four sequences): 16 columns per work-group so
// that even a 576-column projection spreads over 36 CUs. All four waves
// stage a K-chunk of the 16-column weight slab into LDS with coalesced
// loads; lanes (row, column) of wave 0 then walk k in order.
constexpr int kSmallColumns = 16;
constexpr int kSmallRows = 4;
constexpr int kSmallChunk = 384;

template <int EPI>
__global__ __launch_bounds__(256) void gemm_small_kernel(const float* __restrict__ x, int ldx,
                                                         int rows, int inner,
                                                         const float* __restrict__ w,
                                                         const float* __restrict__ w2,
                                                         int columns, int ldw, float* out, int ldo,
                                                         int tiles) {
    __shared__ float xs[kSmallRows * kSmallChunk];
    __shared__ float ws[kSmallChunk * kSmallColumns];
    __shared__ float ws2[EPI == kSwiglu ? kSmallChunk * kSmallColumns : 1];
    const int tid = threadIdx.x;
    const int n0 = xcd_tile(blockIdx.x, tiles) * kSmallColumns;
    const int r = tid / kSmallColumns, c = tid % kSmallColumns;
    const int n = n0 + c;
    float acc = 0.0f, acc2 = 0.0f;
    for (int k0 = 0; k0 < inner; k0 += kSmallChunk) {
        const int kc = min(kSmallChunk, inner - k0);
        for (int i = tid; i < rows * kc; i += 256) {
            const int rr = i / kc, kk = i - rr * kc;
            xs[rr * kSmallChunk + kk] = x[(size_t)rr * ldx + k0 + kk];
        }
        for (int i = tid; i < kc * kSmallColumns; i += 256) {
            const int kk = i / kSmallColumns, cc = i % kSmallColumns;
            const bool in = n0 + cc < columns;
            const size_t off = (size_t)(k0 + kk) * ldw + n0 + cc;
            ws[i] = in ? w[off] : 0.0f;
            if (EPI == kSwiglu) ws2[i] = in ? w2[off] : 0.0f;
        }
        __syncthreads();
        if (r < rows) {
            const float* xr = xs + r * kSmallChunk;
            int k = 0;
            for (; k + 4 <= kc; k += 4) {
                const float4 xv = *reinterpret_cast<const float4*>(xr + k);
                const float* wk = ws + k * kSmallColumns + c;
                acc = acc + xv.x * wk[0];
                acc = acc + xv.y * wk[kSmallColumns];
                acc = acc + xv.z * wk[2 * kSmallColumns];
                acc = acc + xv.w * wk[3 * kSmallColumns];
                if (EPI == kSwiglu) {
                    const float* uk = ws2 + k * kSmallColumns + c;
                    acc2 = acc2 + xv.x * uk[0];
                    acc2 = acc2 + xv.y * uk[kSmallColumns];
                    acc2 = acc2 + xv.z * uk[2 * kSmallColumns];
                    acc2 = acc2 + xv.w * uk[3 * kSmallColumns];
                }
            }
            for (; k < kc; ++k) {
                acc = acc + xr[k] * ws[k * kSmallColumns + c];
                if (EPI == kSwiglu) acc2 = acc2 + xr[k] * ws2[k * kSmallColumns + c];
            }
        }
        __syncthreads();
    }
    if (r < rows && n < columns) store_result<EPI>(out + (size_t)r * ldo + n, acc, acc2);
}

// Many rows (batched decode, prefill chunks): 64 columns x 16 rows per
// 1024-thread work-group, one output chain per lane (lane = column,
// wave = row). A K-chunk of the weight tile is shared by the 16 waves
// through LDS and double-buffered through registers.
constexpr int kWideColumns = 64;
constexpr int kWideRows = 16;

template <int EPI>
__global__ __launch_bounds__(1024) void gemm_wide_kernel(const float* __restrict__ x, int ldx,
                                                         int rows, int inner,
                                                         const float* __restrict__ w,
                                                         const float* __restrict__ w2,
                                                         int columns, int ldw, float* out, int ldo,
                                                         int column_tiles) {
    constexpr int kDual = EPI == kSwiglu ? 2 : 1;
    constexpr int kChunk = EPI == kSwiglu ? 32 : 64;          // k rows per chunk
    constexpr int kPerThread = kChunk * kWideColumns / 1024;  // weight floats per thread
    constexpr int kXThreads = kWideRows * kChunk / 4;         // threads staging x (float4 each)
    __shared__ float ws[2][kDual][kChunk * kWideColumns];
    __shared__ float4 xs4[2][kXThreads];
    const int tid = threadIdx.x;
    const int wave = tid / kWave, lane = tid % kWave;
    const int column_tile = xcd_tile(blockIdx.x, column_tiles);
    const int n0 = column_tile * kWideColumns, r0 = blockIdx.y * kWideRows;
    const int n = n0 + lane, row = r0 + wave;
    const int lr = tid / (kChunk / 4), lk = (tid % (kChunk / 4)) * 4;
    float wreg[kDual][kPerThread];
    float4 xreg = make_float4(0.f, 0.f, 0.f, 0.f);
    auto fetch = [&](int k0) {
#pragma unroll
        for (int m = 0; m < kDual; ++m) {
            const float* src = m == 0 ? w : w2;
#pragma unroll
            for (int j = 0; j < kPerThread; ++j) {
                const int e = tid + j * 1024;
                const int kk = e / kWideColumns, cc = e % kWideColumns;
                const bool in = (k0 + kk < inner) && (n0 + cc < columns);
                wreg[m][j] = in ? src[(size_t)(k0 + kk) * ldw + n0 + cc] : 0.0f;
            }
        }
        if (tid < kXThreads) {
            const int gr = r0 + lr;
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                v[j] = (gr < rows && k0 + lk + j < inner) ? x[(size_t)gr * ldx + k0 + lk + j] : 0.0f;
            xreg = make_float4(v[0], v[1], v[2], v[3]);
        }
    };
    auto stash = [&](int buffer) {
#pragma unroll
        for (int m = 0; m < kDual; ++m)
#pragma unroll
            for (int j = 0; j < kPerThread; ++j) ws[buffer][m][tid + j * 1024] = wreg[m][j];
        if (tid < kXThreads) xs4[buffer][tid] = xreg;
    };
    float acc = 0.0f, acc2 = 0.0f;
    const int chunks = (inner + kChunk - 1) / kChunk;
    fetch(0);
    stash(0);
    __syncthreads();
    for (int chunk = 0; chunk < chunks; ++chunk) {
        const int buffer = chunk & 1;
        if (chunk + 1 < chunks) fetch((chunk + 1) * kChunk);
        const int kc = min(kChunk, inner - chunk * kChunk);
        const float* xr = reinterpret_cast<const float*>(xs4[buffer]) + wave * kChunk;
        const float* wk = ws[buffer][0] + lane;
        const float* uk = ws[buffer][kDual - 1] + lane;
        int k = 0;
        for (; k + 4 <= kc; k += 4) {
            const float4 xv = *reinterpret_cast<const float4*>(xr + k);
            acc = acc + xv.x * wk[(k + 0) * kWideColumns];
            acc = acc + xv.y * wk[(k + 1) * kWideColumns];
            acc = acc + xv.z * wk[(k + 2) * kWideColumns];
            acc = acc + xv.w * wk[(k + 3) * kWideColumns];
            if (EPI == kSwiglu) {
                acc2 = acc2 + xv.x * uk[(k + 0) * kWideColumns];
                acc2 = acc2 + xv.y * uk[(k + 1) * kWideColumns];
                acc2 = acc2 + xv.z * uk[(k + 2) * kWideColumns];
                acc2 = acc2 + xv.w * uk[(k + 3) * kWideColumns];
            }
        }
        for (; k < kc; ++k) {
            acc = acc + xr[k] * wk[k * kWideColumns];
            if (EPI == kSwiglu) acc2 = acc2 + xr[k] * uk[k * kWideColumns];
        }
        if (chunk + 1 < chunks) stash(buffer ^ 1);
        __syncthreads();
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

// One work-group per (row, kv head): the group's query heads share every K
// and V byte. Reference order per (row, head) (llama_runner.cpp:86-92):
//   s_t = (sum_d q_d k_td, sequential d) / sqrt(dim)
//   m   = max_t s_t
//   e_t = expf(s_t - m);  den = sum_t e_t, sequential t
//   out_d = sum_t (e_t/den) * v_td, sequential t
// Scores are parallel over t; the denominator runs in one lane per head and
// each (head, d) output chain in one lane.
struct AttentionRow {
    const float* q;
    const int32_t* table;
    int length;
    float* out;
};

__device__ void attention_row(const AttentionRow& row, const float* keys, const float* values,
                              int layer, int layers, int block_tokens, int kv_width, int group,
                              int dim, int kh, float* scores_global) {
    __shared__ float qs[kMaxGroup * kMaxDim];
    __shared__ float lds_scores[kAttentionLdsScores];
    __shared__ float reduce[kAttentionThreads / kWave];
    __shared__ float den_shared[kMaxGroup];
    __shared__ float max_shared[kMaxGroup];
    const int tid = threadIdx.x;
    const int length = row.length;
    // Score rows padded to a multiple of 4 for vector reads.
    const int stride = (length + 3) & ~3;
    float* scores = group * stride <= kAttentionLdsScores ? lds_scores : scores_global;
    for (int i = tid; i < group * dim; i += kAttentionThreads) qs[i] = row.q[i];
    __syncthreads();
    // Scores: one token per thread, `group` sequential dot products.
    float local_max[kMaxGroup];
    for (int h = 0; h < group; ++h) local_max[h] = -INFINITY;
    const float root = sqrtf((float)dim);
    for (int t = tid; t < length; t += kAttentionThreads) {
        const float* k = keys + pool_offset(row.table, t, layer, layers, block_tokens, kv_width) +
                         (size_t)kh * dim;
        float s[kMaxGroup];
        for (int h = 0; h < group; ++h) s[h] = 0.0f;
        for (int d = 0; d < dim; d += 4) {
            const float4 kv4 = *reinterpret_cast<const float4*>(k + d);
            for (int h = 0; h < group; ++h) {
                const float* qh = qs + h * dim + d;
                s[h] = s[h] + qh[0] * kv4.x;
                s[h] = s[h] + qh[1] * kv4.y;
                s[h] = s[h] + qh[2] * kv4.z;
                s[h] = s[h] + qh[3] * kv4.w;
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
        for (int t = tid; t < length; t += kAttentionThreads)
            scores[h * stride + t] = ref_expf(scores[h * stride + t] - m);
    }
    __syncthreads();
    if (tid < group) {
        const float* e = scores + tid * stride;
        float den = 0.0f;
        int t = 0;
        for (; t + 4 <= length; t += 4) {
            const float4 v = *reinterpret_cast<const float4*>(e + t);
            den = den + v.x;
            den = den + v.y;
            den = den + v.z;
            den = den + v.w;
        }
        for (; t < length; ++t) den = den + e[t];
        den_shared[tid] = den;
    }
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
        const float* vbase = values + (size_t)kh * dim + d;
        float total = 0.0f;
        int t = 0;
        for (; t + 4 <= length; t += 4) {
            const float v0 = vbase[pool_offset(row.table, t + 0, layer, layers, block_tokens, kv_width)];
            const float v1 = vbase[pool_offset(row.table, t + 1, layer, layers, block_tokens, kv_width)];
            const float v2 = vbase[pool_offset(row.table, t + 2, layer, layers, block_tokens, kv_width)];
            const float v3 = vbase[pool_offset(row.table, t + 3, layer, layers, block_tokens, kv_width)];
            const float4 pv = *reinterpret_cast<const float4*>(p + t);
            total = total + pv.x * v0;
            total = total + pv.y * v1;
            total = total + pv.z * v2;
            total = total + pv.w * v3;
        }
        for (; t < length; ++t)
            total = total + p[t] * vbase[pool_offset(row.table, t, layer, layers, block_tokens, kv_width)];
        row.out[h * dim + d] = total;
    }
    __syncthreads();
}

__global__ __launch_bounds__(kAttentionThreads) void attention_kernel(
    const float* __restrict__ qkv, int ldq, int heads, int kv_heads, int dim, RowMeta meta,
    PagedKv kv, int layer, float* __restrict__ out, int ldo, float* scratch,
    size_t scratch_row_floats) {
    const int r = blockIdx.x, kh = blockIdx.y;
    const int group = heads / kv_heads;
    AttentionRow row;
    row.q = qkv + (size_t)r * ldq + (size_t)kh * group * dim;
    row.table = kv.tables + (size_t)meta.seq_slot[meta.row_seq[r]] * kv.table_stride;
    row.length = meta.row_pos[r] + 1;
    row.out = out + (size_t)r * ldo + (size_t)kh * group * dim;
    float* scores_global =
        scratch ? scratch + ((size_t)r * kv_heads + kh) * scratch_row_floats : nullptr;
    attention_row(row, kv.keys, kv.values, layer, kv.layers, kv.block_tokens, kv.kv_width, group,
                  dim, kh, scores_global);
}

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
    const size_t stride = (size_t)((length + 3) & ~3) * group;
    float* scores_global = scratch ? scratch + (size_t)kh * stride : nullptr;
    attention_row(row, keys, values, layer, layers, block_tokens, kv_heads * dim, group, dim, kh,
                  scores_global);
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
    if (bad) atomicOr(nonfinite, 1);
    __syncthreads();
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
        switch (epilogue) {
        case kStore: gemm_wide_kernel<kStore><<<grid, 1024, 0, s>>>(x, ldx, rows, inner, w, w2, columns, ldw, out, ldo, tiles); break;
        case kResidual: gemm_wide_kernel<kResidual><<<grid, 1024, 0, s>>>(x, ldx, rows, inner, w, w2, columns, ldw, out, ldo, tiles); break;
        case kSwiglu: gemm_wide_kernel<kSwiglu><<<grid, 1024, 0, s>>>(x, ldx, rows, inner, w, w2, columns, ldw, out, ldo, tiles); break;
        }
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

hipError_t launch_attention(hipStream_t s, const float* qkv, int ldq, int rows, int heads,
                            int kv_heads, int dim, const RowMeta& meta, const PagedKv& kv,
                            int layer, float* out, int ldo, float* scratch,
                            size_t scratch_row_floats) {
    if (rows <= 0) return hipSuccess;
    if (heads / kv_heads > kMaxGroup || dim > kMaxDim || dim % 4) return hipErrorInvalidValue;
    attention_kernel<<<dim3(rows, kv_heads), kAttentionThreads, 0, s>>>(
        qkv, ldq, heads, kv_heads, dim, meta, kv, layer, out, ldo, scratch, scratch_row_floats);
    return hipGetLastError();
}

hipError_t launch_attention_single(hipStream_t s, const float* q, const float* keys,
                                   const float* values, const int32_t* table, int length,
                                   int layer, int layers, int block_tokens, int heads,
                                   int kv_heads, int dim, float* out, float* scratch) {
    if (heads / kv_heads > kMaxGroup || dim > kMaxDim || dim % 4) return hipErrorInvalidValue;
    attention_single_kernel<<<dim3(1, kv_heads), kAttentionThreads, 0, s>>>(
        q, keys, values, table, length, layer, layers, block_tokens, heads, kv_heads, dim, out,
        scratch);
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
