// Stand-alone paged GQA decode attention over caller-owned pools in the
// reference layout ([block][layer][slot][kv_width], paged_kv.cpp:53-56): the
// single-operation entry point mp_hip_paged_attention_decode.
//
// Every reduction that the reference CPU path performs sequentially
// (miniprefix/src/backend/cpu/llama_runner.cpp:85-93) runs in ONE lane in the
// same order, with multiply and add rounded separately (this file is
// compiled with -ffp-contract=off). Parallelism comes from independent
// outputs: tokens for scores, (head, d) for the PV sums.
#include "exact_math.h"
#include "kernels.h"
#include "layout.h"

namespace mphip {
namespace {

constexpr int kWave = 64;

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
// register copies between them.
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

}  // namespace

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


}  // namespace mphip
