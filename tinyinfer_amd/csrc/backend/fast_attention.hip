// Decode attention of the fast arithmetic mode: flash-decoding over the
// paged pools. The reference computes each (row, head) with an explicit
// two-pass softmax and sequential sums (llama_runner.cpp:85-93); here the
// context is cut into page-aligned splits, each split keeps a running
// maximum, denominator and weighted sum (the order of the floating-point
// sums differs; the result matches the reference within 1e-4 absolute on
// the reference's scale of inputs).
//
// One wavefront per work item (row, KV head, split): it serves the G query
// heads of the KV head, so each K and V byte is read once. Per page (16
// tokens of one layer and KV head, 4 KB of K then 4 KB of V, device page
// order of layout.h):
//  - scores: lane = (token t = lane/4, quarter dq = lane%4 of the 64 dims);
//    a lane reads 4 float4 of K (dims 16dq..16dq+15 of token t, the 16 lanes
//    of one float4 index forming a 256-byte run) and the four quarters are
//    summed across lanes;
//  - output: lane = dim d; a lane reads 4 float4 of V (4 tokens each for
//    its d, a 1 KB run per float4 index) and the page's probabilities from
//    LDS.
// The next page's K and V loads are issued before the current page is used.
// A merge kernel then combines the splits of every (row, head).
#include "kernels.h"
#include "layout.h"

namespace mphip {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kDim = 64;
constexpr int kPage = 16;
constexpr int kMaxGroup = 4;

template <int G>
__global__ __launch_bounds__(64) void fast_attention_split_kernel(const float* __restrict__ qkv, int ldq, int heads,
                                                                  RowMeta meta, PagedKv kv, int layer,
                                                                  FastAttentionWork w) {
    __shared__ float p_s[G][kPage];
    const int lane = threadIdx.x;
    const int4 item = reinterpret_cast<const int4*>(w.items)[blockIdx.x];
    const int row = item.x, kvh = item.y, t0 = item.z, n = item.w;
    const int length = meta.row_pos[row] + 1;
    const int32_t* table = kv.tables + (size_t)meta.seq_slot[meta.row_seq[row]] * kv.table_stride;
    const int t = lane >> 2, dq = lane & 3;
    // q of the group's heads, dims 16dq..16dq+15 (rotated, quad layout).
    f4 q[G][4];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = (kvh * G + h) * kDim + dq * 16 + j * 4;
            q[h][j] = *reinterpret_cast<const f4*>(qkv + quad_index(row, c, ldq));
        }
    const size_t head_base = (size_t)kvh * kPage * kDim;  // floats into a page-layer span
    auto page_ptr = [&](const float* pool, int page) {
        return pool + kv_page_base(table[page], layer, kv.layers, kPage, kv.kv_width) + head_base;
    };
    auto load = [&](int page, f4 (&kk)[4], f4 (&vv)[4]) {
        const f4* kp = reinterpret_cast<const f4*>(page_ptr(kv.keys, page));
        const f4* vp = reinterpret_cast<const f4*>(page_ptr(kv.values, page));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            kk[j] = __builtin_nontemporal_load(kp + (dq * 4 + j) * kPage + t);
            vv[j] = __builtin_nontemporal_load(vp + j * kDim + lane);
        }
    };
    float m[G], l[G], acc[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        m[h] = -__builtin_inff();
        l[h] = 0.0f;
        acc[h] = 0.0f;
    }
    const float scale = 0.125f;  // 1/sqrt(64)
    const int first = t0 / kPage, last = (t0 + n - 1) / kPage;
    f4 kc[4], vc[4], kn[4], vn[4];
    load(first, kc, vc);
    for (int page = first; page <= last; ++page) {
        if (page < last) load(page + 1, kn, vn);
        const int tok = page * kPage + t;
        const bool valid = tok < length && tok >= t0 && tok < t0 + n;
        float p[G];
#pragma unroll
        for (int h = 0; h < G; ++h) {
            f4 prod = q[h][0] * kc[0];
            prod += q[h][1] * kc[1];
            prod += q[h][2] * kc[2];
            prod += q[h][3] * kc[3];
            float s = (prod.x + prod.y) + (prod.z + prod.w);
            s += __shfl_xor(s, 1);
            s += __shfl_xor(s, 2);
            s = valid ? s * scale : -__builtin_inff();
            float mx = s;
            mx = fmaxf(mx, __shfl_xor(mx, 4));
            mx = fmaxf(mx, __shfl_xor(mx, 8));
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float m_new = fmaxf(m[h], mx);  // finite: every page holds a valid token
            const float keep = __expf(m[h] - m_new);
            p[h] = valid ? __expf(s - m_new) : 0.0f;
            float ps = p[h];
            ps += __shfl_xor(ps, 4);
            ps += __shfl_xor(ps, 8);
            ps += __shfl_xor(ps, 16);
            ps += __shfl_xor(ps, 32);
            l[h] = l[h] * keep + ps;
            acc[h] *= keep;
            m[h] = m_new;
        }
        if (dq == 0)
#pragma unroll
            for (int h = 0; h < G; ++h) p_s[h][t] = p[h];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const f4* pp = reinterpret_cast<const f4*>(p_s[h]);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f4 pv = pp[g];
                acc[h] += pv.x * vc[g].x + pv.y * vc[g].y + pv.z * vc[g].z + pv.w * vc[g].w;
            }
        }
        __builtin_amdgcn_wave_barrier();
        if (page < last) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                kc[j] = kn[j];
                vc[j] = vn[j];
            }
        }
    }
    const size_t it = blockIdx.x;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        w.partial_out[(it * G + h) * kDim + lane] = acc[h];
        if (lane == 0) {
            w.partial_ml[(it * G + h) * 2] = m[h];
            w.partial_ml[(it * G + h) * 2 + 1] = l[h];
        }
    }
}

// out[row][h*64 + d] for every head: the splits of (row, h/G) combined.
__global__ void fast_attention_merge_kernel(int heads, int kv_heads, FastAttentionWork w, float* __restrict__ out,
                                            int ldo) {
    const int row = blockIdx.x;
    const int G = heads / kv_heads;
    const int2 ri = reinterpret_cast<const int2*>(w.row_items)[row];
    for (int i = threadIdx.x; i < heads * kDim; i += blockDim.x) {
        const int h = i / kDim, d = i % kDim;
        const int kvh = h / G, hg = h % G;
        const int base = ri.x + kvh * ri.y;
        float mx = -__builtin_inff();
        for (int s = 0; s < ri.y; ++s) mx = fmaxf(mx, w.partial_ml[((size_t)(base + s) * G + hg) * 2]);
        float den = 0.0f, num = 0.0f;
        for (int s = 0; s < ri.y; ++s) {
            const size_t at = (size_t)(base + s) * G + hg;
            const float f = __expf(w.partial_ml[at * 2] - mx);
            den += w.partial_ml[at * 2 + 1] * f;
            num += w.partial_out[at * kDim + d] * f;
        }
        out[quad_index(row, i, ldo)] = num / den;
    }
}

template <int G>
void launch_split(hipStream_t s, const float* qkv, int ldq, int heads, const RowMeta& meta, const PagedKv& kv,
                  int layer, const FastAttentionWork& w) {
    fast_attention_split_kernel<G><<<w.items_count, 64, 0, s>>>(qkv, ldq, heads, meta, kv, layer, w);
}

}  // namespace

hipError_t launch_fast_attention(hipStream_t s, const float* qkv, int ldq, int rows, int heads, int kv_heads,
                                 const RowMeta& meta, const PagedKv& kv, int layer, float* out, int ldo,
                                 const FastAttentionWork& w) {
    const int G = heads / kv_heads;
    if (rows <= 0) return hipSuccess;
    if (kv.block_tokens != kPage || kv.kv_width != kv_heads * kDim || G > kMaxGroup || G < 1)
        return hipErrorInvalidValue;
    switch (G) {
    case 1: launch_split<1>(s, qkv, ldq, heads, meta, kv, layer, w); break;
    case 2: launch_split<2>(s, qkv, ldq, heads, meta, kv, layer, w); break;
    case 3: launch_split<3>(s, qkv, ldq, heads, meta, kv, layer, w); break;
    default: launch_split<4>(s, qkv, ldq, heads, meta, kv, layer, w); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    fast_attention_merge_kernel<<<rows, 256, 0, s>>>(heads, kv_heads, w, out, ldo);
    return hipGetLastError();
}

}  // namespace mphip
