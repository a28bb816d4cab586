// Paged GQA attention of the MiniPrefix forward (decode rows and chunked
// prefill row blocks) on gfx950, in the reference CPU path's evaluation
// order (miniprefix/src/backend/cpu/llama_runner.cpp:85-93), per (row, head):
//   s_t   = (sum_d q_d k_td, d sequential, multiply and add rounded
//            separately) / sqrt(dim)
//   m     = max_t s_t
//   e_t   = expf(s_t - m);   den = sum_t e_t, t sequential
//   out_d = sum_t (e_t / den) * v_td, t sequential
// (this file is compiled with -ffp-contract=off).
//
// A row block is up to 16 consecutive rows (positions) of one sequence;
// decode rows are blocks of one. Two kernels per layer:
//   scores: one work-group per (row block, kv head, 256-token chunk), thread
//           = token: every (row, head) of the block that sees the token gets
//           its score; per-chunk maxima go beside the scores.
//   pv:     one single-wavefront work-group per (row, head) task: the
//           softmax (maximum, e_t, the sequential denominator, p_t) and the
//           output chains, lane = d.
// Blocks arrive sorted by decreasing length so the longest chains start
// first.
#include "exact_math.h"
#include "kernels.h"
#include "layout.h"

namespace mphip {
namespace {

constexpr int kScoreChunk = 256;
constexpr int kMaxRowHeads = 48;
constexpr int kMaxTable = 2048;  // pages of one sequence (the host enforces it)
constexpr int kMaxDim = 64;  // lane = d in the output chains

// Wavefront maximum with DPP row shifts and row broadcasts (the maximum is
// order-free); lane 63 ends up with the result, which is then broadcast.
__device__ __forceinline__ float wave_max(float v) {
    const int ninf = __float_as_int(-INFINITY);
    int x = __float_as_int(v);
    x = __float_as_int(fmaxf(__int_as_float(x), __int_as_float(__builtin_amdgcn_update_dpp(ninf, x, 0x111, 0xf, 0xf, false))));
    x = __float_as_int(fmaxf(__int_as_float(x), __int_as_float(__builtin_amdgcn_update_dpp(ninf, x, 0x112, 0xf, 0xf, false))));
    x = __float_as_int(fmaxf(__int_as_float(x), __int_as_float(__builtin_amdgcn_update_dpp(ninf, x, 0x114, 0xf, 0xf, false))));
    x = __float_as_int(fmaxf(__int_as_float(x), __int_as_float(__builtin_amdgcn_update_dpp(ninf, x, 0x118, 0xf, 0xf, false))));
    x = __float_as_int(fmaxf(__int_as_float(x), __int_as_float(__builtin_amdgcn_update_dpp(ninf, x, 0x142, 0xa, 0xf, false))));
    x = __float_as_int(fmaxf(__int_as_float(x), __int_as_float(__builtin_amdgcn_update_dpp(ninf, x, 0x143, 0xc, 0xf, false))));
    return __int_as_float(__builtin_amdgcn_readlane(x, 63));
}

// BT/DIM: compile-time page size and head dim (0: runtime).
template <int BT, int DIM>
__global__ __launch_bounds__(kScoreChunk) void attn_scores_kernel(const float* __restrict__ qkv, int ldq, int heads,
                                                                  int kv_heads, int dim_rt, RowMeta meta, PagedKv kv,
                                                                  int layer, AttentionWork w) {
    __shared__ float partial[kScoreChunk / 64][kMaxRowHeads];
    __shared__ float4 q_s[kMaxRowHeads * kMaxDim / 4];
    const int dim = DIM ? DIM : dim_rt;
    const int bt = BT ? BT : kv.block_tokens;
    const int2 item = w.items[blockIdx.x];
    const int2 blk = w.blocks[item.x];
    const int kvh = blockIdx.y, chunk = item.y;
    const int r0 = blk.x, nr = blk.y;
    const int group = heads / kv_heads, rh = nr * group;
    const int pos0 = meta.row_pos[r0];
    const int last_length = pos0 + nr;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int32_t* table = kv.tables + (size_t)meta.seq_slot[meta.row_seq[r0]] * kv.table_stride;
    const int t = chunk * kScoreChunk + tid;
    const bool live = t < last_length;
    const int tc = live ? t : last_length - 1;
    const float* kbase = kv.keys + kv_page_base(table[tc / bt], layer, kv.layers, bt, kv.kv_width) +
                         key_offset(tc % bt, kvh, 0, bt, dim);
    // The block's q rows (rh x dim) in LDS, all loads in flight together
    // with this token's K row.
    const int dq = dim / 4;
    for (int e = tid; e < rh * dq; e += kScoreChunk) {
        const int i = e / dq, c = e - i * dq;
        const int r = i / group, h = i - r * group;
        q_s[e] = *reinterpret_cast<const float4*>(qkv + quad_index(r0 + r, (kvh * group + h) * dim + 4 * c, ldq));
    }
    float4 kreg[DIM ? DIM / 4 : 1];
    if (DIM) {
#pragma unroll
        for (int c = 0; c < DIM / 4; ++c) kreg[c] = *reinterpret_cast<const float4*>(kbase + (size_t)c * bt * 4);
    }
    __syncthreads();
    const float root = sqrtf((float)dim);
    for (int i = 0; i < rh; ++i) {
        const int r = i / group, h = i - r * group;
        const float4* q4 = q_s + i * dq;
        float acc = 0.0f;
        if (DIM) {
#pragma unroll
            for (int c = 0; c < DIM / 4; ++c) {
                const float4 q = q4[c];
                acc = acc + q.x * kreg[c].x;
                acc = acc + q.y * kreg[c].y;
                acc = acc + q.z * kreg[c].z;
                acc = acc + q.w * kreg[c].w;
            }
        } else {
            for (int c = 0; c < dq; ++c) {
                const float4 q = q4[c];
                const float4 k = *reinterpret_cast<const float4*>(kbase + (size_t)c * bt * 4);
                acc = acc + q.x * k.x;
                acc = acc + q.y * k.y;
                acc = acc + q.z * k.z;
                acc = acc + q.w * k.w;
            }
        }
        const float score = acc / root;
        const bool keep = live && t <= pos0 + r;
        if (keep) w.scores[((size_t)(r0 + r) * heads + kvh * group + h) * w.stride + t] = score;
        const float m = wave_max(keep ? score : -INFINITY);
        if (lane == 0) partial[wave][i] = m;
    }
    __syncthreads();
    if (tid < rh) {
        float m = partial[0][tid];
#pragma unroll
        for (int j = 1; j < kScoreChunk / 64; ++j) m = fmaxf(m, partial[j][tid]);
        const int r = tid / group, h = tid - r * group;
        w.chunk_max[((size_t)(r0 + r) * heads + kvh * group + h) * w.chunks + chunk] = m;
    }
}

// One single-wavefront work-group per task: P heads (P = 1 for decode, the
// whole group for prefill) of one row. It forms the row's softmax and its
// output chains (lane = d):
//   m  = max of the row's chunk maxima;
//   e_t = expf(s_t - m) staged in LDS (kPWindow tokens at a time);
//   den = sum_t e_t in token order (lane h of the wavefront, one chain per
//         head); p_t = e_t / den;
//   out_d = sum_t p_t v_td in token order.
// V pages stream through a ring of registers; the first pages are already
// in flight while the denominators are summed. grid =
// (blocks, kv heads, tasks per block): for decode the 3 heads of a
// (sequence, kv head) are 192 work-groups apart in dispatch order, which
// keeps them on one XCD (shared L2) but on different CUs.
constexpr int kPWindow = 2048;
constexpr int kRingPages = 8;  // V pages in flight per wavefront (16 VGPRs each)

template <int BT, int DIM, int P>
__global__ __launch_bounds__(64) void attn_pv_kernel(int heads, int kv_heads, int dim_rt, RowMeta meta, PagedKv kv,
                                                     int layer, AttentionWork w, float* __restrict__ out, int ldo) {
    __shared__ int32_t table_s[kMaxTable];
    __shared__ float4 p_s[P][kPWindow / 4];
    __shared__ float den_s[P];
    const int dim = DIM ? DIM : dim_rt;
    const int bt = BT ? BT : kv.block_tokens;
    const int2 blk = w.blocks[blockIdx.x];
    const int kvh = blockIdx.y, task = blockIdx.z;
    const int r0 = blk.x, nr = blk.y;
    const int group = heads / kv_heads;
    const int per_row = group / P;
    if (task >= nr * per_row) return;
    const int r = task / per_row, hg = task - r * per_row;
    const int pos0 = meta.row_pos[r0];
    const int row = r0 + r, len = pos0 + r + 1;
    const int h0 = kvh * group + hg * P;
    const int lane = threadIdx.x;
    const int32_t* table_g = kv.tables + (size_t)meta.seq_slot[meta.row_seq[r0]] * kv.table_stride;
    const int pages = (len + bt - 1) / bt;
    const float* srow = w.scores + ((size_t)row * heads + h0) * w.stride;
    const int nc = (len + kScoreChunk - 1) / kScoreChunk;
    // Page table and chunk maxima: loads go out 8 per lane at a time
    // (unrolled, clamped), one memory latency per 8.
    for (int i0 = 0; i0 < pages; i0 += 64 * 8) {
        int32_t tv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) tv[j] = table_g[min(i0 + 64 * j + lane, pages - 1)];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (i0 + 64 * j + lane < pages) table_s[i0 + 64 * j + lane] = tv[j];
    }
    float mx[P];
#pragma unroll
    for (int h = 0; h < P; ++h) {
        const float* cm = w.chunk_max + ((size_t)row * heads + h0 + h) * w.chunks;
        float m = -INFINITY;
        for (int c0 = 0; c0 < nc; c0 += 64 * 4) {
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = cm[min(c0 + 64 * j + lane, nc - 1)];
#pragma unroll
            for (int j = 0; j < 4; ++j) m = fmaxf(m, v[j]);
        }
        mx[h] = wave_max(m);
    }
    // e_t = expf(s_t - m) for tokens [u0, u0+n) into p_s.
    auto stage_e = [&](int u0, int n) {
        const int n4 = (n + 3) / 4;
#pragma unroll
        for (int h = 0; h < P; ++h) {
            const float4* src = reinterpret_cast<const float4*>(srow + (size_t)h * w.stride + u0);
            for (int i0 = 0; i0 < n4; i0 += 64 * 8) {
                float4 t[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) t[j] = src[min(i0 + 64 * j + lane, n4 - 1)];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int e = i0 + 64 * j + lane;
                    if (e < n4) {
                        const float m = mx[h];
                        const int u = 4 * e;  // padding past n is never read
                        p_s[h][e] = make_float4(ref_expf(t[j].x - m), u + 1 < n ? ref_expf(t[j].y - m) : 0.0f,
                                                u + 2 < n ? ref_expf(t[j].z - m) : 0.0f,
                                                u + 3 < n ? ref_expf(t[j].w - m) : 0.0f);
                    }
                }
            }
        }
    };
    // Lane h < P adds head h's staged e_t (tokens [0, n)) in order.
    auto chain = [&](int n, float& den) {
        if (lane < P) {
            const float4* e4 = p_s[lane];
            const int full = n >> 2;
            int q = 0;
            if (full >= 16) {
                float4 a[8], b[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) a[j] = e4[j];
                for (; q + 16 <= full; q += 16) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) b[j] = e4[q + 8 + j];
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        den = den + a[j].x;
                        den = den + a[j].y;
                        den = den + a[j].z;
                        den = den + a[j].w;
                    }
                    const int nq = min(q + 16, full - 8);
#pragma unroll
                    for (int j = 0; j < 8; ++j) a[j] = e4[nq + j];
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        den = den + b[j].x;
                        den = den + b[j].y;
                        den = den + b[j].z;
                        den = den + b[j].w;
                    }
                }
                if (q + 8 <= full) {  // `a` holds quads q..q+7
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        den = den + a[j].x;
                        den = den + a[j].y;
                        den = den + a[j].z;
                        den = den + a[j].w;
                    }
                    q += 8;
                }
            }
            for (; q < full; ++q) {
                const float4 v = e4[q];
                den = den + v.x;
                den = den + v.y;
                den = den + v.z;
                den = den + v.w;
            }
            const float* e = reinterpret_cast<const float*>(e4);
            for (int u = full * 4; u < n; ++u) den = den + e[u];
        }
    };
    const int d = lane < dim ? lane : 0;
    // Ring of kRingPages V pages in registers (16-token pages, dim 64):
    // lane d holds the page's 16 values of d as 4 float4 (tokens 4j..4j+3),
    // each float4 load one contiguous 1 KB run across the wavefront.
    float4 ring[kRingPages][4];
    auto load_page = [&](int pg, float4 (&v)[4]) {
        const int block = __builtin_amdgcn_readfirstlane(table_s[pg]);
        const float4* src = reinterpret_cast<const float4*>(
            kv.values + kv_page_base(block, layer, kv.layers, 16, kv.kv_width) + value_offset(0, kvh, 0, 16, 64));
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = src[64 * j + lane];
    };
    // Ring invariant at a group boundary pg: ring[s] holds page
    // min(pg + s, last).
    auto prologue = [&](int pg_first, int pg_end) {
#pragma unroll
        for (int s = 0; s < kRingPages; ++s) load_page(min(pg_first + s, pg_end - 1), ring[s]);
    };
    constexpr bool kRing = BT == 16 && DIM == 64;
    // Denominators. One window: e is staged once, the first V pages are
    // requested, and the chain runs while they arrive. Several windows: a
    // first pass sums the denominators; the window loop forms e again.
    // (The ring is first filled at a single place in the window loop so that
    // every path reaches the page loop with the same loads in flight.)
    const bool one_window = len <= kPWindow;
    float den = 0.0f;
    if (!one_window) {
        for (int u0 = 0; u0 < len; u0 += kPWindow) {
            stage_e(u0, min(kPWindow, len - u0));
            chain(min(kPWindow, len - u0), den);
        }
        if (lane < P) den_s[lane] = den;
    }
    float acc[P];
#pragma unroll
    for (int h = 0; h < P; ++h) acc[h] = 0.0f;
    for (int u0 = 0; u0 < len; u0 += kPWindow) {
        const int n_win = min(kPWindow, len - u0);
        stage_e(u0, n_win);
        if (kRing) prologue(u0 >> 4, (u0 + n_win + 15) >> 4);
        if (one_window) {
            chain(len, den);
            if (lane < P) den_s[lane] = den;
        }
        // p_t = e_t / den in place.
#pragma unroll
        for (int h = 0; h < P; ++h) {
            const float dn = den_s[h];
            for (int e = lane; e < (n_win + 3) / 4; e += 64) {
                const float4 v = p_s[h][e];
                p_s[h][e] = make_float4(v.x / dn, v.y / dn, v.z / dn, v.w / dn);
            }
        }
        if (kRing) {
            const int pg_first = u0 >> 4;
            const int pg_end = (u0 + n_win + 15) >> 4;
            const int full_end = (u0 + n_win) >> 4;
            auto page_sum = [&](const float4 (&v)[4], int pg, int n) {
                const int q0 = (pg - pg_first) * 4;
#pragma unroll
                for (int h = 0; h < P; ++h) {
                    float a = acc[h];
#pragma unroll
                    for (int s4 = 0; s4 < 4; ++s4) {
                        const float4 p = p_s[h][q0 + s4];
                        if (n == 16) {
                            a = a + p.x * v[s4].x;
                            a = a + p.y * v[s4].y;
                            a = a + p.z * v[s4].z;
                            a = a + p.w * v[s4].w;
                        } else {
                            if (4 * s4 + 0 < n) a = a + p.x * v[s4].x;
                            if (4 * s4 + 1 < n) a = a + p.y * v[s4].y;
                            if (4 * s4 + 2 < n) a = a + p.z * v[s4].z;
                            if (4 * s4 + 3 < n) a = a + p.w * v[s4].w;
                        }
                    }
                    acc[h] = a;
                }
            };
            const int last = pg_end - 1;
            int pg = pg_first;
            for (; pg + kRingPages <= full_end; pg += kRingPages) {
#pragma unroll
                for (int s = 0; s < kRingPages; ++s) {
                    page_sum(ring[s], pg + s, 16);
                    load_page(min(pg + s + kRingPages, last), ring[s]);
                    // Keep each page's LDS reads next to its use (no
                    // hoisting across pages: register pressure).
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            // Fewer than kRingPages full pages and the partial page remain.
#pragma unroll
            for (int s = 0; s < kRingPages; ++s)
                if (pg + s < pg_end) page_sum(ring[s], pg + s, pg + s < full_end ? 16 : u0 + n_win - ((pg + s) << 4));
            // Drain the clamped refills past the window so that the next
            // window starts with no ring load in flight (the compiler then
            // keeps exact per-page waits in the loop above).
            if (!one_window) __builtin_amdgcn_s_waitcnt(0);
        } else {
            for (int u = 0; u < n_win; ++u) {
                const int tt = u0 + u, pg = tt / bt, slot = tt - pg * bt;
                const float v = kv.values[kv_page_base(table_s[pg], layer, kv.layers, bt, kv.kv_width) +
                                          value_offset(slot, kvh, d, bt, dim)];
#pragma unroll
                for (int h = 0; h < P; ++h) acc[h] = acc[h] + reinterpret_cast<const float*>(p_s[h])[u] * v;
            }
        }
    }
    if (lane < dim) {
#pragma unroll
        for (int j = 0; j < P; ++j) out[quad_index(row, (h0 + j) * dim + lane, ldo)] = acc[j];
    }
}

template <int BT, int DIM>
hipError_t launch_pair(hipStream_t s, const float* qkv, int ldq, int heads, int kv_heads, int dim,
                       const RowMeta& meta, const PagedKv& kv, int layer, float* out, int ldo,
                       const AttentionWork& w, bool decode) {
    attn_scores_kernel<BT, DIM><<<dim3(w.items_count, kv_heads), kScoreChunk, 0, s>>>(qkv, ldq, heads, kv_heads, dim,
                                                                                      meta, kv, layer, w);
    const int group = heads / kv_heads;
    const int block_rows = attention_row_block(heads, kv_heads, dim);
    if (decode) {
        attn_pv_kernel<BT, DIM, 1><<<dim3(w.blocks_count, kv_heads, group), 64, 0, s>>>(heads, kv_heads, dim, meta,
                                                                                       kv, layer, w, out, ldo);
    } else {
        const dim3 grid(w.blocks_count, kv_heads, block_rows);
        switch (group) {
        case 2: attn_pv_kernel<BT, DIM, 2><<<grid, 64, 0, s>>>(heads, kv_heads, dim, meta, kv, layer, w, out, ldo); break;
        case 3: attn_pv_kernel<BT, DIM, 3><<<grid, 64, 0, s>>>(heads, kv_heads, dim, meta, kv, layer, w, out, ldo); break;
        case 4: attn_pv_kernel<BT, DIM, 4><<<grid, 64, 0, s>>>(heads, kv_heads, dim, meta, kv, layer, w, out, ldo); break;
        default:
            attn_pv_kernel<BT, DIM, 1><<<dim3(w.blocks_count, kv_heads, block_rows * group), 64, 0, s>>>(
                heads, kv_heads, dim, meta, kv, layer, w, out, ldo);
            break;
        }
    }
    return hipGetLastError();
}

}  // namespace

int attention_row_block(int heads, int kv_heads, int dim) {
    (void)dim;
    const int group = heads / kv_heads;
    const int rows = kMaxRowHeads / group;
    return rows < 16 ? rows : 16;
}

hipError_t launch_attention(hipStream_t s, const float* qkv, int ldq, int rows, int heads, int kv_heads, int dim,
                            const RowMeta& meta, const PagedKv& kv, int layer, float* out, int ldo,
                            const AttentionWork& w, bool decode) {
    if (rows <= 0 || w.blocks_count <= 0) return hipSuccess;
    const int group = heads / kv_heads;
    if (group > kMaxRowHeads || dim % 4 || dim > kMaxDim || kv.block_tokens % 4 ||
        kv.table_stride > kMaxTable)
        return hipErrorInvalidValue;
    if (kv.block_tokens == 16 && dim == 64)
        return launch_pair<16, 64>(s, qkv, ldq, heads, kv_heads, dim, meta, kv, layer, out, ldo, w, decode);
    return launch_pair<0, 0>(s, qkv, ldq, heads, kv_heads, dim, meta, kv, layer, out, ldo, w, decode);
}

}  // namespace mphip
