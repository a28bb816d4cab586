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
#include <hip/hip_ext.h>

#include <type_traits>

#include "dpp.h"
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
// ROPE (decode blocks of one row, 16-token pages, head dim 64): q is
// rotated while it is staged in LDS, and the block holding the row's new
// token rotates that token's k, writes it and the v row to the pools and
// uses the rotated k for the token's own score (the arithmetic of
// rope_append_kernel; no other block reads that token).
template <int BT, int DIM, bool ROPE = false>
__global__ __launch_bounds__(kScoreChunk) void attn_scores_kernel(const float* __restrict__ qkv, int ldq, int heads,
                                                                  int kv_heads, int dim_rt, RowMeta meta, PagedKv kv,
                                                                  int layer, AttentionWork w, RopeTables rope) {
    static_assert(!ROPE || (BT == 16 && DIM == 64), "fused RoPE shape");
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
    // (a, b) -> (a*cos - b*sin, b*cos + a*sin); inputs by value, so lo and hi
    // may be the inputs' own registers.
    auto rotate = [](const float4 a, const float4 b, const float4 cs, const float4 sn, float4& lo, float4& hi) {
        lo = make_float4(a.x * cs.x - b.x * sn.x, a.y * cs.y - b.y * sn.y, a.z * cs.z - b.z * sn.z,
                         a.w * cs.w - b.w * sn.w);
        hi = make_float4(b.x * cs.x + a.x * sn.x, b.y * cs.y + a.y * sn.y, b.z * cs.z + a.z * sn.z,
                         b.w * cs.w + a.w * sn.w);
    };
    const float4* cs4 = ROPE ? reinterpret_cast<const float4*>(rope.cos + (size_t)pos0 * (DIM / 2)) : nullptr;
    const float4* sn4 = ROPE ? reinterpret_cast<const float4*>(rope.sin + (size_t)pos0 * (DIM / 2)) : nullptr;
    __shared__ float4 rope_s[ROPE ? 2 * (DIM / 8) : 1];  // cos then sin of the row's position
    const bool new_token = ROPE && t == pos0;
    const int hidden = heads * (DIM ? DIM : dim);
    if (ROPE) {
        // One row (nr = 1): quads c and c + 8 of each head form the rotated pairs.
        for (int e = tid; e < group * (DIM / 8); e += kScoreChunk) {
            const int h = e / (DIM / 8), c = e - h * (DIM / 8);
            const int col = (kvh * group + h) * DIM;
            const float4 a = *reinterpret_cast<const float4*>(qkv + quad_index(r0, col + 4 * c, ldq));
            const float4 b = *reinterpret_cast<const float4*>(qkv + quad_index(r0, col + DIM / 2 + 4 * c, ldq));
            rotate(a, b, cs4[c], sn4[c], q_s[h * (DIM / 4) + c], q_s[h * (DIM / 4) + c + DIM / 8]);
        }
        if (tid < 2 * (DIM / 8)) rope_s[tid] = tid < DIM / 8 ? cs4[tid] : sn4[tid - DIM / 8];
    } else {
        for (int e = tid; e < rh * dq; e += kScoreChunk) {
            const int i = e / dq, c = e - i * dq;
            const int r = i / group, h = i - r * group;
            q_s[e] = *reinterpret_cast<const float4*>(qkv + quad_index(r0 + r, (kvh * group + h) * dim + 4 * c, ldq));
        }
    }
    // This token's K row; the row's new token takes its unrotated k from the
    // projection instead (rotated below, then written to the page).
    float4 kreg[DIM ? DIM / 4 : 1];
    if (DIM) {
        // Consecutive quads of a row are 256 floats apart in the quad layout,
        // bt*4 apart in a K page.
        const float* src = new_token ? qkv + quad_index(r0, hidden + kvh * DIM, ldq) : kbase;
        const int step = new_token ? 256 : BT * 4;
        // K is read once per step: non-temporal loads (measured ~10% faster
        // for this kernel than the default policy).
#pragma unroll
        for (int c = 0; c < DIM / 4; ++c) {
            const f4v k4 = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(src + c * step));
            kreg[c] = make_float4(k4.x, k4.y, k4.z, k4.w);
        }
    }
    // The wavefront holding the new token copies its v row at the end (lane = d).
    const bool v_wave = ROPE && pos0 >= chunk * kScoreChunk + wave * 64 && pos0 < chunk * kScoreChunk + wave * 64 + 64;
    float vnew = 0.0f;
    if (v_wave) vnew = qkv[quad_index(r0, hidden + kv.kv_width + kvh * DIM + lane, ldq)];
    __syncthreads();
    if (new_token) {
#pragma unroll
        for (int c = 0; c < DIM / 8; ++c) rotate(kreg[c], kreg[c + DIM / 8], rope_s[c], rope_s[DIM / 8 + c], kreg[c], kreg[c + DIM / 8]);
#pragma unroll
        for (int c = 0; c < DIM / 4; ++c) *reinterpret_cast<float4*>(kv.keys + (kbase - kv.keys) + (size_t)c * BT * 4) = kreg[c];
    }
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
    if (v_wave) {
        const size_t base = kv_page_base(table[pos0 / BT], layer, kv.layers, BT, kv.kv_width);
        kv.values[base + value_offset(pos0 % BT, kvh, lane, BT, DIM)] = vnew;
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
    auto load_block = [&](int block_id, float4 (&v)[4]) {
        const int block = __builtin_amdgcn_readfirstlane(block_id);
        const float4* src = reinterpret_cast<const float4*>(
            kv.values + kv_page_base(block, layer, kv.layers, 16, kv.kv_width) + value_offset(0, kvh, 0, 16, 64));
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = src[64 * j + lane];
    };
    auto load_page = [&](int pg, float4 (&v)[4]) { load_block(table_s[pg], v); };
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
            // Products p_t * v_td (rounded as the reference rounds them) are
            // formed one page ahead of their additions and interleaved with
            // them in program order (each dependent add is followed by
            // independent multiplies), so the add chain is the only latency.
            auto read_p = [&](int pg, float4 (&o)[P][4]) {
                const int q0 = (pg - pg_first) * 4;
#pragma unroll
                for (int h = 0; h < P; ++h)
#pragma unroll
                    for (int s4 = 0; s4 < 4; ++s4) o[h][s4] = p_s[h][q0 + s4];
            };
            auto lane4 = [](const float4& v, int c) { return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w; };
            auto products = [&](const float4 (&v)[4], const float4 (&pp)[P][4], float (&o)[P][16]) {
#pragma unroll
                for (int h = 0; h < P; ++h)
#pragma unroll
                    for (int t = 0; t < 16; ++t) o[h][t] = lane4(pp[h][t >> 2], t & 3) * lane4(v[t >> 2], t & 3);
            };
            // acc += products of the first n tokens of a page, in order.
            auto add_page = [&](const float (&o)[P][16], int n) {
#pragma unroll
                for (int t = 0; t < 16; ++t)
                    if (n == 16 || t < n) {
#pragma unroll
                        for (int h = 0; h < P; ++h) acc[h] = acc[h] + o[h][t];
                    }
            };
            const int last = pg_end - 1;
            int pg = pg_first;
            float pr[P][16];  // products of page pg
            {
                float4 pp[P][4];
                read_p(pg, pp);
                products(ring[0], pp, pr);
            }
            for (; pg + kRingPages <= full_end; pg += kRingPages) {
                // Block ids of this group's refills, read together.
                int32_t refill[kRingPages];
#pragma unroll
                for (int s = 0; s < kRingPages; ++s) refill[s] = table_s[min(pg + kRingPages + s, last)];
#pragma unroll
                for (int s = 0; s < kRingPages; ++s) {
                    // ring[s] (page pg+s) is consumed: refill it; add page
                    // pg+s while forming the products of page pg+s+1
                    // (ring[s+1], or the refilled ring[0] at the end of the
                    // group).
                    load_block(refill[s], ring[s]);
                    float4 pp[P][4];
                    read_p(min(pg + s + 1, last), pp);
                    const float4 (&vn)[4] = ring[(s + 1) % kRingPages];
                    float nx[P][16];
#pragma unroll
                    for (int t = 0; t < 16; ++t) {
#pragma unroll
                        for (int h = 0; h < P; ++h) acc[h] = acc[h] + pr[h][t];
                        // The first adds run while the next page's p and V
                        // arrive; from the 4th on, each add is followed by
                        // the multiplies of the next page.
                        if (t >= 3) {
                            const int t0 = (t - 3) * 16 / 13, t1 = (t - 2) * 16 / 13;
#pragma unroll
                            for (int u = t0; u < t1; ++u)
#pragma unroll
                                for (int h = 0; h < P; ++h)
                                    nx[h][u] = lane4(pp[h][u >> 2], u & 3) * lane4(vn[u >> 2], u & 3);
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
#pragma unroll
                    for (int h = 0; h < P; ++h)
#pragma unroll
                        for (int t = 0; t < 16; ++t) pr[h][t] = nx[h][t];
                }
            }
            // Fewer than kRingPages full pages and the partial page remain;
            // ring[s] holds page pg+s and pr the products of page pg.
#pragma unroll
            for (int s = 0; s < kRingPages; ++s) {
                if (pg + s < pg_end) {
                    if (s) {
                        float4 pp[P][4];
                        read_p(pg + s, pp);
                        products(ring[s], pp, pr);
                    }
                    add_page(pr, pg + s < full_end ? 16 : u0 + n_win - ((pg + s) << 4));
                }
            }
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

// Decode rows with 16-token pages and head dim 64, contexts up to
// kFusedMaxT, after the scores kernel: one work-group of 8 wavefronts per
// (sequence row, KV head) forms the softmax and the output of its G query
// heads.
//   1-3. wavefronts G..7 (producers): m = maximum of each head's chunk
//      maxima (order-free); e_t = expf(s_t - m) for 64-token batches, lane
//      = token, into LDS, then a per-batch ready flag;
//      wavefront h < G (consumer): den of head h, adding e_t in token order
//      batch by batch as the flags come up (every lane runs the same chain
//      from LDS broadcast reads);
//   4. p_t = e_t / den, all threads;
//   5. output: wavefront h adds p_t * v_td (product rounded as the reference
//      rounds it; each dependent add is followed by the next multiply) in
//      token order, lane = d, with V pages streamed through a ring of
//      registers kRingPages ahead (the producers touched the first pages
//      after their e_t). The G wavefronts read the same pages, so two of three
//      reads hit the work-group's L1. p_t reaches the lanes by DPP row
//      broadcast from one f4 per lane per 64 tokens.
constexpr int kFusedMaxT = 4096;
constexpr int kFusedThreads = 512;
// Producer wavefronts touch up to this many V pages each after their e_t
// (more floods HBM while the softmax still needs it).
constexpr int kTouchPages = 16;

typedef __attribute__((address_space(3))) uint32_t LdsU32;

// Work-group barrier that orders LDS only: this wavefront's LDS accesses
// complete (lgkmcnt(0)) before the barrier; global loads stay in flight.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt 63, expcnt 7, lgkmcnt 0
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int G>
__global__ __launch_bounds__(kFusedThreads) void attn_decode_kernel(int heads, RowMeta meta, PagedKv kv, int layer,
                                                                    AttentionWork w, float* __restrict__ out,
                                                                    int ldo) {
    static_assert(G >= 1 && G < kFusedThreads / 64, "waves per head");
    __shared__ float4 sc4[G][kFusedMaxT / 4];  // s_t, then e_t, then p_t
    __shared__ float den_s[G];
    __shared__ uint64_t exp_tab[32];
    __shared__ uint32_t ready_s[G][kFusedMaxT / 64];  // e of batch b of head h is in LDS
    __shared__ uint32_t voff_s[kFusedMaxT / 16];  // page pg's V of this KV head, in float4 from kv.values
    float* const sc = reinterpret_cast<float*>(&sc4[0][0]);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kvh = blockIdx.y;
    const int row = w.blocks[blockIdx.x].x;
    const int len = meta.row_pos[row] + 1;
    const int pages = (len + 15) >> 4;
    const int last_page = pages - 1;
    const int32_t* table_g = kv.tables + (size_t)meta.seq_slot[meta.row_seq[row]] * kv.table_stride;
    // Float4 offsets of the pages' V for this KV head (the pool holds fewer
    // than 2^32 float4: checked at creation).
    const uint32_t page_f4 = (uint32_t)(16 * kv.kv_width / 4);
    for (int i = tid; i < pages; i += kFusedThreads)
        voff_s[i] = ((uint32_t)table_g[i] * (uint32_t)kv.layers + (uint32_t)layer) * page_f4 + (uint32_t)kvh * 256u;
    // Producers (wavefronts G..7) start their first loads before the
    // barrier: head h's scores of their first batch and its chunk maxima.
    constexpr int kProducers = kFusedThreads / 64 - G;
    const int batches = (len + 63) >> 6;  // 64-token batches, 64 * batches <= kFusedMaxT
    const int nch = (len + 255) >> 8;     // at most 16 chunk maxima
    // Every batch a producer will handle (b = wave - G + i * kProducers) has
    // its scores requested here, so the producers wait on one round trip.
    constexpr int kProducerBatches = (kFusedMaxT / 64 + kProducers - 1) / kProducers;
    float sall[kProducerBatches][G], cmax[G];
    float touch[kTouchPages];  // producers: V pages read ahead, see below
    if (wave >= G) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const size_t rh = (size_t)row * heads + kvh * G + h;
            cmax[h] = w.chunk_max[rh * w.chunks + min(lane, nch - 1)];
        }
#pragma unroll
        for (int i = 0; i < kProducerBatches; ++i)
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float* srow = w.scores + ((size_t)row * heads + kvh * G + h) * w.stride;
                sall[i][h] = srow[min(64 * (wave - G + i * kProducers) + lane, len - 1)];
            }
    }
    for (int i = tid; i < G * (kFusedMaxT / 64); i += kFusedThreads) (&ready_s[0][0])[i] = 0u;
    if (tid < 32) exp_tab[tid] = kExp2Table[tid];
    __syncthreads();

    // ---- 1-3. e_t into LDS by the producer wavefronts, den by wavefront h
    if (wave >= G) {
        // Producers: batch b goes to wavefront G + b % kProducers; lane =
        // token. m of each head is the maximum of its chunk maxima.
        float m[G];
#pragma unroll
        for (int h = 0; h < G; ++h) m[h] = wave_max(cmax[h]);
#pragma unroll
        for (int i = 0; i < kProducerBatches; ++i) {
            const int b = wave - G + i * kProducers;
            if (b >= batches) break;
#pragma unroll
            for (int h = 0; h < G; ++h)
                sc[h * kFusedMaxT + 64 * b + lane] = ref_expf_select(sall[i][h] - m[h], exp_tab);
            // The e writes above precede the flags in this wavefront's LDS order.
            if (lane == 0) {
#pragma unroll
                for (int h = 0; h < G; ++h) ((volatile LdsU32*)ready_s[h])[b] = 1u;
            }
        }
        // Then touch this KV head's V pages (one dword per 64 bytes, a page
        // per instruction; this wavefront's share of the first
        // kTouchPages * kProducers pages, all in flight together) so that the
        // output chains find them in cache rather than in HBM. The loaded
        // values are consumed only when the producers leave (phase 5): the
        // barriers in between wait for LDS work only, not for these loads.
        const float* vf = kv.values;
#pragma unroll
        for (int i = 0; i < kTouchPages; ++i)
            touch[i] = vf[(size_t)voff_s[min(wave - G + i * kProducers, last_page)] * 4 + lane * 16];
    } else {
        // Consumer: its adds are the work-group's critical path, so it takes
        // issue priority over the producer sharing its SIMD until den is out.
        __builtin_amdgcn_s_setprio(3);
        // Consumer: head h = wave sums its e_t in token order, every lane the
        // same chain, a batch as soon as its flag is up. The wait is bounded;
        // every flag below `batches` is set by a producer.
        const float4* es4 = sc4[wave];
        const float* es = sc + wave * kFusedMaxT;
        // Flags are checked four batches at a time (one 16-byte read); a flag
        // at or past `batches` counts as set.
        typedef uint32_t u4v __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) u4v LdsU4;
        volatile LdsU4* const flags4 = (volatile LdsU4*)ready_s[wave];
        // A wait that runs out (it cannot while every producer runs) records
        // a device error that the host turns into a failed forward; the
        // work-group still runs to its end so every wave leaves normally.
        auto wait_group = [&](int g) {
            bool ok = false;
            for (int spin = 0; spin < (1 << 16) && !ok; ++spin) {
                const u4v f = flags4[g];
                const int b = 4 * g;
                const bool set = (f.x | (b >= batches)) && (f.y | (b + 1 >= batches)) &&
                                 (f.z | (b + 2 >= batches)) && (f.w | (b + 3 >= batches));
                ok = __builtin_amdgcn_readfirstlane(set ? 1 : 0) != 0;
                if (!ok) __builtin_amdgcn_s_sleep(1);
            }
            if (!ok && lane == 0 && w.error) __hip_atomic_fetch_or(w.error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            asm volatile("" ::: "memory");
        };
        auto read_batch = [&](int b, float4 (&ev)[16]) {
#pragma unroll
            for (int j = 0; j < 16; ++j) ev[j] = es4[16 * b + j];
        };
        float den = 0.0f;
        auto add_batch = [&](const float4 (&ev)[16]) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                den = den + ev[j].x;
                den = den + ev[j].y;
                den = den + ev[j].z;
                den = den + ev[j].w;
            }
        };
        // Full batches in groups of four; within a group batch b+1 is read
        // while batch b is added.
        const int full = len >> 6;
        float4 e0[16], e1[16];
        for (int g = 0; 4 * g < full; ++g) {
            const int b = 4 * g;
            wait_group(g);
            read_batch(b, e0);
            if (b + 1 < full) read_batch(b + 1, e1);
            add_batch(e0);
            if (b + 1 < full) {
                if (b + 2 < full) read_batch(b + 2, e0);
                add_batch(e1);
                if (b + 2 < full) {
                    if (b + 3 < full) read_batch(b + 3, e1);
                    add_batch(e0);
                    if (b + 3 < full) add_batch(e1);
                }
            }
        }
        if (full < batches) {
            wait_group(full >> 2);
            for (int t = 64 * full; t < len; ++t) den = den + es[t];
        }
        if (lane == 0) den_s[wave] = den;
        __builtin_amdgcn_s_setprio(0);
    }
    lds_barrier();
    // ---- 4. p_t = e_t / den
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float dn = den_s[h];
        for (int t = tid; t < len; t += kFusedThreads) sc[h * kFusedMaxT + t] = sc[h * kFusedMaxT + t] / dn;
    }
    lds_barrier();

    // ---- 5. output chains (no barrier from here on)
    if (wave >= G) {
        float sink = 0.0f;
#pragma unroll
        for (int i = 0; i < kTouchPages; ++i) sink += touch[i];
        asm volatile("" ::"v"(sink));
        return;
    }
    // p of 64-token group g: lane l holds p[64g + 4(l%16) .. +3], so the p of
    // token 64g + 4i + c is component c of lane i of every 16-lane row and
    // reaches all lanes through a DPP row broadcast folded into the multiply.
    const f4v* pg4 = reinterpret_cast<const f4v*>(sc4[wave]) + (lane & 15);
    auto read_group = [&](int g) { return pg4[16 * min(g, kFusedMaxT / 64 - 1)]; };
    const float4* vbase = reinterpret_cast<const float4*>(kv.values);
    auto lane4 = [](const float4& v, int c) { return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w; };
    auto lane4v = [](const f4v& v, int c) { return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w; };
    float4 ring[kRingPages][4];
    auto load_page = [&](uint32_t off, float4 (&v)[4]) {
        const float4* src = vbase + __builtin_amdgcn_readfirstlane(off);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = src[64 * j + lane];
    };
    float acc = 0.0f;
    // acc += p_t * v_td over full page K (0..3) of a group: each dependent
    // add is followed by the next token's multiply.
    auto add_page = [&](auto kpage, const float4 (&v)[4], const f4v& pv) {
        constexpr int K = decltype(kpage)::value;
        float prod = mul_bcast<4 * K>(pv.x, v[0].x);
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const float cur = prod;
            if (t < 15) {
                const int u = t + 1;
                prod = mul_bcast_at(4 * K + (u >> 2), lane4v(pv, u & 3), lane4(v[u >> 2], u & 3));
            }
            acc = acc + cur;
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    static_assert(kRingPages == 8, "two p groups per ring turn");
    // Ring invariant at a turn boundary pg (a multiple of 8): ring[r] holds
    // page min(pg + r, last_page) and pgrp holds the p groups of pages
    // pg..pg+7.
#pragma unroll
    for (int r = 0; r < kRingPages; ++r) load_page(voff_s[min(r, last_page)], ring[r]);
    f4v pgrp[2] = {read_group(0), read_group(1)};
    const int full_pages = len >> 4;
    int pg = 0;
    for (; pg + kRingPages <= full_pages; pg += kRingPages) {
        uint32_t refill[kRingPages];
#pragma unroll
        for (int r = 0; r < kRingPages; ++r) refill[r] = voff_s[min(pg + kRingPages + r, last_page)];
        const f4v next[2] = {read_group((pg >> 2) + 2), read_group((pg >> 2) + 3)};
        add_page(std::integral_constant<int, 0>(), ring[0], pgrp[0]); load_page(refill[0], ring[0]);
        add_page(std::integral_constant<int, 1>(), ring[1], pgrp[0]); load_page(refill[1], ring[1]);
        add_page(std::integral_constant<int, 2>(), ring[2], pgrp[0]); load_page(refill[2], ring[2]);
        add_page(std::integral_constant<int, 3>(), ring[3], pgrp[0]); load_page(refill[3], ring[3]);
        add_page(std::integral_constant<int, 0>(), ring[4], pgrp[1]); load_page(refill[4], ring[4]);
        add_page(std::integral_constant<int, 1>(), ring[5], pgrp[1]); load_page(refill[5], ring[5]);
        add_page(std::integral_constant<int, 2>(), ring[6], pgrp[1]); load_page(refill[6], ring[6]);
        add_page(std::integral_constant<int, 3>(), ring[7], pgrp[1]); load_page(refill[7], ring[7]);
        pgrp[0] = next[0];
        pgrp[1] = next[1];
    }
    // Fewer than kRingPages full pages and the partial page remain.
#pragma unroll
    for (int r = 0; r < kRingPages; ++r) {
        const int q = pg + r;
        if (q < pages) {
            const f4v& pv = pgrp[r >> 2];
            if (q < full_pages) {
                switch (r & 3) {
                case 0: add_page(std::integral_constant<int, 0>(), ring[r], pv); break;
                case 1: add_page(std::integral_constant<int, 1>(), ring[r], pv); break;
                case 2: add_page(std::integral_constant<int, 2>(), ring[r], pv); break;
                default: add_page(std::integral_constant<int, 3>(), ring[r], pv); break;
                }
            } else {
                const int n = len - 16 * q;
#pragma unroll
                for (int t = 0; t < 16; ++t)
                    if (t < n)
                        acc = acc + mul_bcast_at(4 * (r & 3) + (t >> 2), lane4v(pv, t & 3), lane4(ring[r][t >> 2], t & 3));
            }
        }
    }
    out[quad_index(row, (kvh * G + wave) * 64 + lane, ldo)] = acc;
}

// A launch that records `start` as the kernel begins and `stop` as it ends
// (events carried by the dispatch itself, so timing adds no packets to the
// stream), or a plain launch when both are null.
template <typename... P, typename... A>
void launch_timed(void (*kernel)(P...), dim3 grid, dim3 block, hipStream_t s, hipEvent_t start, hipEvent_t stop,
                  A... args) {
    if (start || stop)
        hipExtLaunchKernelGGL(kernel, grid, block, 0, s, start, stop, 0, args...);
    else
        kernel<<<grid, block, 0, s>>>(args...);
}

hipError_t launch_fused_decode(hipStream_t s, const float* qkv, int ldq, int heads, int kv_heads,
                               const RowMeta& meta, const PagedKv& kv, int layer, float* out, int ldo,
                               const AttentionWork& w, const RopeTables& rope, const LaunchEvents& ev) {
    launch_timed(attn_scores_kernel<16, 64, true>, dim3(w.items_count, kv_heads), dim3(kScoreChunk), s, ev.start,
                 nullptr, qkv, ldq, heads, kv_heads, 64, meta, kv, layer, w, rope);
    const dim3 grid(w.blocks_count, kv_heads);
    switch (heads / kv_heads) {
    case 1: launch_timed(attn_decode_kernel<1>, grid, dim3(kFusedThreads), s, nullptr, ev.stop, heads, meta, kv, layer, w, out, ldo); break;
    case 2: launch_timed(attn_decode_kernel<2>, grid, dim3(kFusedThreads), s, nullptr, ev.stop, heads, meta, kv, layer, w, out, ldo); break;
    case 3: launch_timed(attn_decode_kernel<3>, grid, dim3(kFusedThreads), s, nullptr, ev.stop, heads, meta, kv, layer, w, out, ldo); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int BT, int DIM>
hipError_t launch_pair(hipStream_t s, const float* qkv, int ldq, int heads, int kv_heads, int dim,
                       const RowMeta& meta, const PagedKv& kv, int layer, float* out, int ldo,
                       const AttentionWork& w, bool decode, const LaunchEvents& ev) {
    launch_timed(attn_scores_kernel<BT, DIM>, dim3(w.items_count, kv_heads), dim3(kScoreChunk), s, ev.start, nullptr,
                 qkv, ldq, heads, kv_heads, dim, meta, kv, layer, w, RopeTables{nullptr, nullptr});
    const int group = heads / kv_heads;
    const int block_rows = attention_row_block(heads, kv_heads, dim);
    const dim3 wg(64);
    if (decode) {
        launch_timed(attn_pv_kernel<BT, DIM, 1>, dim3(w.blocks_count, kv_heads, group), wg, s, nullptr, ev.stop, heads,
                     kv_heads, dim, meta, kv, layer, w, out, ldo);
    } else {
        const dim3 grid(w.blocks_count, kv_heads, block_rows);
        switch (group) {
        case 2: launch_timed(attn_pv_kernel<BT, DIM, 2>, grid, wg, s, nullptr, ev.stop, heads, kv_heads, dim, meta, kv, layer, w, out, ldo); break;
        case 3: launch_timed(attn_pv_kernel<BT, DIM, 3>, grid, wg, s, nullptr, ev.stop, heads, kv_heads, dim, meta, kv, layer, w, out, ldo); break;
        case 4: launch_timed(attn_pv_kernel<BT, DIM, 4>, grid, wg, s, nullptr, ev.stop, heads, kv_heads, dim, meta, kv, layer, w, out, ldo); break;
        default:
            launch_timed(attn_pv_kernel<BT, DIM, 1>, dim3(w.blocks_count, kv_heads, block_rows * group), wg, s, nullptr,
                         ev.stop, heads, kv_heads, dim, meta, kv, layer, w, out, ldo);
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

hipError_t launch_attention(hipStream_t s, float* qkv, int ldq, int rows, int heads, int kv_heads, int dim,
                            const RowMeta& meta, const PagedKv& kv, int layer, float* out, int ldo,
                            const AttentionWork& w, bool decode, const RopeTables& rope, const LaunchEvents& ev) {
    if (rows <= 0 || w.blocks_count <= 0) return hipSuccess;
    const int group = heads / kv_heads;
    if (group > kMaxRowHeads || dim % 4 || dim > kMaxDim || kv.block_tokens % 4 ||
        kv.table_stride > kMaxTable)
        return hipErrorInvalidValue;
    // Decode rows of 16-token pages, head dim 64, at most 3 query heads per
    // KV head and contexts up to kFusedMaxT (stride = longest context
    // rounded up to 16): one fused kernel.
    if (decode && kv.block_tokens == 16 && dim == 64 && group <= 3 && w.stride <= kFusedMaxT)
        return launch_fused_decode(s, qkv, ldq, heads, kv_heads, meta, kv, layer, out, ldo, w, rope, ev);
    const hipError_t e = launch_rope_append(s, qkv, ldq, rows, heads, kv_heads, dim, rope.cos, rope.sin, meta, kv, layer);
    if (e != hipSuccess) return e;
    if (kv.block_tokens == 16 && dim == 64)
        return launch_pair<16, 64>(s, qkv, ldq, heads, kv_heads, dim, meta, kv, layer, out, ldo, w, decode, ev);
    return launch_pair<0, 0>(s, qkv, ldq, heads, kv_heads, dim, meta, kv, layer, out, ldo, w, decode, ev);
}

}  // namespace mphip
