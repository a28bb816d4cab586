// Decode attention of the fast arithmetic mode: flash-decoding over the
// paged pools. The reference computes each (row, head) with an explicit
// two-pass softmax and sequential sums (llama_runner.cpp:85-93); here the
// context is cut into page-aligned splits (fast_attention_split: 128
// tokens, 256 in rows of more than 4,096; a row of up to 256 tokens in 8
// splits), each split keeps
// a running maximum, denominator and weighted sum per query head, and the
// splits are combined at the end (the order of the floating-point sums
// differs; the result matches the reference within 1e-4 absolute on the
// reference's scale of inputs). The splits depend on nothing but the row,
// so a row's result does not depend on the rest of the batch.
//
// One wavefront per work item (row, KV head, split: the item carries the
// row's table slot beside the KV head and the row's sequence, whose index
// places the split's partial results), four items per work-group; the
// wavefront serves the G query heads of the KV head, so each K and V byte
// is read once. It walks the split's (up to 16) pages with two pages in
// flight in a ring of registers: the loads of page k+2 are issued as soon
// as page k has been used (with 2,000-3,000 wavefronts in flight a third
// page only deepens the queues at HBM). Per page (16 tokens of one layer
// and KV head, 4 KB of K then 4 KB of V, device page order of layout.h):
//  - scores: lane = (token t = lane/4, quarter dq = lane%4 of the 64 dims);
//    a lane reads 4 float4 of K (dims 16dq..16dq+15 of token t, the 16 lanes
//    of one float4 index forming a 256-byte run) and the four quarters are
//    summed across lanes;
//  - output: lane = dim d; a lane reads 4 float4 of V (4 tokens each for
//    its d, a 1 KB run per float4 index) and the page's probabilities from
//    LDS (written by one lane per token, read back as a broadcast).
// Cross-lane sums and maxima use DPP and lane reads (lanes.h). The softmax
// keeps a reference maximum per head that is raised only when a score
// exceeds it by more than 16 (probabilities then stay below e^16 and the
// sums are rescaled), so most pages need no cross-lane maximum.
// Whole splits (8 or 16 pages; 2 for a short row's 32-token splits) run the
// page loop compiled for their page count, which loads exactly their pages.
// A row's last split, of any length, keeps every load unconditional, so that
// each page's wait counts a fixed number of later loads: its loads past the
// last page re-read that page. Rows of up to 256 tokens (at most 8 splits)
// run as one work-group per (row, KV head) that combines its splits in LDS;
// the splits of longer rows write partials that a merge kernel combines.
// (Combining in the last split to finish costs each split a store
// completion and an atomic round trip at its end, more than the extra
// launch; with a device-scope release fence it would also write back the
// whole L2 on this chip.)
#include <algorithm>

#include "kernels.h"
#include "lanes.h"
#include "layout.h"

// The fast mode's own summation order: multiply-adds may be fused.
#pragma clang fp contract(fast)

namespace mphip {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kDim = 64;
constexpr int kPage = 16;
constexpr int kMaxGroup = 4;
constexpr int kSplitPages = 8;   // splits of a short row (wavefronts of its work-group)
constexpr int kMaxPages = 16;    // pages of one split
constexpr int kRing = 2;                           // pages in flight per wavefront
constexpr int kItemsPerGroup = 4;
constexpr int kMergeHeld = 16;  // splits per lane group whose partials the merge loads in one round
constexpr float kScale = 0.125f;  // 1/sqrt(64)
constexpr float kRescale = 16.0f;  // probabilities stay below e^16 before a rescale

// Activation addressing: the forward's row-tile quad layout (layout.h), or
// plain row-major rows (the stand-alone entry point).
template <bool PLAIN>
__device__ __forceinline__ size_t act_index(int row, int column, int width) {
    return PLAIN ? (size_t)row * width + column : quad_index(row, column, width);
}

// Slice `touch` (8 KB) of the weights to prefetch: lane i reads one dword
// of line i (128 bytes) of the slice; slices past the ranges read nothing.
__device__ __forceinline__ float touch_weights(const FastAttentionWork& w, uint64_t touch, int lane) {
    uint64_t at = (touch * 64 + lane) * 128;
    const char* line = nullptr;
#pragma unroll
    for (int r = 0; r < FastAttentionWork::kPrefetchRanges; ++r) {
        if (!line && at < w.prefetch_bytes[r]) line = reinterpret_cast<const char*>(w.prefetch[r]) + at;
        if (!line) at -= w.prefetch_bytes[r];
    }
    return line ? *reinterpret_cast<const float*>(line) : 0.0f;
}

// One split: tokens t0..t0+n-1 (t0 page-aligned, at most kMaxPages pages)
// of the row whose page ids are `table` (its page table, or the page ids a
// short item carries), for the G query heads of KV head
// kvh. Gives per head the reference maximum m, the denominator l and lane
// d's weighted sum acc (not yet divided). `touch` numbers this wavefront's
// 8 KB slice of the weight prefetch; p_s is the wavefront's own LDS.
// NP > 0: the split is NP whole pages (n == NP * kPage), so the ring loads
// exactly its pages. NP == 0: any split; the ring's loads are unconditional
// (so that each page's wait counts a fixed number of later loads), and those
// past the split's last page re-read it -- two page loads per wavefront that
// the whole-page variants avoid.
template <int G, bool PLAIN, int NP = 0>
__device__ __forceinline__ void attend_split(const float* __restrict__ qkv, int ldq, const PagedKv& kv, int layer,
                                             const FastAttentionWork& w, const int32_t* table, int row, int kvh,
                                             int t0, int n, uint64_t touch, float (&p_s)[G][kPage], float (&m)[G],
                                             float (&l)[G], float (&acc)[G]) {
    const int lane = threadIdx.x & 63;
    const int t = lane >> 2, dq = lane & 3;
    const int end = t0 + n;           // tokens t0..end-1 (t0 page-aligned)
    const int first = t0 / kPage;     // the split's first page
    static_assert(NP >= 0 && NP <= kMaxPages && (NP == 0 || NP >= kRing), "whole-page splits fill the ring");
    constexpr int kPages = NP > 0 ? NP : kMaxPages;  // iterations of the page loop
    const int np = NP > 0 ? NP : (end + kPage - 1) / kPage - first;  // 1..kMaxPages
    int page_id[kMaxPages];
#pragma unroll
    for (int k = 0; k < kPages; ++k) page_id[k] = table[first + (NP > 0 ? k : min(k, np - 1))];
    const size_t head_base = (size_t)kvh * kPage * kDim;  // floats into a page-layer span
    f4 kb[kRing][4], vb[kRing][4];
    auto load = [&](int k, f4 (&kk)[4], f4 (&vv)[4]) {
        const size_t base = kv_page_base(page_id[k], layer, kv.layers, kPage, kv.kv_width) + head_base;
        const f4* kp = reinterpret_cast<const f4*>(kv.keys + base);
        const f4* vp = reinterpret_cast<const f4*>(kv.values + base);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            kk[j] = __builtin_nontemporal_load(kp + (dq * 4 + j) * kPage + t);
            vv[j] = __builtin_nontemporal_load(vp + j * kDim + lane);
        }
    };
    // q of the group's heads, dims 16dq..16dq+15 (rotated); loaded before
    // the pages, as loads complete in order.
    f4 q[G][4];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = (kvh * G + h) * kDim + dq * 16 + j * 4;
            q[h][j] = *reinterpret_cast<const f4*>(qkv + act_index<PLAIN>(row, c, ldq));
        }
    __builtin_amdgcn_sched_barrier(0);
    const float touched = touch_weights(w, touch, lane);
#pragma unroll
    for (int k = 0; k < kRing; ++k) load(k, kb[k], vb[k]);
    // Keep the loads where they are: the scheduler would otherwise sink
    // them to their first use and take the pages out of flight.
    __builtin_amdgcn_sched_barrier(0);
    // Per head: the reference maximum m (uniform), this lane's share of the
    // denominator (the probabilities of its token; quad-uniform) and lane
    // d's output. Probabilities are exp(s - m) with m raised only when a
    // score exceeds it by more than kRescale (then the sums are rescaled),
    // so a page costs no cross-lane maximum unless the scores climb.
    float lp[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        lp[h] = 0.0f;
        acc[h] = 0.0f;
    }
#pragma unroll
    for (int k = 0; k < kPages; ++k) {
        if (NP == 0 && k > 0 && k >= np) break;  // np >= 1
        f4(&kc)[4] = kb[k % kRing];
        f4(&vc)[4] = vb[k % kRing];
        const int tok0 = (first + k) * kPage;
        const bool valid = tok0 + t < end;
        float s[G];
#pragma unroll
        for (int h = 0; h < G; ++h) {
            // Four independent chains (one per float4), then their sum.
            float dj[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                dj[j] = q[h][j].x * kc[j].x;
                dj[j] += q[h][j].y * kc[j].y;
                dj[j] += q[h][j].z * kc[j].z;
                dj[j] += q[h][j].w * kc[j].w;
            }
            const float d = quad_sum((dj[0] + dj[1]) + (dj[2] + dj[3]));  // token t's score in its four lanes
            s[h] = valid ? d * kScale : -__builtin_inff();
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
            if (k == 0) {
                m[h] = rows_max(row_quads_max(s[h]));  // finite: the first page holds a valid token
            } else if (__builtin_amdgcn_ballot_w64(s[h] > m[h] + kRescale)) {
                const float m_new = fmaxf(m[h], rows_max(row_quads_max(s[h])));
                const float keep = __expf(m[h] - m_new);
                lp[h] *= keep;
                acc[h] *= keep;
                m[h] = m_new;
            }
            const float p = valid ? __expf(s[h] - m[h]) : 0.0f;
            lp[h] += p;
            if (dq == 0) p_s[h][t] = p;
        }
        // Slots past the context (last page only) hold stale values: they
        // take no part, whatever they are.
        f4 v[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) v[g] = vc[g];
        if (tok0 + kPage > end) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int tok = tok0 + 4 * g;
                if (tok + 0 >= end) v[g].x = 0.0f;
                if (tok + 1 >= end) v[g].y = 0.0f;
                if (tok + 2 >= end) v[g].z = 0.0f;
                if (tok + 3 >= end) v[g].w = 0.0f;
            }
        }
        __builtin_amdgcn_wave_barrier();
        // Lane d: sum over the page's tokens of p_t * V[t][d], p read back
        // from LDS as four float4 (the same address in every lane).
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float ag[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f4 pv = reinterpret_cast<const f4*>(p_s[h])[g];
                ag[g] = pv.x * v[g].x;
                ag[g] += pv.y * v[g].y;
                ag[g] += pv.z * v[g].z;
                ag[g] += pv.w * v[g].w;
            }
            acc[h] += (ag[0] + ag[1]) + (ag[2] + ag[3]);
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if (k + kRing < kPages) load(k + kRing, kb[k % kRing], vb[k % kRing]);
        __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("" ::"v"(touched));  // the prefetch's value is not used
#pragma unroll
    for (int h = 0; h < G; ++h) l[h] = rows_sum(row_quads_sum(lp[h]));  // each token once
}

// Splits of rows of more than 256 tokens, one wavefront per work item.
template <int G, bool PLAIN>
__global__ __launch_bounds__(kItemsPerGroup * 64) void fast_attention_kernel(const float* __restrict__ qkv, int ldq,
                                                                             RowMeta meta, PagedKv kv, int layer,
                                                                             FastAttentionWork w,
                                                                             float* __restrict__ out, int ldo) {
    const int lane = threadIdx.x & 63;
    __shared__ float p_s[kItemsPerGroup][G][kPage];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int index = blockIdx.x * kItemsPerGroup + wave;
    // The item (within the list's capacity) and, for a launch that a graph
    // replays, the step's count from device memory are loaded together.
    int4 item = {0, 0, 0, 0};
    if (index < w.items_capacity) item = reinterpret_cast<const int4*>(w.items)[index];
    if (index >= (w.counts ? w.counts[0] : w.items_count)) {
        // A wavefront past the items (batches with few splits) only touches
        // its slice of the weights to prefetch.
        const float touched = touch_weights(w, (uint64_t)index, lane);
        asm volatile("" ::"v"(touched));
        return;
    }
    const int row = item.x, kvh = item.y % w.kv_heads, seq = item.z;
    const int n = item.w & 0x1FF, sp = (item.w >> 9) & 0x7FFF, t0 = sp << (item.w >> 24);
    const int32_t* table = kv.tables + (size_t)(item.y / w.kv_heads) * kv.table_stride;
    float m[G], l[G], acc[G];
    // Whole 128- and 256-token splits (all but each row's last) take the
    // variants that load exactly their pages.
    const int pages = __builtin_amdgcn_readfirstlane(n == 8 * kPage ? 8 : n == 16 * kPage ? 16 : 0);
    if (pages == 8)
        attend_split<G, PLAIN, 8>(qkv, ldq, kv, layer, w, table, row, kvh, t0, n, (uint64_t)index, p_s[wave], m, l, acc);
    else if (pages == 16)
        attend_split<G, PLAIN, 16>(qkv, ldq, kv, layer, w, table, row, kvh, t0, n, (uint64_t)index, p_s[wave], m, l, acc);
    else
        attend_split<G, PLAIN>(qkv, ldq, kv, layer, w, table, row, kvh, t0, n, (uint64_t)index, p_s[wave], m, l, acc);
    const size_t slot = ((size_t)seq * w.kv_heads + kvh) * w.split_stride + sp;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const size_t at = slot * G + h;
        w.partial_out[at * kDim + lane] = acc[h];
        if (lane == 0) {
            w.partial_ml[at * 2] = m[h];
            w.partial_ml[at * 2 + 1] = l[h];
        }
    }
}

// Rows of up to 256 tokens (fast_attention_short: at most kSplitPages
// splits of 16 or 32 tokens): one work-group per (row, KV head) of
// w.short_items, wavefront s takes split s, and the splits are combined
// through LDS in split order by one wavefront per query head, so these
// rows need no merge launch. A row of one split gives acc / l exactly.
template <int G, bool PLAIN>
__global__ __launch_bounds__(kSplitPages * 64) void fast_attention_short_kernel(const float* __restrict__ qkv,
                                                                                int ldq, RowMeta meta, PagedKv kv,
                                                                                int layer, FastAttentionWork w,
                                                                                float* __restrict__ out, int ldo) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    __shared__ float p_s[kSplitPages][G][kPage];
    __shared__ float part_ml[kSplitPages][G][2];
    __shared__ float part_acc[kSplitPages][G][kDim];
    // (row, slot * kv_heads + KV head, tokens, 0, page ids): the length and
    // the pages ride in the item, loaded together with the count, so the
    // pages' loads depend on one load only.
    const int32_t* it = w.short_items + (size_t)min((int)blockIdx.x, w.short_capacity - 1) * kShortItemInts;
    int4 item = reinterpret_cast<const int4*>(it)[0];
    if ((int)blockIdx.x >= w.short_capacity) item = {0, 0, 1, 0};
    if ((int)blockIdx.x >= (w.counts ? w.counts[1] : w.short_count)) {
        // A work-group past the items (small batches, whose items leave
        // most CUs idle) only touches its slices of the weights to prefetch.
        const float touched = touch_weights(w, (uint64_t)blockIdx.x * kSplitPages + wave, lane);
        asm volatile("" ::"v"(touched));
        return;
    }
    const int row = item.x, kvh = item.y % w.kv_heads, length = item.z;
    const int32_t* table = it + 4;
    const int split = fast_attention_split(length);
    const int splits = (length + split - 1) / split;  // 1..kSplitPages
    if (wave < splits) {
        float m[G], l[G], acc[G];
        const int t0 = wave * split;
        const int n = min(split, length - t0);
        const uint64_t touch = (uint64_t)blockIdx.x * kSplitPages + wave;
        if (n == 2 * kPage)  // whole 32-token splits: exactly their two pages
            attend_split<G, PLAIN, 2>(qkv, ldq, kv, layer, w, table, row, kvh, t0, n, touch, p_s[wave], m, l, acc);
        else
            attend_split<G, PLAIN>(qkv, ldq, kv, layer, w, table, row, kvh, t0, n, touch, p_s[wave], m, l, acc);
#pragma unroll
        for (int h = 0; h < G; ++h) {
            part_acc[wave][h][lane] = acc[h];
            if (lane == 0) {
                part_ml[wave][h][0] = m[h];
                part_ml[wave][h][1] = l[h];
            }
        }
    }
    __syncthreads();
    if (wave >= G) return;
    // Query head h: lane s < splits holds split s's (maximum, denominator)
    // (all in the first 16-lane row), lane d sums its dimension over the
    // splits in order.
    const int h = wave;
    const bool mine = lane < splits;
    const int sl = min(lane, kSplitPages - 1);
    const float ms = mine ? part_ml[sl][h][0] : -__builtin_inff();
    const float ls = mine ? part_ml[sl][h][1] : 0.0f;
    float mx = fmaxf(ms, dpp<kDppQuadXor1>(ms));
    mx = fmaxf(mx, dpp<kDppQuadXor2>(mx));
    mx = lane_value(row_quads_max(mx), 0);
    const float f = mine ? (splits == 1 ? 1.0f : __expf(ms - mx)) : 0.0f;
    const float den = lane_value(row_sum(ls * f), 0);
    float num = 0.0f;
#pragma unroll
    for (int s = 0; s < kSplitPages; ++s)
        if (s < splits) num += part_acc[s][h][lane] * lane_value(f, s);
    out[act_index<PLAIN>(row, (kvh * G + h) * kDim + lane, ldo)] = num / den;
}

// out[row][h*64 + d] for the listed rows (w.merge_rows: one-token rows of
// more than 256 tokens, with their sequences): the splits of (row, h/G)
// combined. One wavefront
// per (row, head), as four groups of 16 lanes: lane 16g + c holds dims
// 4c..4c+3, and group g takes splits g,
// g+4, g+8, ... with its own running maximum, denominator and weighted sum,
// kMergeHeld splits' partials loaded per round (a row of up to 64 splits,
// 16k tokens in 256-token splits, takes one round of loads). The four
// groups are then rescaled to the common maximum and summed as
// (g0 + g1) + (g2 + g3). The order depends on nothing but the row's split
// count. The row's list entry carries its split count, so the first round
// of loads depends on that one load only and reads no slot past the row's
// splits.
template <bool PLAIN>
__global__ __launch_bounds__(256) void fast_attention_merge_kernel(int heads, int kv_heads, RowMeta meta,
                                                                   FastAttentionWork w, float* __restrict__ out,
                                                                   int ldo) {
    const int lane = threadIdx.x & 63;
    const int pair = blockIdx.x * 4 + (threadIdx.x >> 6);
    int4 rs = {0, 0, 1, 0};  // row, sequence, splits
    if (pair / heads < w.merge_capacity) rs = reinterpret_cast<const int4*>(w.merge_rows)[pair / heads];
    if (pair >= (w.counts ? w.counts[2] : w.merge_count) * heads) return;
    const int row = rs.x, h = pair % heads, splits = rs.z;
    const int G = heads / kv_heads, kvh = h / G, hg = h % G;
    const int grp = lane >> 4, c = lane & 15;
    const size_t slot0 = ((size_t)rs.y * kv_heads + kvh) * w.split_stride;  // split 0 of (sequence, kvh)
    auto at = [&](int sp) { return (slot0 + sp) * G + hg; };
    float gm = -__builtin_inff(), gl = 0.0f;
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    float mv[kMergeHeld] = {}, lv[kMergeHeld] = {};
    f4 ov[kMergeHeld] = {};
    // Round r: this group's splits grp + 4(r*kMergeHeld + j) for the j whose
    // split of group 0 is below `count` (a wave-uniform bound), clamped to
    // split count - 1 (loads past the row's splits are not used).
    auto load = [&](int r, int count) {
#pragma unroll
        for (int j = 0; j < kMergeHeld; ++j) {
            if (4 * (r * kMergeHeld + j) >= count) break;
            const int sp = min(grp + 4 * (r * kMergeHeld + j), count - 1);
            mv[j] = w.partial_ml[at(sp) * 2];
            lv[j] = w.partial_ml[at(sp) * 2 + 1];
            ov[j] = reinterpret_cast<const f4*>(w.partial_out + at(sp) * kDim)[c];
        }
    };
    auto combine = [&](int r, int splits) {
        float rm = gm;
#pragma unroll
        for (int j = 0; j < kMergeHeld; ++j)
            if (grp + 4 * (r * kMergeHeld + j) < splits) rm = fmaxf(rm, mv[j]);
        // 0 when the group's first splits arrive, 1 while it has none (its sums are 0).
        const float keep = gm == rm ? 1.0f : __expf(gm - rm);
        gl *= keep;
        acc *= keep;
#pragma unroll
        for (int j = 0; j < kMergeHeld; ++j) {
            const bool valid = grp + 4 * (r * kMergeHeld + j) < splits;
            const float f = valid ? __expf(mv[j] - rm) : 0.0f;
            gl = valid ? gl + lv[j] * f : gl;
            acc = valid ? acc + ov[j] * f : acc;
        }
        gm = rm;
    };
    load(0, splits);
    combine(0, splits);
    for (int r = 1; 4 * r * kMergeHeld < splits; ++r) {
        load(r, splits);
        combine(r, splits);
    }
    // Groups to the common maximum (group 0 holds split 0, so it is finite).
    float m = fmaxf(gm, __shfl_xor(gm, 16));
    m = fmaxf(m, __shfl_xor(m, 32));
    const float f = __expf(gm - m);
    float den = gl * f;
    f4 num = acc * f;
    den += __shfl_xor(den, 16);
    den += __shfl_xor(den, 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        num[i] += __shfl_xor(num[i], 16);
        num[i] += __shfl_xor(num[i], 32);
    }
    if (grp == 0) *reinterpret_cast<f4*>(out + act_index<PLAIN>(row, h * kDim + 4 * c, ldo)) = num / den;
}

// Grids: the step's counts, or with w.capacity_grids the capacities of the
// lists this step uses (a launch captured once for the steps of one shape,
// whose lists are empty or not alike; the kernels read each step's counts
// from w.counts).
template <int G, bool PLAIN>
void launch_items(hipStream_t s, const float* qkv, int ldq, const RowMeta& meta, const PagedKv& kv, int layer,
                  const FastAttentionWork& w, float* out, int ldo) {
    // Slices of 8 KB (one per wavefront) that cover the weights to prefetch.
    uint64_t bytes = 0;
    for (int r = 0; r < FastAttentionWork::kPrefetchRanges; ++r) bytes += w.prefetch_bytes[r];
    const uint64_t slices = (bytes + 64 * 128 - 1) / (64 * 128);
    const int items = w.capacity_grids && w.items_count > 0 ? w.items_capacity : w.items_count;
    const int shorts = w.capacity_grids && w.short_count > 0 ? w.short_capacity : w.short_count;
    if (shorts > 0) {
        // Without split items (whose launch covers the slices), enough
        // work-groups for every slice.
        int groups = shorts;
        if (items <= 0)
            groups = (int)std::max<uint64_t>((uint64_t)groups, (slices + kSplitPages - 1) / kSplitPages);
        fast_attention_short_kernel<G, PLAIN><<<groups, kSplitPages * 64, 0, s>>>(qkv, ldq, meta, kv, layer, w, out, ldo);
    }
    if (items > 0) {
        const uint64_t waves = std::max<uint64_t>((uint64_t)items, slices);
        fast_attention_kernel<G, PLAIN><<<(int)((waves + kItemsPerGroup - 1) / kItemsPerGroup), kItemsPerGroup * 64, 0,
                                   s>>>(qkv, ldq, meta, kv, layer, w, out, ldo);
    }
}

template <bool PLAIN>
hipError_t launch_all(hipStream_t s, const float* qkv, int ldq, int heads, int kv_heads, const RowMeta& meta,
                      const PagedKv& kv, int layer, float* out, int ldo, const FastAttentionWork& w) {
    switch (heads / kv_heads) {
    case 1: launch_items<1, PLAIN>(s, qkv, ldq, meta, kv, layer, w, out, ldo); break;
    case 2: launch_items<2, PLAIN>(s, qkv, ldq, meta, kv, layer, w, out, ldo); break;
    case 3: launch_items<3, PLAIN>(s, qkv, ldq, meta, kv, layer, w, out, ldo); break;
    default: launch_items<4, PLAIN>(s, qkv, ldq, meta, kv, layer, w, out, ldo); break;
    }
    hipError_t e = hipGetLastError();
    const int merges = w.capacity_grids && w.merge_count > 0 ? w.merge_capacity : w.merge_count;
    if (e != hipSuccess || w.items_count <= 0 || merges <= 0) return e;
    fast_attention_merge_kernel<PLAIN><<<(merges * heads + 3) / 4, 256, 0, s>>>(heads, kv_heads, meta, w, out, ldo);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_fast_attention(hipStream_t s, const float* qkv, int ldq, int rows, int heads, int kv_heads,
                                 const RowMeta& meta, const PagedKv& kv, int layer, float* out, int ldo,
                                 const FastAttentionWork& w, bool plain) {
    const int G = heads / kv_heads;
    if (rows <= 0) return hipSuccess;
    if (kv.block_tokens != kPage || kv.kv_width != kv_heads * kDim || G > kMaxGroup || G < 1 ||
        G * kv_heads != heads || w.kv_heads != kv_heads || (w.items_count > 0 && w.split_stride < w.max_splits) ||
        (w.capacity_grids && !w.counts) || w.items_count > w.items_capacity || w.short_count > w.short_capacity ||
        w.merge_count > w.merge_capacity)
        return hipErrorInvalidValue;
    return plain ? launch_all<true>(s, qkv, ldq, heads, kv_heads, meta, kv, layer, out, ldo, w)
                 : launch_all<false>(s, qkv, ldq, heads, kv_heads, meta, kv, layer, out, ldo, w);
}

}  // namespace mphip
