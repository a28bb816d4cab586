// Launchers for the gfx950 kernels of the MiniPrefix device forward.
// All launchers enqueue on `stream` and return hipGetLastError().
// Activations use the row-tile quad layout of layout.h; projection weights
// are stored transposed ([out][in]).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace mphip {

// Per-call row metadata resident on the device. Row r of a forward call is
// token tokens[r] of sequence row_seq[r] at absolute position row_pos[r];
// sequence s reads its page table at tables + seq_slot[s]*table_stride and
// its last row is seq_last_row[s].
struct RowMeta {
    const int32_t* tokens;
    const int32_t* row_seq;
    const int32_t* row_pos;
    const int32_t* seq_slot;
    const int32_t* seq_last_row;
};

struct PagedKv {
    float* keys;
    float* values;
    const int32_t* tables;
    int32_t table_stride;  // entries per sequence table
    int32_t layers, block_tokens, kv_width;
};

// kRope is of the fast mode only (launch_fast_gemm).
enum Epilogue { kStore = 0, kResidual = 1, kSwiglu = 2, kHead = 3, kRope = 4 };

// out[r][n] = epilogue(sum_k x[r][k] * w[n][k]) with k accumulated in order
// from 0, multiply and add rounded separately. x is `rows` x `inner` (quad
// layout), w is [columns][inner]. kStore writes out (quad layout, `columns`
// wide); kResidual adds into out; kSwiglu computes (g/(1+exp(-g)))*u from the
// chains of w (g) and w2 (u); kHead writes, per row and per group of
// kHeadColumns columns, the first maximum and a non-finite flag into the
// partial arrays, and the logits row-major into `out` when it is non-null.
struct GemmArgs {
    const float* x;
    const float* w;
    const float* w2;
    float* out;
    int rows, inner, columns;
    // RMSNorm folded into the projection (launch_gemm_normed): x is the raw
    // residual stream and norm the RMSNorm weights of width `inner`.
    const float* norm;
    float eps;
    float* best_value;
    int32_t* best_index;
    int32_t* bad;
    int groups;
};
constexpr int kHeadColumns = 64;
int head_groups(int columns);
hipError_t launch_gemm(hipStream_t s, Epilogue epilogue, const GemmArgs& args);
// The same projection of RMSNorm(x) (llama_runner.cpp:10-16 then :30-36)
// in one launch where the shape allows (one row tile, inner <= 576 and a
// multiple of 64, kStore or kSwiglu); false when it does not, and nothing
// is launched.
bool gemm_normed_fits(Epilogue epilogue, const GemmArgs& args);
hipError_t launch_gemm_normed(hipStream_t s, Epilogue epilogue, const GemmArgs& args);
// argmax[r] = first index of the row maximum, nonfinite[r] = any non-finite
// logit, from the kHead partials of `args`.
hipError_t launch_head_argmax(hipStream_t s, const GemmArgs& args, int32_t* argmax, int32_t* nonfinite);

// Fast arithmetic mode (fast_gemm.hip): the same projections on FP32 matrix
// cores, in their summation order. x and out in the quad layout (kHead:
// logits row-major [rows][columns]); w (and w2, the up matrix of kSwiglu) is
// [columns][inner] in the fragment order of layout.h. inner and columns
// multiples of 16.
// - rope_columns (kStore): the first rope_columns output columns (q and k
//   of a q|k|v projection) are stored pair-permuted within each 64-wide head
//   (fast_rope_column) and are written back in natural order.
// - norm (kStore, kSwiglu, kHead): RMSNorm of x with weights `norm`; the row
//   sums of squares come from ssq_in: ssq_parts partial sums per row at
//   ssq_in[p*ssq_stride + row] (written by the producer of x).
// - kResidual: out += result, and ssq_out[c*ssq_stride + row] = sum of
//   squares of the updated row over columns 16c..16c+15.
// - kHead: row i of the result reads x row row_map[i] (row i when row_map is
//   null); per row and column group, the first maximum into
//   best_value/best_index/bad [rows][groups], logits written when `logits`
//   is non-null
//   (groups = columns/fast_head_group_columns(columns)).
// - kRope (norm required; head dim 64; columns = q|k|v of `heads` query and
//   kv.kv_width/64 KV heads, q and k columns pair-permuted as for
//   rope_columns): split-half RoPE at meta.row_pos with the
//   per-row rotation row_rope[row][64] (cos of dims 0..31, then sin) and
//   page row_block[row] (launch_embed writes both); rotated q into out (quad
//   layout), rotated k and v into the pools of `kv` at `layer` and the
//   row's position.
struct FastGemmArgs {
    const float* x;
    const float* w;
    const float* w2;
    float* out;
    int rows, inner, columns;
    const float* norm;
    float eps;
    const float* ssq_in;
    float* ssq_out;
    int ssq_parts, ssq_stride;
    const int32_t* row_map;
    float* logits;
    float* best_value;
    int32_t* best_index;
    int32_t* bad;
    int groups;
    RowMeta meta;
    PagedKv kv;
    int layer, heads;
    const int32_t* row_block;
    const float* row_rope;
    int rope_columns;
};
// Source column of stored column n of a q or k matrix whose 64-wide heads are
// pair-permuted for the fast RoPE projection: within a head, stored column
// 16b + c holds dim 8b + c%8 + 32(c/8), so each 16-column block carries 8
// whole split-half pairs (d, d + 32).
__host__ __device__ inline int fast_rope_column(int n) {
    const int h = n & ~63, b = (n >> 4) & 3, c = n & 15;
    return h + 8 * b + (c & 7) + 32 * (c >> 3);
}
bool fast_gemm_fits(const FastGemmArgs& args);
// Columns per LM-head argmax group of the fast head.
int fast_head_group_columns(int columns);
hipError_t launch_fast_gemm(hipStream_t s, Epilogue epilogue, const FastGemmArgs& args);
// Per-16-column sums of squares of x's rows (quad layout, `width` columns)
// into ssq[p*stride + row], for the first RMSNorm after the embedding.
hipError_t launch_fast_ssq(hipStream_t s, const float* x, int rows, int width, float* ssq, int stride);

// Fast-mode projections of a decode step of up to four sequences
// (fast_gemv.hip): GEMV on the vector ALU over row-major [columns][inner]
// weights, one wavefront per output (per RoPE pair for kRope). x and out are
// rows 0..rows-1 of quad-layout matrices (`inner` and `columns` wide).
// kRope: RMSNorm (weights `norm`, eps) then q|k|v of `heads` query and
// kv.kv_width/64 KV heads in natural column order, RoPE at each row's
// position (meta.row_pos[r], row_rope[r], page row_block[r]), q into out, K
// and V into the pools of `kv` at `layer`; kResidual: out += x W^T (no
// norm); kSwiglu: RMSNorm then the SwiGLU of the w (gate) and w2 (up) rows.
// Shapes: inner 576 (kRope, kSwiglu, kResidual) or 1536 (kResidual), head
// dim 64, rows 1..4. A row's result does not depend on the other rows.
struct GemvArgs {
    const float* x;
    const float* w;
    const float* w2;
    float* out;
    const float* norm;
    float eps;
    int rows, inner, columns, heads, layer;
    PagedKv kv;
    RowMeta meta;
    const int32_t* row_block;
    const float* row_rope;
};
constexpr int kGemvRows = 4;
bool gemv_fits(int hidden, int intermediate, int heads, int kv_heads);
hipError_t launch_gemv(hipStream_t s, Epilogue epilogue, const GemvArgs& args);

// Fast-mode decode attention (fast_attention.hip): every row is one new
// token (already rotated q, its K/V already in the pools). Flash-decoding
// split over the context: work item (row, KV head, split of
// fast_attention_split(length) tokens, page-aligned) computes a maximum,
// denominator and output per query head; a merge kernel combines the splits
// of every (row, head). Head dim 64, page 16.
//
// Tokens per split of a row of `length` tokens: 8 pages (128 tokens); 16
// pages (256 tokens) for rows of more than 4,096 tokens, whose merge then
// reads half as many partials (a 16k-token row: 64 splits, one round of
// loads); and for rows of up to 256 tokens the row in (at most) 8 splits of
// whole pages, so that a short row is still spread over several wavefronts
// (a small batch of short rows is bound by one wavefront's chain of pages).
// A function of the row alone: a decoding row's result does not depend on
// the rest of the batch.
__host__ __device__ inline int fast_attention_split(int length) {
    const int pages = (length + 15) / 16;
    return pages <= 16 ? 16 * ((pages + 7) / 8) : pages > 256 ? 256 : 128;
}
// Rows of up to 256 tokens (at most 8 splits) are combined inside one
// work-group; longer rows through the partials and the merge kernel.
__host__ __device__ inline bool fast_attention_short(int length) { return (length + 15) / 16 <= 16; }
constexpr int kShortItemInts = 20;
// The most splits a row that is not short has, over every length up to
// `length` (0 when every such row is short): the stride of the partial
// results per (sequence, KV head), fixed by the context limit so that the
// partials never grow during a decode.
inline int fast_attention_max_splits(int length) {
    if (fast_attention_short(length)) return 0;
    const int below = (length < 4096 ? length : 4096) + 127;  // 128-token splits up to 4,096 tokens
    const int above = length > 4096 ? (length + 255) / 256 : 0;
    return below / 128 > above ? below / 128 : above;
}
// Work item of a split (int4): row, table slot * kv_heads + KV head,
// sequence (the partials' index), tokens | split index << 9 | log2(split
// tokens) << 24 (the split's first token is split index << log2).
inline int fast_attention_item_w(int tokens, int split_index, int split_tokens) {
    int lg = 0;
    while ((1 << lg) < split_tokens) ++lg;
    return tokens | (split_index << 9) | (lg << 24);
}
struct FastAttentionWork {
    // With capacity_grids, the lists' lengths as the kernels read them:
    // device int32 [3] = split items, short items, merged rows (equal to the
    // host counts below); null otherwise (the kernels take the host counts).
    const int32_t* counts;
    // splits of the rows longer than 256 tokens (fast_attention_item_w), in
    // any order (the forward puts every row's whole splits before the
    // shorter last ones)
    const int32_t* items;
    int items_count, items_capacity;
    // per row of up to 256 tokens and KV head, kShortItemInts int32: row,
    // table slot * kv_heads + KV head, tokens, 0, then the row's page ids
    // (16; past the row's last page, its last page again), so that the
    // pages are found without a dependent load of the table
    const int32_t* short_items;
    int short_count, short_capacity;
    // the rows whose splits the merge kernel combines (the one-token rows
    // longer than 256 tokens), as (row, sequence, splits, 0) int4s
    const int32_t* merge_rows;
    int merge_count, merge_capacity;
    // Grids sized by the capacities instead of the counts (a launch that a
    // graph replays for several steps).
    bool capacity_grids;
    // Splits of the longest row (of those longer than 256 tokens; 0 if
    // none); the partial results of (sequence, KV head, split) sit at slot
    // (sequence * kv_heads + KV head) * split_stride + split, split_stride >=
    // max_splits (the merge's first round of loads is bounded by it).
    int max_splits;
    int split_stride;
    float* partial_out;  // [slot][G][64]
    float* partial_ml;   // [slot][G][2]: running maximum, denominator
    int kv_heads;
    // Weights the next projections read, touched by the attention's
    // wavefronts (one dword per 128-byte line, 8 KB per wavefront, results
    // unused) so that they are in the memory-side cache when those
    // projections run: up to kPrefetchRanges ranges of `bytes` each. A
    // launch with fewer wavefronts than slices adds wavefronts that only
    // touch, enough for all of the ranges.
    static constexpr int kPrefetchRanges = 6;
    const float* prefetch[kPrefetchRanges];
    uint64_t prefetch_bytes[kPrefetchRanges];
};
// Prefill attention of the fast mode: work items (int4) of up to 16
// consecutive rows of one sequence's chunk and one KV head: first row,
// table slot * kv_heads + KV head, position of the first row, rows. The
// rows' K/V must already be in the pools (launch_rope_append).
bool fast_prefill_fits(int heads, int kv_heads, const PagedKv& kv);
hipError_t launch_fast_prefill(hipStream_t s, const float* qkv, int ldq, int heads, int kv_heads, const PagedKv& kv,
                               int layer, const int32_t* items, int count, float* out, int ldo);
// `plain`: q rows (ldq wide) and out rows (ldo wide) are row-major instead
// of the quad layout (the stand-alone entry point).
hipError_t launch_fast_attention(hipStream_t s, const float* qkv, int ldq, int rows, int heads, int kv_heads,
                                 const RowMeta& meta, const PagedKv& kv, int layer, float* out, int ldo,
                                 const FastAttentionWork& work, bool plain = false);

// Per-row RoPE inputs of a forward for the fast q|k|v projection: for row r
// at position p = meta.row_pos[r], block[r] = the page holding p (from the
// row's sequence table) and rope[r][0..half) = cos_table[p][..],
// rope[r][half..2half) = sin_table[p][..].
struct RowRope {
    RowMeta meta;
    const int32_t* tables;
    int32_t table_stride, block_tokens, half;
    const float* cos_table;
    const float* sin_table;
    int32_t* block;
    float* rope;
};

// x = embedding rows of `tokens` (the embedding [vocab][hidden] row-major,
// or in the fragment order of layout.h when `fragments`); also clears the
// forward's device error word `error` (may be null) and fills `rope` when it
// is non-null.
hipError_t launch_embed(hipStream_t s, const float* embedding, const int32_t* tokens, float* x, int rows,
                        int hidden, int32_t* error, const RowRope* rope = nullptr, bool fragments = false);
// dst = the n_out x k_in matrix W (W[n][k]: output n, input k) in the
// fragment order of layout.h; src holds it [k_in][n_out] (in_out) or
// [n_out][k_in]. n_out and k_in are multiples of 16. With rope_heads, the
// stored output n is the source's fast_rope_column(n) (n_out a multiple of
// 64).
hipError_t launch_to_fragments(hipStream_t s, const float* src, float* dst, int n_out, int k_in, bool in_out,
                               bool rope_heads = false);

// out[r] = (x[r']*scale_r')*w with scale = 1/sqrt(sequential sum of squares/width + eps);
// r' = row_map[r] when row_map is non-null, else r.
hipError_t launch_rms(hipStream_t s, const float* x, const int32_t* row_map, const float* weight, float* out,
                      int rows, int width, float eps);

// Split-half RoPE of q and k (from host-computed cos/sin tables) for every
// row, in place for q, and the row's rotated K and its V written into the
// pools through the page table. qkv is `width` = heads*dim + 2*kv_width wide.
hipError_t launch_rope_append(hipStream_t s, float* qkv, int width, int rows, int heads, int kv_heads, int dim,
                              const float* cos_table, const float* sin_table, const RowMeta& meta,
                              const PagedKv& kv, int layer);

// Causal GQA attention for every row in the reference two-pass softmax
// order. q rows at qkv (quad layout, ldq wide); out is quad layout, ldo
// wide. Rows are grouped in row blocks (first row, row count): consecutive
// positions of one sequence, at most attention_row_block() rows each,
// ordered by decreasing attended length. `items` lists (block, 256-token
// chunk) for every chunk each block reaches. Scratch: scores
// [rows][heads][stride] (stride >= max length, multiple of 16) and chunk
// maxima [rows][heads][chunks]. `decode` = every block has one row. Head
// dim at most 64 (lane = d), at most 2048 pages per sequence.
struct AttentionWork {
    const int2* blocks;
    const int2* items;
    int blocks_count, items_count;
    float* scores;
    float* chunk_max;
    int stride, chunks;
    // Device error word (set non-zero by a kernel that had to give up a
    // bounded wait); cleared by launch_embed at the start of each forward.
    int32_t* error;
};
int attention_row_block(int heads, int kv_heads, int dim);
// Optional timing: `start` is recorded as the first kernel of a launch
// begins and `stop` as its last kernel ends (events carried by the kernel
// dispatches, adding nothing to the stream between kernels).
struct LaunchEvents {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};
// RoPE tables [position][dim/2] (cos, sin) of the rows' positions.
struct RopeTables {
    const float* cos;
    const float* sin;
};
// Attention of the rows, including RoPE of q and k and the append of the
// rows' K/V to the pools (rope_append_kernel ahead of the attention kernels,
// or folded into the scores kernel on the fused decode path). qkv is
// [rows][heads*dim + 2*kv_width] in quad layout; q may be rotated in place.
hipError_t launch_attention(hipStream_t s, float* qkv, int ldq, int rows, int heads, int kv_heads, int dim,
                            const RowMeta& meta, const PagedKv& kv, int layer, float* out, int ldo,
                            const AttentionWork& work, bool decode, const RopeTables& rope,
                            const LaunchEvents& events = LaunchEvents());
// Stand-alone single-row variant over a caller page table (plain layouts).
hipError_t launch_attention_single(hipStream_t s, const float* q, const float* keys, const float* values,
                                   const int32_t* table, int length, int layer, int layers, int block_tokens,
                                   int heads, int kv_heads, int dim, float* out, float* scratch);
// Score floats per row that fit in LDS.
constexpr int kAttentionLdsScores = 10240;

// One copy-on-write: the first `valid` token slots of page `source` into
// page `destination` (block ids), every layer, both pools.
struct TailCopy {
    int32_t destination, source, valid;
};

// `count` copies-on-write (device array), in the device page order of
// layout.h, as one launch; no copy reads or writes a page another one writes.
hipError_t launch_copy_tails(hipStream_t s, float* keys, float* values, const TailCopy* copies, int count,
                             int layers, int block_tokens, int kv_heads, int dim);

// tables[updates[i].x] = updates[i].y for i < count (queued block-table
// entries; the indices are distinct).
hipError_t launch_table_update(hipStream_t s, int32_t* tables, const int2* updates, int count);

// dst[c*ld_dst + r] = src[r*cols + c] for a rows x cols matrix.
hipError_t launch_transpose(hipStream_t s, const float* src, float* dst, int rows, int cols, int ld_dst);

}  // namespace mphip
