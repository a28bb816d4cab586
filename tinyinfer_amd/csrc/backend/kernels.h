// Launchers for the gfx950 kernels of the MiniPrefix device forward.
// All launchers enqueue on `stream` and return hipGetLastError().
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

enum Epilogue { kStore = 0, kResidual = 1, kSwiglu = 2 };

hipError_t launch_embed(hipStream_t s, const float* embedding, const int32_t* tokens, float* x,
                        int rows, int hidden);

// out[r] = (x[r]*scale_r)*w with scale_r = 1/sqrt(sequential sum of squares/width + eps);
// row r reads x row row_map[r] when row_map is non-null.
hipError_t launch_rms(hipStream_t s, const float* x, int ldx, const int32_t* row_map,
                      const float* weight, float* out, int ldo, int rows, int width, float eps);

// out[r][n] = epilogue(sum_k x[r][k]*w[k][n]) with k accumulated in order,
// multiply and add rounded separately. kResidual adds into out; kSwiglu
// combines the chains of w and w2 as (g/(1+exp(-g)))*u.
hipError_t launch_gemm(hipStream_t s, Epilogue epilogue, const float* x, int ldx, int rows,
                       int inner, const float* w, const float* w2, int columns, int ldw,
                       float* out, int ldo);

// Split-half RoPE of q and k (from host-computed cos/sin tables) for every
// row, in place for q, and the row's rotated K and its V written into the
// pools through the page table.
hipError_t launch_rope_append(hipStream_t s, float* qkv, int ldqkv, int rows, int heads,
                              int kv_heads, int dim, const float* cos_table,
                              const float* sin_table, const RowMeta& meta, const PagedKv& kv,
                              int layer);

// Causal GQA attention for every row in the reference two-pass softmax
// order. q rows at qkv (stride ldq); out rows stride ldo. Rows are grouped
// in `blocks` row blocks (first row, row count): consecutive positions of
// one sequence, at most attention_row_block() rows each. Scratch holds
// rows*heads score rows of `stride` floats (max length padded to 16) and
// rows*heads*chunks chunk maxima (chunks = ceil(max length / 256)).
struct AttentionScratch {
    float* scores;
    float* chunk_max;
    int stride;
    int chunks;
    const int2* row_blocks;
    int blocks;
};
int attention_row_block(int heads, int kv_heads, int dim);
hipError_t launch_attention(hipStream_t s, const float* qkv, int ldq, int rows, int heads,
                            int kv_heads, int dim, const RowMeta& meta, const PagedKv& kv,
                            int layer, float* out, int ldo, const AttentionScratch& scratch);
// Stand-alone single-row variant over a caller page table.
hipError_t launch_attention_single(hipStream_t s, const float* q, const float* keys,
                                   const float* values, const int32_t* table, int length,
                                   int layer, int layers, int block_tokens, int heads,
                                   int kv_heads, int dim, float* out, float* scratch);
// Score floats per row that fit in LDS.
constexpr int kAttentionLdsScores = 10240;

// First index of the maximum of each row of logits (std::max_element), and
// per row a flag: 1 when any value of the row is not finite, else 0.
hipError_t launch_argmax(hipStream_t s, const float* logits, int rows, int vocabulary,
                         int32_t* argmax, int32_t* nonfinite);

// Copies a strided region inside both pools (rows x width floats, pitch apart).
hipError_t launch_copy_region(hipStream_t s, float* keys, float* values, uint64_t destination,
                              uint64_t source, uint64_t pitch, uint64_t width, uint64_t rows);

// dst[c][r] = src[r][c] for a rows x cols matrix.
hipError_t launch_transpose(hipStream_t s, const float* src, float* dst, int rows, int cols);

}  // namespace mphip
