// Device data layouts of the MiniPrefix forward.
//
// Activations (the residual stream, normalized rows, q|k|v, attention
// context, SwiGLU output) use a "row-tile quad" layout so that a wavefront
// whose lanes are 64 consecutive rows reads 4 consecutive columns of every
// row with one coalesced 1 KB load: a matrix of R rows and W columns (W a
// multiple of 4) is ceil(R/64) row tiles; tile t is W/4 quads, quad q holds
// [64 rows][4 columns] = columns 4q..4q+3 of rows 64t..64t+63.
//
// Projection weights are stored transposed, [out][in] (each output column's
// weights contiguous along k), so a wavefront that owns one output column
// reads its weights as a broadcast. The fast arithmetic stores them (and
// the embedding, which is the tied LM head) in the matrix cores' fragment
// order instead: for output block nb (16 outputs) and input step s (16
// inputs), fragment nb * (in/16) + s is 64 float4, float4 l holding
// W[16nb + l%16][16s + 4(l/16) .. 16s + 4(l/16) + 3], the B operand of lane
// l for the four 16x16x4 MFMAs of the step.
//
// K/V pages: block b of layer l starts at float (b*layers + l)*bt*kv_width,
// as in the reference pool (paged_kv.cpp:53-56), so page tables, block ids
// and copy-on-write regions keep the reference's meaning. Inside a
// (block, layer) the order differs: kv head major, then for keys
// [d/4][slot][4] (a wavefront whose lanes are consecutive tokens reads one
// float4 of d per lane as contiguous 256-byte runs) and for values
// [slot/4][d][4] (a wavefront whose lanes are the d of one head reads 4
// consecutive tokens per lane as one contiguous run of dim*16 bytes).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace mphip {

constexpr int kTileRows = 64;

__host__ __device__ __forceinline__ size_t quad_index(int row, int column, int width) {
    return ((size_t)(row >> 6) * (size_t)(width >> 2) + (size_t)(column >> 2)) * 256 +
           (size_t)((row & 63) * 4 + (column & 3));
}

// Floats of a quad-layout matrix with `rows` rows (padded to whole tiles).
__host__ __device__ __forceinline__ size_t quad_floats(int rows, int width) {
    return (size_t)((rows + 63) / 64) * 64 * (size_t)width;
}

__host__ __device__ __forceinline__ size_t kv_page_base(int block, int layer, int layers, int bt, int kv_width) {
    return ((size_t)block * layers + layer) * (size_t)bt * kv_width;
}
__host__ __device__ __forceinline__ size_t key_offset(int slot, int kv_head, int d, int bt, int dim) {
    return (size_t)kv_head * bt * dim + (size_t)(d >> 2) * bt * 4 + (size_t)slot * 4 + (d & 3);
}
__host__ __device__ __forceinline__ size_t value_offset(int slot, int kv_head, int d, int bt, int dim) {
    return (size_t)kv_head * bt * dim + (size_t)(slot >> 2) * dim * 4 + (size_t)d * 4 + (slot & 3);
}

}  // namespace mphip
