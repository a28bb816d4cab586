// Row-wise kernels of the MiniPrefix forward on the row-tile quad layout:
// embedding gather, RMSNorm, RoPE + paged K/V append, the copy-on-write tail
// copy and the weight transpose used at upload. Reference order:
// miniprefix/src/backend/cpu/llama_runner.cpp:10-22 (rms, rope), :71-73
// (embedding) and :81-83 (K/V write).
#include <algorithm>

#include "kernels.h"
#include "layout.h"

namespace mphip {
namespace {

// x[r][:] = E[tokens[r]][:] for rows < rows; padding rows of the last tile
// are zeroed so that later kernels only ever see finite values there.
__global__ __launch_bounds__(256) void embed_kernel(const float* __restrict__ embedding,
                                                    const int32_t* __restrict__ tokens,
                                                    float* __restrict__ x, int rows, int hidden,
                                                    int32_t* __restrict__ error, RowRope rope, bool fragments) {
    if (error && blockIdx.x == 0 && threadIdx.x == 0) *error = 0;
    if (rope.rope) {
        const int per = 2 * rope.half + 1;  // cos, sin, then the page
        for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < rows * per; i += gridDim.x * blockDim.x) {
            const int r = i / per, c = i % per;
            const int pos = rope.meta.row_pos[r];
            if (c < 2 * rope.half) {
                const float* src = c < rope.half ? rope.cos_table : rope.sin_table;
                rope.rope[(size_t)r * 2 * rope.half + c] = src[(size_t)pos * rope.half + c % rope.half];
            } else {
                const int32_t* table =
                    rope.tables + (size_t)rope.meta.seq_slot[rope.meta.row_seq[r]] * rope.table_stride;
                rope.block[r] = table[pos / rope.block_tokens];
            }
        }
    }
    const int quads = hidden >> 2;
    const size_t total = (size_t)((rows + 63) >> 6) * quads * 64;
    float4* x4 = reinterpret_cast<float4*>(x);
    const float4* e4 = reinterpret_cast<const float4*>(embedding);
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const int r_in = (int)(i & 63);
        const size_t tq = i >> 6;  // tile * quads + q
        const int q = (int)(tq % quads);
        const int row = (int)(tq / quads) * 64 + r_in;
        if (row >= rows) {
            x4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            continue;
        }
        const int t = tokens[row];
        // Fragment order: quad q of row t is the float4 of lane
        // t%16 + 16(q%4) in the (t/16, q/4) fragment.
        x4[i] = fragments ? e4[((size_t)(t >> 4) * (quads >> 2) + (q >> 2)) * 64 + (t & 15) + 16 * (q & 3)]
                          : e4[(size_t)t * quads + q];
    }
}

// out[r] = (x[src(r)] * scale) * weight with scale = 1/sqrt(sum/width + eps),
// sum = sequential float sum of squares (llama_runner.cpp:10-16).
// A work-group of kRmsWaves wavefronts per (64-row tile, column slice),
// lane = row. The row tile is taken kRmsWaves*kRmsPer quads (4 columns) at
// a time, all loads in flight together. Wavefront 0 sums its own quads
// (squares formed between the adds) while wavefronts 1.. write the squares
// of theirs to LDS; wavefront 0 then continues with adds only over the LDS
// squares (the next 8 quads read while 8 are added). Every work-group of a
// tile computes the same scales and writes only its slice of columns: from
// the wavefronts' registers when the row fits one pass
// (width <= 4*kRmsWaves*kRmsPer), else from global memory.
constexpr int kRmsWaves = 4;
constexpr int kRmsPer = 36;    // quads per wavefront per pass (144 VGPRs)
constexpr int kRmsSlices = 8;  // work-groups per row tile

__global__ __launch_bounds__(kRmsWaves * 64) void rms_kernel(const float* __restrict__ x,
                                                             const int32_t* __restrict__ row_map,
                                                             const float* __restrict__ weight,
                                                             float* __restrict__ out, int rows, int width,
                                                             float eps) {
    __shared__ float4 sq_s[(kRmsWaves - 1) * kRmsPer * 64];
    __shared__ float4 w_s[kRmsWaves * kRmsPer];
    __shared__ float scale_s[64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tile = blockIdx.x, slice = blockIdx.y;
    const int quads = width >> 2;
    const bool one_pass = quads <= kRmsWaves * kRmsPer;
    const int row = tile * 64 + lane;
    const int src = row < rows ? (row_map ? row_map[row] : row) : -1;
    const int src_c = src < 0 ? 0 : src;
    // Quad q of this lane's source row.
    const float4* xrow = reinterpret_cast<const float4*>(x) + (size_t)(src_c >> 6) * quads * 64 + (src_c & 63);
    const float4* w4 = reinterpret_cast<const float4*>(weight);
    if (one_pass && tid < quads) w_s[tid] = w4[tid];
    // Wavefront 0's chain; the squares of the next quad are formed between
    // the four dependent adds of the pending one. pp starts as four zero
    // squares, whose adds leave sum at +0.0f as the reference starts it.
    float sum = 0.0f;
    float pp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto step = [&](const float4& n) {
        sum = sum + pp[0];
        pp[0] = n.x * n.x;
        __builtin_amdgcn_sched_barrier(0);
        sum = sum + pp[1];
        pp[1] = n.y * n.y;
        __builtin_amdgcn_sched_barrier(0);
        sum = sum + pp[2];
        pp[2] = n.z * n.z;
        __builtin_amdgcn_sched_barrier(0);
        sum = sum + pp[3];
        pp[3] = n.w * n.w;
        __builtin_amdgcn_sched_barrier(0);
    };
    auto add_sq = [&](const float4& q) {
        sum = sum + q.x;
        sum = sum + q.y;
        sum = sum + q.z;
        sum = sum + q.w;
    };
    float4 v[kRmsPer];
    int q0 = 0;
    for (int p0 = 0; p0 < quads; p0 += kRmsWaves * kRmsPer) {
        q0 = p0 + wave * kRmsPer;  // this wavefront's quads
#pragma unroll
        for (int i = 0; i < kRmsPer; ++i) v[i] = xrow[(size_t)min(q0 + i, quads - 1) * 64];
        if (wave == 0) {
#pragma unroll
            for (int i = 0; i < kRmsPer; ++i)
                if (q0 + i < quads) step(v[i]);
            sum = sum + pp[0];
            sum = sum + pp[1];
            sum = sum + pp[2];
            sum = sum + pp[3];
            pp[0] = pp[1] = pp[2] = pp[3] = 0.0f;
        } else {
#pragma unroll
            for (int i = 0; i < kRmsPer; ++i)
                sq_s[((wave - 1) * kRmsPer + i) * 64 + lane] =
                    make_float4(v[i].x * v[i].x, v[i].y * v[i].y, v[i].z * v[i].z, v[i].w * v[i].w);
        }
        __syncthreads();
        if (wave == 0) {
            const int n = min(quads - (p0 + kRmsPer), (kRmsWaves - 1) * kRmsPer);
            const float4* t4 = sq_s + lane;
            auto read8 = [&](int q, float4 (&u)[8]) {
#pragma unroll
                for (int j = 0; j < 8; ++j) u[j] = t4[min(q + j, n - 1) * 64];
            };
            int q = 0;
            if (n >= 8) {
                float4 u0[8], u1[8];
                read8(0, u0);
                for (; q + 16 <= n; q += 16) {
                    read8(q + 8, u1);
#pragma unroll
                    for (int j = 0; j < 8; ++j) add_sq(u0[j]);
                    read8(q + 16, u0);
#pragma unroll
                    for (int j = 0; j < 8; ++j) add_sq(u1[j]);
                }
                if (q + 8 <= n) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) add_sq(u0[j]);
                    q += 8;
                }
            }
            for (; q < n; ++q) add_sq(t4[q * 64]);
        }
        __syncthreads();
    }
    if (wave == 0) scale_s[lane] = 1.0f / sqrtf(sum / (float)width + eps);
    __syncthreads();
    if (src < 0) return;
    const float scale = scale_s[lane];
    float4* o4 = reinterpret_cast<float4*>(out) + (size_t)tile * quads * 64 + lane;
    const int per = (quads + kRmsSlices - 1) / kRmsSlices;
    const int qs = slice * per, qe = min(quads, qs + per);
    auto emit = [&](int q, const float4& v_, const float4& w) {
        o4[(size_t)q * 64] =
            make_float4(v_.x * scale * w.x, v_.y * scale * w.y, v_.z * scale * w.z, v_.w * scale * w.w);
    };
    if (one_pass) {
        // The slice's quads that this wavefront holds (q0 = wave*kRmsPer).
#pragma unroll
        for (int i = 0; i < kRmsPer; ++i) {
            const int q = q0 + i;
            if (q >= qs && q < qe) emit(q, v[i], w_s[q]);
        }
    } else {
        for (int q = qs + wave; q < qe; q += kRmsWaves) emit(q, xrow[(size_t)q * 64], w4[q]);
    }
}

// llama_runner.cpp:17-22 and :81-83: split-half rotation of every q and k
// head at the row's position (cos/sin from the host table of
// float(pos)/powf(theta, 2d/dim), so the rotation is bit-identical); q is
// rotated in place, the rotated k and the v row go to the pools (device page
// layout of layout.h).
__global__ void rope_append_kernel(float* __restrict__ qkv, int width, int heads, int kv_heads, int dim,
                                   const float* __restrict__ cos_table, const float* __restrict__ sin_table,
                                   RowMeta meta, PagedKv kv, int layer) {
    const int r = blockIdx.x;
    const int pos = meta.row_pos[r];
    const int32_t* table = kv.tables + (size_t)meta.seq_slot[meta.row_seq[r]] * kv.table_stride;
    const int half = dim / 2;
    const float* cs_row = cos_table + (size_t)pos * half;
    const float* sn_row = sin_table + (size_t)pos * half;
    const int bt = kv.block_tokens, slot = pos % bt;
    const size_t base = kv_page_base(table[pos / bt], layer, kv.layers, bt, kv.kv_width);
    const int hidden = heads * dim;
    for (int p = threadIdx.x; p < heads * half; p += blockDim.x) {
        const int h = p / half, d = p % half;
        const int i = h * dim + d, j = i + half;
        float* qi = qkv + quad_index(r, i, width);
        float* qj = qkv + quad_index(r, j, width);
        const float a = *qi, b = *qj, cs = cs_row[d], sn = sn_row[d];
        *qi = a * cs - b * sn;
        *qj = b * cs + a * sn;
    }
    for (int p = threadIdx.x; p < kv_heads * half; p += blockDim.x) {
        const int h = p / half, d = p % half;
        const int i = h * dim + d, j = i + half;
        const float a = qkv[quad_index(r, hidden + i, width)], b = qkv[quad_index(r, hidden + j, width)];
        const float cs = cs_row[d], sn = sn_row[d];
        kv.keys[base + key_offset(slot, h, d, bt, dim)] = a * cs - b * sn;
        kv.keys[base + key_offset(slot, h, d + half, bt, dim)] = b * cs + a * sn;
    }
    for (int i = threadIdx.x; i < kv.kv_width; i += blockDim.x)
        kv.values[base + value_offset(slot, i / dim, i % dim, bt, dim)] =
            qkv[quad_index(r, hidden + kv.kv_width + i, width)];
}

// Copy-on-write of the first `valid` token slots of a page, every layer, in
// both pools (block x = layer, block y = pool, block z = copy). In the device
// page order the valid slots of a key page are, per (KV head, group of 4
// dims), a run of `valid` float4 (key_offset); those of a value page are, per
// KV head, the first ceil(valid/4) groups of dim float4 (value_offset; the
// last group may carry slots past the tail, which later appends overwrite
// before any read). `page4` is one page-layer span in float4; a block id
// times `layers` page-layer spans is the (page, layer 0) span.
__global__ void copy_tails_kernel(float4* keys, float4* values, const TailCopy* __restrict__ copies,
                                  uint32_t page4, int layers, int block_tokens, int kv_heads, int dim) {
    const TailCopy c = copies[blockIdx.z];
    const int valid = c.valid;
    const uint64_t destination = (uint64_t)c.destination * layers * page4;
    const uint64_t source = (uint64_t)c.source * layers * page4;
    const bool is_key = blockIdx.y == 0;
    float4* pool = is_key ? keys : values;
    const uint64_t layer = blockIdx.x;
    float4* dst = pool + destination + layer * page4;
    const float4* src = pool + source + layer * page4;
    const int head4 = block_tokens * dim / 4;  // float4 per KV head in a page-layer span
    if (is_key) {
        const int runs = kv_heads * (dim / 4);  // runs of block_tokens float4, one per (head, 4 dims)
        for (int i = threadIdx.x; i < runs * valid; i += blockDim.x) {
            const int run = i / valid, slot = i % valid;
            const int at = run * block_tokens + slot;
            dst[at] = src[at];
        }
    } else {
        const int per_head = (valid + 3) / 4 * dim;  // float4 of the valid slot groups of one head
        for (int i = threadIdx.x; i < kv_heads * per_head; i += blockDim.x) {
            const int at = (i / per_head) * head4 + i % per_head;
            dst[at] = src[at];
        }
    }
}

// tables[updates[i].x] = updates[i].y; the indices are distinct.
__global__ void table_update_kernel(int32_t* __restrict__ tables, const int2* __restrict__ updates, int count) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += gridDim.x * blockDim.x)
        tables[updates[i].x] = updates[i].y;
}

// W[n][k] (n < n_out, k < k_in) to the fragment order of layout.h: float4
// f of the destination is lane f%64 of fragment f/64 = (n/16) * (k_in/16) +
// k/16, holding W[16(n/16) + lane%16][16(k/16) + 4(lane/16) .. +3] (with
// rope_heads, stored output n holds source output fast_rope_column(n)).
__global__ void to_fragments_kernel(const float* __restrict__ src, float* __restrict__ dst, int n_out, int k_in,
                                    bool in_out, bool rope_heads) {
    const size_t total = (size_t)n_out * k_in;
    const int steps = k_in >> 4;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const int c = (int)(i & 3);
        const int lane = (int)((i >> 2) & 63);
        const size_t fragment = i >> 8;
        const int stored = (int)(fragment / steps) * 16 + (lane & 15);
        const int n = rope_heads ? fast_rope_column(stored) : stored;
        const int k = (int)(fragment % steps) * 16 + 4 * (lane >> 4) + c;
        dst[i] = in_out ? src[(size_t)k * n_out + n] : src[(size_t)n * k_in + k];
    }
}

__global__ void transpose_kernel(const float* __restrict__ src, float* __restrict__ dst, int rows, int cols,
                                 int ld_dst) {
    __shared__ float tile[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    for (int i = threadIdx.y; i < 32; i += blockDim.y) {
        const int r = r0 + i, c = c0 + threadIdx.x;
        if (r < rows && c < cols) tile[i][threadIdx.x] = src[(size_t)r * cols + c];
    }
    __syncthreads();
    for (int i = threadIdx.y; i < 32; i += blockDim.y) {
        const int c = c0 + i, r = r0 + threadIdx.x;
        if (r < rows && c < cols) dst[(size_t)c * ld_dst + r] = tile[threadIdx.x][i];
    }
}

}  // namespace

hipError_t launch_embed(hipStream_t s, const float* embedding, const int32_t* tokens, float* x, int rows,
                        int hidden, int32_t* error, const RowRope* rope, bool fragments) {
    if (rows <= 0) return hipSuccess;
    if (fragments && hidden % 16) return hipErrorInvalidValue;
    const size_t total = quad_floats(rows, hidden) / 4;
    const int blocks = (int)std::min<size_t>((total + 255) / 256, 4096);
    RowRope rr{};
    if (rope) rr = *rope;
    embed_kernel<<<blocks, 256, 0, s>>>(embedding, tokens, x, rows, hidden, error, rr, fragments);
    return hipGetLastError();
}

hipError_t launch_to_fragments(hipStream_t s, const float* src, float* dst, int n_out, int k_in, bool in_out,
                               bool rope_heads) {
    if (n_out % 16 || k_in % 16 || (rope_heads && n_out % 64)) return hipErrorInvalidValue;
    to_fragments_kernel<<<4096, 256, 0, s>>>(src, dst, n_out, k_in, in_out, rope_heads);
    return hipGetLastError();
}

hipError_t launch_rms(hipStream_t s, const float* x, const int32_t* row_map, const float* weight, float* out,
                      int rows, int width, float eps) {
    if (rows <= 0) return hipSuccess;
    rms_kernel<<<dim3((rows + 63) / 64, kRmsSlices), kRmsWaves * 64, 0, s>>>(x, row_map, weight, out, rows, width,
                                                                             eps);
    return hipGetLastError();
}

hipError_t launch_rope_append(hipStream_t s, float* qkv, int width, int rows, int heads, int kv_heads, int dim,
                              const float* cos_table, const float* sin_table, const RowMeta& meta,
                              const PagedKv& kv, int layer) {
    if (rows <= 0) return hipSuccess;
    rope_append_kernel<<<rows, 256, 0, s>>>(qkv, width, heads, kv_heads, dim, cos_table, sin_table, meta, kv,
                                            layer);
    return hipGetLastError();
}

hipError_t launch_copy_tails(hipStream_t s, float* keys, float* values, const TailCopy* copies, int count,
                             int layers, int block_tokens, int kv_heads, int dim) {
    if (layers <= 0 || count <= 0) return hipSuccess;
    const uint32_t page4 = (uint32_t)(block_tokens * kv_heads * dim / 4);
    copy_tails_kernel<<<dim3((unsigned)layers, 2, (unsigned)count), 256, 0, s>>>(
        reinterpret_cast<float4*>(keys), reinterpret_cast<float4*>(values), copies, page4, layers, block_tokens,
        kv_heads, dim);
    return hipGetLastError();
}

hipError_t launch_table_update(hipStream_t s, int32_t* tables, const int2* updates, int count) {
    if (count <= 0) return hipSuccess;
    table_update_kernel<<<std::min((count + 255) / 256, 64), 256, 0, s>>>(tables, updates, count);
    return hipGetLastError();
}

hipError_t launch_transpose(hipStream_t s, const float* src, float* dst, int rows, int cols, int ld_dst) {
    transpose_kernel<<<dim3((cols + 31) / 32, (rows + 31) / 32), dim3(32, 8), 0, s>>>(src, dst, rows, cols,
                                                                                     ld_dst);
    return hipGetLastError();
}

}  // namespace mphip
