// Projections of the fast arithmetic mode on FP32 matrix cores
// (v_mfma_f32_16x16x4f32): out[r][n] = epilogue(sum_k a[r][k] * w[n][k]) in
// the matrix cores' summation order, not the reference's sequential one
// (the reference's result is matched to 1e-3 relative on the logits and
// its greedy tokens are checked, instead of bit for bit).
//
// Operand layout of one 16x16x4 MFMA (measured on gfx950): lane l supplies
// A[l%16][l/16] and B[l/16][l%16]; result register i of lane l is
// D[4*(l/16)+i][l%16]. Each lane loads a float4 of 4 consecutive k for its
// row (A) and its column (B); MFMA j of a 16-k step takes component j of
// both, so the four lane groups l/16 cover k, k+4, k+8, k+12 of the step.
// The weights are stored in that fragment order (layout.h), so a
// wavefront's B operand of one step is one contiguous 1 KB load.
//
// A work-group of eight wavefronts computes RB 16-row blocks x CB 16-column
// blocks. The 16-k steps of K are dealt to the wavefronts in turn (step s to
// wavefront s % 8) and a wavefront issues the loads of all its steps (up to
// CH at a time) before its first multiply: at decode sizes a projection is
// bound by memory latency, not bandwidth, so the loads of a launch must be
// in flight together, and so are everything the epilogue reads (RMSNorm
// partials, the residual's old values, the RoPE rows). The partial tiles
// are then summed through LDS in a fixed order by the wavefront that owns
// their row block (row block rb to wavefront rb % min(RB, 4)), which runs
// the epilogue for it, as ((p0 + p4) + (p1 + p5)) + ((p2 + p6) + (p3 + p7)):
// with up to 4 tiles from all eight partials after one barrier, with more
// in two levels (wavefronts 4-7 into 0-3, then the four). A row's result
// depends on nothing but the row.
//
// Work-group b runs on XCD b % 8. Up to 256 rows (decode), the work-groups
// sharing a column group (one per row group) go to the same XCD and share
// its L2 for the weights: the 8-strided sequence of one XCD walks the row
// groups of a column group first. Above 256 rows (prefill, many rounds of
// work-groups) each XCD takes an equal run of consecutive tiles in
// column-group-major order (XCD x: tiles x*P .. x*P + P - 1, P = tiles / 8
// rounded up): with 9 column groups of 64 the decode layout gives XCD 0
// twice the tiles of the others (prefill O and down ran at half the rate of
// gate/up), while at decode sizes the equal runs were 1.4% slower.
//
// Epilogues: store; residual (x += result) writing, for the next RMSNorm,
// the sum of squares of the updated x over each 16-column block; SwiGLU
// (gate and up accumulated side by side); LM head (per row and column group
// of 16*CB columns, the first maximum and a non-finite flag, logits
// row-major on request); RoPE (the q|k|v projection of a decode step, over
// q and k columns stored pair-permuted so that each 16-column block holds
// whole split-half pairs (d, d+32) in lanes c and c+8; q is rotated in
// place, the rotated k and the v go to the paged pools at the row's
// position).
// RMSNorm on the input (NORM): a[r][k] = x[r][k] * g[k], and the result is
// scaled by 1/sqrt(sum_k x[r][k]^2 / K + eps), the sum assembled from the
// producer's per-block partials.
#include <type_traits>

#include "kernels.h"
#include "lanes.h"
#include "layout.h"

// The fast mode's own summation order: multiply-adds may be fused.
#pragma clang fp contract(fast)

namespace mphip {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kXcds = 8;
constexpr int kSpreadRows = 256;  // above: tiles in equal runs per XCD
constexpr int kRopeDim = 64;
constexpr int kSsqSlots = 8;  // threads per row summing the RMSNorm partials
constexpr int kSsqHeld = 8;   // partials per thread loaded up front (hidden <= 1024)

__device__ __forceinline__ f4 ld4(const float* p) { return *reinterpret_cast<const f4*>(p); }

// Order-preserving key of a finite float (larger value -> larger key; -0 is
// taken as +0) with the column in the low half (smaller column -> larger
// key), so that the maximum key is the first maximum. 0 means no finite
// value.
__device__ __forceinline__ uint64_t argmax_key(float v, int col) {
    const uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
    const uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)k << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)col);
}
__device__ __forceinline__ float key_value(uint64_t key) {
    const uint32_t k = (uint32_t)(key >> 32);
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// The larger of this lane's key and the key of the lane DPP control kCtrl
// names (the reduction steps of a 16-lane row).
template <int kCtrl>
__device__ __forceinline__ uint64_t max_key(uint64_t key) {
    const uint64_t k = ((uint64_t)dpp_u<kCtrl>((uint32_t)(key >> 32)) << 32) | dpp_u<kCtrl>((uint32_t)key);
    return k > key ? k : key;
}

// The q and k columns of the RoPE projection are stored pair-permuted
// within each 64-wide head (fast_rope_column): column 16b + c of a head is
// dim rope_dim = 8b + c%8 + 32(c/8), so each 16-column block holds 8 whole
// split-half pairs (d, d + 32) in lanes c and c + 8; rope_pair is the
// pair's rotation index d % 32.
__device__ __forceinline__ int rope_dim(int cb, int lane) { return fast_rope_column(cb * 16 + (lane & 15)) & 63; }
__device__ __forceinline__ int rope_pair(int cb, int lane) { return 8 * (cb & 3) + (lane & 7); }

template <int EPI, bool NORM, bool GATHER, int RB, int CB, int CH>
__global__ __launch_bounds__(kWaves * 64, CH == 1 ? 4 : 1) void fast_gemm_kernel(FastGemmArgs a) {
    static_assert(EPI != kRope || CB == 1, "the RoPE epilogue takes one column block");
    constexpr int M = EPI == kSwiglu ? 2 : 1;
    constexpr int NB = CB * M;  // B operands per step
    constexpr int T = RB * NB;  // accumulator tiles
    constexpr int OW = RB < 4 ? RB : 4;  // wavefronts that own row blocks
    // Up to 4 tiles, every wavefront's partials go to LDS at once and one
    // barrier precedes the owners' sums; more tiles are summed in two levels
    // (wavefronts 4-7 into 0-3, then to the owners) to halve the LDS.
    constexpr bool kOneSync = T <= 4;
    __shared__ f4 part_s[kOneSync ? kWaves : kWaves / 2][T][64];
    __shared__ float ssq_s[NORM ? RB * 16 : 1][kSsqSlots];
    __shared__ float inv_s[RB * 16];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Work-group -> (row group, column group), XCD-grouped.
    const int nrg = (((a.rows + 15) >> 4) + RB - 1) / RB;
    const int ncg = (a.columns >> 4) / CB;
    int cg, rg;
    if (a.rows > kSpreadRows) {
        const int tiles = nrg * ncg, per_xcd = (tiles + kXcds - 1) / kXcds;
        const int t = (blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
        if (t >= tiles) return;
        cg = t / nrg;
        rg = t % nrg;
    } else {
        const int g = blockIdx.x / kXcds, xcd = blockIdx.x % kXcds;
        rg = g % nrg;
        cg = (g / nrg) * kXcds + xcd;
        if (cg >= ncg) return;
    }
    int cblock[CB];
#pragma unroll
    for (int j = 0; j < CB; ++j) cblock[j] = cg * CB + j;
    const int row0 = rg * RB * 16;
    const int K = a.inner, Q = K >> 2, steps = K >> 4;
    // A: row row0 + 16rb + l%16 (gathered), quads 4s + l/16.
    const float* xa[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int r = min(row0 + rb * 16 + (lane & 15), a.rows - 1);
        const int xrow = GATHER && a.row_map ? a.row_map[r] : r;
        xa[rb] = a.x + ((size_t)(xrow >> 6) * Q * 64 + (xrow & 63)) * 4 + (size_t)(lane >> 4) * 256;
    }
    // B: column 16cblock + l%16, k 16s + 4(l/16): lane l's float4 of the
    // (cblock, s) fragment (weights in fragment order), one contiguous 1 KB
    // per wavefront and step.
    const float* wb[NB];
#pragma unroll
    for (int j = 0; j < CB; ++j) {
        const size_t off = (size_t)cblock[j] * steps * 256 + (size_t)lane * 4;
        wb[j * M] = a.w + off;
        if (M == 2) wb[j * M + M - 1] = a.w2 + off;
    }
    const float* gn = NORM ? a.norm + (lane >> 4) * 4 : nullptr;
    // RMSNorm: the producer's per-16-column partial sums of squares of each
    // row, summed by 8 threads per row (slot u takes partials u, u+8, ...).
    // The order of the sums is fixed per row (slots in order), whatever RB is.
    const int ssq_row = threadIdx.x / kSsqSlots, ssq_slot = threadIdx.x % kSsqSlots;
    float ssv[kSsqHeld];
    if (NORM) {
        const int r = min(row0 + ssq_row, a.rows - 1);
        const int pr = GATHER && a.row_map ? a.row_map[r] : r;
#pragma unroll
        for (int u = 0; u < kSsqHeld; ++u) {
            const int p = ssq_slot + u * kSsqSlots;
            ssv[u] = ssq_row < RB * 16 && p < a.ssq_parts ? a.ssq_in[(size_t)p * a.ssq_stride + pr] : 0.0f;
        }
    }
    // The residual's old values (small tiles: wavefront 0 owns the only row block).
    constexpr bool kEarly = EPI == kResidual && RB * CB == 1;
    float old[4];
    if (kEarly && wave == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = min(row0 + 4 * (lane >> 4) + i, a.rows - 1);
            old[i] = a.out[quad_index(row, cblock[0] * 16 + (lane & 15), a.columns)];
        }
    }
    // RoPE rows of the owned row block: position, page and rotation (cos,
    // sin of rotation index rope_pair() at the row's position; CB == 1).
    int rope_pos[4], rope_block[4];
    float rope_cs[4], rope_sn[4];
    if (EPI == kRope && wave < OW) {
        const int rd = rope_pair(cblock[0], lane);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = min(row0 + wave * 16 + 4 * (lane >> 4) + i, a.rows - 1);
            rope_pos[i] = a.meta.row_pos[row];
            rope_block[i] = a.row_block[row];
            rope_cs[i] = a.row_rope[(size_t)row * kRopeDim + rd];
            rope_sn[i] = a.row_rope[(size_t)row * kRopeDim + kRopeDim / 2 + rd];
        }
    }

    f4 acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
    const int mine = steps > wave ? (steps - wave + kWaves - 1) / kWaves : 0;  // this wavefront's steps
    // Steps i0 .. i0+CH-1 of this wavefront: their operands, then their MFMAs
    // (steps in order, whatever the chunking).
    auto load = [&](int i0, f4 (&av)[CH][RB], f4 (&bv)[CH][NB], f4 (&gv)[CH]) {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            if (i0 + c < mine) {
                const size_t s = wave + (size_t)kWaves * (i0 + c);
                if (NORM) gv[c] = ld4(gn + s * 16);
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) av[c][rb] = ld4(xa[rb] + s * 1024);  // 4 quads x 64 rows x 4
#pragma unroll
                for (int j = 0; j < NB; ++j)
                    bv[c][j] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(wb[j] + s * 256));
            }
        }
    };
    auto multiply = [&](int i0, const f4 (&av)[CH][RB], const f4 (&bv)[CH][NB], const f4 (&gv)[CH]) {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            if (i0 + c < mine) {
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) {
                    const f4 x = NORM ? av[c][rb] * gv[c] : av[c][rb];
#pragma unroll
                    for (int j = 0; j < NB; ++j) {
                        f4& d = acc[rb * NB + j];
                        d = __builtin_amdgcn_mfma_f32_16x16x4f32(x.x, bv[c][j].x, d, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x4f32(x.y, bv[c][j].y, d, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x4f32(x.z, bv[c][j].z, d, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x4f32(x.w, bv[c][j].w, d, 0, 0, 0);
                    }
                }
            }
        }
    };
    if constexpr (CH == 2) {
        // Short chunks (the many-step tiles of the LM head and of prefill):
        // two operand buffers, the next chunk's loads in flight during this
        // chunk's MFMAs.
        f4 av0[CH][RB], bv0[CH][NB], gv0[CH], av1[CH][RB], bv1[CH][NB], gv1[CH];
        load(0, av0, bv0, gv0);
        for (int i0 = 0; i0 < mine; i0 += 2 * CH) {
            if (i0 + CH < mine) load(i0 + CH, av1, bv1, gv1);
            __builtin_amdgcn_sched_barrier(0);
            multiply(i0, av0, bv0, gv0);
            if (i0 + CH >= mine) break;
            if (i0 + 2 * CH < mine) load(i0 + 2 * CH, av0, bv0, gv0);
            __builtin_amdgcn_sched_barrier(0);
            multiply(i0 + CH, av1, bv1, gv1);
        }
    } else {
        for (int i0 = 0; i0 < mine; i0 += CH) {
            f4 av[CH][RB], bv[CH][NB], gv[CH];
            load(i0, av, bv, gv);
            multiply(i0, av, bv, gv);
        }
    }
    if (NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int u = 0; u < kSsqHeld; ++u) ss += ssv[u];
        const int r = min(row0 + ssq_row, a.rows - 1);
        const int pr = GATHER && a.row_map ? a.row_map[r] : r;
        for (int p = ssq_slot + kSsqHeld * kSsqSlots; p < a.ssq_parts; p += kSsqSlots)
            ss += a.ssq_in[(size_t)p * a.ssq_stride + pr];
        if constexpr (kOneSync) {
            // A row's kSsqSlots = 8 slots are 8 consecutive lanes: lane 8r
            // gets their sum (quads, then the other quad of the eight).
            ss += dpp<kDppQuadXor1>(ss);
            ss += dpp<kDppQuadXor2>(ss);
            ss += __shfl_xor(ss, 4);
            // 1/sqrt(mean square + eps) of the group's rows.
            if (ssq_slot == 0 && ssq_row < RB * 16) inv_s[ssq_row] = 1.0f / sqrtf(ss / (float)K + a.eps);
        } else if (ssq_row < RB * 16) {
            ssq_s[ssq_row][ssq_slot] = ss;
        }
    }
    if constexpr (kOneSync) {
        // Every wavefront's partial tiles, one barrier, then each tile's
        // eight partials to its owner.
#pragma unroll
        for (int t = 0; t < T; ++t) part_s[wave][t][lane] = acc[t];
        __syncthreads();
        if (wave >= OW) return;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            if (rb % OW != wave) continue;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int t = rb * NB + j;
                // The order of the two-level sums below (wavefront w with
                // w + 4, then the four in order), whatever the tile count.
                const f4 q0 = part_s[0][t][lane] + part_s[4][t][lane], q1 = part_s[1][t][lane] + part_s[5][t][lane];
                const f4 q2 = part_s[2][t][lane] + part_s[6][t][lane], q3 = part_s[3][t][lane] + part_s[7][t][lane];
                acc[t] = (q0 + q1) + (q2 + q3);
            }
        }
    } else {
        // Wavefronts 4-7 into 0-3.
        if (wave >= kWaves / 2)
#pragma unroll
            for (int t = 0; t < T; ++t) part_s[wave - kWaves / 2][t][lane] = acc[t];
        __syncthreads();
        if (wave < kWaves / 2)
#pragma unroll
            for (int t = 0; t < T; ++t) acc[t] += part_s[wave][t][lane];
        if (NORM && threadIdx.x < RB * 16) {
            // 1/sqrt(mean square + eps) of the group's rows, the slots
            // summed in the order of the lane sums above.
            const float* u = ssq_s[threadIdx.x];
            const float ss = ((u[0] + u[1]) + (u[2] + u[3])) + ((u[4] + u[5]) + (u[6] + u[7]));
            inv_s[threadIdx.x] = 1.0f / sqrtf(ss / (float)K + a.eps);
        }
        __syncthreads();
        // Then each tile's four partials to its owner.
        if (wave < kWaves / 2)
#pragma unroll
            for (int t = 0; t < T; ++t) part_s[wave][t][lane] = acc[t];
        __syncthreads();
        if (wave >= OW) return;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            if (rb % OW != wave) continue;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int t = rb * NB + j;
                acc[t] = (part_s[0][t][lane] + part_s[1][t][lane]) + (part_s[2][t][lane] + part_s[3][t][lane]);
            }
        }
    }

    const int N = a.columns;
    if (EPI == kRope) {
        // One column block (CB == 1) of the pair-permuted q|k|v columns:
        // lanes c and c + 8 of a q or k block hold the split-half pair
        // (d, d + 32) of one head (rope_dim), exchanged by a DPP rotation of
        // the 16-lane row by 8; v blocks are in natural order. RB <= 4, so
        // wavefront w owns row block w.
        const int rb = wave;
        const int cb = cblock[0];
        const int hcol = cb * 16 / kRopeDim * kRopeDim;  // the head's first column
        const int hidden = a.heads * kRopeDim, kvw = a.kv.kv_width;
        const int bt = a.kv.block_tokens;
        const bool rotate = hcol < hidden + kvw;
        const int d = rotate ? rope_dim(cb, lane) : (cb * 16) % kRopeDim + (lane & 15);
        const bool low = (lane & 8) == 0;  // the d < 32 half of a pair
        float x[4], xp[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v = 0.0f;
#pragma unroll
            for (int r2 = 0; r2 < RB; ++r2)
                if (r2 == rb) v = acc[r2][i];
            x[i] = v * inv_s[rb * 16 + 4 * (lane >> 4) + i];
            xp[i] = dpp<kDppRowRor8>(x[i]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = row0 + rb * 16 + 4 * (lane >> 4) + i;
            if (row >= a.rows) continue;
            const float cs = rope_cs[i], sn = rope_sn[i];
            const float y = !rotate ? x[i] : low ? x[i] * cs - xp[i] * sn : x[i] * cs + xp[i] * sn;
            if (hcol < hidden) {
                a.out[quad_index(row, hcol + d, N)] = y;
                continue;
            }
            const size_t base = kv_page_base(rope_block[i], a.layer, a.kv.layers, bt, kvw);
            const int slot = rope_pos[i] % bt;
            if (rotate) a.kv.keys[base + key_offset(slot, (hcol - hidden) / kRopeDim, d, bt, kRopeDim)] = y;
            else a.kv.values[base + value_offset(slot, (hcol - hidden - kvw) / kRopeDim, d, bt, kRopeDim)] = y;
        }
        return;
    }
    if (EPI == kHead) {
        // Per row of the owned row blocks: the first maximum over the column
        // group's 16*CB columns (lane: columns cblock[j]*16 + l%16, j in
        // order), then across the 16 lanes of the row's lane group.
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            if (rb % OW != wave) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int rl = 4 * (lane >> 4) + i;
                const int row = row0 + rb * 16 + rl;
                const bool live = row < a.rows;
                const float inv = NORM ? inv_s[rb * 16 + rl] : 1.0f;
                uint64_t key = 0;
                bool bad = false;
#pragma unroll
                for (int j = 0; j < CB; ++j) {
                    const float x = acc[rb * NB + j][i] * inv;
                    const int col = cblock[j] * 16 + (lane & 15);
                    if (live && a.logits) a.logits[(size_t)row * N + col] = x;
                    const bool finite = __builtin_isfinite(x);
                    bad |= !finite;
                    const uint64_t k = finite ? argmax_key(x, col) : 0;
                    key = k > key ? k : key;
                }
                key = max_key<kDppQuadXor1>(key);
                key = max_key<kDppQuadXor2>(key);
                key = max_key<kDppRowRor4>(key);
                key = max_key<kDppRowRor8>(key);
                const uint64_t bads = __ballot(bad);
                if (live && (lane & 15) == 0) {
                    const size_t at = (size_t)row * a.groups + cg;
                    a.best_value[at] = key ? key_value(key) : -__builtin_inff();
                    a.best_index[at] = key ? (int)(0xFFFFFFFFu - (uint32_t)key) : -1;
                    a.bad[at] = ((bads >> (lane & 48)) & 0xFFFFull) != 0;
                }
            }
        }
        return;
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        if (rb % OW != wave) continue;
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            // Lane l, register i: row row0 + 16rb + 4(l/16) + i, column 16cblock + l%16.
            const int col = cblock[j] * 16 + (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int rl = 4 * (lane >> 4) + i;
                const int row = row0 + rb * 16 + rl;
                const bool live = row < a.rows;
                float v[M];
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const float s = acc[rb * NB + j * M + m][i];
                    v[m] = NORM ? s * inv_s[rb * 16 + rl] : s;
                }
                if (EPI == kStore) {
                    const int oc = col < a.rope_columns ? fast_rope_column(col) : col;
                    if (live) a.out[quad_index(row, oc, N)] = v[0];
                } else if (EPI == kResidual) {
                    float nx = 0.0f;
                    if (live) {
                        float* o = a.out + quad_index(row, col, N);
                        nx = (kEarly ? old[i] : *o) + v[0];
                        *o = nx;
                    }
                    // The row's 16 columns sit in the 16 lanes of this lane's group.
                    const float sq = row_sum(nx * nx);
                    if (live && (lane & 15) == 0) a.ssq_out[(size_t)cblock[j] * a.ssq_stride + row] = sq;
                } else {  // kSwiglu
                    const float gt = v[0];
                    if (live) a.out[quad_index(row, col, N)] = (gt / (1.0f + __expf(-gt))) * v[M - 1];
                }
            }
        }
    }
}

// LM head over the tied embedding for hidden size K. The tiles above cut K
// into eight per work-group and sum eight partial tiles through LDS; for the
// head (768 groups of 64 columns, 36 steps each) that took 50.5 us at 64
// rows and 25 us at 1 row. Here one work-group per CU holds the rows of a
// pass (up to 64, times the RMSNorm weights, in fragment order) in LDS, and
// each of its kHeadWaves wavefronts streams the weights of one 16-column
// block from HBM through a ring of kHeadRing steps in flight: one MFMA chain
// per output over the 16-k steps in order, the row blocks' MFMAs of a
// sub-step issued together (41.7 us at 64 rows, 20.5 us at 16, measured in
// isolation). The order depends on K only, so a row's logits do not depend
// on the batch or on the rows sharing its pass; rows beyond 64 take further
// passes over the same columns. Epilogue as above: the row's 1/sqrt(mean
// square + eps) (its per-16-column partials summed in a fixed order), logits
// on request, and per row and 64-column group the first maximum and a
// non-finite flag, the four wavefronts of a group combined through LDS.
constexpr int kHeadWaves = 12;  // 16-column blocks per work-group: 3 groups of 64
constexpr int kHeadRing = 12;   // weight steps in flight per wavefront

template <int K, int RB>
__global__ __launch_bounds__(kHeadWaves * 64, 1) void fast_head_kernel(FastGemmArgs a) {
    constexpr int S = K / 16;
    constexpr int R = RB * 16;
    constexpr int kThreads = kHeadWaves * 64;
    constexpr int kFill = (RB * S * 64 + kThreads - 1) / kThreads;
    constexpr int kParts = S / 4;  // RMSNorm partials per quarter
    static_assert(K % 16 == 0 && S % kHeadRing == 0 && S % 4 == 0, "whole rings of steps, quarters of partials");
    __shared__ f4 a_s[RB * S * 64];
    __shared__ f4 g_s[S][4];
    __shared__ uint64_t key_s[kHeadWaves][R];
    __shared__ int32_t bad_s[kHeadWaves][R];
    __shared__ float ssq_s[4][R];
    __shared__ float inv_s[R];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nblocks = a.columns >> 4;
    const int cb = blockIdx.x * kHeadWaves + wave;
    const bool active = cb < nblocks;
    // Lane l's float4 of fragment (cb, s): W[16cb + l%16][16s + 4(l/16) .. +3].
    const float* wb = a.w + (size_t)min(cb, nblocks - 1) * S * 256 + (size_t)lane * 4;
    for (int r0 = 0; r0 < a.rows; r0 += R) {
        // The thread index, opaque to the compiler in each pass: otherwise
        // it keeps every fill address live across the passes (spilled).
        int tid = threadIdx.x;
        asm volatile("" : "+v"(tid));
        // The pass's rows (gathered, clamped to the last row), the RMSNorm
        // weights and the first ring of weights, all loads issued before the
        // first wait.
        f4 xv[kFill], gv = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < kFill; ++u) {
            const int i = min(tid + u * kThreads, RB * S * 64 - 1);
            const int l = i & 63, s = (i >> 6) % S, rb = (i >> 6) / S;
            const int r = min(r0 + rb * 16 + (l & 15), a.rows - 1);
            const int xrow = a.row_map ? a.row_map[r] : r;
            xv[u] = ld4(a.x + ((size_t)(xrow >> 6) * (K / 4) * 64 + (xrow & 63)) * 4 + (size_t)(4 * s + (l >> 4)) * 256);
        }
        if (r0 == 0 && tid < S * 4) gv = ld4(a.norm + 4 * tid);
        // The row's S per-16-column sums of squares: quarter q (partials
        // qS/4 .. (q+1)S/4 - 1, in order) by thread qR + row.
        float ss = 0.0f;
        if (tid < 4 * R) {
            const int q = tid / R;
            const int r = min(r0 + tid % R, a.rows - 1);
            const int pr = a.row_map ? a.row_map[r] : r;
            float part[kParts];
#pragma unroll
            for (int p = 0; p < kParts; ++p) part[p] = a.ssq_in[(size_t)(q * kParts + p) * a.ssq_stride + pr];
#pragma unroll
            for (int p = 0; p < kParts; ++p) ss += part[p];
        }
        f4 ring[kHeadRing];
#pragma unroll
        for (int j = 0; j < kHeadRing; ++j)
            ring[j] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(wb + (size_t)j * 256));
        if (r0 == 0 && tid < S * 4) g_s[tid / 4][tid % 4] = gv;
        if (tid < 4 * R) ssq_s[tid / R][tid % R] = ss;
        __syncthreads();
        // The rows times the RMSNorm weights (so that the MFMA loop has no
        // multiplies).
#pragma unroll
        for (int u = 0; u < kFill; ++u) {
            const int i = tid + u * kThreads;
            if (i < RB * S * 64) a_s[i] = xv[u] * g_s[(i >> 6) % S][(i >> 4) & 3];
        }
        __syncthreads();
        if (tid < R) {
            const float* u = &ssq_s[0][tid];
            inv_s[tid] = 1.0f / sqrtf(((u[0] + u[R]) + (u[2 * R] + u[3 * R])) / (float)K + a.eps);
        }
        f4 acc[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[rb] = f4{0.f, 0.f, 0.f, 0.f};
        // Rounds of kHeadRing steps (a loop, then the last round on its own),
        // each step's ring slot reloaded with the step kHeadRing ahead once
        // consumed (but in the last round, which would only re-read the
        // last step: 12 KB of surplus loads per wavefront), and the next
        // step's rows read from LDS before this step's MFMAs (the scheduling
        // barriers keep the compiler from hoisting more of them). The MFMAs
        // of a step go sub-step by sub-step across the row blocks, so that
        // consecutive ones are independent.
        f4 xc[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) xc[rb] = a_s[rb * S * 64 + lane];
        auto round = [&](int s0, auto reload) {
#pragma unroll
            for (int j = 0; j < kHeadRing; ++j) {
                const int s = s0 + j;
                const f4 b = ring[j];
                if constexpr (decltype(reload)::value)
                    ring[j] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(wb + (size_t)(s + kHeadRing) * 256));
                const int sn = min(s + 1, S - 1);
                f4 xn[RB];
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) xn[rb] = a_s[(rb * S + sn) * 64 + lane];
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) acc[rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xc[rb].x, b.x, acc[rb], 0, 0, 0);
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) acc[rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xc[rb].y, b.y, acc[rb], 0, 0, 0);
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) acc[rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xc[rb].z, b.z, acc[rb], 0, 0, 0);
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) acc[rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xc[rb].w, b.w, acc[rb], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) xc[rb] = xn[rb];
            }
        };
#pragma unroll 1
        for (int s0 = 0; s0 + kHeadRing < S; s0 += kHeadRing) round(s0, std::true_type{});
        round(S - kHeadRing, std::false_type{});
        __syncthreads();  // inv_s
        // Lane l, register i: row r0 + 16rb + 4(l/16) + i, column 16cb + l%16.
        // (A transpose through LDS, each lane then scanning one row's 16
        // columns, measured slower: 45.9 vs 41.7 us at 64 rows.)
        const int N = a.columns;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int rl = rb * 16 + 4 * (lane >> 4) + i;
                const int row = r0 + rl;
                const bool live = active && row < a.rows;
                const float x = acc[rb][i] * inv_s[rl];
                const int col = cb * 16 + (lane & 15);
                if (live && a.logits) a.logits[(size_t)row * N + col] = x;
                const bool finite = __builtin_isfinite(x);
                uint64_t key = live && finite ? argmax_key(x, col) : 0;
                key = max_key<kDppQuadXor1>(key);
                key = max_key<kDppQuadXor2>(key);
                key = max_key<kDppRowRor4>(key);
                key = max_key<kDppRowRor8>(key);
                const uint64_t bads = __ballot(live && !finite);
                if ((lane & 15) == 0) {
                    key_s[wave][rl] = key;
                    bad_s[wave][rl] = ((bads >> (lane & 48)) & 0xFFFFull) != 0;
                }
            }
        }
        __syncthreads();
        // Per row and 64-column group: the first maximum of its four blocks.
        if (tid < (kHeadWaves / 4) * R) {
            const int gl = tid / R, rl = tid % R;
            const int cg = blockIdx.x * (kHeadWaves / 4) + gl, row = r0 + rl;
            if (4 * cg < nblocks && row < a.rows) {
                uint64_t key = 0;
                int32_t bad = 0;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint64_t k = key_s[4 * gl + w][rl];
                    key = k > key ? k : key;
                    bad |= bad_s[4 * gl + w][rl];
                }
                const size_t at = (size_t)row * a.groups + cg;
                a.best_value[at] = key ? key_value(key) : -__builtin_inff();
                a.best_index[at] = key ? (int)(0xFFFFFFFFu - (uint32_t)key) : -1;
                a.bad[at] = bad;
            }
        }
        __syncthreads();  // the next pass rewrites a_s, key_s and bad_s
    }
}

// x rows' per-16-column sums of squares (the partials a NORM projection
// reads), for x written by something other than a residual projection.
__global__ __launch_bounds__(256) void fast_ssq_kernel(const float* __restrict__ x, int rows, int width,
                                                       float* __restrict__ ssq, int stride) {
    const int parts = width >> 4;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * parts) return;
    const int r = i % rows, p = i / rows;
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        const float v = x[quad_index(r, p * 16 + c, width)];
        s += v * v;
    }
    ssq[(size_t)p * stride + r] = s;
}

template <int EPI, bool NORM, bool GATHER, int RB, int CB, int CH>
hipError_t launch_fast(hipStream_t s, const FastGemmArgs& a) {
    const int nrg = ((a.rows + 15) / 16 + RB - 1) / RB;
    const int ncg = a.columns / 16 / CB;
    const int blocks = a.rows > kSpreadRows ? (nrg * ncg + kXcds - 1) / kXcds * kXcds
                                            : (ncg + kXcds - 1) / kXcds * nrg * kXcds;
    fast_gemm_kernel<EPI, NORM, GATHER, RB, CB, CH><<<blocks, kWaves * 64, 0, s>>>(a);
    return hipGetLastError();
}

// Tile shape by size. At decode sizes (one row tile) the tiles are small,
// for many work-groups (SwiGLU over more than 32 rows takes two row blocks:
// its two weight matrices make its column blocks the heaviest; up to 32 rows one,
// 6.3-6.5 instead of 8.0-8.7 us at 1 and 32 rows), and so up to 256 rows
// (at 256 rows they beat the larger tiles below: O 6.6 vs 7.5, down 12.5 vs
// 14.8, gate/up 16.9 vs 18.9 us). The LM head takes tiles of 64 columns
// and 16, 32 or 64 rows, and a projection of more than 256 rows takes
// 64 x 64 tiles when they still
// give every CU a work-group: they read each weight and each activation a
// quarter as often. Otherwise the largest of 64 x 16, 32 x 16 and 16 x 16
// that gives every CU a work-group. (The q|k|v+RoPE projection keeps
// 64 x 16 or 32 x 16 tiles above 64 rows: 11.2 vs 16.0 us at 256 rows.)
constexpr int kCus = 256;
bool head_wide(int columns) { return columns % 64 == 0; }
int tiles(const FastGemmArgs& a, int rb, int cb) { return ((a.rows + 15) / 16 + rb - 1) / rb * (a.columns / 16 / cb); }

template <int EPI, bool NORM, bool GATHER>
hipError_t launch_sized(hipStream_t s, const FastGemmArgs& a) {
    constexpr int M = EPI == kSwiglu ? 2 : 1;
    if constexpr (EPI == kHead) {
        if (a.inner == 576 && a.ssq_parts == 576 / 16 && head_wide(a.columns) && a.norm && a.ssq_in) {
            const int blocks = (a.columns / 16 + kHeadWaves - 1) / kHeadWaves;
            if (a.rows <= 16) fast_head_kernel<576, 1><<<blocks, kHeadWaves * 64, 0, s>>>(a);
            else if (a.rows <= 32) fast_head_kernel<576, 2><<<blocks, kHeadWaves * 64, 0, s>>>(a);
            else fast_head_kernel<576, 4><<<blocks, kHeadWaves * 64, 0, s>>>(a);
            return hipGetLastError();
        }
        if (head_wide(a.columns)) {
            // Row blocks as the batch needs them (B=1: 24.6 instead of 52.4
            // us; B=32: 35.0 instead of 48.6), 64-column groups throughout.
            if (a.rows <= 16) return launch_fast<EPI, NORM, GATHER, 1, 4, 1>(s, a);
            if (a.rows <= 32) return launch_fast<EPI, NORM, GATHER, 2, 4, 1>(s, a);
            return launch_fast<EPI, NORM, GATHER, 4, 4, 1>(s, a);
        }
        return launch_fast<EPI, NORM, GATHER, 1, 1, 6>(s, a);
    } else {
        if (a.rows > 256) {
            if (a.columns % 64 == 0 && tiles(a, 4, 4 / M) >= kCus)
                return launch_fast<EPI, NORM, GATHER, 4, 4 / M, 2>(s, a);
            if (tiles(a, 4, 1) >= kCus) return launch_fast<EPI, NORM, GATHER, 4, 1, 2>(s, a);
            if (tiles(a, 2, 1) >= kCus) return launch_fast<EPI, NORM, GATHER, 2, 1, 6>(s, a);
        }
        if constexpr (M == 2) {
            if (a.rows > 32) return launch_fast<EPI, NORM, GATHER, 2, 1, 6>(s, a);
        }
        return launch_fast<EPI, NORM, GATHER, 1, 1, 12>(s, a);
    }
}

}  // namespace

int fast_head_group_columns(int columns) { return head_wide(columns) ? 64 : 16; }

bool fast_gemm_fits(const FastGemmArgs& a) {
    return a.rows > 0 && a.inner > 0 && a.inner % 16 == 0 && a.columns > 0 && a.columns % 16 == 0;
}

hipError_t launch_fast_gemm(hipStream_t s, Epilogue epilogue, const FastGemmArgs& a) {
    if (!fast_gemm_fits(a)) return hipErrorInvalidValue;
    const bool norm = a.norm != nullptr;
    switch (epilogue) {
    case kStore: return norm ? launch_sized<kStore, true, false>(s, a) : launch_sized<kStore, false, false>(s, a);
    case kResidual: return launch_sized<kResidual, false, false>(s, a);
    case kSwiglu: return norm ? launch_sized<kSwiglu, true, false>(s, a) : launch_sized<kSwiglu, false, false>(s, a);
    case kHead:
        if (a.groups != a.columns / fast_head_group_columns(a.columns)) return hipErrorInvalidValue;
        return launch_sized<kHead, true, true>(s, a);
    case kRope:
        // q|k|v of 64-wide heads: column groups pair blocks j and j+2 of a head.
        if (a.columns % kRopeDim || a.heads * kRopeDim + 2 * a.kv.kv_width != a.columns || !norm ||
            a.kv.block_tokens <= 0 || !a.row_block || !a.row_rope)
            return hipErrorInvalidValue;
        if (a.rows > 64 && tiles(a, 4, 1) >= kCus) return launch_fast<kRope, true, false, 4, 1, 2>(s, a);
        if (a.rows > 64 && tiles(a, 2, 1) >= kCus) return launch_fast<kRope, true, false, 2, 1, 6>(s, a);
        return launch_fast<kRope, true, false, 1, 1, 12>(s, a);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_fast_ssq(hipStream_t s, const float* x, int rows, int width, float* ssq, int stride) {
    if (rows <= 0) return hipSuccess;
    const int total = rows * (width / 16);
    fast_ssq_kernel<<<(total + 255) / 256, 256, 0, s>>>(x, rows, width, ssq, stride);
    return hipGetLastError();
}

}  // namespace mphip
