// Prefill attention of the fast arithmetic mode on FP32 matrix cores
// (v_mfma_f32_16x16x4f32): for a block of up to 16 consecutive rows of one
// sequence's chunk and one KV head, the G query heads' scores against each
// 16-token page and the weighted sum of its values, with a reference maximum
// (raised only when a score exceeds it by more than 16) and a denominator
// per row (flash attention). The reference computes each
// (row, head) with an explicit two-pass softmax and sequential sums
// (llama_runner.cpp:85-93); the order of the floating-point sums differs
// here, and a row's result depends only on the row (its query and keys),
// not on the block, the chunking or the batch.
//
// One work-group per work item (first row, table slot * kv_heads + KV head,
// position of the first row, rows): wavefront w of W walks pages w, w + W,
// ... with its own running maxima and sums, and wavefront 0
// combines the W results in order through LDS. The page-to-wavefront map
// depends only on the page, so the order of the sums is a function of the
// row. Per wavefront and page, with the MFMA operand layout (gfx950): lane l
// supplies A[l%16][l/16] and B[l/16][l%16]; result register i of lane l is
// D[4(l/16)+i][l%16]. With c = l%16 and g = l/16:
//  - scores S = Q K^T, 16 MFMAs per head over the 64 dims: lane (c, g)
//    holds Q[row c][dim 4j+g] (A, kept in registers for the whole walk) and
//    K[key c][dim 4j+g] (B: one dword of the page's key order [d/4][slot][4],
//    a contiguous 256 bytes per MFMA); S[row 4g+i][key c] comes back in
//    register i;
//  - the row maxima and sums of the page over the 16 lanes of a lane group
//    (DPP), the probabilities to LDS as P[row][key], read back as the A
//    operand P[row c][key 4m+g];
//  - O += P V, 4 MFMAs per 16-dim block over the page's 16 keys: lane
//    (c, g) holds V[key 4m+g][dim 16n+c] (B: one dword of the page's value
//    order [slot/4][d][4]); O[row 4g+i][dim 16n+c] accumulates in register i.
// Keys past the row's position are masked; keys past the block's last
// position (the rest of the last page) are masked for every row and their
// values taken as zero, so stale slots take no part, whatever they hold.
#include "kernels.h"
#include "lanes.h"
#include "layout.h"

// The fast mode's own summation order: multiply-adds may be fused.
#pragma clang fp contract(fast)

namespace mphip {
namespace {

constexpr int kDim = 64;
constexpr int kPage = 16;
// Wavefronts per work item, each over every fourth page: one per SIMD. Eight
// (two per SIMD, for G <= 3) took 4% less time on 16384-token prompts but 25%
// more on prompts of 256 to 2048 tokens, whose wavefronts then hold few pages.
constexpr int kWaves = 4;
constexpr float kScale = 0.125f;  // 1/sqrt(64)
constexpr float kRescale = 16.0f;  // probabilities stay below e^16 before a rescale

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp<kDppQuadXor1>(v));
    v = fmaxf(v, dpp<kDppQuadXor2>(v));
    return row_quads_max(v);
}

template <int G, int W = kWaves>
__global__ __launch_bounds__(W * 64) void fast_prefill_kernel(const float* __restrict__ qkv, int ldq,
                                                                            PagedKv kv, int layer,
                                                                            const int4* __restrict__ items, int count,
                                                                            int kv_heads, float* __restrict__ out,
                                                                            int ldo) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    __shared__ float p_s[W][G][kPage][kPage + 1];
    // The other wavefronts' results, combined by wavefront 0: output tiles
    // (per lane, as held) and per row the running maximum and denominator.
    __shared__ f4 o_s[W - 1][G][4][64];
    __shared__ float ml_s[W][G][kPage][2];
    const int index = blockIdx.x;  // one work item per work-group (uniform)
    if (index >= count) return;
    const int4 item = items[index];
    const int row0 = item.x, kvh = item.y % kv_heads, pos0 = item.z, nrows = item.w;
    const int32_t* table = kv.tables + (size_t)(item.y / kv_heads) * kv.table_stride;
    const int last = pos0 + nrows - 1;  // the block's last position
    const int pages = last / kPage + 1;
    const int c = lane & 15, g = lane >> 4;
    // Q of the block's rows (row c, clamped to the block), scaled by 1/8.
    float qa[G][16];
    {
        const int qrow = row0 + min(c, nrows - 1);
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int j = 0; j < 16; ++j)
                qa[h][j] = qkv[quad_index(qrow, (kvh * G + h) * kDim + 4 * j + g, ldq)] * kScale;
    }
    f4 o[G][4];
    float mx[G][4], ls[G][4];  // per row 4g+i: running maximum (lane-group uniform), this lane's share of the sum
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o[h][i] = f4{0.f, 0.f, 0.f, 0.f};
            mx[h][i] = -__builtin_inff();
            ls[h][i] = 0.0f;
        }
    const size_t head_base = (size_t)kvh * kPage * kDim;
    // Page p goes to wavefront p % W, whatever the block.
    for (int p = wave; p < pages; p += W) {
        const size_t base = kv_page_base(table[p], layer, kv.layers, kPage, kv.kv_width) + head_base;
        const float* kp = kv.keys + base;
        const float* vp = kv.values + base;
        float kb[16], vb[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) kb[j] = kp[j * 64 + c * 4 + g];
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int n = 0; n < 4; ++n) vb[m * 4 + n] = vp[m * 256 + (16 * n + c) * 4 + g];
        if (p == pages - 1) {
            // Value slots past the block's last position: zero.
#pragma unroll
            for (int m = 0; m < 4; ++m)
                if (p * kPage + 4 * m + g > last)
#pragma unroll
                    for (int n = 0; n < 4; ++n) vb[m * 4 + n] = 0.0f;
        }
        const int key = p * kPage + c;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            f4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 16; ++j) s = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[h][j], kb[j], s, 0, 0, 0);
            // Per row a reference maximum, raised (and the sums rescaled)
            // only when one of the row's scores exceeds it by more than
            // kRescale, so the probabilities stay below e^16 and most pages
            // need no row maximum at all. A row with no unmasked key yet in
            // this wavefront's pages keeps maximum -inf and sums 0. Each
            // row's raises depend on its own scores only.
            float sv[4];
            bool need = false;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int qpos = min(pos0 + 4 * g + i, last);
                sv[i] = key <= qpos ? s[i] : -__builtin_inff();
                need |= sv[i] > mx[h][i] + kRescale;
            }
            if (__builtin_amdgcn_ballot_w64(need)) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float pm = row16_max(sv[i]);
                    if (pm > mx[h][i] + kRescale) {  // uniform in the row's lane group
                        const float keep = __expf(mx[h][i] - pm);  // 0 from maximum -inf
                        ls[h][i] *= keep;
                        o[h][0][i] *= keep;
                        o[h][1][i] *= keep;
                        o[h][2][i] *= keep;
                        o[h][3][i] *= keep;
                        mx[h][i] = pm;
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float pv = sv[i] != -__builtin_inff() ? __expf(sv[i] - mx[h][i]) : 0.0f;
                ls[h][i] += pv;
                p_s[wave][h][4 * g + i][c] = pv;
            }
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const float a = p_s[wave][h][c][4 * m + g];
#pragma unroll
                for (int n = 0; n < 4; ++n) o[h][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vb[m * 4 + n], o[h][n], 0, 0, 0);
            }
        __builtin_amdgcn_wave_barrier();
    }
    // Each row's denominator: the sum of its 16 lanes' shares (lane group g
    // holds rows 4g..4g+3). A wavefront without pages holds maximum -inf,
    // sums 0 and outputs 0, and takes no part below.
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float l = row_sum(ls[h][i]);
            if (c == 0) {
                ml_s[wave][h][4 * g + i][0] = mx[h][i];
                ml_s[wave][h][4 * g + i][1] = l;
            }
        }
    if (wave > 0)
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int n = 0; n < 4; ++n) o_s[wave - 1][h][n][lane] = o[h][n];
    __syncthreads();
    if (wave != 0) return;
    // Wavefront 0: the wavefronts' results in order, then the block's rows.
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 4 * g + i;
            float m = ml_s[0][h][r][0];
#pragma unroll
            for (int w = 1; w < W; ++w) m = fmaxf(m, ml_s[w][h][r][0]);  // finite: page 0 is wave 0's
            float f[W], l = 0.0f;
#pragma unroll
            for (int w = 0; w < W; ++w) {
                f[w] = __expf(ml_s[w][h][r][0] - m);
                l += ml_s[w][h][r][1] * f[w];
            }
#pragma unroll
            for (int n = 0; n < 4; ++n) {
                float v = o[h][n][i] * f[0];
#pragma unroll
                for (int w = 1; w < W; ++w) v += o_s[w - 1][h][n][lane][i] * f[w];
                if (r < nrows) out[quad_index(row0 + r, (kvh * G + h) * kDim + 16 * n + c, ldo)] = v / l;
            }
        }
}

}  // namespace

bool fast_prefill_fits(int heads, int kv_heads, const PagedKv& kv) {
    const int G = kv_heads > 0 ? heads / kv_heads : 0;
    return kv.block_tokens == kPage && kv.kv_width == kv_heads * kDim && G >= 1 && G <= 4 && G * kv_heads == heads;
}

hipError_t launch_fast_prefill(hipStream_t s, const float* qkv, int ldq, int heads, int kv_heads, const PagedKv& kv,
                               int layer, const int32_t* items, int count, float* out, int ldo) {
    if (count <= 0) return hipSuccess;
    if (!fast_prefill_fits(heads, kv_heads, kv)) return hipErrorInvalidValue;
    const dim3 grid(count);
    const int4* it = reinterpret_cast<const int4*>(items);
    switch (heads / kv_heads) {
    case 1: fast_prefill_kernel<1><<<grid, kWaves * 64, 0, s>>>(qkv, ldq, kv, layer, it, count, kv_heads, out, ldo); break;
    case 2: fast_prefill_kernel<2><<<grid, kWaves * 64, 0, s>>>(qkv, ldq, kv, layer, it, count, kv_heads, out, ldo); break;
    case 3: fast_prefill_kernel<3><<<grid, kWaves * 64, 0, s>>>(qkv, ldq, kv, layer, it, count, kv_heads, out, ldo); break;
    default: fast_prefill_kernel<4><<<grid, kWaves * 64, 0, s>>>(qkv, ldq, kv, layer, it, count, kv_heads, out, ldo); break;
    }
    return hipGetLastError();
}

}  // namespace mphip
