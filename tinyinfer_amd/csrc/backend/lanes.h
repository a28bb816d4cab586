// Cross-lane helpers of the fast-mode kernels on the vector ALU: DPP row
// operations within a row of 16 lanes and lane reads into scalar registers,
// instead of LDS permutes (a __shfl_xor is a ds_bpermute, ~100 cycles of
// latency per step). All lanes of the wavefront must be active.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mphip {

// DPP controls (GFX9): quad permutations and rotations within a 16-lane row.
constexpr int kDppQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppRowRor4 = 0x124;
constexpr int kDppRowRor8 = 0x128;

template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, true));
}
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, kCtrl, 0xF, 0xF, true);
}

// Sum / max over the 4 lanes of a quad (every lane gets the result).
__device__ __forceinline__ float quad_sum(float v) {
    v += dpp<kDppQuadXor1>(v);
    return v + dpp<kDppQuadXor2>(v);
}
// Over lanes i, i+4, i+8, i+12 of a 16-lane row (every lane gets the
// result): with quad-uniform values, the row's 4 quads.
__device__ __forceinline__ float row_quads_sum(float v) {
    v += dpp<kDppRowRor4>(v);
    return v + dpp<kDppRowRor8>(v);
}
__device__ __forceinline__ float row_quads_max(float v) {
    v = fmaxf(v, dpp<kDppRowRor4>(v));
    return fmaxf(v, dpp<kDppRowRor8>(v));
}
// Over all 16 lanes of a row.
__device__ __forceinline__ float row_sum(float v) { return row_quads_sum(quad_sum(v)); }

// Lane `l`'s value, uniform across the wavefront.
__device__ __forceinline__ float lane_value(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
// Of row-uniform values: the sum / max over the four rows, in row order.
__device__ __forceinline__ float rows_sum(float v) {
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}
__device__ __forceinline__ float rows_max(float v) {
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

}  // namespace mphip
