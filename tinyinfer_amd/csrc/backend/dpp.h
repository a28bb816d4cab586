// Row broadcasts through DPP (gfx950). A wavefront's 64 lanes form four
// 16-lane rows; row_newbcast:I hands lane I of each row to the whole row.
// Data replicated across the four rows (lane l holding element l % 16 of a
// 16-element vector) therefore reaches every lane with no LDS or scalar
// traffic, and the compiler folds the broadcast into the consuming VALU
// instruction (v_mul_f32_dpp).
#pragma once
#include <hip/hip_runtime.h>

namespace mphip {

typedef float f4v __attribute__((ext_vector_type(4)));

// w (lane I of this lane's 16-lane row) * x, rounded once.
template <int I>
__device__ __forceinline__ float mul_bcast(float w, float x) {
    static_assert(I >= 0 && I < 16, "row lane");
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(w), 0x150 + I, 0xf, 0xf, false)) * x;
}

// The same with the row lane chosen by an expression that is constant once
// the enclosing loops are unrolled.
__device__ __forceinline__ float mul_bcast_at(int i, float w, float x) {
    switch (i) {
    case 0: return mul_bcast<0>(w, x);
    case 1: return mul_bcast<1>(w, x);
    case 2: return mul_bcast<2>(w, x);
    case 3: return mul_bcast<3>(w, x);
    case 4: return mul_bcast<4>(w, x);
    case 5: return mul_bcast<5>(w, x);
    case 6: return mul_bcast<6>(w, x);
    case 7: return mul_bcast<7>(w, x);
    case 8: return mul_bcast<8>(w, x);
    case 9: return mul_bcast<9>(w, x);
    case 10: return mul_bcast<10>(w, x);
    case 11: return mul_bcast<11>(w, x);
    case 12: return mul_bcast<12>(w, x);
    case 13: return mul_bcast<13>(w, x);
    case 14: return mul_bcast<14>(w, x);
    default: return mul_bcast<15>(w, x);
    }
}

}  // namespace mphip
