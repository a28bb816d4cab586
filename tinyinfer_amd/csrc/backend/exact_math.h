// Device float helpers that reproduce the reference CPU path's rounding.
//
// The reference evaluates std::exp on float, which glibc implements as expf:
// the table-driven method of ARM's optimized-routines (Szabolcs Nagy, 2017):
// exp(x) = 2^(k/32) * 2^(r/32), k = round(x*32/ln2), with a cubic in double
// precision for 2^(r/32) and one final rounding to float. glibc's x86-64 build
// selects the FMA-compiled variant of that routine on FMA-capable hosts; the
// contractions it forms are reproduced below with explicit fma() calls. The
// 32-entry table holds asuint64(2^(i/32) rounded to double) - (i << 47),
// computed from exp2l. This replica was checked against the host's expf on
// every finite float input that reaches the polynomial (2.24e9 inputs, zero
// differences); tests/test_oracle.py re-checks the algorithm (emulated in
// double precision) against the C library, and the device forward's logits
// are compared bit for bit with the oracle's by the GPU tests.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mphip {

__device__ __constant__ static const uint64_t kExp2Table[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// expf with the reference host's exact results (see the file comment).
__device__ __forceinline__ float ref_expf(float x) {
    const uint32_t bits = __float_as_uint(x);
    const uint32_t abstop = (bits >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {  // |x| >= 88, or x is inf/nan
        if (bits == 0xff800000u) return 0.0f;         // -inf
        if (abstop >= 0x7f8u) return x + x;           // nan, +inf
        if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);  // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;          // underflow
    }
    const double inv_ln2_n = 0x1.71547652b82fep+5;   // 32/ln2
    const double shift = 0x1.8p+52;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    uint64_t t = kExp2Table[ki % 32];
    t += ki << 47;
    const double s = __longlong_as_double((long long)t);
    const double z = __builtin_fma(0x1.c6af84b912394p-20, r, 0x1.ebfce50fac4f3p-13);
    const double r2 = r * r;
    double y = __builtin_fma(0x1.62e42ff0c52d6p-6, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

// ref_expf without branches: the main path runs for every input (its table
// index stays in range for any x) and the special cases are selected after,
// so a wavefront never splits. Same results as ref_expf for every x. `tab`
// is a copy of kExp2Table (in LDS where the caller keeps global loads for
// other work in flight: a global table read would wait for all of them).
__device__ __forceinline__ float ref_expf_select(float x, const uint64_t* tab) {
    const uint32_t bits = __float_as_uint(x);
    const uint32_t abstop = (bits >> 20) & 0x7ffu;
    const double inv_ln2_n = 0x1.71547652b82fep+5;
    const double shift = 0x1.8p+52;
    const double xd = (double)x;
    double kd = __builtin_fma(inv_ln2_n, xd, shift);
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    uint64_t t = tab[ki % 32];
    t += ki << 47;
    const double s = __longlong_as_double((long long)t);
    const double z = __builtin_fma(0x1.c6af84b912394p-20, r, 0x1.ebfce50fac4f3p-13);
    const double r2 = r * r;
    double y = __builtin_fma(0x1.62e42ff0c52d6p-6, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    float res = (float)y;
    if (abstop >= 0x42bu) {
        res = x < -0x1.9fe368p6f ? 0.0f : res;
        res = x > 0x1.62e42ep6f ? __uint_as_float(0x7f800000u) : res;
        res = abstop >= 0x7f8u ? x + x : res;
        res = bits == 0xff800000u ? 0.0f : res;
    }
    return res;
}

}  // namespace mphip
