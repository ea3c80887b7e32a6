// sc_arith.hpp - exact arithmetic shortcuts of the quantizing tiles, on the hardware's fast instructions.
//
// div127(a): a / 127 for a >= 0 (not NaN), equal to the IEEE quotient: one product with the correctly rounded 1/127
// and one fused correction (Markstein's method: P. Markstein, "Computation of elementary functions on the IBM RISC
// System/6000 processor", IBM J. Res. Dev. 34(1), 1990).  127 = 1.984375 x 2^6 is one of the divisors the test
// suite's exhaustive quotient check covers, so the result is the IEEE quotient wherever nothing leaves the normal
// range; below it (a < 2^-100) both lie far below the smallest binary16 and round to the same +0.  +inf stays +inf.
//
// recip_normal(d): 1 / d from v_rcp_f32 (accurate to 1 ulp) and one fused Newton correction, equal to the IEEE
// quotient 1.0f / d for every d with 2^-126 <= |d| < 2^126 (recip_normal_ok), checked over every such binary32 input
// on the device (tests/test_gpu_convert.py).  Outside that range v_rcp_f32 does not keep subnormal inputs or
// results, and the caller divides.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sc {

__device__ __forceinline__ float div127(float a) {
#pragma clang fp contract(off)
    constexpr float kInv127 = 1.0f / 127.0f;
    const float q0 = a * kInv127;
    const float q = __builtin_fmaf(__builtin_fmaf(-q0, 127.0f, a), kInv127, q0);
    return a == __builtin_inff() ? a : q;
}

__device__ __forceinline__ bool recip_normal_ok(float d) {
    const float m = __builtin_fabsf(d);
    return m >= 0x1p-126f && m < 0x1p126f;
}

__device__ __forceinline__ float recip_normal(float d) {
#pragma clang fp contract(off)
    const float r0 = __builtin_amdgcn_rcpf(d);
    return __builtin_fmaf(__builtin_fmaf(-d, r0, 1.0f), r0, r0);
}

}  // namespace sc
