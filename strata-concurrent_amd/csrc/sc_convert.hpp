// sc_convert.hpp - binary32 <-> binary16 conversions of the handoff kernels, on the conversion instructions.
//
// f16_bits_rne: IEEE-754 binary32 -> binary16, round to nearest even, as raw bits.  Finite values too large for f16
// become infinities, an f32 infinity stays one and a NaN becomes the quiet NaN sign | 0x7C00 | 0x200, the convention
// of the reference's f16_from_f32 (include/strata/kernels/f16_bits.hpp:37-70).  v_cvt_f16_f32 rounds by the mode
// register (round to nearest even, f16 denormals kept: the HIP defaults); only its NaN payload differs from that
// convention, so a NaN takes the convention's bits by a select.
//
// f16_bits_rne_not_nan: the same for inputs that are never NaN, without the select.
//
// f32_of_f16: binary16 -> binary32 (v_cvt_f32_f16), exact for every non-NaN value including the subnormals.
//
// Both are checked over every input on the device against the CPU oracle (all 2^32 binary32 patterns, all 2^16
// binary16 patterns) by a probe library of the test suite that includes this header.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sc {

__device__ __forceinline__ uint32_t f16_bits_rne(uint32_t x) {
    const float f = __uint_as_float(x);
    const uint32_t h = uint32_t(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f)));
    return f != f ? (((x >> 16) & 0x8000u) | 0x7E00u) : h;
}

// f16_bits_rne for an input known not to be NaN (the conversion instruction alone).
__device__ __forceinline__ uint32_t f16_bits_rne_not_nan(float f) {
    return uint32_t(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f)));
}

__device__ __forceinline__ float f32_of_f16(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

}  // namespace sc
