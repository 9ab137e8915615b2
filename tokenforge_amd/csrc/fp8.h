// OCP float8_e4m3fn encoding from the format definition (no vendor conversion routine).
//
// e4m3fn: 1 sign bit, 4 exponent bits with bias 7, 3 mantissa bits, no infinities,
// S.1111.111 is NaN. Largest finite value 448 = 1.75 * 2^8, smallest normal 2^-6,
// subnormals are m * 2^-9 for m = 1..7.
#pragma once

#include "tf_common.h"

namespace tf {

// Round-to-nearest-even of an fp32 value with |v| <= 448 (or NaN) onto e4m3fn, the
// rounding that rmsnorm_fp8.py:29-41 applies before its cast. Signed zeros are kept.
__device__ __forceinline__ uint8_t e4m3_encode(float v) {
  const uint32_t bits = as_u32(v);
  const uint32_t sign = (bits >> 24) & 0x80u;
  const uint32_t a = bits & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint8_t)(sign | 0x7Fu);  // NaN
  if (a < 0x3C800000u) {
    // |v| < 2^-6: fixed quantum 2^-9. |v| * 512 is exact; rint rounds half to even.
    // A result of 8 is the code 0x08, i.e. the smallest normal 2^-6.
    const float t = as_f32(a) * 512.0f;
    return (uint8_t)(sign | (uint32_t)__builtin_rintf(t));
  }
  // Normal: keep 3 of the 23 mantissa bits, ties to even; a carry out of the mantissa
  // correctly bumps the exponent. Re-bias the exponent from 127 to 7.
  const uint32_t r = a + 0x7FFFFu + ((a >> 20) & 1u);
  return (uint8_t)(sign | ((r >> 20) - (120u << 3)));
}

// The same rounding through v_cvt_pk_fp8_f32 (two values per instruction on gfx950). It
// agrees with e4m3_encode on every fp32 with |v| <= 448 (checked exhaustively on MI355X) and
// writes 0xFF for every NaN; NaN inputs therefore take e4m3_encode, which keeps the sign.
__device__ __forceinline__ uint8_t e4m3_encode_hw(float v) {
  if (v != v) return e4m3_encode(v);
  return (uint8_t)((uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v, 0.0f, 0, false) & 0xFFu);
}

}  // namespace tf
