// Exact fp32 quotients of the fused RMSNorm + e4m3 quantization (reference.py:37-49), shared by
// the kernel (rmsnorm_fp8.hip) and the exhaustive on-device check of the dynamic-scale form
// (probes/norm_probes.hip).
//
// Quotient y / scale (reference.py:47-49), two exact forms:
// * static scales: fp32(fp64(y) * fp64(1 / scale)) with the reciprocal correctly rounded in
//   fp64. This equals the IEEE fp32 division for every fp16 y and fp32 scale: the fp64 product
//   is within 2^-52 (relative) of y / scale, while a quotient of an 11-bit by a 24-bit
//   significand that is not exactly representable lies at least ~2^-49 (relative) away from
//   every fp32 rounding boundary, so both round alike (the zero, infinite and NaN cases follow
//   IEEE multiplication by 0, inf or NaN the same way).
// * dynamic scales: Markstein's correction in fp32, r = fp32(1 / scale) correctly rounded,
//   q0 = y * r, e = fma(q0, scale, -y) (exact), q = fma(-e, r, q0). Three fp32 operations on
//   the fp16 y instead of two conversions and an fp64 product. It equals the IEEE division
//   for every finite fp16 y and every scale a row can produce, max(fp32(amax / 448),
//   1 / (448 * 512)) over all finite fp16 amax: checked exhaustively on MI355X (31743 scales
//   x 63488 y). The residual is formed as q0 * scale - y, not y - q0 * scale, so that y = -0
//   gives q = -0 (the other sign order would sum +0 and -0 to +0).
//
// Per-row divisions: mean = fp32(fp64(sum) * fp64(1 / h)) and amax / 448 =
// fp32(fp64(amax) * fp64(1 / 448)) equal the IEEE fp32 quotients. A quotient of a 24-bit
// (11-bit) significand by an integer below 2^15 is either exactly representable, or at least
// 2^-40 (relative) away from every fp32 rounding boundary, as its significand is an integer
// over the divisor's odd part; the fp64 product is within 2^-52 of it.
#pragma once

#include "tf_common.h"

namespace tf {

constexpr float kFp8Max = 448.0f;
constexpr float kMinScale = 1.0f / (448.0f * 512.0f);  // reference.py:10

// The dynamic scale of a row from its absmax (reference.py:47-48): max(fp32(amax / 448),
// kMinScale), the quotient as fp32(fp64(amax) * fp64(1 / 448)); clamp(min=...) keeps NaN.
__device__ __forceinline__ float dynamic_scale(float amax) {
  const float raw = (float)((double)amax * (1.0 / (double)kFp8Max));
  return (raw < kMinScale) ? kMinScale : raw;
}

__device__ __forceinline__ float quotient(_Float16 y, double rcp) { return (float)((double)(float)y * rcp); }

// fp32(y) * r for the fp16 y in the low (HI false) or high half of `pair`, as one v_fma_mix_f32
// that reads the fp16 operand directly (the backend does not form it from a multiply). The
// addend is -0, so the sum is the rounded product for every sign, zeros included.
template <bool HI>
__device__ __forceinline__ float mul_f16_f32(uint32_t pair, float r) {
  float q;
  if (HI)
    __asm__("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(q) : "v"(pair), "v"(r), "v"(-0.0f));
  else
    __asm__("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(q) : "v"(pair), "v"(r), "v"(-0.0f));
  return q;
}

// y / s for the fp16 y in half HI of `pair` and a dynamic scale s, given r = fp32(1 / s)
// (Markstein's correction, see the top of this file).
template <bool HI>
__device__ __forceinline__ float quotient_dynamic(h2 pair, float s, float r) {
  const float yf = (float)pair[HI ? 1 : 0];
  const float q0 = mul_f16_f32<HI>(as_u32(pair), r);
  const float e = __builtin_fmaf(q0, s, -yf);
  return __builtin_fmaf(-e, r, q0);
}

// Four clamped fp32 values -> four e4m3fn codes in one word (bytes in order).
__device__ __forceinline__ uint32_t encode4_clamped(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, __builtin_bit_cast(int, a), false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

}  // namespace tf
