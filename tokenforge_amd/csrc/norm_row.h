// Row arithmetic of the fused RMSNorm + e4m3 quantization (reference.py:37-49): the exact
// fp32 quotients, the roundings, the encode and decode of the codes and the wave reductions.
// Shared by the norm kernel (rmsnorm_fp8.hip), the decode GEMV's RMSNorm prologue
// (gemv_stream.hip) and the exhaustive on-device check of the dynamic-scale form
// (probes/norm_probes.hip), so that all of them compute the same bits.
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

#include "fp8.h"
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


// y / s for a row that is not on the fast path (a NaN or infinite absmax, or a static scale
// that is not positive and finite), given rcp = fp64(1 / s): clamped to +-448 with compares
// that keep NaN, then encoded with the sign of a NaN kept (e4m3_encode).
__device__ __forceinline__ uint8_t encode_slow(_Float16 y, double rcp) {
  float v = quotient(y, rcp);
  v = (v < -kFp8Max) ? -kFp8Max : v;
  v = (v > kFp8Max) ? kFp8Max : v;
  return e4m3_encode(v);
}

// fp16(fp32(a * b)): reference.py:39 rounds x * rstd to fp32 and then to fp16. Left alone,
// the backend folds the multiply and the conversion into v_fma_mixlo_f16, which rounds once,
// straight to fp16, and differs from the double rounding on ~6e-5 of the elements. The empty
// asm makes the fp32 product a register value, so it is rounded to fp32 first.
__device__ __forceinline__ _Float16 mul_round_f32_then_f16(float a, float b) {
  float p = a * b;
  __asm__ volatile("" : "+v"(p));
  return (_Float16)p;
}

__device__ __forceinline__ uint32_t f16_bits_of(_Float16 v) { return __builtin_bit_cast(uint16_t, v); }

// fp16(fp32(code) * s) of four codes (one word): the activation a W4A16 linear reads when it is
// fed from the codes, as `(q.to(float32) * scale).to(float16)` computes it. Every e4m3fn code,
// NaN included, decodes exactly; the product is rounded to fp32 and then to fp16.
__device__ __forceinline__ u2 dequant_codes4(uint32_t codes, float s) {
  const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)codes, false);
  const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)codes, true);
  const uint32_t h0 = f16_bits_of(mul_round_f32_then_f16(lo[0], s));
  const uint32_t h1 = f16_bits_of(mul_round_f32_then_f16(lo[1], s));
  const uint32_t h2 = f16_bits_of(mul_round_f32_then_f16(hi[0], s));
  const uint32_t h3 = f16_bits_of(mul_round_f32_then_f16(hi[1], s));
  return u2{h0 | (h1 << 16), h2 | (h3 << 16)};
}

// Lane exchanges inside a row of 16 lanes (DPP, no LDS): swap neighbours, swap pairs, mirror
// each half row, mirror the row. Applied in that order, each pairs every lane with one holding
// a disjoint set of the row's lanes, so four steps leave the row's total in all 16 lanes.
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1, 0, 3, 2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfRowMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint64_t lo = dpp_u32<CTRL>((uint32_t)b), hi = dpp_u32<CTRL>((uint32_t)(b >> 32));
  return __builtin_bit_cast(double, lo | (hi << 32));
}
__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, lane);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), lane);
  return __builtin_bit_cast(double, lo | (hi << 32));
}

// Sum of a wave's 64 lanes (every lane active), wave-uniform: four DPP steps leave each row of
// 16 lanes holding its row's total, then the four row totals are read and added. The order is
// pairwise over the lane index ((l0 + l1) + (l2 + l3), ...; fp add commutes, so every lane of
// a step forms the same sums), which the fixed sum-of-squares order below relies on.
__device__ __forceinline__ double wave_sum_f64(double v) {
  v += dpp_f64<kDppQuadXor1>(v);
  v += dpp_f64<kDppQuadXor2>(v);
  v += dpp_f64<kDppHalfRowMirror>(v);
  v += dpp_f64<kDppRowMirror>(v);
  return (readlane_f64(v, 0) + readlane_f64(v, 16)) + (readlane_f64(v, 32) + readlane_f64(v, 48));
}

// ------------------------------------------------------------------ sum of squares order
//
// Every form of the norm adds the squares of a row in one fixed order, so a row's var does not
// depend on the form, the batch size or the fusion (reference.py:37 leaves the order to torch):
// elements in chunks of 8 (the row zero-padded), each chunk as ((e0 + e1) + (e2 + e3)) +
// ((e4 + e5) + (e6 + e7)) with e = fp64(x)^2 (exact for fp16 x), then the chunk sums pairwise,
// bottom up over the chunk index, the count zero-padded to a power of two (zeros change no
// partial sum, so any larger power of two gives the same total). The forms write their chunk
// sums to LDS and each wave reduces them: lane l adds the R consecutive sums l R .. l R + R - 1
// pairwise (the low bits of the chunk index), then the 64 lane totals are added pairwise by
// wave_sum_f64 (the next six bits).

// Sum of squares of one 8-element chunk (four fp16 pairs, element 2j in the low half of pair j).
// fma(d0, d0, d1 * d1) rounds d0^2 + d1^2 once, as the add of the two exact squares does.
__device__ __forceinline__ double chunk_sum_squares(const h2 (&v)[4]) {
  double p[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const double d0 = (double)(float)v[j][0], d1 = (double)(float)v[j][1];
    p[j] = __builtin_fma(d0, d0, d1 * d1);
  }
  return (p[0] + p[1]) + (p[2] + p[3]);
}

// Pairwise sum of the R values at p[0 .. R) (R a power of two), recursive halves.
template <int R>
__device__ __forceinline__ double pairwise_lds(const double* p) {
  if constexpr (R == 1) {
    return p[0];
  } else if constexpr (R == 2) {
    const double2 v = *reinterpret_cast<const double2*>(p);
    return v.x + v.y;
  } else {
    return pairwise_lds<R / 2>(p) + pairwise_lds<R / 2>(p + R / 2);
  }
}

// Unsigned max of a wave's 64 lanes (every lane active), wave-uniform.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = __builtin_elementwise_max(v, dpp_u32<kDppQuadXor1>(v));
  v = __builtin_elementwise_max(v, dpp_u32<kDppQuadXor2>(v));
  v = __builtin_elementwise_max(v, dpp_u32<kDppHalfRowMirror>(v));
  v = __builtin_elementwise_max(v, dpp_u32<kDppRowMirror>(v));
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return __builtin_elementwise_max(__builtin_elementwise_max(a, b), __builtin_elementwise_max(c, d));
}

// The row total of 64 R chunk sums in LDS (R a power of two; entries past the row's chunks hold
// zeros) in the fixed order, computed by one wave (every lane active); wave-uniform.
template <int R>
__device__ __forceinline__ double row_total_lds(const double* sums) {
  const int lane = threadIdx.x & 63;
  return wave_sum_f64(pairwise_lds<R>(sums + lane * R));
}

// The same for a runtime count of chunks: R = L / 64 (L, a power of two from 64 to 64 RMAX, at
// least the chunk count); each lane reads its R sums into a zero-filled set of RMAX, which has
// the same pairwise total as the R.
template <int RMAX>
__device__ __forceinline__ double row_total_lds_rt(const double* sums, int r) {
  const int lane = threadIdx.x & 63;
  double v[RMAX];
#pragma unroll
  for (int i = 0; i < RMAX; ++i) v[i] = i < r ? sums[lane * r + i] : 0.0;
#pragma unroll
  for (int w = RMAX; w > 1; w /= 2)
#pragma unroll
    for (int i = 0; i < w / 2; ++i) v[i] = v[2 * i] + v[2 * i + 1];
  return wave_sum_f64(v[0]);
}

}  // namespace tf
