// Shared device helpers for the gfx950 kernels of the quantized-linear path.
//
// Conventions:
//  * fp16 values travel as raw 16-bit patterns (uint16_t) across the C ABI and as
//    clang _Float16 vectors inside kernels, so every conversion is explicit.
//  * Packed int4 words use the AWQ nibble order: nibble i (bits 4i..4i+3) holds offset
//    AWQ_ORDER[i] = {0,2,4,6,1,3,5,7}[i]; offset j lives in nibble (j%2)*4 + j/2
//    (pack.py:32-36 in the reference).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/tokenforge_hip.h"

namespace tf {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------------ host-side errors

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

// ------------------------------------------------------------------ bit casts

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ float as_f32(uint32_t v) { return __builtin_bit_cast(float, v); }
__device__ __forceinline__ uint32_t as_u32(float v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ float half_bits_to_float(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}

// Nibble position of offset j inside a packed word: AWQ_REVERSE_ORDER[j] = (j%2)*4 + j/2.
__host__ __device__ __forceinline__ uint32_t awq_nibble_of(uint32_t j) {
  return (j & 1u) * 4u + (j >> 1);
}

// ------------------------------------------------------------------ buffer loads

// Raw buffer resources (V#): base, byte size, no stride. A load whose byte offset lies at
// or past the size returns zeros without touching memory, which is how the kernels handle
// ragged edges without branches. Dword 3 = 0x00020000 selects the raw 32-bit data format of
// the gfx9 family (gfx950 included).
constexpr int kBufferFlags = 0x00020000;
constexpr uint32_t kOutOfRange = 0x80000000u;  // any offset >= every size used here

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferFlags);
}
__device__ __forceinline__ u4 load_b128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t load_b32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ __forceinline__ uint32_t load_b16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}
__device__ __forceinline__ u2 load_b64(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
}

// Eight OCP e4m3fn codes (two words) -> eight fp16 values, exactly (every e4m3fn value, NaN
// included, is an fp16 value; the round-toward-zero pack therefore does not round).
__device__ __forceinline__ u4 e4m3x8_to_f16(u2 codes) {
  u4 r;
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)codes[w], false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)codes[w], true);
    r[2 * w] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo[0], lo[1]));
    r[2 * w + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(hi[0], hi[1]));
  }
  return r;
}

// ------------------------------------------------------------------ zero/scale operands

// Per-(group, column) constants for the dequantization of one packed word.
//   zlo = fp16x2(1024 + z): subtrahend for nibbles at bits 0-3 / 16-19 (0x6400 magic)
//   zhi = fp16x2(64 + z):   subtrahend for nibbles at bits 4-7 / 20-23 (0x5400 magic)
//   s   = fp16x2(scale)
struct QuantParams {
  h2 zlo;
  h2 zhi;
  h2 s;
};

__device__ __forceinline__ QuantParams make_params(uint32_t z, uint32_t scale_bits) {
  QuantParams p;
  const uint32_t lo = 0x6400u | z;          // 1024 + z  (ulp of 1024 is 1)
  const uint32_t hi = 0x5400u | (z << 4);   // 64 + z    (ulp of 64 is 1/16)
  p.zlo = as_h2(lo | (lo << 16));
  p.zhi = as_h2(hi | (hi << 16));
  p.s = as_h2(scale_bits | (scale_bits << 16));
  return p;
}

// Zero-point nibble of column n from its qzeros word (pack.py:35; w4a16.py:38-40).
__device__ __forceinline__ uint32_t zero_of(uint32_t zword, uint32_t n) {
  return (zword >> (4u * awq_nibble_of(n & 7u))) & 0xFu;
}

// Unpack masks and magic exponents kept in VGPRs: gfx9 VOP3 takes no literal operands, so
// with literals the compiler splits (w & m) | e into two instructions; from registers it is
// a single v_and_or_b32.
struct UnpackConsts {
  uint32_t m_lo;  // 0x000F000F
  uint32_t m_hi;  // 0x00F000F0
  uint32_t e_lo;  // 0x64006400: fp16x2 1024
  uint32_t e_hi;  // 0x54005400: fp16x2 64
};

__device__ __forceinline__ UnpackConsts unpack_consts() {
  UnpackConsts c{0x000F000Fu, 0x00F000F0u, 0x64006400u, 0x54005400u};
  __asm__ volatile("" : "+v"(c.m_lo), "+v"(c.m_hi), "+v"(c.e_lo), "+v"(c.e_hi));
  return c;
}

// Dequantize the eight int4 values of one packed word into fp16, K order:
// out[i] holds offsets (2i, 2i+1). (word & 0x000F000F) | 0x6400_6400 is the fp16x2 pair
// (1024 + q0, 1024 + q1) because nibble 0 holds offset 0 and nibble 4 offset 1; the 0x00F0
// nibbles become 64 + q with the 0x5400 magic. Subtracting (1024 + z) or (64 + z) is exact
// in fp16, so fp16(q - z) * s rounds exactly once (v_pk_mul_f16), matching pack.py:194 and
// w4a16.py:95 bit for bit.
__device__ __forceinline__ void dequant_word(uint32_t w, const QuantParams& p, const UnpackConsts& k,
                                             h2 out[4]) {
  const uint32_t w8 = w >> 8;
  const h2 a0 = as_h2((w & k.m_lo) | k.e_lo);
  const h2 a1 = as_h2((w & k.m_hi) | k.e_hi);
  const h2 a2 = as_h2((w8 & k.m_lo) | k.e_lo);
  const h2 a3 = as_h2((w8 & k.m_hi) | k.e_hi);
  out[0] = (a0 - p.zlo) * p.s;
  out[1] = (a1 - p.zhi) * p.s;
  out[2] = (a2 - p.zlo) * p.s;
  out[3] = (a3 - p.zhi) * p.s;
}

__device__ __forceinline__ void dequant_word(uint32_t w, const QuantParams& p, h2 out[4]) {
  dequant_word(w, p, UnpackConsts{0x000F000Fu, 0x00F000F0u, 0x64006400u, 0x54005400u}, out);
}

__device__ __forceinline__ h8 pack_h8(const h2 v[4]) {
  h8 r;
  r[0] = v[0][0]; r[1] = v[0][1];
  r[2] = v[1][0]; r[3] = v[1][1];
  r[4] = v[2][0]; r[5] = v[2][1];
  r[6] = v[3][0]; r[7] = v[3][1];
  return r;
}

// ------------------------------------------------------------------ cross-lane (DPP)

// Sum of v over the four lanes of each quad, fixed tree: (0+1)+(2+3) in every lane.
__device__ __forceinline__ float quad_sum(float v) {
  // quad_perm [1,0,3,2] = 0xB1, then [2,3,0,1] = 0x4E.
  float t = as_f32(__builtin_amdgcn_update_dpp(0, (int)as_u32(v), 0xB1, 0xF, 0xF, false));
  v = v + t;
  t = as_f32(__builtin_amdgcn_update_dpp(0, (int)as_u32(v), 0x4E, 0xF, 0xF, false));
  return v + t;
}

// ------------------------------------------------------------------ XCD placement

// MI355X hands workgroup b of a launch to XCD b % 8 (round robin over its 8 XCDs, each with
// its own L2). xcd_tile renumbers workgroups so every XCD works on one contiguous range of
// tiles: neighbouring tiles share cache lines (per-column scales and zero points, operand
// panels), which are then fetched into one L2 instead of several. A bijection on [0, nb).
constexpr int kXcds = 8;

__device__ __forceinline__ int xcd_tile(int b, int nb) {
  const int q = nb / kXcds;
  const int r = nb % kXcds;
  const int x = b % kXcds;
  return x * q + (x < r ? x : r) + b / kXcds;
}

// ------------------------------------------------------------------ misc

__host__ __device__ constexpr int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace tf
