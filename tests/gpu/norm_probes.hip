// Exhaustive on-device check of the RMSNorm+FP8 dynamic-scale quotient (norm_row.h), run
// by tests/gpu/test_norm_quotient.py. A test fixture: built into a library of its own
// (tests/gpu/lib/libtokenforge_norm_probes.so), which the product library never contains or calls.
//
// Workgroup b takes the fp16 absmax with bits b + 1 (every positive finite fp16), derives the
// row scale s with dynamic_scale() and r = fp32(1 / s) as the kernel does, and runs every
// finite fp16 y of both signs through the kernel's encode (quotient_dynamic, v_med3 clamp,
// encode4_clamped). The reference is the IEEE fp32 division y / s, clamped with compares and
// encoded by e4m3_encode, the encoder pinned against torch's cast. Three counts per absmax:
//   bad_codes:   codes that differ (the claim under test: zero);
//   bad_scale:   1 when dynamic_scale(amax) != max(IEEE amax / 448, 1 / (448 * 512));
//   uncorrected: y for which fp32(y * r) alone differs from y / s, which shows that the
//                correction is needed and that the check sees a wrong quotient.
#include "../../tokenforge_amd/csrc/fp8.h"
#include "../../tokenforge_amd/csrc/norm_row.h"

namespace {

constexpr int kThreads = 256;
constexpr int kScales = 0x7BFF;  // positive finite fp16 bit patterns 0x0001 .. 0x7BFF

__device__ uint8_t reference_code(float y, float s) {
  float v = y / s;
  v = (v < -tf::kFp8Max) ? -tf::kFp8Max : v;
  v = (v > tf::kFp8Max) ? tf::kFp8Max : v;
  return tf::e4m3_encode(v);
}

__device__ uint32_t block_total(uint32_t v, uint32_t* red) {
  red[threadIdx.x] = v;
  __syncthreads();
  for (int off = kThreads / 2; off > 0; off >>= 1) {
    if ((int)threadIdx.x < off) red[threadIdx.x] += red[threadIdx.x + off];
    __syncthreads();
  }
  return red[0];
}

__global__ __launch_bounds__(kThreads) void norm_quotient_check_kernel(uint32_t* bad_codes, uint32_t* bad_scale,
                                                                       uint32_t* uncorrected) {
  __shared__ uint32_t red[kThreads];
  const int b = blockIdx.x;  // grid = kScales: b + 1 <= 0x7BFF
  const float amax = (float)__builtin_bit_cast(_Float16, (uint16_t)(b + 1));
  const float s = tf::dynamic_scale(amax);
  const float s_ieee = amax / tf::kFp8Max;
  const float s_ref = (s_ieee < tf::kMinScale) ? tf::kMinScale : s_ieee;
  const float r = 1.0f / s;
  uint32_t nbad = 0, nunc = 0;
  for (uint32_t y = threadIdx.x; y < 0x8000u; y += kThreads) {
    if (y >= 0x7C00u) continue;  // inf and NaN: rows holding them take the exact slow path
    const uint32_t bits = y | ((y | 0x8000u) << 16);  // +y in the low half, -y in the high half
    const tf::h2 pair = tf::as_h2(bits);
    const float lo = __builtin_amdgcn_fmed3f(tf::quotient_dynamic<false>(pair, s, r), -tf::kFp8Max, tf::kFp8Max);
    const float hi = __builtin_amdgcn_fmed3f(tf::quotient_dynamic<true>(pair, s, r), -tf::kFp8Max, tf::kFp8Max);
    const uint32_t got = tf::encode4_clamped(lo, hi, 0.0f, 0.0f) & 0xFFFFu;
    const float yf = (float)pair[0];
    const uint32_t want = (uint32_t)reference_code(yf, s) | ((uint32_t)reference_code(-yf, s) << 8);
    nbad += got != want;
    nunc += tf::as_u32(yf * r) != tf::as_u32(yf / s);
  }
  const uint32_t tb = block_total(nbad, red);
  __syncthreads();
  const uint32_t tu = block_total(nunc, red);
  if (threadIdx.x == 0) {
    bad_codes[b] = tb;
    uncorrected[b] = tu;
    bad_scale[b] = tf::as_u32(s) != tf::as_u32(s_ref);
  }
}

}  // namespace

// Fills three arrays of 0x7BFF counts (one per positive finite fp16 absmax, in bit order):
// code mismatches, scale mismatches and uncorrected-quotient differences (see above).
// Returns 0, 1 (null pointer) or 2 (launch error).
extern "C" int tfp_norm_quotient_check(uint32_t* bad_codes, uint32_t* bad_scale, uint32_t* uncorrected,
                                       void* stream) {
  if (!bad_codes || !bad_scale || !uncorrected) return 1;
  norm_quotient_check_kernel<<<kScales, kThreads, 0, (hipStream_t)stream>>>(bad_codes, bad_scale, uncorrected);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Number of counts each array of tfp_norm_quotient_check holds.
extern "C" int tfp_norm_quotient_scales() { return kScales; }
