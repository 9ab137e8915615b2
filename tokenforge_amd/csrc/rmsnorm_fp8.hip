// Fused RMSNorm + OCP e4m3fn quantization: one HBM read of x, one write of the codes.
//
// One workgroup per token row. The row stays in registers between the two reductions
// (sum of squares, then absmax). The sum of squares is accumulated in fp64: every x^2 of
// an fp16 x is exact, so the fp64 total is the exact sum up to ~2^-53 relative and its
// rounding to fp32 does not depend on the summation order. The kernel is therefore
// deterministic and matches a correctly rounded fp32 restatement bit for bit; torch's
// fp32 `mean` (reference.py:37) can differ from it by an ulp of var on some rows.
#include "fp8.h"
#include "tf_common.h"

namespace tf {
namespace {

constexpr float kFp8Max = 448.0f;

// fp16(fp32(a * b)): reference.py:39 rounds x * rstd to fp32 and then to fp16. Left alone,
// the backend folds the multiply and the conversion into v_fma_mixlo_f16, which rounds once,
// straight to fp16, and differs from the double rounding on ~6e-5 of the elements. The empty
// asm makes the fp32 product a register value, so it is rounded to fp32 first.
__device__ __forceinline__ _Float16 mul_round_f32_then_f16(float a, float b) {
  float p = a * b;
  __asm__ volatile("" : "+v"(p));
  return (_Float16)p;
}
constexpr float kMinScale = 1.0f / (448.0f * 512.0f);  // reference.py:10

__device__ __forceinline__ float nan_max(float a, float b) { return (a > b || a != a) ? a : b; }

template <int WAVES>
__device__ __forceinline__ double block_sum(double v, double* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  double t = red[0];
#pragma unroll
  for (int i = 1; i < WAVES; ++i) t += red[i];
  return t;
}

template <int WAVES>
__device__ __forceinline__ float block_nan_max(float v, float* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = nan_max(v, __shfl_xor(v, off, 64));
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int i = 1; i < WAVES; ++i) t = nan_max(t, red[i]);
  return t;
}

// CPT: 8-element chunks per thread. VEC: 16-byte x / weight loads and 8-byte code stores.
template <int WAVES, int CPT, bool VEC>
__global__ __launch_bounds__(WAVES * 64) void rmsnorm_fp8_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ w,
    uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale, int static_scale, int h,
    float eps) {
  constexpr int kThreads = WAVES * 64;
  __shared__ double red_d[WAVES];
  __shared__ float red_f[WAVES];

  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * ldx;
  const int tid = threadIdx.x;

  _Float16 xv[CPT][8];
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int e0 = (tid + i * kThreads) * 8;
    if (VEC) {
      if (e0 < h) {
        const u4 raw = *reinterpret_cast<const u4*>(xr + e0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const h2 p = as_h2(raw[j]);
          xv[i][2 * j] = p[0];
          xv[i][2 * j + 1] = p[1];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[i][j] = (_Float16)0.0f;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        xv[i][j] = (e0 + j < h) ? __builtin_bit_cast(_Float16, xr[e0 + j]) : (_Float16)0.0f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const double d = (double)(float)xv[i][j];
      ss += d * d;
    }
  }
  const double total = block_sum<WAVES>(ss, red_d);

  // reference.py:37-38: var = mean(x^2) in fp32, rstd = 1 / sqrt(var + eps), IEEE ops.
  const float var = (float)total / (float)h;
  const float rstd = 1.0f / __builtin_sqrtf(var + eps);

  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int e0 = (tid + i * kThreads) * 8;
    _Float16 wv[8];
    if (VEC) {
      if (e0 < h) {
        const u4 raw = *reinterpret_cast<const u4*>(w + e0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const h2 p = as_h2(raw[j]);
          wv[2 * j] = p[0];
          wv[2 * j + 1] = p[1];
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) wv[j] = (_Float16)0.0f;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        wv[j] = (e0 + j < h) ? __builtin_bit_cast(_Float16, w[e0 + j]) : (_Float16)0.0f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      // reference.py:39: fp16(x * rstd) in fp32 then cast, times weight in fp16 (one rounding).
      const _Float16 nrm = mul_round_f32_then_f16((float)xv[i][j], rstd);
      const _Float16 y = nrm * wv[j];
      xv[i][j] = y;  // the row is reused in place for y
      if (e0 + j < h) amax = nan_max(amax, __builtin_fabsf((float)y));
    }
  }

  float s;
  if (static_scale) {
    s = scale[0];
  } else {
    __syncthreads();  // red_f is disjoint from red_d, but keep the two reductions ordered
    const float m = block_nan_max<WAVES>(amax, red_f);
    const float raw = m / kFp8Max;
    s = (raw < kMinScale) ? kMinScale : raw;  // clamp(min=...) keeps NaN
    if (tid == 0) scale[row] = s;
  }

  uint8_t* qr = q + row * ldq;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int e0 = (tid + i * kThreads) * 8;
    uint8_t codes[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float v = (float)xv[i][j] / s;
      v = (v < -kFp8Max) ? -kFp8Max : v;
      v = (v > kFp8Max) ? kFp8Max : v;
      codes[j] = e4m3_encode(v);
    }
    if (VEC) {
      if (e0 < h) {
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          lo |= (uint32_t)codes[j] << (8 * j);
          hi |= (uint32_t)codes[4 + j] << (8 * j);
        }
        *reinterpret_cast<uint2*>(qr + e0) = make_uint2(lo, hi);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (e0 + j < h) qr[e0 + j] = codes[j];
    }
  }
}

template <int WAVES, int CPT>
int launch_cpt(bool vec, const uint16_t* x, int64_t ldx, const uint16_t* w, uint8_t* q, int64_t ldq,
               float* scale, int static_scale, int64_t t, int h, float eps, hipStream_t stream) {
  if (vec)
    rmsnorm_fp8_kernel<WAVES, CPT, true>
        <<<(unsigned)t, WAVES * 64, 0, stream>>>(x, ldx, w, q, ldq, scale, static_scale, h, eps);
  else
    rmsnorm_fp8_kernel<WAVES, CPT, false>
        <<<(unsigned)t, WAVES * 64, 0, stream>>>(x, ldx, w, q, ldq, scale, static_scale, h, eps);
  return check_launch("tf_rmsnorm_fp8_quant");
}

template <int WAVES>
int launch_waves(int cpt, bool vec, const uint16_t* x, int64_t ldx, const uint16_t* w, uint8_t* q,
                 int64_t ldq, float* scale, int static_scale, int64_t t, int h, float eps,
                 hipStream_t stream) {
  switch (cpt) {
    case 1: return launch_cpt<WAVES, 1>(vec, x, ldx, w, q, ldq, scale, static_scale, t, h, eps, stream);
    case 2: return launch_cpt<WAVES, 2>(vec, x, ldx, w, q, ldq, scale, static_scale, t, h, eps, stream);
    case 4: return launch_cpt<WAVES, 4>(vec, x, ldx, w, q, ldq, scale, static_scale, t, h, eps, stream);
    case 8: return launch_cpt<WAVES, 8>(vec, x, ldx, w, q, ldq, scale, static_scale, t, h, eps, stream);
    default: return launch_cpt<WAVES, 16>(vec, x, ldx, w, q, ldq, scale, static_scale, t, h, eps, stream);
  }
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace
}  // namespace tf

using namespace tf;

extern "C" int tf_rmsnorm_fp8_quant(const uint16_t* x, int64_t ldx, const uint16_t* weight,
                                    uint8_t* q, int64_t ldq, float* scale, int32_t static_scale,
                                    int64_t t, int64_t h, float eps, void* stream) {
  if (!x || !weight || !q || !scale) return fail(TF_EINVAL, "tf_rmsnorm_fp8_quant: null pointer");
  if (t < 0 || h <= 0) return fail(TF_EINVAL, "tf_rmsnorm_fp8_quant: need t >= 0 and h > 0");
  if (ldx < h || ldq < h) return fail(TF_EINVAL, "tf_rmsnorm_fp8_quant: row stride smaller than h");
  if (t > 0x7FFFFFFF) return fail(TF_EINVAL, "tf_rmsnorm_fp8_quant: too many rows");
  if (h > 16 * 8 * 256) return fail(TF_EINVAL, "tf_rmsnorm_fp8_quant: h above 32768 is not supported");
  if (t == 0) return TF_OK;
  const int64_t chunks = cdiv(h, 8);
  const int waves = chunks >= 512 ? 4 : (chunks >= 256 ? 2 : 1);
  const int64_t per = cdiv(chunks, waves * 64);
  const int cpt = per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : per <= 8 ? 8 : 16;
  const bool vec = (h % 8 == 0) && (ldx % 8 == 0) && (ldq % 8 == 0) && aligned(x, 16) &&
                   aligned(weight, 16) && aligned(q, 8);
  hipStream_t s = (hipStream_t)stream;
  const int hh = (int)h;
  switch (waves) {
    case 1: return launch_waves<1>(cpt, vec, x, ldx, weight, q, ldq, scale, static_scale, t, hh, eps, s);
    case 2: return launch_waves<2>(cpt, vec, x, ldx, weight, q, ldq, scale, static_scale, t, hh, eps, s);
    default: return launch_waves<4>(cpt, vec, x, ldx, weight, q, ldq, scale, static_scale, t, hh, eps, s);
  }
}
