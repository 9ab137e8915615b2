// Shared plumbing of the W4A16 linear kernels: argument bundle and variant registry.
#pragma once

#include "tf_common.h"

namespace tf {

// One W4A16 linear call (w4a16.py:178-232). Pointers are device pointers; x rows and the
// qweight_t rows are 16-byte aligned (checked by tf_w4a16_linear).
struct LinearArgs {
  const uint16_t* x;       // fp16 [m, k], row stride ldx
  int64_t ldx;
  const uint32_t* qw;      // qweight_t [n, k/8]
  const uint16_t* scales;  // fp16 [k/g, n]
  const uint32_t* qz;      // qzeros [k/g, n/8]
  const uint16_t* bias;    // fp16 [n] or nullptr
  uint16_t* out;           // fp16 [m, n], row stride ldo
  int64_t ldo;
  int m;
  int n;
  int k;
  int log2g;               // log2(group_size)
  // Epilogue (TF_EPILOGUE_*): NONE writes y; RESIDUAL writes fp16(residual + fp16(y)) (out may
  // be residual itself, element for element); SILU_MUL writes [m, n / 2]:
  // fp16(fp16(silu(fp16(y[:, j]))) * fp16(y[:, n / 2 + j])).
  int epilogue = TF_EPILOGUE_NONE;
  const uint16_t* residual = nullptr;  // fp16 [m, n], row stride ldr
  int64_t ldr = 0;
  // W4A8 input (tf_w4a8_linear_ex): e4m3fn codes [m, k] with row stride ldx8 bytes, read by
  // the kernels that stage x (others get x converted to fp16 in `x`), and the fp32 row scales
  // of x applied to each row's sum before the bias: y = xscale[m] * sum + bias.
  const uint8_t* x8 = nullptr;
  int64_t ldx8 = 0;
  const float* xscale = nullptr;  // [m] with stride xscale_stride (0: one scale for all rows)
  int64_t xscale_stride = 0;
  // RMSNorm + e4m3 prologue (tf_rmsnorm_fp8_w4a16_linear, decode GEMV stream form only): x holds
  // the rows before the norm; the kernel normalizes each with weight norm_w (fp16 [k], 16-byte
  // aligned) and norm_eps, quantizes it to e4m3 with its dynamic scale and multiplies with
  // fp16(code * scale), the activation rmsnorm_fp8_quant_dq writes for the row.
  const uint16_t* norm_w = nullptr;
  float norm_eps = 0.0f;
  double norm_inv_k = 0.0;  // fp64(1 / k)
};

// Row scale of row m (1 without a W4A8 input, and for rows past m, which are never stored).
__device__ __forceinline__ float row_scale(const LinearArgs& a, int m) {
  return (a.xscale != nullptr && m < a.m) ? a.xscale[(int64_t)m * a.xscale_stride] : 1.0f;
}

// Column mapping of the fused SiLU*mul epilogue for kernels that hold a 16-column group in
// one row of 16 lanes: local column l of the tile at n_base takes the gate row
// n_base / 2 + 8 (l / 16) + l % 8 when l % 16 < 8, else the up row n / 2 + that; lanes l and
// l ^ 8 then hold the gate and up values of one output column. Without the epilogue the
// mapping is the identity n_base + l.
__device__ __forceinline__ int phys_col(const LinearArgs& a, int n_base, int l) {
  if (a.epilogue != TF_EPILOGUE_SILU_MUL) return n_base + l;
  const int j = (n_base >> 1) + ((l >> 4) << 3) + (l & 7);
  return (l & 8) ? (a.n >> 1) + j : j;
}

// Output column of local column l under the SiLU*mul mapping (valid on the gate lanes).
__device__ __forceinline__ int silu_out_col(int n_base, int l) { return (n_base >> 1) + ((l >> 4) << 3) + (l & 7); }

// True when the physical column of local column l holds data (inside N; for SiLU*mul, its
// output column inside n / 2).
__device__ __forceinline__ bool col_valid(const LinearArgs& a, int n_base, int l) {
  if (a.epilogue != TF_EPILOGUE_SILU_MUL) return n_base + l < a.n;
  return silu_out_col(n_base, l) < (a.n >> 1);
}

__device__ __forceinline__ uint16_t f16_bits(float v) { return __builtin_bit_cast(uint16_t, (_Float16)v); }

// fp16(residual + fp16(v)): the unfused `residual + linear(x)` of two fp16 tensors.
__device__ __forceinline__ uint16_t finish_residual(float v, uint16_t r) {
  const float y = (float)(_Float16)v;
  return f16_bits(y + half_bits_to_float(r));
}

// fp16(fp16(silu(fp16(g))) * fp16(u)): torch's fp16 silu (x / (1 + exp(-x)) in fp32, one
// rounding) followed by its fp16 multiply, on the rounded linear outputs.
__device__ __forceinline__ uint16_t finish_silu_mul(float g, float u) {
  const float g16 = (float)(_Float16)g;
  const float u16 = (float)(_Float16)u;
  const float s16 = (float)(_Float16)(g16 / (1.0f + expf(-g16)));
  return f16_bits(s16 * u16);
}

// Write one output value v (= acc + bias, fp32) of row m, physical column n under the
// NONE / RESIDUAL epilogues.
__device__ __forceinline__ void store_out(const LinearArgs& a, int m, int n, float v) {
  uint16_t r = f16_bits(v);
  if (a.epilogue == TF_EPILOGUE_RESIDUAL) r = finish_residual(v, a.residual[(int64_t)m * a.ldr + n]);
  a.out[(int64_t)m * a.ldo + n] = r;
}

// Kernels whose accumulators hold runs of four consecutive output columns of one row (the
// MFMA with the weight fragment as its first operand) store each run as one 8-byte piece where
// N, the row strides and the pointers are in 4-element units.
__device__ __forceinline__ bool run_store_ok(const LinearArgs& a, const uint16_t* dst, int64_t ldd, bool residual) {
  return (a.n & 3) == 0 && (ldd & 3) == 0 && (reinterpret_cast<uintptr_t>(dst) & 7) == 0 &&
         (!residual || ((a.ldr & 3) == 0 && (reinterpret_cast<uintptr_t>(a.residual) & 7) == 0));
}

// Columns n .. n + 3 of row m (v: acc * row scale + bias in fp32) to dst (row stride ldd) as
// fp16, or as fp16(residual + fp16(v)) under the residual epilogue: the values store_out
// writes. vec: run_store_ok holds (then a run is inside N or past it); else per value, the
// columns past N skipped.
__device__ __forceinline__ void store_run4(const LinearArgs& a, uint16_t* dst, int64_t ldd, bool residual, int m,
                                           int n, const float (&v)[4], bool vec) {
  if (vec) {
    uint16_t h[4];
    if (residual) {
      const u2 res = *reinterpret_cast<const u2*>(a.residual + (int64_t)m * a.ldr + n);
#pragma unroll
      for (int j = 0; j < 4; ++j) h[j] = finish_residual(v[j], (uint16_t)(res[j >> 1] >> (16 * (j & 1))));
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) h[j] = f16_bits(v[j]);
    }
    *reinterpret_cast<u2*>(dst + (int64_t)m * ldd + n) =
        u2{(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
    return;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (n + j >= a.n) break;
    uint16_t r = f16_bits(v[j]);
    if (residual) r = finish_residual(v[j], a.residual[(int64_t)m * a.ldr + n + j]);
    dst[(int64_t)m * ldd + n + j] = r;
  }
}

// ------------------------------------------------------------------ launch helpers

// LDS bytes one workgroup may use on the current device (160 KiB on gfx950), queried once
// per device.
inline size_t device_max_lds() {
  static size_t cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 64 * 1024;
  if (cache[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
      v = 64 * 1024;
    cache[dev] = (size_t)v;
  }
  return cache[dev];
}

// Dynamic LDS above 64 KiB must be enabled per kernel before the launch.
template <typename Kernel>
inline int reserve_lds(Kernel kernel, size_t bytes, const char* name) {
  if (bytes > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)bytes) != hipSuccess)
    return fail(TF_ELAUNCH, std::string("tf_w4a16_linear: cannot reserve LDS for ") + name);
  return TF_OK;
}

// Buffer offsets are 32-bit: every byte offset into qweight_t, scales, qzeros and x must fit
// (the streaming kernels address them through buffer resources).
inline int check_offsets(const LinearArgs& a) {
  const int64_t x_bytes = ((int64_t)(a.m - 1) * a.ldx + a.k) * 2;
  const int64_t w_bytes = (int64_t)a.n * (a.k / 2);
  if (x_bytes >= (int64_t)kOutOfRange || w_bytes >= (int64_t)kOutOfRange)
    return fail(TF_EINVAL, "tf_w4a16_linear: gemv kernels need x and qweight_t below 2 GiB");
  return TF_OK;
}

using LaunchFn = int (*)(const LinearArgs&, const tf_gemm_config&, float* workspace,
                         hipStream_t stream);
using WorkspaceFn = int64_t (*)(const LinearArgs&, const tf_gemm_config&);
// The checks a launch function makes before it launches anything (TF_OK or an error), for
// callers that must reject a call before they queue work of their own (tf_w4a8_linear_ex).
using CheckFn = int (*)(const LinearArgs&, const tf_gemm_config&);

// A compiled kernel variant: cfg holds (kernel, block_m, block_n, block_k, num_warps,
// num_stages) with split_k = 1. check may be null when the launch function rejects nothing
// beyond what tf_w4a16_linear_ex checks first.
struct Variant {
  tf_gemm_config cfg;
  LaunchFn launch;
  WorkspaceFn workspace;
  CheckFn check = nullptr;
};

const Variant* gemv_variants(int* count);
const Variant* gemv_stream_variants(int* count);
const Variant* gemm_variants(int* count);
const Variant* gemm2_variants(int* count);
const Variant* gemm3_variants(int* count);
const Variant* gemm4_variants(int* count);
const Variant* gemm8_variants(int* count);

int check_group_size(int32_t group_size, int64_t k, const char* name);
int log2_group(int32_t g);

// Upper bound on the split-K factor of any kernel.
constexpr int kMaxSplitK = 16;

}  // namespace tf
