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
};

using LaunchFn = int (*)(const LinearArgs&, const tf_gemm_config&, float* workspace,
                         hipStream_t stream);
using WorkspaceFn = int64_t (*)(const LinearArgs&, const tf_gemm_config&);

// A compiled kernel variant: cfg holds (kernel, block_m, block_n, block_k, num_warps,
// num_stages) with split_k = 1.
struct Variant {
  tf_gemm_config cfg;
  LaunchFn launch;
  WorkspaceFn workspace;
};

const Variant* gemv_variants(int* count);
const Variant* gemm_variants(int* count);
const Variant* gemm2_variants(int* count);
const Variant* gemm3_variants(int* count);

int check_group_size(int32_t group_size, int64_t k, const char* name);
int log2_group(int32_t g);

// Upper bound on the split-K factor of any kernel.
constexpr int kMaxSplitK = 16;

}  // namespace tf
