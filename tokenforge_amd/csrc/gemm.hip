// Prefill-shaped W4A16 GEMM (M >= 16): LDS-staged tiles feeding v_mfma_f32_32x32x16_f16.
//
// Per K block (BK <= group size, so one scale and one zero per column per block):
//   * x tile [BM][BK] fp16 is copied global -> registers -> LDS;
//   * the packed weight tile (BN columns x BK, tile layout) is loaded with 128-bit loads, dequantized in
//     registers (fp16(q - z) * s, one rounding) and stored to LDS as fp16 [BN][BK];
//   * each wave reads its A/B fragments (8 consecutive K values per lane, the operand
//     layout of the 32x32x16 MFMA) and accumulates fp32.
// Two LDS buffers: the global loads of block i+1 are issued before the MFMAs of block i,
// and their LDS stores after, so one barrier per K block suffices. LDS rows are padded by
// 16 bytes so the 16-byte fragment reads of 16 consecutive rows hit distinct banks.
//
// Split-K (grid.z > 1) writes fp32 partials [split][M][N] to the caller's workspace; a
// second kernel sums them in split order, adds the bias and rounds once (w4a16.py:227-232),
// so the result does not depend on scheduling.
#include "linear.h"
#include "tile_layout.h"

namespace tf {
namespace {

template <int BM, int BN, int BK, int WM, int WN>
__global__ __launch_bounds__(WM * WN * 64) void gemm_kernel(LinearArgs a, float* __restrict__ ws,
                                                            int split_k) {
  constexpr int T = WM * WN * 64;
  constexpr int LD = BK + 8;  // fp16 elements per LDS row
  constexpr int TM = BM / WM / 32;
  constexpr int TN = BN / WN / 32;
  constexpr int A_CHUNKS = BM * BK / 8;     // 16-byte chunks of the x tile
  constexpr int B_CHUNKS = BN * BK / 32;    // 16-byte chunks (4 words) of the weight tile
  constexpr int A_PER = (A_CHUNKS + T - 1) / T;
  constexpr int B_PER = (B_CHUNKS + T - 1) / T;
  static_assert(TM >= 1 && TN >= 1, "wave tile must hold at least one 32x32 MFMA tile");
  static_assert(BK % 32 == 0, "BK must be a multiple of 32");

  __shared__ __attribute__((aligned(16))) _Float16 As[2][BM][LD];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN][LD];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int z = blockIdx.z;
  const int nkb = a.k / BK;
  const int kb0 = (int)(((int64_t)z * nkb) / split_k);
  const int kb1 = (int)(((int64_t)(z + 1) * nkb) / split_k);
  const int64_t q_total = a.k >> 5;
  const int64_t groups = a.k >> a.log2g;

  u4 ra[A_PER];
  u4 rb[B_PER];
  uint32_t rs[B_PER];
  uint32_t rz[B_PER];

  auto load_global = [&](int kb) {
    const int k0 = kb * BK;
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const int id = tid + i * T;
      const int row = id / (BK / 8);
      const int c8 = id % (BK / 8);
      const int m = m0 + row;
      if (id < A_CHUNKS && m < a.m)
        ra[i] = *reinterpret_cast<const u4*>(a.x + (int64_t)m * a.ldx + k0 + c8 * 8);
      else
        ra[i] = u4{0u, 0u, 0u, 0u};
    }
    const int grp = k0 >> a.log2g;
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const int id = tid + i * T;
      const int col = id / (BK / 32);
      const int kc = id % (BK / 32);
      const int n = n0 + col;
      if (id < B_CHUNKS && n < a.n) {  // tile layout (tile_layout.h)
        rb[i] = *reinterpret_cast<const u4*>(a.qw + tile_chunk(n, (k0 >> 5) + kc, a.n, q_total) * 4);
        rs[i] = a.scales[tile_scale(grp, n, a.n, groups)];
        rz[i] = a.qz[tile_zero(grp, n >> 3, a.n, groups)];
      } else {
        rb[i] = u4{0u, 0u, 0u, 0u};
        rs[i] = 0u;
        rz[i] = 0u;
      }
    }
  };

  auto store_lds = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_PER; ++i) {
      const int id = tid + i * T;
      if (id < A_CHUNKS) {
        const int row = id / (BK / 8);
        const int c8 = id % (BK / 8);
        *reinterpret_cast<u4*>(&As[buf][row][c8 * 8]) = ra[i];
      }
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      const int id = tid + i * T;
      if (id < B_CHUNKS) {
        const int col = id / (BK / 32);
        const int kc = id % (BK / 32);
        const QuantParams p = make_params(zero_of(rz[i], (uint32_t)(n0 + col)), rs[i]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          h2 d[4];
          dequant_word(rb[i][j], p, d);
          u4 o;
          o[0] = as_u32(d[0]);
          o[1] = as_u32(d[1]);
          o[2] = as_u32(d[2]);
          o[3] = as_u32(d[3]);
          *reinterpret_cast<u4*>(&Bs[buf][col][kc * 32 + j * 8]) = o;
        }
      }
    }
  };

  f16v acc[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[tm][tn][r] = 0.0f;

  if (kb0 < kb1) {
    load_global(kb0);
    store_lds(0);
  }
  __syncthreads();

  int buf = 0;
  for (int kb = kb0; kb < kb1; ++kb) {
    const bool more = kb + 1 < kb1;
    if (more) load_global(kb + 1);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      h8 af[TM];
      h8 bf[TN];
      const int kcol = kk * 16 + (lane >> 5) * 8;
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        af[tm] = *reinterpret_cast<const h8*>(&As[buf][(wm * TM + tm) * 32 + (lane & 31)][kcol]);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
        bf[tn] = *reinterpret_cast<const h8*>(&Bs[buf][(wn * TN + tn) * 32 + (lane & 31)][kcol]);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
          acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[tm], bf[tn], acc[tm][tn], 0, 0, 0);
    }
    if (more) store_lds(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }

  // D layout of the 32x32 MFMA: register r of lane l is row 8*(r/4) + 4*(l/32) + r%4,
  // column l%32. A SiLU*mul epilogue pairs columns n and n + N/2 of different tiles: without
  // split-K the fp16 y goes to the workspace for silu_mul_kernel, with split-K the fp32
  // partials go to the reduce kernel.
  const bool partials = split_k > 1;
  const bool stage_y = !partials && a.epilogue == TF_EPILOGUE_SILU_MUL;
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int n = n0 + (wn * TN + tn) * 32 + (lane & 31);
      if (n >= a.n) continue;
      const float b = (!partials && a.bias) ? half_bits_to_float(a.bias[n]) : 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + (wm * TM + tm) * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
        if (m >= a.m) continue;
        const float v = acc[tm][tn][r] * row_scale(a, m) + b;
        if (stage_y)
          reinterpret_cast<uint16_t*>(ws)[(int64_t)m * a.n + n] = f16_bits(v);
        else if (!partials)
          store_out(a, m, n, v);
        else
          ws[((int64_t)z * a.m + m) * a.n + n] = acc[tm][tn][r];
      }
    }
}

// Sum of the split partials of element (row, col) in split order, times the row scale, plus
// bias.
__device__ __forceinline__ float reduce_partials(const float* __restrict__ ws, const uint16_t* __restrict__ bias,
                                                 int64_t total, int64_t i, int64_t col, int split, float rs) {
  float v = ws[i];
  for (int s = 1; s < split; ++s) v += ws[(int64_t)s * total + i];
  v = v * rs;
  if (bias) v += half_bits_to_float(bias[col]);
  return v;
}

// One thread per output element; under SiLU*mul the output has N/2 columns and each thread
// reduces its gate column j and up column N/2 + j.
__global__ void splitk_reduce_kernel(LinearArgs a, const float* __restrict__ ws, int split) {
  const int n_out = a.epilogue == TF_EPILOGUE_SILU_MUL ? a.n >> 1 : a.n;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.m * n_out) return;
  const int64_t row = i / n_out;
  const int64_t col = i % n_out;
  const int64_t total = (int64_t)a.m * a.n;
  const float rs = row_scale(a, (int)row);
  const float v = reduce_partials(ws, a.bias, total, row * a.n + col, col, split, rs);
  if (a.epilogue == TF_EPILOGUE_SILU_MUL) {
    const float u = reduce_partials(ws, a.bias, total, row * a.n + n_out + col, n_out + col, split, rs);
    a.out[row * a.ldo + col] = finish_silu_mul(v, u);
  } else {
    store_out(a, (int)row, (int)col, v);
  }
}

// Four consecutive columns per thread (NONE / RESIDUAL epilogues, N and the strides in
// 4-element units): every split's 16-byte load is issued before the sums, which add in split
// order as reduce_partials does, and the run is stored as one 8-byte piece.
__global__ __launch_bounds__(256) void splitk_reduce4_kernel(LinearArgs a, const float* __restrict__ ws, int split) {
  const int64_t total = (int64_t)a.m * a.n;
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i >= total) return;
  const int row = (int)(i / a.n);
  const int col = (int)(i - (int64_t)row * a.n);
  f4 p[kMaxSplitK];
#pragma unroll
  for (int s = 0; s < kMaxSplitK; ++s)
    if (s < split) p[s] = *reinterpret_cast<const f4*>(ws + (int64_t)s * total + i);
  const float rs = row_scale(a, row);
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float acc = p[0][j];
#pragma unroll
    for (int s = 1; s < kMaxSplitK; ++s)
      if (s < split) acc += p[s][j];
    acc = acc * rs;
    if (a.bias) acc += half_bits_to_float(a.bias[col + j]);
    v[j] = acc;
  }
  store_run4(a, a.out, a.ldo, a.epilogue == TF_EPILOGUE_RESIDUAL, row, col, v, true);
}

}  // namespace

// SiLU*mul over an fp16 y [m, n] (row stride n) staged in the workspace.
__global__ void silu_mul_kernel(LinearArgs a, const uint16_t* __restrict__ y) {
  const int half = a.n >> 1;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)a.m * half) return;
  const int64_t row = i / half;
  const int64_t col = i % half;
  a.out[row * a.ldo + col] =
      finish_silu_mul(half_bits_to_float(y[row * a.n + col]), half_bits_to_float(y[row * a.n + half + col]));
}

int silu_mul_staged(const LinearArgs& a, const float* ws, hipStream_t stream) {
  const int64_t total = (int64_t)a.m * (a.n >> 1);
  silu_mul_kernel<<<(unsigned)cdiv(total, 256), 256, 0, stream>>>(a, reinterpret_cast<const uint16_t*>(ws));
  return check_launch("tf_w4a16_linear(silu_mul)");
}

int splitk_reduce(const LinearArgs& a, const float* ws, int split, hipStream_t stream) {
  const bool residual = a.epilogue == TF_EPILOGUE_RESIDUAL;
  const auto al = [](const void* p, uintptr_t b) { return (reinterpret_cast<uintptr_t>(p) & (b - 1)) == 0; };
  if (a.epilogue != TF_EPILOGUE_SILU_MUL && split <= kMaxSplitK && (a.n & 3) == 0 && (a.ldo & 3) == 0 &&
      al(a.out, 8) && al(ws, 16) && (!residual || ((a.ldr & 3) == 0 && al(a.residual, 8)))) {
    const int64_t runs = (int64_t)a.m * a.n / 4;
    splitk_reduce4_kernel<<<(unsigned)cdiv(runs, 256), 256, 0, stream>>>(a, ws, split);
    return check_launch("tf_w4a16_linear(splitk_reduce)");
  }
  const int64_t total = (int64_t)a.m * (a.epilogue == TF_EPILOGUE_SILU_MUL ? a.n >> 1 : a.n);
  splitk_reduce_kernel<<<(unsigned)cdiv(total, 256), 256, 0, stream>>>(a, ws, split);
  return check_launch("tf_w4a16_linear(splitk_reduce)");
}

// Workspace of an LDS-tile GEMM launch: fp32 partials under split-K, the fp16 y under a
// SiLU*mul epilogue without split-K, else none.
int64_t lds_gemm_workspace(const LinearArgs& a, int split) {
  if (split > 1) return (int64_t)split * a.m * a.n * (int64_t)sizeof(float);
  if (a.epilogue == TF_EPILOGUE_SILU_MUL) return (int64_t)a.m * a.n * 2;
  return 0;
}

// The kernel after an LDS-tile GEMM launch, if any.
int lds_gemm_finish(const LinearArgs& a, const float* ws, int split, hipStream_t stream) {
  if (split > 1) return splitk_reduce(a, ws, split, stream);
  if (a.epilogue == TF_EPILOGUE_SILU_MUL) return silu_mul_staged(a, ws, stream);
  return TF_OK;
}

namespace {

int effective_split(const LinearArgs& a, const tf_gemm_config& cfg) {
  const int nkb = a.k / cfg.block_k;
  return cfg.split_k < nkb ? cfg.split_k : (nkb > 0 ? nkb : 1);
}

int64_t gemm_workspace(const LinearArgs& a, const tf_gemm_config& cfg) {
  return lds_gemm_workspace(a, effective_split(a, cfg));
}

template <int BM, int BN, int BK, int WM, int WN>
int launch_gemm(const LinearArgs& a, const tf_gemm_config& cfg, float* ws, hipStream_t stream) {
  const int split = effective_split(a, cfg);
  if (lds_gemm_workspace(a, split) > 0 && ws == nullptr)
    return fail(TF_EINVAL, "tf_w4a16_linear: this config needs a workspace");
  const dim3 grid((unsigned)cdiv(a.n, BN), (unsigned)cdiv(a.m, BM), (unsigned)split);
  gemm_kernel<BM, BN, BK, WM, WN><<<grid, WM * WN * 64, 0, stream>>>(a, ws, split);
  if (int rc = check_launch("tf_w4a16_linear(gemm_mfma)")) return rc;
  return lds_gemm_finish(a, ws, split, stream);
  return TF_OK;
}

#define TF_GEMM(BM, BN, BK, WM, WN) \
  {{TF_KERNEL_GEMM_MFMA, BM, BN, BK, 1, WM * WN, 2}, (launch_gemm<BM, BN, BK, WM, WN>), gemm_workspace}

const Variant kGemmVariants[] = {
    TF_GEMM(64, 64, 64, 2, 2),   TF_GEMM(64, 128, 64, 2, 2),  TF_GEMM(128, 64, 64, 2, 2),
    TF_GEMM(128, 128, 64, 2, 2), TF_GEMM(128, 256, 64, 2, 2), TF_GEMM(256, 128, 64, 2, 2),
    TF_GEMM(256, 256, 64, 2, 2), TF_GEMM(64, 64, 32, 2, 2),   TF_GEMM(128, 128, 32, 2, 2),
    TF_GEMM(256, 128, 32, 2, 2),
};

}  // namespace

const Variant* gemm_variants(int* count) {
  *count = (int)(sizeof(kGemmVariants) / sizeof(kGemmVariants[0]));
  return kGemmVariants;
}

}  // namespace tf
