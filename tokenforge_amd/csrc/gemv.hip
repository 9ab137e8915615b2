// Decode-shaped W4A16 kernels (small M): stream the packed weights once, dequantize in
// registers, accumulate in fp32.
//
// Work split: a workgroup owns block_n = 16 * RT consecutive rows of qweight_t (output
// columns); its num_warps waves take disjoint, contiguous K ranges of those rows (on-chip
// split-K) and their partial sums are added in wave order through LDS, so results are
// bit-identical from run to run. No workspace, no atomics.
//
// Memory stream: a "step" is 16 rows x 128 K values. Per step each lane issues one 128-bit
// buffer load per 16-row tile (4 packed words = 32 weights of one row), so each row receives
// a 64-byte run per load and consecutive steps complete the 128-byte lines. Every wave keeps
// a ring of P steps in flight: the loads of step s + P are issued as soon as step s has been
// consumed, so the HBM queue never drains while the wave computes. Buffer loads return zeros
// past the end of a tensor, which handles ragged N, partial last steps and unused M rows
// without branches.
//
//  * gemv_dot  (TF_KERNEL_GEMV_DOT): lane = (row c = lane/4, chunk g = lane%4). Each lane
//    accumulates its products with v_dot2_f32_f16; quads are reduced with DPP.
//  * gemv_mfma (TF_KERNEL_GEMV_MFMA): lane = (row c = lane%16, chunk g = lane/16), exactly the
//    B-operand layout of v_mfma_f32_16x16x32_f16 (8 consecutive K values per lane = one
//    packed word). The dequantized word goes straight into the MFMA and x rows are the A
//    operand, so the matrix core does the dot products and the VALU only unpacks and scales.
//    A rows m >= M only feed output rows that are discarded, so they need no masking.
#include "linear.h"

namespace tf {
namespace {

__device__ __forceinline__ void k_range(int wave, int waves, int nsteps, int* s0, int* s1) {
  *s0 = (int)(((int64_t)wave * nsteps) / waves);
  *s1 = (int)(((int64_t)(wave + 1) * nsteps) / waves);
}

// Buffer resources and per-launch constants shared by both kernels.
struct Streams {
  __amdgpu_buffer_rsrc_t qw, sc, qz, x;
  uint32_t row_bytes;  // K / 2
  int nchunks;         // K / 32
  int log2g;
  int n;
};

__device__ __forceinline__ Streams make_streams(const LinearArgs& a) {
  Streams s;
  s.row_bytes = (uint32_t)(a.k >> 1);
  s.qw = make_rsrc(a.qw, (uint32_t)a.n * s.row_bytes);
  s.sc = make_rsrc(a.scales, (uint32_t)((a.k >> a.log2g) * a.n * 2));
  s.qz = make_rsrc(a.qz, (uint32_t)((a.k >> a.log2g) * (a.n >> 3) * 4));
  s.x = make_rsrc(a.x, (uint32_t)(((int64_t)(a.m - 1) * a.ldx + a.k) * 2));
  s.nchunks = a.k >> 5;
  s.log2g = a.log2g;
  s.n = a.n;
  return s;
}

// Weights, scales and zero words of one step for RT row tiles.
template <int RT>
struct WeightSlot {
  u4 w[RT];
  uint32_t s[RT];
  uint32_t z[RT];
};

// Loads of (row n_base + rt*16 + c, chunk ch) for every rt; zeros when invalid.
template <int RT>
__device__ __forceinline__ void issue_weights(WeightSlot<RT>& slot, const Streams& st, int n_base,
                                              int c, int ch, bool kvalid) {
  const uint32_t grp = (uint32_t)(ch << 5) >> st.log2g;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int n = n_base + rt * 16 + c;
    const bool ok = kvalid && n < st.n;
    const uint32_t wo = ok ? (uint32_t)n * st.row_bytes + (uint32_t)ch * 16u : kOutOfRange;
    const uint32_t so = ok ? (grp * (uint32_t)st.n + (uint32_t)n) * 2u : kOutOfRange;
    const uint32_t zo = ok ? (grp * (uint32_t)(st.n >> 3) + (uint32_t)(n >> 3)) * 4u : kOutOfRange;
    slot.w[rt] = load_b128(st.qw, wo);
    slot.s[rt] = load_b16(st.sc, so);
    slot.z[rt] = load_b32(st.qz, zo);
  }
}

// ------------------------------------------------------------------------ gemv_dot

template <int MAXM, int RT>
struct DotSlot {
  WeightSlot<RT> wt;
  u4 x[MAXM][4];  // x[m][32 values of this lane's chunk]
};

template <int MAXM, int RT, int P, int MAXW>
__global__ __launch_bounds__(MAXW * 64) void gemv_dot_kernel(LinearArgs a) {
  extern __shared__ __attribute__((aligned(16))) float red[];  // [(waves - 1)][MAXM][RT][16]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const int g = lane & 3;
  const int c = lane >> 2;
  const int n_base = blockIdx.x * 16 * RT;
  const Streams st = make_streams(a);
  const int nsteps = (st.nchunks + 3) >> 2;
  int s0, s1;
  k_range(wave, waves, nsteps, &s0, &s1);
  const UnpackConsts uc = unpack_consts();

  auto issue = [&](DotSlot<MAXM, RT>& slot, int step) {
    const int ch = step * 4 + g;
    const bool kvalid = step < s1 && ch < st.nchunks;
    issue_weights<RT>(slot.wt, st, n_base, c, ch, kvalid);
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
      const uint32_t xo = (kvalid && m < a.m) ? (uint32_t)(((int64_t)m * a.ldx + ch * 32) * 2) : kOutOfRange;
#pragma unroll
      for (int j = 0; j < 4; ++j) slot.x[m][j] = load_b128(st.x, xo + 16u * j);
    }
  };

  float acc[MAXM][RT];
#pragma unroll
  for (int m = 0; m < MAXM; ++m)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[m][rt] = 0.0f;

  DotSlot<MAXM, RT> ring[P];
#pragma unroll
  for (int p = 0; p < P; ++p) issue(ring[p], s0 + p);

  for (int s = s0; s < s1; s += P) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      if (s + p < s1) {
        DotSlot<MAXM, RT>& slot = ring[p];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const int n = n_base + rt * 16 + c;
          const QuantParams qp = make_params(zero_of(slot.wt.z[rt], (uint32_t)n), slot.wt.s[rt]);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            h2 wd[4];
            dequant_word(slot.wt.w[rt][j], qp, uc, wd);
#pragma unroll
            for (int m = 0; m < MAXM; ++m)
#pragma unroll
              for (int i = 0; i < 4; ++i)
                acc[m][rt] = __builtin_amdgcn_fdot2(as_h2(slot.x[m][j][i]), wd[i], acc[m][rt], false);
          }
        }
        issue(slot, s + p + P);
      }
    }
  }

#pragma unroll
  for (int m = 0; m < MAXM; ++m)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[m][rt] = quad_sum(acc[m][rt]);

  if (waves > 1) {
    if (wave > 0 && g == 0) {
#pragma unroll
      for (int m = 0; m < MAXM; ++m)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) red[(((wave - 1) * MAXM + m) * RT + rt) * 16 + c] = acc[m][rt];
    }
    __syncthreads();
    if (wave == 0) {
      for (int w = 1; w < waves; ++w)
#pragma unroll
        for (int m = 0; m < MAXM; ++m)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) acc[m][rt] += red[(((w - 1) * MAXM + m) * RT + rt) * 16 + c];
    }
  }
  if (wave == 0 && g == 0) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int n = n_base + rt * 16 + c;
      if (n >= a.n) continue;
      const float b = a.bias ? half_bits_to_float(a.bias[n]) : 0.0f;
#pragma unroll
      for (int m = 0; m < MAXM; ++m) {
        if (m < a.m)
          a.out[(int64_t)m * a.ldo + n] = __builtin_bit_cast(uint16_t, (_Float16)(acc[m][rt] + b));
      }
    }
  }
}

// ------------------------------------------------------------------------ gemv_mfma

template <int MT, int RT>
struct MfmaSlot {
  WeightSlot<RT> wt;
  h8 x[MT][4];  // A operand: row (m_base + mt*16 + c), the 32 values of this lane's chunk
};

template <int MT, int RT, int P, int MAXW>
__global__ __launch_bounds__(MAXW * 64) void gemv_mfma_kernel(LinearArgs a) {
  extern __shared__ __attribute__((aligned(16))) float red[];  // [(waves - 1)][MT][RT][64][4]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const int c = lane & 15;
  const int g = lane >> 4;
  const int n_base = blockIdx.x * 16 * RT;
  const int m_base = blockIdx.y * 16 * MT;
  const Streams st = make_streams(a);
  const int nsteps = (st.nchunks + 3) >> 2;
  int s0, s1;
  k_range(wave, waves, nsteps, &s0, &s1);
  const UnpackConsts uc = unpack_consts();

  auto issue = [&](MfmaSlot<MT, RT>& slot, int step) {
    const int ch = step * 4 + g;
    const bool kvalid = step < s1 && ch < st.nchunks;
    issue_weights<RT>(slot.wt, st, n_base, c, ch, kvalid);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = m_base + mt * 16 + c;
      const uint32_t xo = (kvalid && m < a.m) ? (uint32_t)(((int64_t)m * a.ldx + ch * 32) * 2) : kOutOfRange;
#pragma unroll
      for (int j = 0; j < 4; ++j) slot.x[mt][j] = __builtin_bit_cast(h8, load_b128(st.x, xo + 16u * j));
    }
  };

  f4 acc[MT][RT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[mt][rt] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  MfmaSlot<MT, RT> ring[P];
#pragma unroll
  for (int p = 0; p < P; ++p) issue(ring[p], s0 + p);

  for (int s = s0; s < s1; s += P) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      if (s + p < s1) {
        MfmaSlot<MT, RT>& slot = ring[p];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const int n = n_base + rt * 16 + c;
          const QuantParams qp = make_params(zero_of(slot.wt.z[rt], (uint32_t)n), slot.wt.s[rt]);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            h2 wd[4];
            dequant_word(slot.wt.w[rt][j], qp, uc, wd);
            const h8 b = pack_h8(wd);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              acc[mt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(slot.x[mt][j], b, acc[mt][rt], 0, 0, 0);
          }
        }
        issue(slot, s + p + P);
      }
    }
  }

  if (waves > 1) {
    if (wave > 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
          *reinterpret_cast<f4*>(&red[((((wave - 1) * MT + mt) * RT + rt) * 64 + lane) * 4]) = acc[mt][rt];
    }
    __syncthreads();
    if (wave == 0) {
      for (int w = 1; w < waves; ++w)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt)
            acc[mt][rt] += *reinterpret_cast<const f4*>(&red[((((w - 1) * MT + mt) * RT + rt) * 64 + lane) * 4]);
    }
  }
  if (wave == 0) {
    // D layout of v_mfma_f32_16x16x32_f16: lane holds rows 4*(lane/16) + r, column lane%16.
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int n = n_base + rt * 16 + c;
      if (n >= a.n) continue;
      const float b = a.bias ? half_bits_to_float(a.bias[n]) : 0.0f;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m_base + mt * 16 + 4 * g + r;
          if (m < a.m)
            a.out[(int64_t)m * a.ldo + n] = __builtin_bit_cast(uint16_t, (_Float16)(acc[mt][rt][r] + b));
        }
    }
  }
}

// ------------------------------------------------------------------------ launchers

int64_t no_workspace(const LinearArgs&, const tf_gemm_config&) { return 0; }

// Buffer offsets are 32-bit: every byte offset into qweight_t, scales, qzeros and x must fit.
int check_offsets(const LinearArgs& a) {
  const int64_t x_bytes = ((int64_t)(a.m - 1) * a.ldx + a.k) * 2;
  const int64_t w_bytes = (int64_t)a.n * (a.k / 2);
  if (x_bytes >= (int64_t)kOutOfRange || w_bytes >= (int64_t)kOutOfRange)
    return fail(TF_EINVAL, "tf_w4a16_linear: gemv kernels need x and qweight_t below 2 GiB");
  return TF_OK;
}

template <int MAXM, int RT, int P, int MAXW>
int launch_dot(const LinearArgs& a, const tf_gemm_config& cfg, float*, hipStream_t stream) {
  if (a.m > MAXM) return fail(TF_EINVAL, "tf_w4a16_linear: gemv_dot variant needs m <= block_m");
  if (int rc = check_offsets(a)) return rc;
  const int waves = cfg.num_warps;
  const dim3 grid((unsigned)cdiv(a.n, 16 * RT));
  const size_t lds = (size_t)(waves - 1) * MAXM * RT * 16 * sizeof(float);
  gemv_dot_kernel<MAXM, RT, P, MAXW><<<grid, waves * 64, lds, stream>>>(a);
  return check_launch("tf_w4a16_linear(gemv_dot)");
}

template <int MT, int RT, int P, int MAXW>
int launch_mfma(const LinearArgs& a, const tf_gemm_config& cfg, float*, hipStream_t stream) {
  if (int rc = check_offsets(a)) return rc;
  const int waves = cfg.num_warps;
  const dim3 grid((unsigned)cdiv(a.n, 16 * RT), (unsigned)cdiv(a.m, 16 * MT));
  const size_t lds = (size_t)(waves - 1) * MT * RT * 64 * 4 * sizeof(float);
  gemv_mfma_kernel<MT, RT, P, MAXW><<<grid, waves * 64, lds, stream>>>(a);
  return check_launch("tf_w4a16_linear(gemv_mfma)");
}

// One table row per (variant, num_warps): num_warps ranges over 1..MAXW (powers of two).
#define TF_W1(K, BM, BN, ST, FN) {{K, BM, BN, 128, 1, 1, ST}, FN, no_workspace}
#define TF_W2(K, BM, BN, ST, FN) TF_W1(K, BM, BN, ST, FN), {{K, BM, BN, 128, 1, 2, ST}, FN, no_workspace}
#define TF_W4(K, BM, BN, ST, FN) TF_W2(K, BM, BN, ST, FN), {{K, BM, BN, 128, 1, 4, ST}, FN, no_workspace}
#define TF_W8(K, BM, BN, ST, FN) TF_W4(K, BM, BN, ST, FN), {{K, BM, BN, 128, 1, 8, ST}, FN, no_workspace}
#define TF_W16(K, BM, BN, ST, FN) TF_W8(K, BM, BN, ST, FN), {{K, BM, BN, 128, 1, 16, ST}, FN, no_workspace}

#define TF_DOT(BM, RT, P, MAXW) \
  TF_W##MAXW(TF_KERNEL_GEMV_DOT, BM, 16 * RT, P, (launch_dot<BM, RT, P, MAXW>))
#define TF_MFMA(MT, RT, P, MAXW) \
  TF_W##MAXW(TF_KERNEL_GEMV_MFMA, 16 * MT, 16 * RT, P, (launch_mfma<MT, RT, P, MAXW>))

const Variant kGemvVariants[] = {
    TF_DOT(1, 1, 2, 16), TF_DOT(1, 1, 4, 16), TF_DOT(1, 2, 2, 16), TF_DOT(1, 2, 4, 8),
    TF_DOT(1, 4, 2, 8),  TF_DOT(1, 4, 3, 8),  TF_DOT(2, 1, 2, 16), TF_DOT(2, 2, 2, 8),
    TF_DOT(4, 1, 2, 8),
    TF_MFMA(1, 1, 2, 16), TF_MFMA(1, 1, 4, 16), TF_MFMA(1, 2, 2, 16), TF_MFMA(1, 2, 3, 16),
    TF_MFMA(1, 2, 4, 8),  TF_MFMA(1, 4, 2, 8),  TF_MFMA(1, 4, 3, 8),  TF_MFMA(2, 1, 2, 16),
    TF_MFMA(2, 2, 2, 8),
};

}  // namespace

const Variant* gemv_variants(int* count) {
  *count = (int)(sizeof(kGemvVariants) / sizeof(kGemvVariants[0]));
  return kGemvVariants;
}

}  // namespace tf
