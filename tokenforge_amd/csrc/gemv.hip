// Decode-shaped W4A16 kernels (small M): stream the packed weights once, dequantize in
// registers, accumulate in fp32.
//
// Both kernels tile N into 16-row tiles of qweight_t (block_n = 16 * RT rows per
// workgroup). Inside a 16-row tile, a wavefront covers 16 rows x 4 consecutive 32-value
// chunks of K per step: every lane issues one 128-bit load (4 packed words = 32 weights),
// so each row receives a 64-byte contiguous run per load and adjacent steps complete the
// 128-byte lines. The num_warps waves of a workgroup take disjoint, contiguous K ranges
// of the same rows (on-chip split-K); their partial sums are added in wave order through
// LDS, so results are bit-identical from run to run. No workspace, no atomics.
//
//  * gemv_dot  (TF_KERNEL_GEMV_DOT): lane = (row c = lane/4, chunk g = lane%4). Each lane
//    accumulates its 32 products per row with v_dot2_f32_f16; quads are reduced with DPP.
//  * gemv_mfma (TF_KERNEL_GEMV_MFMA): lane = (row c = lane%16, chunk g = lane/16), which is
//    exactly the B-operand layout of v_mfma_f32_16x16x32_f16 (8 consecutive K values per
//    lane = one packed word). The dequantized word goes straight into the MFMA; x rows are
//    the A operand (M <= 16 per M tile). The matrix core replaces the VALU dot products,
//    so VALU work per weight is only the unpack + (q - z) * s.
#include "linear.h"

namespace tf {
namespace {

__device__ __forceinline__ void k_range(int wave, int waves, int nsteps, int* s0, int* s1) {
  *s0 = (int)(((int64_t)wave * nsteps) / waves);
  *s1 = (int)(((int64_t)(wave + 1) * nsteps) / waves);
}

// ------------------------------------------------------------------------ gemv_dot

template <int MAXM, int RT, int UNROLL>
__global__ __launch_bounds__(1024) void gemv_dot_kernel(LinearArgs a) {
  extern __shared__ float red[];  // [(waves - 1)][MAXM][RT][16]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const int g = lane & 3;
  const int c = lane >> 2;
  const int n_base = blockIdx.x * 16 * RT;
  const int nchunks = a.k >> 5;
  const int nsteps = (nchunks + 3) >> 2;
  const int64_t words_per_row = a.k >> 3;
  int s0, s1;
  k_range(wave, waves, nsteps, &s0, &s1);

  float acc[MAXM][RT];
#pragma unroll
  for (int m = 0; m < MAXM; ++m)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[m][rt] = 0.0f;

  for (int s = s0; s < s1; s += UNROLL) {
    u4 wv[UNROLL][RT];
    uint32_t sc[UNROLL][RT];
    uint32_t zw[UNROLL][RT];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int ch = (s + u) * 4 + g;
      const bool kvalid = (s + u < s1) && (ch < nchunks);
      const int grp = (ch << 5) >> a.log2g;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int n = n_base + rt * 16 + c;
        if (kvalid && n < a.n) {
          wv[u][rt] = *reinterpret_cast<const u4*>(a.qw + (int64_t)n * words_per_row + ch * 4);
          sc[u][rt] = a.scales[(int64_t)grp * a.n + n];
          zw[u][rt] = a.qz[(int64_t)grp * (a.n >> 3) + (n >> 3)];
        } else {
          wv[u][rt] = u4{0u, 0u, 0u, 0u};
          sc[u][rt] = 0u;
          zw[u][rt] = 0u;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int ch = (s + u) * 4 + g;
      const bool kvalid = (s + u < s1) && (ch < nchunks);
      // x[m][32 values of this chunk] as 16 fp16 pairs.
      u4 xv[MAXM][4];
#pragma unroll
      for (int m = 0; m < MAXM; ++m) {
        if (kvalid && m < a.m) {
          const u4* xp = reinterpret_cast<const u4*>(a.x + (int64_t)m * a.ldx + ch * 32);
#pragma unroll
          for (int j = 0; j < 4; ++j) xv[m][j] = xp[j];
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) xv[m][j] = u4{0u, 0u, 0u, 0u};
        }
      }
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int n = n_base + rt * 16 + c;
        const QuantParams p = make_params(zero_of(zw[u][rt], (uint32_t)n), sc[u][rt]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          h2 wd[4];
          dequant_word(wv[u][rt][j], p, wd);
#pragma unroll
          for (int m = 0; m < MAXM; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              acc[m][rt] = __builtin_amdgcn_fdot2(as_h2(xv[m][j][i]), wd[i], acc[m][rt], false);
        }
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

template <int MT, int RT, int UNROLL>
__global__ __launch_bounds__(1024) void gemv_mfma_kernel(LinearArgs a) {
  extern __shared__ __attribute__((aligned(16))) float red[];  // [(waves - 1)][MT][RT][64 lanes][4]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const int c = lane & 15;
  const int g = lane >> 4;
  const int n_base = blockIdx.x * 16 * RT;
  const int m_base = blockIdx.y * 16 * MT;
  const int nchunks = a.k >> 5;
  const int nsteps = (nchunks + 3) >> 2;
  const int64_t words_per_row = a.k >> 3;
  int s0, s1;
  k_range(wave, waves, nsteps, &s0, &s1);

  f4 acc[MT][RT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[mt][rt] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int s = s0; s < s1; s += UNROLL) {
    u4 wv[UNROLL][RT];
    uint32_t sc[UNROLL][RT];
    uint32_t zw[UNROLL][RT];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int ch = (s + u) * 4 + g;
      const bool kvalid = (s + u < s1) && (ch < nchunks);
      const int grp = (ch << 5) >> a.log2g;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int n = n_base + rt * 16 + c;
        if (kvalid && n < a.n) {
          wv[u][rt] = *reinterpret_cast<const u4*>(a.qw + (int64_t)n * words_per_row + ch * 4);
          sc[u][rt] = a.scales[(int64_t)grp * a.n + n];
          zw[u][rt] = a.qz[(int64_t)grp * (a.n >> 3) + (n >> 3)];
        } else {
          wv[u][rt] = u4{0u, 0u, 0u, 0u};
          sc[u][rt] = 0u;
          zw[u][rt] = 0u;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int ch = (s + u) * 4 + g;
      const bool kvalid = (s + u < s1) && (ch < nchunks);
      // A operand: row (m_base + mt*16 + c) of x, the 32 values of this lane's chunk.
      h8 xa[MT][4];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = m_base + mt * 16 + c;
        if (kvalid && m < a.m) {
          const h8* xp = reinterpret_cast<const h8*>(a.x + (int64_t)m * a.ldx + ch * 32);
#pragma unroll
          for (int j = 0; j < 4; ++j) xa[mt][j] = xp[j];
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) xa[mt][j] = h8{0, 0, 0, 0, 0, 0, 0, 0};
        }
      }
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int n = n_base + rt * 16 + c;
        const QuantParams p = make_params(zero_of(zw[u][rt], (uint32_t)n), sc[u][rt]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          h2 wd[4];
          dequant_word(wv[u][rt][j], p, wd);
          const h8 b = pack_h8(wd);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            acc[mt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[mt][j], b, acc[mt][rt], 0, 0, 0);
        }
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

template <int MAXM, int RT, int UNROLL>
int launch_dot(const LinearArgs& a, const tf_gemm_config& cfg, float*, hipStream_t stream) {
  if (a.m > MAXM) return fail(TF_EINVAL, "tf_w4a16_linear: gemv_dot variant needs m <= block_m");
  const int waves = cfg.num_warps;
  const dim3 grid((unsigned)cdiv(a.n, 16 * RT));
  const size_t lds = (size_t)(waves - 1) * MAXM * RT * 16 * sizeof(float);
  gemv_dot_kernel<MAXM, RT, UNROLL><<<grid, waves * 64, lds, stream>>>(a);
  return check_launch("tf_w4a16_linear(gemv_dot)");
}

template <int MT, int RT, int UNROLL>
int launch_mfma(const LinearArgs& a, const tf_gemm_config& cfg, float*, hipStream_t stream) {
  const int waves = cfg.num_warps;
  const dim3 grid((unsigned)cdiv(a.n, 16 * RT), (unsigned)cdiv(a.m, 16 * MT));
  const size_t lds = (size_t)(waves - 1) * MT * RT * 64 * 4 * sizeof(float);
  gemv_mfma_kernel<MT, RT, UNROLL><<<grid, waves * 64, lds, stream>>>(a);
  return check_launch("tf_w4a16_linear(gemv_mfma)");
}

#define TF_WAVES_5(KERNEL, BM, BN, ST, FN)                                              \
  {{KERNEL, BM, BN, 128, 1, 1, ST}, FN, no_workspace},                                  \
      {{KERNEL, BM, BN, 128, 1, 2, ST}, FN, no_workspace},                              \
      {{KERNEL, BM, BN, 128, 1, 4, ST}, FN, no_workspace},                              \
      {{KERNEL, BM, BN, 128, 1, 8, ST}, FN, no_workspace},                              \
      {{KERNEL, BM, BN, 128, 1, 16, ST}, FN, no_workspace}

#define TF_DOT(BM, RT, ST) TF_WAVES_5(TF_KERNEL_GEMV_DOT, BM, 16 * RT, ST, (launch_dot<BM, RT, ST>))
#define TF_MFMA(MT, RT, ST) TF_WAVES_5(TF_KERNEL_GEMV_MFMA, 16 * MT, 16 * RT, ST, (launch_mfma<MT, RT, ST>))

const Variant kGemvVariants[] = {
    TF_DOT(1, 1, 1), TF_DOT(1, 1, 2), TF_DOT(1, 1, 4),
    TF_DOT(1, 2, 1), TF_DOT(1, 2, 2), TF_DOT(1, 2, 4),
    TF_DOT(1, 4, 1), TF_DOT(1, 4, 2),
    TF_DOT(2, 1, 1), TF_DOT(2, 1, 2), TF_DOT(2, 2, 1), TF_DOT(2, 2, 2),
    TF_DOT(4, 1, 1), TF_DOT(4, 1, 2), TF_DOT(4, 2, 1),
    TF_MFMA(1, 1, 1), TF_MFMA(1, 1, 2), TF_MFMA(1, 1, 4),
    TF_MFMA(1, 2, 1), TF_MFMA(1, 2, 2), TF_MFMA(1, 2, 4),
    TF_MFMA(1, 4, 1), TF_MFMA(1, 4, 2),
    TF_MFMA(2, 1, 1), TF_MFMA(2, 1, 2), TF_MFMA(2, 2, 1), TF_MFMA(2, 2, 2),
};

}  // namespace

const Variant* gemv_variants(int* count) {
  *count = (int)(sizeof(kGemvVariants) / sizeof(kGemvVariants[0]));
  return kGemvVariants;
}

}  // namespace tf
