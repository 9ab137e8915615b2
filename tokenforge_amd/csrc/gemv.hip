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
// consumed. Buffer loads return zeros past the end of a tensor, which handles ragged N and a
// partial last step without branches.
//
// Only the weight stream uses the vector-memory path inside the loop. Before the loop each
// wave stages what it will reuse in its own LDS region (no barrier needed, a wave reads only
// what it wrote): the dequantization operands (1024 + z, 64 + z, scale as fp16 pairs) of every
// (group, column) of its K range, and, in the XLDS variants, its slice of x. Measured on
// MI355X, per-step scale/zero/x loads cost more than the dequantization arithmetic.
//
//  * gemv_dot  (TF_KERNEL_GEMV_DOT): lane = (row c = lane/4, chunk g = lane%4). Each lane
//    accumulates its products with v_dot2_f32_f16; quads are reduced with DPP.
//  * gemv_mfma (TF_KERNEL_GEMV_MFMA): lane = (row c = lane%16, chunk g = lane/16), exactly the
//    B-operand layout of v_mfma_f32_16x16x32_f16 (8 consecutive K values per lane = one
//    packed word). The dequantized word goes straight into the MFMA and x rows are the A
//    operand, so the matrix core does the dot products and the VALU only unpacks and scales.
//    A rows m >= M only feed output rows that are discarded, so they read any staged row.
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
  int nsteps;          // ceil(K / 128)
  int groups;          // K / G
  int log2g;
  int n;
};

__device__ __forceinline__ Streams make_streams(const LinearArgs& a) {
  Streams s;
  s.row_bytes = (uint32_t)(a.k >> 1);
  s.groups = a.k >> a.log2g;
  s.qw = make_rsrc(a.qw, (uint32_t)a.n * s.row_bytes);
  s.sc = make_rsrc(a.scales, (uint32_t)(s.groups * a.n * 2));
  s.qz = make_rsrc(a.qz, (uint32_t)(s.groups * (a.n >> 3) * 4));
  s.x = make_rsrc(a.x, (uint32_t)(((int64_t)(a.m - 1) * a.ldx + a.k) * 2));
  s.nchunks = a.k >> 5;
  s.nsteps = (s.nchunks + 3) >> 2;
  s.log2g = a.log2g;
  s.n = a.n;
  return s;
}

// Largest number of 128-wide K steps any wave gets, and the groups such a range can touch.
__host__ __device__ __forceinline__ int max_steps(int nsteps, int waves) { return (nsteps + waves - 1) / waves; }
__host__ __device__ __forceinline__ int max_groups(int steps, int log2g) {
  // A range of `steps` steps starting at a multiple of 128 spans ceil(steps*128 / G) groups
  // (G <= 128 divides 128).
  return (steps * 128) >> log2g;
}

// Per-wave LDS staging area (in 32-bit words).
struct WaveLds {
  uint32_t* params;  // [groups_max][16*RT] x 3 words: fp16x2 (1024+z), (64+z), scale
  _Float16* xs;      // [rows][xstride] x slice (XLDS variants)
};

template <int RT>
__device__ __forceinline__ int params_words(int groups_max) { return groups_max * 16 * RT * 3; }

// Stage the dequantization operands of groups [g_lo, g_lo + ng) x columns [n_base, n_base+16RT)
// into slots [0, slots). Slots past ng (the unused tail of a partial last step) get neutral
// operands, zero point 0 and scale 0, so a zero weight word dequantizes to exactly 0 there.
template <int RT>
__device__ __forceinline__ void stage_params(uint32_t* p, const Streams& st, int n_base, int g_lo, int ng,
                                             int slots, int lane) {
  const int entries = slots * 16 * RT;
  for (int e = lane; e < entries; e += 64) {
    const int gi = e / (16 * RT);
    const int col = e % (16 * RT);
    const int n = n_base + col;
    const bool ok = n < st.n && gi < ng;
    const uint32_t grp = (uint32_t)(g_lo + gi);
    const uint32_t sb = load_b16(st.sc, ok ? (grp * (uint32_t)st.n + (uint32_t)n) * 2u : kOutOfRange);
    const uint32_t zw = load_b32(st.qz, ok ? (grp * (uint32_t)(st.n >> 3) + (uint32_t)(n >> 3)) * 4u : kOutOfRange);
    const QuantParams q = make_params(zero_of(zw, (uint32_t)n), sb);
    uint32_t* d = p + 3 * e;
    d[0] = as_u32(q.zlo);
    d[1] = as_u32(q.zhi);
    d[2] = as_u32(q.s);
  }
}

__device__ __forceinline__ QuantParams read_params(const uint32_t* p, int gi, int col, int cols) {
  const uint32_t* d = p + 3 * (gi * cols + col);
  QuantParams q;
  q.zlo = as_h2(d[0]);
  q.zhi = as_h2(d[1]);
  q.s = as_h2(d[2]);
  return q;
}

// Stage x[m0 + r][k0 .. k0 + kn) for r < rows into xs (row stride xstride halfs); values at
// k >= K are zero (buffer loads past the tensor return zeros only at its very end, so the
// K bound is explicit).
__device__ __forceinline__ void stage_x(_Float16* xs, const LinearArgs& a, const Streams& st, int m0, int rows,
                                        int k0, int kn, int xstride, int lane) {
  const int chunks = kn >> 3;  // 16-byte chunks per row
  for (int e = lane; e < rows * chunks; e += 64) {
    const int r = e / chunks;
    const int q = e % chunks;
    const int k = k0 + q * 8;
    const uint32_t off = (k < a.k) ? (uint32_t)(((int64_t)(m0 + r) * a.ldx + k) * 2) : kOutOfRange;
    *reinterpret_cast<u4*>(xs + r * xstride + q * 8) = load_b128(st.x, off);
  }
}

// Weights of one step for RT row tiles.
template <int RT>
struct WeightSlot {
  u4 w[RT];
};

template <int RT>
__device__ __forceinline__ void issue_weights(WeightSlot<RT>& slot, const Streams& st, const uint32_t* row_off,
                                              int ch, bool kvalid) {
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const uint32_t wo = (kvalid && row_off[rt] != kOutOfRange) ? row_off[rt] + (uint32_t)ch * 16u : kOutOfRange;
    slot.w[rt] = load_b128(st.qw, wo);
  }
}

// ------------------------------------------------------------------------ gemv_dot

template <int MAXM, int RT>
struct DotSlot {
  WeightSlot<RT> wt;
};

template <int MAXM, int RT, int P, int MAXW>
__global__ __launch_bounds__(MAXW * 64) void gemv_dot_kernel(LinearArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const int g = lane & 3;
  const int c = lane >> 2;
  const int n_base = blockIdx.x * 16 * RT;
  const Streams st = make_streams(a);
  int s0, s1;
  k_range(wave, waves, st.nsteps, &s0, &s1);
  const int steps_max = max_steps(st.nsteps, waves);
  const int groups_max = max_groups(steps_max, st.log2g);
  const int xrows = a.m < MAXM ? a.m : MAXM;
  const int xstride = steps_max * 128 + 8;
  const int wave_words = params_words<RT>(groups_max) + (xrows * xstride) / 2;
  uint32_t* my = lds + wave * wave_words;
  uint32_t* prm = my;
  _Float16* xs = reinterpret_cast<_Float16*>(my + params_words<RT>(groups_max));
  const UnpackConsts uc = unpack_consts();
  const int g_lo = (s0 * 128) >> st.log2g;
  const int g_hi = min(st.groups, ((s1 * 128) >> st.log2g));

  stage_params<RT>(prm, st, n_base, g_lo, g_hi - g_lo, groups_max, lane);
  stage_x(xs, a, st, 0, xrows, s0 * 128, (s1 - s0) * 128, xstride, lane);

  uint32_t row_off[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int n = n_base + rt * 16 + c;
    row_off[rt] = n < a.n ? (uint32_t)n * st.row_bytes : kOutOfRange;
  }
  auto issue = [&](DotSlot<MAXM, RT>& slot, int step) {
    const int ch = step * 4 + g;
    issue_weights<RT>(slot.wt, st, row_off, ch, step < s1 && ch < st.nchunks);
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
        const int local = (s + p - s0) * 128 + g * 32;  // this lane's K offset inside the slice
        const int gi = (((s + p) * 128 + g * 32) >> st.log2g) - g_lo;
        u4 xv[MAXM][4];
#pragma unroll
        for (int m = 0; m < MAXM; ++m) {
          const int row = m < xrows ? m : 0;  // rows past M only feed accumulators never stored
#pragma unroll
          for (int j = 0; j < 4; ++j) xv[m][j] = *reinterpret_cast<const u4*>(xs + row * xstride + local + j * 8);
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const QuantParams qp = read_params(prm, gi, rt * 16 + c, 16 * RT);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            h2 wd[4];
            dequant_word(slot.wt.w[rt][j], qp, uc, wd);
#pragma unroll
            for (int m = 0; m < MAXM; ++m)
#pragma unroll
              for (int i = 0; i < 4; ++i)
                acc[m][rt] = __builtin_amdgcn_fdot2(as_h2(xv[m][j][i]), wd[i], acc[m][rt], false);
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
    float* red = reinterpret_cast<float*>(lds + waves * wave_words);  // [(waves - 1)][MAXM][RT][16]
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

template <int MT, int RT, bool XLDS>
struct MfmaSlot {
  WeightSlot<RT> wt;
  h8 x[XLDS ? 1 : MT][XLDS ? 1 : 4];  // A operand from global when x is not staged
};

template <int MT, int RT, int P, int MAXW, bool XLDS>
__global__ __launch_bounds__(MAXW * 64) void gemv_mfma_kernel(LinearArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const int c = lane & 15;
  const int g = lane >> 4;
  const int n_base = blockIdx.x * 16 * RT;
  const int m_base = blockIdx.y * 16 * MT;
  const Streams st = make_streams(a);
  int s0, s1;
  k_range(wave, waves, st.nsteps, &s0, &s1);
  const int steps_max = max_steps(st.nsteps, waves);
  const int groups_max = max_groups(steps_max, st.log2g);
  const int xrows = min(16 * MT, a.m - m_base);   // rows staged by this workgroup
  const int xalloc = min(16 * MT, a.m);           // rows allocated per wave (same in every workgroup)
  const int xstride = steps_max * 128 + 8;
  const int wave_words = params_words<RT>(groups_max) + (XLDS ? (xalloc * xstride) / 2 : 0);
  uint32_t* my = lds + wave * wave_words;
  uint32_t* prm = my;
  _Float16* xs = reinterpret_cast<_Float16*>(my + params_words<RT>(groups_max));
  const UnpackConsts uc = unpack_consts();
  const int g_lo = (s0 * 128) >> st.log2g;
  const int g_hi = min(st.groups, ((s1 * 128) >> st.log2g));

  stage_params<RT>(prm, st, n_base, g_lo, g_hi - g_lo, groups_max, lane);
  if (XLDS) stage_x(xs, a, st, m_base, xrows, s0 * 128, (s1 - s0) * 128, xstride, lane);

  uint32_t row_off[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int n = n_base + rt * 16 + c;
    row_off[rt] = n < a.n ? (uint32_t)n * st.row_bytes : kOutOfRange;
  }
  auto issue = [&](MfmaSlot<MT, RT, XLDS>& slot, int step) {
    const int ch = step * 4 + g;
    const bool kvalid = step < s1 && ch < st.nchunks;
    issue_weights<RT>(slot.wt, st, row_off, ch, kvalid);
    if (!XLDS) {
#pragma unroll
      for (int mt = 0; mt < (XLDS ? 0 : MT); ++mt) {
        const int m = m_base + mt * 16 + c;
        const uint32_t xo = (kvalid && m < a.m) ? (uint32_t)(((int64_t)m * a.ldx + ch * 32) * 2) : kOutOfRange;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          slot.x[XLDS ? 0 : mt][XLDS ? 0 : j] = __builtin_bit_cast(h8, load_b128(st.x, xo + 16u * j));
      }
    }
  };

  f4 acc[MT][RT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[mt][rt] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  MfmaSlot<MT, RT, XLDS> ring[P];
#pragma unroll
  for (int p = 0; p < P; ++p) issue(ring[p], s0 + p);

  for (int s = s0; s < s1; s += P) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      if (s + p < s1) {
        MfmaSlot<MT, RT, XLDS>& slot = ring[p];
        const int local = (s + p - s0) * 128 + g * 32;
        const int gi = (((s + p) * 128 + g * 32) >> st.log2g) - g_lo;
        h8 xa[MT][4];
        if (XLDS) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const int r = mt * 16 + c;
            const int row = r < xrows ? r : 0;  // rows past M feed discarded outputs
#pragma unroll
            for (int j = 0; j < 4; ++j) xa[mt][j] = *reinterpret_cast<const h8*>(xs + row * xstride + local + j * 8);
          }
        } else {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int j = 0; j < 4; ++j) xa[mt][j] = slot.x[XLDS ? 0 : mt][XLDS ? 0 : j];
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const QuantParams qp = read_params(prm, gi, rt * 16 + c, 16 * RT);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            h2 wd[4];
            dequant_word(slot.wt.w[rt][j], qp, uc, wd);
            const h8 b = pack_h8(wd);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              acc[mt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[mt][j], b, acc[mt][rt], 0, 0, 0);
          }
        }
        issue(slot, s + p + P);
      }
    }
  }

  if (waves > 1) {
    float* red = reinterpret_cast<float*>(lds + waves * wave_words);  // [(waves - 1)][MT][RT][64][4]
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

// LDS bytes one workgroup may use on the current device (160 KiB on gfx950), queried once
// per device.
size_t device_max_lds() {
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
int reserve_lds(Kernel kernel, size_t bytes, const char* name) {
  if (bytes > device_max_lds())
    return fail(TF_EINVAL, std::string("tf_w4a16_linear: ") + name +
                               " variant needs more LDS than the device has for this K; use more waves");
  if (bytes > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)bytes) != hipSuccess)
    return fail(TF_ELAUNCH, std::string("tf_w4a16_linear: cannot reserve LDS for ") + name);
  return TF_OK;
}

// Buffer offsets are 32-bit: every byte offset into qweight_t, scales, qzeros and x must fit.
int check_offsets(const LinearArgs& a) {
  const int64_t x_bytes = ((int64_t)(a.m - 1) * a.ldx + a.k) * 2;
  const int64_t w_bytes = (int64_t)a.n * (a.k / 2);
  if (x_bytes >= (int64_t)kOutOfRange || w_bytes >= (int64_t)kOutOfRange)
    return fail(TF_EINVAL, "tf_w4a16_linear: gemv kernels need x and qweight_t below 2 GiB");
  return TF_OK;
}

// LDS bytes of a gemv launch: per-wave staging plus the cross-wave reduction buffer.
size_t gemv_lds(const LinearArgs& a, int waves, int rt, int x_rows, size_t red_per_wave) {
  const int nsteps = ((a.k >> 5) + 3) >> 2;
  const int steps = max_steps(nsteps, waves);
  const int groups = max_groups(steps, a.log2g);
  const size_t words = (size_t)groups * 16 * rt * 3 + (size_t)(x_rows * (steps * 128 + 8)) / 2;
  return (size_t)waves * words * 4 + (size_t)(waves - 1) * red_per_wave;
}

template <int MAXM, int RT, int P, int MAXW>
int launch_dot(const LinearArgs& a, const tf_gemm_config& cfg, float*, hipStream_t stream) {
  if (a.m > MAXM) return fail(TF_EINVAL, "tf_w4a16_linear: gemv_dot variant needs m <= block_m");
  if (int rc = check_offsets(a)) return rc;
  const int waves = cfg.num_warps;
  const size_t lds = gemv_lds(a, waves, RT, a.m < MAXM ? a.m : MAXM, (size_t)MAXM * RT * 16 * sizeof(float));
  if (int rc = reserve_lds(gemv_dot_kernel<MAXM, RT, P, MAXW>, lds, "gemv_dot")) return rc;
  const dim3 grid((unsigned)cdiv(a.n, 16 * RT));
  gemv_dot_kernel<MAXM, RT, P, MAXW><<<grid, waves * 64, lds, stream>>>(a);
  return check_launch("tf_w4a16_linear(gemv_dot)");
}

template <int MT, int RT, int P, int MAXW, bool XLDS>
int launch_mfma(const LinearArgs& a, const tf_gemm_config& cfg, float*, hipStream_t stream) {
  if (int rc = check_offsets(a)) return rc;
  const int waves = cfg.num_warps;
  const size_t lds = gemv_lds(a, waves, RT, XLDS ? (a.m < 16 * MT ? a.m : 16 * MT) : 0,
                              (size_t)MT * RT * 64 * 4 * sizeof(float));
  if (int rc = reserve_lds(gemv_mfma_kernel<MT, RT, P, MAXW, XLDS>, lds, "gemv_mfma")) return rc;
  const dim3 grid((unsigned)cdiv(a.n, 16 * RT), (unsigned)cdiv(a.m, 16 * MT));
  gemv_mfma_kernel<MT, RT, P, MAXW, XLDS><<<grid, waves * 64, lds, stream>>>(a);
  return check_launch("tf_w4a16_linear(gemv_mfma)");
}

// One table row per (variant, num_warps): num_warps ranges over 1..MAXW (powers of two).
#define TF_W1(K, BM, BN, BK, ST, FN) {{K, BM, BN, BK, 1, 1, ST}, FN, no_workspace}
#define TF_W2(K, BM, BN, BK, ST, FN) TF_W1(K, BM, BN, BK, ST, FN), {{K, BM, BN, BK, 1, 2, ST}, FN, no_workspace}
#define TF_W4(K, BM, BN, BK, ST, FN) TF_W2(K, BM, BN, BK, ST, FN), {{K, BM, BN, BK, 1, 4, ST}, FN, no_workspace}
#define TF_W8(K, BM, BN, BK, ST, FN) TF_W4(K, BM, BN, BK, ST, FN), {{K, BM, BN, BK, 1, 8, ST}, FN, no_workspace}
#define TF_W16(K, BM, BN, BK, ST, FN) TF_W8(K, BM, BN, BK, ST, FN), {{K, BM, BN, BK, 1, 16, ST}, FN, no_workspace}

// block_k = 128 marks x staged in LDS, 64 marks x streamed from global with the weights.
#define TF_DOT(BM, RT, P, MAXW) \
  TF_W##MAXW(TF_KERNEL_GEMV_DOT, BM, 16 * RT, 128, P, (launch_dot<BM, RT, P, MAXW>))
#define TF_MFMA(MT, RT, P, MAXW) \
  TF_W##MAXW(TF_KERNEL_GEMV_MFMA, 16 * MT, 16 * RT, 128, P, (launch_mfma<MT, RT, P, MAXW, true>))
#define TF_MFMA_GX(MT, RT, P, MAXW) \
  TF_W##MAXW(TF_KERNEL_GEMV_MFMA, 16 * MT, 16 * RT, 64, P, (launch_mfma<MT, RT, P, MAXW, false>))

const Variant kGemvVariants[] = {
    TF_DOT(1, 1, 2, 16), TF_DOT(1, 1, 4, 16), TF_DOT(1, 1, 8, 16), TF_DOT(1, 2, 2, 16),
    TF_DOT(1, 2, 4, 8),  TF_DOT(1, 4, 2, 8),  TF_DOT(2, 1, 2, 16), TF_DOT(2, 2, 2, 8),
    TF_DOT(4, 1, 2, 8),
    TF_MFMA(1, 1, 2, 16), TF_MFMA(1, 1, 4, 16), TF_MFMA(1, 1, 8, 16), TF_MFMA(1, 2, 2, 16),
    TF_MFMA(1, 2, 4, 16), TF_MFMA(1, 4, 2, 8),  TF_MFMA(2, 1, 2, 16), TF_MFMA(2, 2, 2, 8),
    TF_MFMA_GX(1, 1, 2, 16), TF_MFMA_GX(1, 2, 2, 16), TF_MFMA_GX(1, 4, 2, 8), TF_MFMA_GX(2, 1, 2, 16),
    TF_MFMA_GX(2, 2, 2, 8),
};

}  // namespace

const Variant* gemv_variants(int* count) {
  *count = (int)(sizeof(kGemvVariants) / sizeof(kGemvVariants[0]));
  return kGemvVariants;
}

}  // namespace tf
