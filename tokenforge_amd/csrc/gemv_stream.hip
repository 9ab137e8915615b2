// Decode W4A16 kernel for M <= 4 (and M <= 8, MAXM = 8) in the interleaved-stream form, on the
// gfx950 tile layout.
//
// Work split. Workgroup b owns a contiguous range of 16-row tiles [t0, t1) (XCD-aware order),
// i.e. (t1 - t0) * nst consecutive 1 KB step blocks of qweight_t (nst = K / 128; in the tile
// layout the blocks of consecutive tiles and steps are consecutive in memory). Its W waves take
// each tile's steps round robin (wave w every W-th step, from a per-tile phase), so at any
// moment the waves of a workgroup read W neighbouring 1 KB blocks, and their scale and zero
// words are neighbours too, instead of every wave streaming its own distant range: on MI355X the
// same bytes read with neighbouring addresses in flight come back 10-25% sooner, most of it on
// the small scale and zero reads. The grid is sized to be resident at once, with about 32 KB of
// weights in flight per CU (workgroups per CU = 32 / (W * P), within the occupancy the kernel
// allows): more bytes in flight per CU were measured slower, fewer leave HBM idle.
//
// Per step a lane does what the MFMA GEMV does: lane 16 g + c holds chunk (column c, K block g)
// of the step block, the 16 bytes that are the B operand of four v_mfma_f32_16x16x32_f16; the
// exact dequantization fp16(q - z) * s (one rounding) runs in registers; x rows are the A
// operand, read from one copy of x staged in LDS. D rows 0..MAXM-1 (lanes 0..4 MAXM - 1; D lane
// l holds rows 4 (l / 16) .. + 3 of column l % 16) are the outputs.
// When a wave's next step lies in a later tile it writes its partial sums for the tile to LDS;
// after one barrier the workgroup adds each tile's partials in wave order and applies bias, row
// scale and epilogue. A column's sum order depends only on its tile, K and W (not on the grid),
// so results are bit-identical from run to run and between the epilogues.
//
// SiLU*mul: virtual tile v covers outputs 8v..8v+7: lanes c < 8 read gate rows 8v + c, lanes
// c >= 8 the up rows N/2 + 8v + c - 8, i.e. half (v % 2) of physical tile v / 2 and of tile
// N/32 + v / 2 (N % 32 == 0). The lane part of every address is then a per-lane constant and
// the step part a wave-uniform scalar, as without the epilogue.
//
// K split (split_k > 1): workgroup b works on K slice z = b / (nwg / split), steps [z nst / split,
// (z + 1) nst / split) of every tile, and stages only that slice of x, so M rows of a long K
// (down_proj at M = 4 and 8) fit in LDS. It writes each column's fp32 sum over its slice (no
// bias or row scale) to the workspace [split][M][N]; splitk_reduce adds the slices in split
// order, the bias and the row scale and applies the epilogue (SiLU*mul on the physical gate
// and up columns: the kernel runs without the virtual SiLU tiles then).
//
// RMSNorm prologue (NORM, tf_rmsnorm_fp8_w4a16_linear): x holds the rows before an RMSNorm +
// e4m3 quantization. Once x is staged, every workgroup turns each row in LDS into fp16(code *
// scale), the activation rmsnorm_fp8_quant_dq writes, with the norm kernel's arithmetic
// (norm_row.h); the weight ring is already in flight meanwhile. For M <= 4 rows this costs
// each workgroup a few hundred instructions per thread and removes the norm's own launch and
// its round trip through HBM.
#include "linear.h"
#include "norm_row.h"

#include <algorithm>

namespace tf {

int splitk_reduce(const LinearArgs& a, const float* ws, int split, hipStream_t stream);

namespace {

constexpr int kNormMaxM = 4;                   // the RMSNorm prologue serves M <= 4
constexpr int kStreamMaxXBytes = 96 * 1024;    // staged x: M rows of K + 8 halfs
constexpr int kStreamInflightKB = 32;          // weight bytes in flight per CU (KB)
constexpr int kNormMaxK = 8192;                // the RMSNorm prologue serves K up to this

// LDS the RMSNorm prologue adds: the chunk sums of the squares of every row, each row padded to
// lpad = the power of two >= K / 8 (at least 64) entries, then [4][16] words for the maxima,
// then the norm weight (K fp16; staged for the LDS form, which reads it once per row).
__host__ __device__ __forceinline__ int norm_lpad(int k) {
  int l = 64;
  while (l < (k >> 3)) l <<= 1;
  return l;
}
__host__ __device__ __forceinline__ size_t norm_scratch_bytes(int m, int k) {
  return (size_t)m * norm_lpad(k) * 8 + 256 + (size_t)k * 2;
}

// The sum of squares of staged row rs in the fixed order of norm_row.h, from its chunk sums at
// sums[rs * lpad + q] (zeros past the row's chunks; lpad / 64 <= 16 per lane); every lane of the
// wave takes part and gets the total.
__device__ __forceinline__ double staged_row_total(const double* sums, int lpad, int rs) {
  return row_total_lds_rt<16>(sums + rs * lpad, lpad >> 6);
}

__host__ __device__ __forceinline__ int stream_xstride(int k) { return k + 8; }

// Scalar (wave-uniform) byte offsets of step s of (virtual) tile v in the three streams, and
// the steps' strides. SILU: virtual tile v is half v % 2 of physical tiles v / 2 (gate rows)
// and N/32 + v / 2 (up rows; the up part of the offset is in the lane's constant part).
template <bool SILU>
struct StreamGeo {
  int nst, groups, gps;
  __device__ __forceinline__ void at(int v, int s, int& ow, int& os, int& oz) const {
    const int t = SILU ? (v >> 1) : v;
    const int h = SILU ? (v & 1) : 0;
    ow = (t * nst + s) * 1024 + h * 128;
    os = (t * groups + s * gps) * 32 + h * 16;
    oz = (t * groups + s * gps) * 8 + h * 4;
  }
};

// The RMSNorm + e4m3 prologue over the m <= 4 rows of x staged in LDS (row r at xs + r *
// xstride), in place: each row becomes fp16(code * scale) as rmsnorm_fp8.hip computes it for
// the row (reference.py:35-50; dynamic scale): fp64 sum of squares in the fixed order of
// norm_row.h, var = fp32(sum * (1 / k)), rstd = 1 / sqrt(var + eps), y = fp16(fp32(x * rstd)) *
// w in fp16, absmax, scale, codes, then the codes times the scale. All rows go through each
// phase together, one barrier per phase: every row's chunk sums into `sums` (every wave then
// adds each row's), the normalized chunks and their maxima (the W waves meet for each row's
// absmax in red_u[r][w]), then the codes. Thread t takes the 8-element chunks t, t + T, ... of
// the flattened (row, chunk) index.
__device__ __forceinline__ void norm_rows(const LinearArgs& a, _Float16* xs, int xstride, double* sums,
                                          uint32_t* red_u, const u4* gs, int W, int wave, int lane) {
  constexpr int R = kNormMaxM;
  const int T = W * 64;
  const int m = a.m;
  const int chunks = a.k >> 3;
  const int total = m * chunks;
  const int lpad = norm_lpad(a.k);
  const int lshift = __builtin_ctz(lpad);
  auto row_q = [&](int e, int& r, int& q) {
    r = 0;
#pragma unroll
    for (int i = 1; i < R; ++i) r += (int)(e >= i * chunks);
    q = e - r * chunks;
  };
  for (int e = threadIdx.x; e < (m << lshift); e += T) {
    const int r = e >> lshift, q = e & (lpad - 1);
    double v = 0.0;
    if (q < chunks) {
      const u4 x = reinterpret_cast<const u4*>(xs + r * xstride)[q];
      const h2 p[4] = {as_h2(x[0]), as_h2(x[1]), as_h2(x[2]), as_h2(x[3])};
      v = chunk_sum_squares(p);
    }
    sums[e] = v;
  }
  __syncthreads();
  // every row's rstd in every wave (the fixed-order total of norm_row.h)
  float rstd[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    rstd[r] = 0.0f;
    if (r < m) {
      const double t = staged_row_total(sums, lpad, r);  // every lane of the wave takes part
      const float var = (float)((double)(float)t * a.norm_inv_k);
      rstd[r] = 1.0f / __builtin_sqrtf(var + a.norm_eps);
    }
  }
  uint32_t am[R];
#pragma unroll
  for (int r = 0; r < R; ++r) am[r] = 0;
  for (int e = threadIdx.x; e < total; e += T) {
    int r, q;
    row_q(e, r, q);
    float rs = rstd[0];
#pragma unroll
    for (int i = 1; i < R; ++i) rs = r == i ? rstd[i] : rs;
    u4* row = reinterpret_cast<u4*>(xs + r * xstride);
    u4 v = row[q];
    const u4 gw = gs[q];  // the norm weight, staged in LDS
    uint32_t mx = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const h2 x = as_h2(v[j]);
      h2 nrm;
      nrm[0] = mul_round_f32_then_f16((float)x[0], rs);
      nrm[1] = mul_round_f32_then_f16((float)x[1], rs);
      v[j] = as_u32(nrm * as_h2(gw[j]));
      const uint32_t yb = v[j] & 0x7FFF7FFFu;
      mx = __builtin_elementwise_max(mx, __builtin_elementwise_max(yb & 0xFFFFu, yb >> 16));
    }
    row[q] = v;
#pragma unroll
    for (int i = 0; i < R; ++i) am[i] = r == i ? __builtin_elementwise_max(am[i], mx) : am[i];
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r < m) {
      const uint32_t wmax = wave_max_u32(am[r]);
      if (lane == 0) red_u[r * 16 + wave] = wmax;
    }
  }
  __syncthreads();
  float sc[R], r32[R];
  double rcp[R];
  bool fast[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    sc[r] = 1.0f, r32[r] = 0.0f, rcp[r] = 0.0, fast[r] = true;
    if (r < m) {
      uint32_t m_bits = red_u[r * 16];
      for (int w = 1; w < W; ++w) m_bits = __builtin_elementwise_max(m_bits, red_u[r * 16 + w]);
      const float amax = (float)__builtin_bit_cast(_Float16, (uint16_t)m_bits);
      sc[r] = dynamic_scale(amax);
      fast[r] = __builtin_isfinite(amax) && __builtin_isfinite(sc[r]) && sc[r] > 0.0f;
      r32[r] = fast[r] ? 1.0f / sc[r] : 0.0f;
      rcp[r] = fast[r] ? 0.0 : 1.0 / (double)sc[r];
    }
  }
  for (int e = threadIdx.x; e < total; e += T) {
    int r, q;
    row_q(e, r, q);
    float s = sc[0], rr = r32[0];
    double rc = rcp[0];
    bool f = fast[0];
#pragma unroll
    for (int i = 1; i < R; ++i) {
      s = r == i ? sc[i] : s;
      rr = r == i ? r32[i] : rr;
      rc = r == i ? rcp[i] : rc;
      f = r == i ? fast[i] : f;
    }
    u4* row = reinterpret_cast<u4*>(xs + r * xstride);
    const u4 v = row[q];
    uint32_t lo, hi;
    if (f) {
      float ev[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ev[2 * j] = __builtin_amdgcn_fmed3f(quotient_dynamic<false>(as_h2(v[j]), s, rr), -kFp8Max, kFp8Max);
        ev[2 * j + 1] = __builtin_amdgcn_fmed3f(quotient_dynamic<true>(as_h2(v[j]), s, rr), -kFp8Max, kFp8Max);
      }
      lo = encode4_clamped(ev[0], ev[1], ev[2], ev[3]);
      hi = encode4_clamped(ev[4], ev[5], ev[6], ev[7]);
    } else {
      lo = hi = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t code = encode_slow(as_h2(v[j >> 1])[j & 1], rc);
        if (j < 4) lo |= code << (8 * j);
        else hi |= code << (8 * (j - 4));
      }
    }
    const u2 d0 = dequant_codes4(lo, s), d1 = dequant_codes4(hi, s);
    row[q] = u4{d0[0], d0[1], d1[0], d1[1]};
  }
}

// The same prologue when every thread holds at most one 8-element chunk of x (M * K <= 8 T, the
// decode case): the thread's chunk x1 (row r, chunk q; ok false past the end) and its weight
// chunk g1 are already in registers, so the arithmetic runs there; the chunk sums meet in
// `sums` (the fixed order of norm_row.h: every wave adds each row's), the maxima in red_u[r][w],
// one barrier each. x1 becomes the fp16(code * scale) chunk.
__device__ __forceinline__ void norm_chunk(const LinearArgs& a, u4& x1, const u4 g1, int r, int q, bool ok,
                                           double* sums, uint32_t* red_u, int W, int wave, int lane) {
  const int chunks = a.k >> 3;
  const int lpad = norm_lpad(a.k);
  const int lshift = __builtin_ctz(lpad);
  const h2 p[4] = {as_h2(x1[0]), as_h2(x1[1]), as_h2(x1[2]), as_h2(x1[3])};
  if (ok) sums[(r << lshift) + q] = chunk_sum_squares(p);
  for (int e = threadIdx.x; e < (a.m << lshift); e += W * 64)
    if ((e & (lpad - 1)) >= chunks) sums[e] = 0.0;
  __syncthreads();
  const int rs = ok ? r : 0;  // threads past the end follow row 0 (their results are not stored)
  double total = 0.0;
  for (int rr = 0; rr < a.m; ++rr) {
    const double t = staged_row_total(sums, lpad, rr);  // every lane of the wave takes part
    total = rr == rs ? t : total;
  }
  const float var = (float)((double)(float)total * a.norm_inv_k);
  const float rstd = 1.0f / __builtin_sqrtf(var + a.norm_eps);

  uint32_t am = 0;
  u4 y;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const h2 x = as_h2(x1[j]);
    h2 nrm;
    nrm[0] = mul_round_f32_then_f16((float)x[0], rstd);
    nrm[1] = mul_round_f32_then_f16((float)x[1], rstd);
    y[j] = as_u32(nrm * as_h2(g1[j]));
    const uint32_t yb = y[j] & 0x7FFF7FFFu;
    am = __builtin_elementwise_max(am, __builtin_elementwise_max(yb & 0xFFFFu, yb >> 16));
  }
  if (!ok) am = 0;
  for (int rr = 0; rr < a.m; ++rr) {
    const uint32_t wmax = wave_max_u32(r == rr ? am : 0u);
    if (lane == 0) red_u[rr * 16 + wave] = wmax;
  }
  __syncthreads();
  uint32_t m_bits = red_u[rs * 16];
  for (int w = 1; w < W; ++w) m_bits = __builtin_elementwise_max(m_bits, red_u[rs * 16 + w]);
  const float amax = (float)__builtin_bit_cast(_Float16, (uint16_t)m_bits);
  const float s = dynamic_scale(amax);
  const bool fast = __builtin_isfinite(amax) && __builtin_isfinite(s) && s > 0.0f;
  uint32_t lo, hi;
  if (fast) {
    const float r32 = 1.0f / s;
    float e[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      e[2 * j] = __builtin_amdgcn_fmed3f(quotient_dynamic<false>(as_h2(y[j]), s, r32), -kFp8Max, kFp8Max);
      e[2 * j + 1] = __builtin_amdgcn_fmed3f(quotient_dynamic<true>(as_h2(y[j]), s, r32), -kFp8Max, kFp8Max);
    }
    lo = encode4_clamped(e[0], e[1], e[2], e[3]);
    hi = encode4_clamped(e[4], e[5], e[6], e[7]);
  } else {
    const double rcp = 1.0 / (double)s;
    lo = hi = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t code = encode_slow(as_h2(y[j >> 1])[j & 1], rcp);
      if (j < 4) lo |= code << (8 * j);
      else hi |= code << (8 * (j - 4));
    }
  }
  const u2 d0 = dequant_codes4(lo, s), d1 = dequant_codes4(hi, s);
  x1 = u4{d0[0], d0[1], d1[0], d1[1]};
}

template <int P, int MAXW, int MAXM, bool SILU, bool X8, bool NORM>
__global__ __launch_bounds__(MAXW * 64) void gemv_stream_kernel(LinearArgs a, int nwg, int tpw, int split,
                                                                float* __restrict__ ws) {
  static_assert(MAXM == 4 || MAXM == 8, "rows per launch");
  static_assert(!NORM || MAXM <= kNormMaxM, "the RMSNorm prologue's scratch serves M <= 4");
  constexpr int kPartLanes = 4 * MAXM;  // lanes whose D registers hold rows < MAXM
  extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
  // Every argument the kernel reads, in SGPRs from the first instruction on: otherwise the
  // compiler loads them next to their first use (x staging, epilogue), each a scalar-memory
  // round trip on the critical path of a short kernel.
  __asm__ volatile("" ::"s"(a.x), "s"(a.x8), "s"(a.ldx), "s"(a.ldx8), "s"(a.qw), "s"(a.scales), "s"(a.qz),
                   "s"(a.bias), "s"(a.out), "s"(a.ldo), "s"(a.residual), "s"(a.ldr), "s"(a.xscale),
                   "s"(a.xscale_stride), "s"(a.m), "s"(a.n), "s"(a.k), "s"(a.log2g), "s"(a.epilogue), "s"(a.norm_w),
                   "s"(a.norm_eps), "s"(a.norm_inv_k), "s"(split), "s"(ws));
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int W = blockDim.x >> 6;
  const int c = lane & 15, g = lane >> 4;

  StreamGeo<SILU> geo;
  geo.nst = a.k >> 7;
  geo.groups = a.k >> a.log2g;
  geo.gps = 128 >> a.log2g;
  const int tiles = a.n >> 4;
  const int half_tiles = a.n >> 5;

  const int bx = xcd_tile(blockIdx.x, nwg);
  // The K slice of this workgroup (the whole of K without a split) and its place among the
  // slice's nps workgroups.
  const int nps = nwg / split;
  const int z = bx / nps;
  const int b = bx - z * nps;
  const int s0 = (int)((uint32_t)(geo.nst * z) / (uint32_t)split);
  const int nst = (int)((uint32_t)(geo.nst * (z + 1)) / (uint32_t)split) - s0;  // steps of the slice
  const int kz = nst * 128;                                                    // K of the slice
  // tiles * nps < 2^31 (checked on the host): 32-bit divisions, far shorter than 64-bit ones.
  const int t0 = (int)((uint32_t)(tiles * b) / (uint32_t)nps);
  const int t1 = (int)((uint32_t)(tiles * (b + 1)) / (uint32_t)nps);
  const int xstride = stream_xstride(kz);
  _Float16* xs = reinterpret_cast<_Float16*>(lds);
  f4* part = reinterpret_cast<f4*>(lds + (a.m * xstride) / 2);  // [W][tpw][4 MAXM]

  // Per-lane parts of the three offsets (see the SiLU*mul note above).
  const uint32_t gl = (uint32_t)((g * 32) >> a.log2g);  // the lane's group inside a step
  uint32_t wl, sl, zl;
  if (SILU) {
    const bool up = c >= 8;
    const uint32_t cl = (uint32_t)(c & 7);
    wl = (up ? (uint32_t)half_tiles * (uint32_t)nst * 1024u : 0u) + (16u * g + cl) * 16u;
    sl = (up ? (uint32_t)half_tiles * (uint32_t)geo.groups * 32u : 0u) + 32u * gl + 2u * (cl & ~1u);
    zl = (up ? (uint32_t)half_tiles * (uint32_t)geo.groups * 8u : 0u) + 8u * gl;
  } else {
    wl = (16u * g + (uint32_t)c) * 16u;
    sl = 32u * gl + 2u * ((uint32_t)c & ~1u);
    zl = 8u * gl + 4u * ((uint32_t)c >> 3);
  }
  const uint32_t zsh = 4u * awq_nibble_of((uint32_t)c & 7u);
  const uint32_t ssel = (c & 1) ? 0x03020302u : 0x01000100u;  // v_perm: this column's scale half
  const uint32_t qw_bytes = (uint32_t)a.n * (uint32_t)(a.k >> 1);
  const uint32_t sc_bytes = (uint32_t)(geo.groups * a.n * 2);
  const uint32_t qz_bytes = (uint32_t)(geo.groups * (a.n >> 3) * 4);

  // Which wave takes which step. Step s of a tile goes to wave (phase(tile) + s) % W, and the
  // phase depends only on the tile's physical position: a column's K steps are summed in the
  // same order whatever the grid (so on any CU count) and under SiLU*mul, whose gate and up
  // tiles u and N/32 + u get one phase (the phase of tile t is that of t mod N/32 when N %
  // 32 == 0). Inside a tile a wave takes every W-th step, so the workgroup's waves read
  // neighbouring blocks; W <= nst gives every wave at least one step of every tile.
  const int wmask = W - 1;
  const int pair_tiles = (a.n & 31) ? tiles : half_tiles;
  auto first_step = [&](int v) {
    const int t = SILU ? (v >> 1) : (v >= pair_tiles ? v - pair_tiles : v);
    return (wave - t * nst) & wmask;
  };
  const int dw = W * 1024, ds = W * geo.gps * 32, dz = W * geo.gps * 8;  // per-issue strides

  // x (all M rows, all of K) is staged in batches of U 16-byte chunks per thread over the
  // flattened (row, chunk) index. The first batch is issued before the weight ring: loads
  // return in order, so x issued behind the ring would reach the workgroup barrier only with
  // the slowest wave's HBM reads (x itself comes from L2 after the first workgroups).
  const int chunks = kz >> 3;
  const int total = a.m * chunks;
  const int64_t kx = (int64_t)s0 * 128;  // first K column of the slice
  const int T = blockDim.x;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)(((int64_t)(a.m - 1) * a.ldx + a.k) * 2));
  const __amdgpu_buffer_rsrc_t rx8 = make_rsrc(a.x8, (uint32_t)((int64_t)(a.m - 1) * a.ldx8 + a.k));
  constexpr int U = 4;
  u4 xv[U];
  auto row_of = [&](int e) {
    int r = 0;
#pragma unroll
    for (int i = 1; i < MAXM; ++i) r += (int)(e >= i * chunks);
    return r;
  };
  auto load_x = [&](int e0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = e0 + u * T;
      const int r = row_of(e), q = e - r * chunks;
      const bool ok = e < total;
      if (X8) {
        const u2 cd = load_b64(rx8, ok ? (uint32_t)((int64_t)r * a.ldx8 + kx + q * 8) : kOutOfRange);
        xv[u] = u4{cd[0], cd[1], 0u, 0u};
      } else {
        xv[u] = load_b128(rx, ok ? (uint32_t)(((int64_t)r * a.ldx + kx + q * 8) * 2) : kOutOfRange);
      }
    }
  };
  auto store_x = [&](int e0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = e0 + u * T;
      const int r = row_of(e), q = e - r * chunks;
      if (e < total)
        *reinterpret_cast<u4*>(xs + r * xstride + q * 8) = X8 ? e4m3x8_to_f16(u2{xv[u][0], xv[u][1]}) : xv[u];
    }
  };
  // One chunk per thread when x is short (M = 1 up to K = 8 T): a single load, no batch.
  const bool one = total <= T;
  u4 x1 = {0u, 0u, 0u, 0u};
  u4 g1 = {0u, 0u, 0u, 0u};  // the norm weight of the thread's chunk (NORM)
  if (one) {
    const int e = threadIdx.x;
    const int r = row_of(e), q = e - r * chunks;
    const bool ok = e < total;
    if (X8) {
      const u2 cd = load_b64(rx8, ok ? (uint32_t)((int64_t)r * a.ldx8 + kx + q * 8) : kOutOfRange);
      x1 = u4{cd[0], cd[1], 0u, 0u};
    } else {
      x1 = load_b128(rx, ok ? (uint32_t)(((int64_t)r * a.ldx + kx + q * 8) * 2) : kOutOfRange);
    }
    if (NORM) g1 = load_b128(make_rsrc(a.norm_w, (uint32_t)a.k * 2u), ok ? (uint32_t)q * 16u : kOutOfRange);
  } else {
    load_x(threadIdx.x);
    // the norm weight's first chunk per thread, issued ahead of the ring like x (NORM)
    if (NORM)
      g1 = load_b128(make_rsrc(a.norm_w, (uint32_t)a.k * 2u),
                     (int)threadIdx.x < chunks ? (uint32_t)threadIdx.x * 16u : kOutOfRange);
  }
  __builtin_amdgcn_sched_barrier(0);

  // Ring of P steps in flight; (iv, is) is the next step this wave issues and (ow, os, oz) its
  // offsets, advanced by the strides inside a tile and recomputed when the wave changes tile.
  u4 rw[P];
  uint32_t rs[P], rz[P];
  int iv = t0, is = first_step(t0), ow, os, oz;
  geo.at(iv, s0 + is, ow, os, oz);
  auto issue = [&](int p) {
    const bool in = iv < t1;
    rw[p] = __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(a.qw, in ? qw_bytes : 0u), (int)wl, in ? ow : 0, 0);
    rs[p] = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(a.scales, in ? sc_bytes : 0u), (int)sl, in ? os : 0, 0);
    rz[p] = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(a.qz, in ? qz_bytes : 0u), (int)zl, in ? oz : 0, 0);
    is += W;
    ow += dw;
    os += ds;
    oz += dz;
    if (is >= nst) {
      ++iv;
      is = first_step(iv);
      geo.at(iv, s0 + is, ow, os, oz);
    }
  };
#pragma unroll
  for (int p = 0; p < P; ++p) {
    issue(p);
    __builtin_amdgcn_sched_barrier(0);  // slot 0 is the oldest load of the ring
  }
  // NORM scratch: the rows' chunk sums, the maxima [4][16], the norm weight [K / 8] chunks
  double* sums = reinterpret_cast<double*>(part + W * tpw * kPartLanes);
  uint32_t* red_u = reinterpret_cast<uint32_t*>(sums + (NORM ? a.m * norm_lpad(a.k) : 0));
  u4* gs = reinterpret_cast<u4*>(red_u + 64);
  if (one) {
    const int e = threadIdx.x;
    const int r = row_of(e), q = e - r * chunks;
    if (NORM) norm_chunk(a, x1, g1, r, q, e < total, sums, red_u, W, wave, lane);
    if (e < total) *reinterpret_cast<u4*>(xs + r * xstride + q * 8) = X8 ? e4m3x8_to_f16(u2{x1[0], x1[1]}) : x1;
  } else {
    store_x(threadIdx.x);
    for (int e0 = threadIdx.x + U * T; e0 < total; e0 += U * T) {
      load_x(e0);
      store_x(e0);
    }
  }
  if (NORM && !one) {
    if ((int)threadIdx.x < chunks) gs[threadIdx.x] = g1;
    for (int q = threadIdx.x + T; q < chunks; q += T)
      gs[q] = load_b128(make_rsrc(a.norm_w, (uint32_t)a.k * 2u), (uint32_t)q * 16u);
    __syncthreads();  // every row of x and the norm weight are in LDS
    norm_rows(a, xs, xstride, sums, red_u, gs, W, wave, lane);
  }
  for (int e = threadIdx.x; e < W * tpw * kPartLanes; e += T) part[e] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  __syncthreads();

  const UnpackConsts uc = unpack_consts();
  const _Float16* xrow = xs + (c < a.m ? c : 0) * xstride + g * 32;  // A operand: row c of x
  f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  int cv = t0, cs = first_step(t0);  // the step this wave consumes next
  while (cv < t1) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      if (cv < t1) {
        const _Float16* xp = xrow + cs * 128;
        h8 xa[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) xa[q] = *reinterpret_cast<const h8*>(xp + q * 8);
        const uint32_t z = (rz[p] >> zsh) & 0xFu;
        const uint32_t zz = z | (z << 16);
        QuantParams qp;
        qp.zlo = as_h2(zz | 0x64006400u);         // 1024 + z (see make_params)
        qp.zhi = as_h2((zz << 4) | 0x54005400u);  // 64 + z
        qp.s = as_h2(__builtin_amdgcn_perm(rs[p], rs[p], ssel));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          h2 wd[4];
          dequant_word(rw[p][q], qp, uc, wd);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[q], pack_h8(wd), acc, 0, 0, 0);
        }
        cs += W;
        if (cs >= nst) {  // the wave leaves this tile: park its partial sums
          if (lane < kPartLanes) part[(wave * tpw + (cv - t0)) * kPartLanes + lane] = acc;
          acc = f4{0.0f, 0.0f, 0.0f, 0.0f};
          ++cv;
          cs = first_step(cv);
        }
      }
      issue(p);
      // Slot boundary: the next slot's work waits for its own loads, not for more of the ring.
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __syncthreads();

  // Each tile's partials in wave order, then bias, row scale and the epilogue. Thread e takes
  // column e % 16 (SiLU*mul: e % 8) of row r and tile tl, (tl, r) = divmod(e / 16, M). Row r
  // of a column is register r % 4 of the lane 16 (r / 4) above the column's.
  const int ntl = t1 - t0;
  const int m = a.m;
  auto divm = [&](int rest, int& tl, int& r) {
    tl = m == 1 ? rest : m == 2 ? (rest >> 1) : m == 4 ? (rest >> 2) : m == 8 ? (rest >> 3) : rest / m;
    r = rest - tl * m;
  };
  if (split > 1) {  // the slice's fp32 sums, for splitk_reduce
    for (int e = threadIdx.x; e < ntl * 16 * m; e += T) {
      int tl, r;
      divm(e >> 4, tl, r);
      const int cc = e & 15;
      float sum = 0.0f;
      for (int w = 0; w < W; ++w) sum += part[(w * tpw + tl) * kPartLanes + 16 * (r >> 2) + cc][r & 3];
      ws[((int64_t)z * m + r) * a.n + 16 * (t0 + tl) + cc] = sum;
    }
  } else if (SILU) {
    for (int e = threadIdx.x; e < ntl * 8 * m; e += T) {
      int tl, r;
      divm(e >> 3, tl, r);
      const int jc = e & 7;
      float gs = 0.0f, us = 0.0f;
      for (int w = 0; w < W; ++w) {
        gs += part[(w * tpw + tl) * kPartLanes + 16 * (r >> 2) + jc][r & 3];
        us += part[(w * tpw + tl) * kPartLanes + 16 * (r >> 2) + 8 + jc][r & 3];
      }
      const int ng = 8 * (t0 + tl) + jc, nu = (a.n >> 1) + ng;
      const float rsc = row_scale(a, r);
      const float vg = gs * rsc + (a.bias ? half_bits_to_float(a.bias[ng]) : 0.0f);
      const float vu = us * rsc + (a.bias ? half_bits_to_float(a.bias[nu]) : 0.0f);
      a.out[(int64_t)r * a.ldo + ng] = finish_silu_mul(vg, vu);
    }
  } else {
    for (int e = threadIdx.x; e < ntl * 16 * m; e += T) {
      int tl, r;
      divm(e >> 4, tl, r);
      const int cc = e & 15;
      float sum = 0.0f;
      for (int w = 0; w < W; ++w) sum += part[(w * tpw + tl) * kPartLanes + 16 * (r >> 2) + cc][r & 3];
      const int n = 16 * (t0 + tl) + cc;
      const float v = sum * row_scale(a, r) + (a.bias ? half_bits_to_float(a.bias[n]) : 0.0f);
      store_out(a, r, n, v);
    }
  }
}

// ------------------------------------------------------------------------ launch plan

struct StreamPlan {
  int nwg = 0;
  int tpw = 0;
  size_t lds = 0;
};

int device_cus() {
  static int cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cache[dev] = v;
  }
  return cache[dev];
}

// K of the longest slice of a K split.
inline int slice_k(int k, int split) { return (int)cdiv(k >> 7, split) * 128; }

// Staged x bytes of a launch: M rows of the longest K slice.
inline size_t stream_x_bytes(const LinearArgs& a, int split) {
  return (size_t)a.m * stream_xstride(slice_k(a.k, split)) * 2;
}

// Workgroups (a multiple of split: the same count on every K slice), tiles per workgroup and
// LDS bytes of a launch (nwg = 0: it does not fit).
template <int MAXM, typename Kernel>
StreamPlan plan_stream(Kernel kernel, const LinearArgs& a, int waves, int depth, int split) {
  StreamPlan p;
  const int tiles = a.n >> 4;
  // The staged x, plus the prologue's reduction scratch behind the partials when it has one.
  const size_t xbytes = stream_x_bytes(a, split) + (a.norm_w ? norm_scratch_bytes(a.m, a.k) : 0);
  const size_t cap = device_max_lds();
  const int per_wave = MAXM * 64;  // bytes of partials per (wave, tile): 4 MAXM lanes x 16
  if (xbytes > (size_t)kStreamMaxXBytes || xbytes + (size_t)waves * per_wave > cap) return p;
  // Fewest tiles per workgroup the LDS allows.
  const int tpw_cap = (int)((cap - xbytes) / ((size_t)waves * per_wave));
  const int min_nps = (int)cdiv(tiles, tpw_cap);
  int per_cu = std::max(1, kStreamInflightKB / (waves * depth));
  for (int pass = 0; pass < 2; ++pass) {
    const int nps = std::max(min_nps, std::min(tiles, std::max(1, device_cus() * per_cu / split)));
    p.nwg = nps * split;
    p.tpw = (int)cdiv(tiles, nps);
    p.lds = xbytes + (size_t)waves * p.tpw * per_wave;
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, waves * 64, p.lds) != hipSuccess || occ <= 0) {
      p.nwg = 0;
      return p;
    }
    if (occ >= per_cu) break;
    per_cu = occ;  // keep the whole grid resident
  }
  return p;
}

// The host-side conditions of the form, before any launch.
template <int MAXM>
int check_stream_shape(const LinearArgs& a, int waves, int split) {
  if (a.m > MAXM)
    return fail(TF_EINVAL, MAXM == 4 ? "tf_w4a16_linear: the gemv stream form (block_k 512, block_m 4) serves M <= 4"
                                     : "tf_w4a16_linear: the gemv stream form (block_k 512, block_m 8) serves M <= 8");
  if ((a.n & 15) || (a.k & 127))
    return fail(TF_EINVAL, "tf_w4a16_linear: the gemv stream form needs N % 16 == 0 and K % 128 == 0");
  if (a.epilogue == TF_EPILOGUE_SILU_MUL && (a.n & 31))
    return fail(TF_EINVAL, "tf_w4a16_linear: the gemv stream form's SiLU*mul epilogue needs N % 32 == 0");
  if ((int64_t)(a.n >> 4) * 65536 >= ((int64_t)1 << 31))
    return fail(TF_EINVAL, "tf_w4a16_linear: the gemv stream form needs N < 2^19");
  if ((a.k >> 7) / split < waves)
    return fail(TF_EINVAL, "tf_w4a16_linear: the gemv stream form needs K / split_k >= 128 * num_warps");
  if (stream_x_bytes(a, split) > (size_t)kStreamMaxXBytes)
    return fail(TF_EINVAL,
                "tf_w4a16_linear: the gemv stream form needs x (M * (K / split_k + 8) halfs) to fit 96 KiB of LDS");
  if (split > 1 && a.norm_w != nullptr)
    return fail(TF_EINVAL, "tf_rmsnorm_fp8_w4a16_linear: the RMSNorm prologue runs without a K split (split_k 1)");
  return check_offsets(a);
}

template <int P, int MAXW, int MAXM>
int check_stream(const LinearArgs& a, const tf_gemm_config& cfg) {
  if (int rc = check_stream_shape<MAXM>(a, cfg.num_warps, cfg.split_k)) return rc;
  if (MAXM > kNormMaxM && a.norm_w != nullptr)
    return fail(TF_EINVAL, "tf_rmsnorm_fp8_w4a16_linear: the RMSNorm prologue runs on the block_m 4 stream form");
  // Every instantiation has the same launch plan (one of them stands for all).
  const StreamPlan plan =
      plan_stream<MAXM>(gemv_stream_kernel<P, MAXW, MAXM, false, false, false>, a, cfg.num_warps, P, cfg.split_k);
  if (plan.nwg == 0)
    return fail(TF_EINVAL, "tf_w4a16_linear: gemv stream variant does not fit the device's LDS");
  return TF_OK;
}

template <int P, int MAXW, int MAXM, bool SILU, bool X8, bool NORM>
int launch_stream_k(const LinearArgs& a, int waves, int split, float* ws, hipStream_t stream) {
  auto kernel = gemv_stream_kernel<P, MAXW, MAXM, SILU, X8, NORM>;
  const StreamPlan plan = plan_stream<MAXM>(kernel, a, waves, P, split);
  if (plan.nwg == 0) return fail(TF_EINVAL, "tf_w4a16_linear: gemv stream variant does not fit the device's LDS");
  if (int rc = reserve_lds(kernel, plan.lds, "gemv_stream")) return rc;
  kernel<<<plan.nwg, waves * 64, plan.lds, stream>>>(a, plan.nwg, plan.tpw, split, ws);
  if (int rc = check_launch("tf_w4a16_linear(gemv stream)")) return rc;
  return split > 1 ? splitk_reduce(a, ws, split, stream) : TF_OK;
}

template <int P, int MAXW, int MAXM>
int launch_stream(const LinearArgs& a, const tf_gemm_config& cfg, float* ws, hipStream_t stream) {
  const int split = cfg.split_k;
  if (int rc = check_stream_shape<MAXM>(a, cfg.num_warps, split)) return rc;
  if (split > 1 && ws == nullptr) return fail(TF_EINVAL, "tf_w4a16_linear: this config needs a workspace");
  const bool x8 = a.x8 != nullptr, norm = a.norm_w != nullptr;
  // With a K split the reduce kernel applies the epilogue: the kernel sums physical columns.
  const bool silu = a.epilogue == TF_EPILOGUE_SILU_MUL && split == 1;
  const int w = cfg.num_warps;
  if (norm && x8) return fail(TF_EINVAL, "tf_w4a16_linear: the RMSNorm prologue takes fp16 x");
  if (norm && a.k > kNormMaxK)
    return fail(TF_EINVAL, "tf_rmsnorm_fp8_w4a16_linear: the RMSNorm prologue serves K <= 8192");
  if constexpr (MAXM <= kNormMaxM) {
    if (norm)
      return silu ? launch_stream_k<P, MAXW, MAXM, true, false, true>(a, w, split, ws, stream)
                  : launch_stream_k<P, MAXW, MAXM, false, false, true>(a, w, split, ws, stream);
  } else {
    if (norm)
      return fail(TF_EINVAL, "tf_rmsnorm_fp8_w4a16_linear: the RMSNorm prologue runs on the block_m 4 stream form");
  }
  if (silu)
    return x8 ? launch_stream_k<P, MAXW, MAXM, true, true, false>(a, w, split, ws, stream)
              : launch_stream_k<P, MAXW, MAXM, true, false, false>(a, w, split, ws, stream);
  return x8 ? launch_stream_k<P, MAXW, MAXM, false, true, false>(a, w, split, ws, stream)
            : launch_stream_k<P, MAXW, MAXM, false, false, false>(a, w, split, ws, stream);
}

// fp32 partials [split][M][N] under a K split, else none.
int64_t stream_workspace(const LinearArgs& a, const tf_gemm_config& cfg) {
  return cfg.split_k > 1 ? (int64_t)cfg.split_k * a.m * a.n * (int64_t)sizeof(float) : 0;
}

#define TF_SW(P, W) \
  {{TF_KERNEL_GEMV_MFMA, 4, 16, 512, 1, W, P}, launch_stream<P, 16, 4>, stream_workspace, check_stream<P, 16, 4>}
#define TF_SW5(P) TF_SW(P, 1), TF_SW(P, 2), TF_SW(P, 4), TF_SW(P, 8), TF_SW(P, 16)
#define TF_SW8(P, W) \
  {{TF_KERNEL_GEMV_MFMA, 8, 16, 512, 1, W, P}, launch_stream<P, 16, 8>, stream_workspace, check_stream<P, 16, 8>}

// block_k 512 marks the stream form; block_m its largest M (4, or 8: 4 M lanes of partials per
// column instead of 1, no RMSNorm prologue); num_stages the ring depth; split_k (runtime) the
// K split across workgroups.
const Variant kStreamVariants[] = {TF_SW5(2), TF_SW5(4),    TF_SW8(2, 4), TF_SW8(2, 8),
                                   TF_SW8(2, 16), TF_SW8(4, 4), TF_SW8(4, 8), TF_SW8(4, 16)};

}  // namespace

const Variant* gemv_stream_variants(int* count) {
  *count = (int)(sizeof(kStreamVariants) / sizeof(kStreamVariants[0]));
  return kStreamVariants;
}

}  // namespace tf
