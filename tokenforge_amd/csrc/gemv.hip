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

// K range [s0, s1) of 128-wide steps owned by `wave`; waves is a power of two (every compiled
// variant's num_warps is). All arguments are wave-uniform, so the range and every loop bound
// derived from it live in scalar registers.
__device__ __forceinline__ void k_range(int wave, int waves, int nsteps, int* s0, int* s1) {
  const int sh = __builtin_ctz((unsigned)waves);
  *s0 = (wave * nsteps) >> sh;
  *s1 = ((wave + 1) * nsteps) >> sh;
}

// Buffer resources and per-launch constants shared by both kernels.
struct Streams {
  __amdgpu_buffer_rsrc_t qw, sc, qz, x, x8;
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
  s.x8 = make_rsrc(a.x8, (uint32_t)((int64_t)(a.m - 1) * a.ldx8 + a.k));
  s.nchunks = a.k >> 5;
  s.nsteps = (s.nchunks + 3) >> 2;
  s.log2g = a.log2g;
  s.n = a.n;
  return s;
}

// Largest number of 128-wide K steps any wave gets.
__host__ __device__ __forceinline__ int max_steps(int nsteps, int waves) { return (nsteps + waves - 1) / waves; }

// One staged (group, column) entry: fp16x2 (1024 + z), fp16x2 (64 + z), fp16x2 scale, unused;
// four words so a lane fetches it with a single ds_read_b128.
constexpr int kParamWords = 4;

// Staging of one window of a wave's K range into its LDS region:
//  * params: the dequantization operands of groups [g_lo, g_lo + ng) x columns
//    the tile's 16 RT columns (phys_col), `slots` groups deep. Slots past ng get neutral operands (zero
//    point 0, scale 0), so any word dequantizes to exactly 0 there.
//  * x (rows > 0): x[m0 + r][k0, k0 + kn) for r < rows, row stride xstride halfs, zero at
//    k >= K (buffer loads past the tensor return zeros only at its very end, so the K bound is
//    explicit).
// Work is split into batches of 64 U entries of each kind: load_batch issues a batch's loads
// into registers, store_batch writes them to LDS, so a batch costs one memory latency and the
// first batch can be issued ahead of the weight ring.
struct Window {
  int n_base, g_lo, ng, pentries;
  int m0, rows, k0, chunks, xentries, xstride;
  float inv_chunks;
  int total;  // max(pentries, xentries)
};

template <int RT>
__device__ __forceinline__ Window make_window(const Streams& st, int n_base, int w0, int w1, int slots, int m0,
                                              int rows, int xstride) {
  Window w;
  w.n_base = n_base;
  w.g_lo = (w0 * 128) >> st.log2g;
  w.ng = min(st.groups, (w1 * 128) >> st.log2g) - w.g_lo;
  w.pentries = w1 > w0 ? slots * 16 * RT : 0;
  w.m0 = m0;
  w.rows = rows;
  w.k0 = w0 * 128;
  w.chunks = (w1 - w0) * 16;  // 16-byte x chunks per row
  w.xentries = rows * w.chunks;
  w.xstride = xstride;
  w.inv_chunks = 1.0f / (float)(w.chunks > 0 ? w.chunks : 1);
  w.total = max(w.pentries, w.xentries);
  return w;
}

template <int U>
struct StageBatch {
  uint32_t sb[U], zw[U];
  u4 xv[U];
  int xr[U], xq[U];
};

template <int RT, int U>
__device__ __forceinline__ void load_batch(StageBatch<U>& b, const Window& w, const LinearArgs& a,
                                           const Streams& st, int base, int lane) {
  constexpr int cols = 16 * RT;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int e = base + u * 64 + lane;
    const int gi = e / cols;
    const int n = phys_col(a, w.n_base, e % cols);
    const bool ok = e < w.pentries && col_valid(a, w.n_base, e % cols) && gi < w.ng;
    const uint32_t grp = (uint32_t)(w.g_lo + gi);
    b.sb[u] = load_b16(st.sc, ok ? (grp * (uint32_t)st.n + (uint32_t)n) * 2u : kOutOfRange);
    b.zw[u] = load_b32(st.qz, ok ? (grp * (uint32_t)(st.n >> 3) + (uint32_t)(n >> 3)) * 4u : kOutOfRange);
    // e = r * chunks + q; the float quotient is off by at most one for e < 2^24.
    int r = (int)((float)e * w.inv_chunks);
    int q = e - r * w.chunks;
    if (q < 0) {
      r -= 1;
      q += w.chunks;
    } else if (q >= w.chunks) {
      r += 1;
      q -= w.chunks;
    }
    b.xr[u] = r;
    b.xq[u] = q;
    const int k = w.k0 + q * 8;
    const bool xok = e < w.xentries && k < a.k;
    if (a.x8 != nullptr) {  // e4m3 codes, converted to fp16 when stored
      const u2 c = load_b64(st.x8, xok ? (uint32_t)((int64_t)(w.m0 + r) * a.ldx8 + k) : kOutOfRange);
      b.xv[u] = u4{c[0], c[1], 0u, 0u};
    } else {
      b.xv[u] = load_b128(st.x, xok ? (uint32_t)((w.m0 + r) * a.ldx + k) * 2u : kOutOfRange);
    }
  }
}

template <int RT, int U>
__device__ __forceinline__ void store_batch(uint32_t* p, _Float16* xs, const StageBatch<U>& b, const Window& w,
                                            const LinearArgs& a, int base, int lane) {
  constexpr int cols = 16 * RT;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int e = base + u * 64 + lane;
    if (e < w.pentries) {
      const int n = phys_col(a, w.n_base, e % cols);
      const QuantParams q = make_params(zero_of(b.zw[u], (uint32_t)n), b.sb[u]);
      *reinterpret_cast<u4*>(p + kParamWords * e) = u4{as_u32(q.zlo), as_u32(q.zhi), as_u32(q.s), 0u};
    }
    if (e < w.xentries)
      *reinterpret_cast<u4*>(xs + b.xr[u] * w.xstride + b.xq[u] * 8) =
          a.x8 != nullptr ? e4m3x8_to_f16(u2{b.xv[u][0], b.xv[u][1]}) : b.xv[u];
  }
}

// Stage the batches of a window from `first` on.
template <int RT, int U>
__device__ __forceinline__ void stage_rest(uint32_t* p, _Float16* xs, const Window& w, const LinearArgs& a,
                                           const Streams& st, int first, int lane) {
  for (int base = first; base < w.total; base += 64 * U) {
    StageBatch<U> b;
    load_batch<RT, U>(b, w, a, st, base, lane);
    store_batch<RT, U>(p, xs, b, w, a, base, lane);
  }
}

__device__ __forceinline__ QuantParams read_params(const uint32_t* p) {
  const u4 v = *reinterpret_cast<const u4*>(p);
  QuantParams q;
  q.zlo = as_h2(v[0]);
  q.zhi = as_h2(v[1]);
  q.s = as_h2(v[2]);
  return q;
}

// Per-lane view of the weight stream: the lane reads 16 bytes (chunk g = 32 K values) of one
// row per row tile and step; its rows are local columns l0 + 16 rt of the tile at n_base
// (phys_col). off[rt] is the byte offset of that run in step 0 (kOutOfRange past N, and still
// out of range after adding any step offset); lane_end is the first step whose chunk lies past
// K for this lane or past the wave's range.
template <int RT>
struct LaneStream {
  uint32_t off[RT];
  int lane_end;

  __device__ __forceinline__ LaneStream(const LinearArgs& a, const Streams& st, int n_base, int l0, int g, int s1) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int l = l0 + rt * 16;
      off[rt] = col_valid(a, n_base, l) ? (uint32_t)phys_col(a, n_base, l) * st.row_bytes + (uint32_t)g * 16u
                                        : kOutOfRange;
    }
    lane_end = min(s1, (st.nchunks - g + 3) >> 2);
  }

  // Every call issues exactly RT loads (zeros when the step is out of range), so the ring
  // below has the same loads in flight on every path and the compiler's vmcnt waits stay
  // exact instead of draining the ring.
  __device__ __forceinline__ void issue(u4 (&w)[RT], const Streams& st, int step) const {
    const bool v = step < lane_end;
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) w[rt] = load_b128(st.qw, v ? off[rt] + (uint32_t)step * 64u : kOutOfRange);
  }
};

// LDS carve-up of one launch. Each wave stages a window of `win` steps: its params for the
// window's groups and (XLDS) the window's x slice; a wave whose range is longer re-stages per
// window. When a range takes several windows, each holds a multiple of the ring depth, so ring
// slot p always holds a step with (step - s0) % P == p.
struct GemvLds {
  int pwords;      // params words per wave
  int xstride;     // halfs per staged x row
  int wave_words;  // params + x words per wave
};

__host__ __device__ __forceinline__ GemvLds gemv_lds_layout(int win, int log2g, int cols, int x_rows) {
  GemvLds l;
  l.pwords = win * (128 >> log2g) * cols * kParamWords;
  l.xstride = win * 128 + 8;
  l.wave_words = l.pwords + (x_rows * l.xstride) / 2;
  return l;
}

// ------------------------------------------------------------------------ gemv_dot

constexpr int kStageU = 2;  // staging entries per lane and batch

template <int MAXM, int RT, int P, int MAXW>
__global__ __launch_bounds__(MAXW * 64) void gemv_dot_kernel(LinearArgs a, int win) {
  extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int waves = blockDim.x >> 6;
  const int g = lane & 3;
  const int c = lane >> 2;
  constexpr int cols = 16 * RT;
  const int n_base = xcd_tile(blockIdx.x, gridDim.x) * cols;
  const Streams st = make_streams(a);
  int s0, s1;
  k_range(wave, waves, st.nsteps, &s0, &s1);
  const int gps = 128 >> st.log2g;
  const int xrows = a.m < MAXM ? a.m : MAXM;
  const GemvLds L = gemv_lds_layout(win, st.log2g, cols, xrows);
  uint32_t* prm = lds + wave * L.wave_words;
  _Float16* xs = reinterpret_cast<_Float16*>(prm + L.pwords);
  const UnpackConsts uc = unpack_consts();
  const LaneStream<RT> ls_w(a, st, n_base, c, g, s1);

  // Lane bases in LDS; a step adds a wave-uniform offset.
  const uint32_t* plane = prm + kParamWords * ((((g * 32) >> st.log2g) * cols) + c);
  const int pstep = kParamWords * gps * cols;
  const _Float16* xl = xs + g * 32;

  float acc[MAXM][RT];
#pragma unroll
  for (int m = 0; m < MAXM; ++m)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[m][rt] = 0.0f;

  // The first staging batch goes out ahead of the weight ring: every wave of the grid issues
  // its ring at once, and the operands that gate the first step must not queue behind it.
  Window win0 = make_window<RT>(st, n_base, s0, min(s1, s0 + win), win * gps, 0, xrows, L.xstride);
  StageBatch<kStageU> first;
  load_batch<RT, kStageU>(first, win0, a, st, 0, lane);
  __builtin_amdgcn_sched_barrier(0);
  u4 ring[P][RT];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    ls_w.issue(ring[p], st, s0 + p);
    __builtin_amdgcn_sched_barrier(0);  // keep slot order: slot 0 must be the oldest ring load
  }
  store_batch<RT, kStageU>(prm, xs, first, win0, a, 0, lane);
  stage_rest<RT, kStageU>(prm, xs, win0, a, st, 64 * kStageU, lane);

  for (int w0 = s0; w0 < s1; w0 += win) {
    const int w1 = min(s1, w0 + win);
    if (w0 != s0) stage_rest<RT, kStageU>(prm, xs, make_window<RT>(st, n_base, w0, w1, win * gps, 0, xrows, L.xstride),
                                         a, st, 0, lane);
    for (int s = w0; s < w1; s += P) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const int step = s + p;
        if (step < w1) {
          const int ls = step - w0;
          u4 xv[MAXM][4];
#pragma unroll
          for (int m = 0; m < MAXM; ++m) {
            const int row = m < xrows ? m : 0;  // rows past M only feed accumulators never stored
#pragma unroll
            for (int j = 0; j < 4; ++j)
              xv[m][j] = *reinterpret_cast<const u4*>(xl + row * L.xstride + ls * 128 + j * 8);
          }
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            const QuantParams qp = read_params(plane + ls * pstep + rt * 16 * kParamWords);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              h2 wd[4];
              dequant_word(ring[p][rt][j], qp, uc, wd);
#pragma unroll
              for (int m = 0; m < MAXM; ++m)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                  acc[m][rt] = __builtin_amdgcn_fdot2(as_h2(xv[m][j][i]), wd[i], acc[m][rt], false);
            }
          }
        }
        ls_w.issue(ring[p], st, step + P);
      }
    }
  }

#pragma unroll
  for (int m = 0; m < MAXM; ++m)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[m][rt] = quad_sum(acc[m][rt]);

  if (waves > 1) {
    float* red = reinterpret_cast<float*>(lds + waves * L.wave_words);  // [(waves - 1)][MAXM][RT][16]
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
  // Lane 4 c (g == 0) holds row c of each row tile. Under SiLU*mul rows c and c ^ 8 are the
  // gate and up columns of one output (phys_col): lanes 4c and 4c ^ 32 swap their values.
  if (wave == 0) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int l = rt * 16 + c;
      const int n = phys_col(a, n_base, l);
      const bool valid = g == 0 && col_valid(a, n_base, l);
      const float b = (a.bias && valid) ? half_bits_to_float(a.bias[n]) : 0.0f;
#pragma unroll
      for (int m = 0; m < MAXM; ++m) {
        const float v = acc[m][rt] * row_scale(a, m) + b;
        if (a.epilogue == TF_EPILOGUE_SILU_MUL) {
          const float u = __shfl_xor(v, 32);
          if (valid && !(l & 8) && m < a.m)
            a.out[(int64_t)m * a.ldo + silu_out_col(n_base, l)] = finish_silu_mul(v, u);
        } else if (valid && m < a.m) {
          store_out(a, m, n, v);
        }
      }
    }
  }
}

// ------------------------------------------------------------------------ gemv_mfma

template <int MT, int RT, int P, int MAXW, bool XLDS>
__global__ __launch_bounds__(MAXW * 64) void gemv_mfma_kernel(LinearArgs a, int win) {
  extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int waves = blockDim.x >> 6;
  const int c = lane & 15;
  const int g = lane >> 4;
  constexpr int cols = 16 * RT;
  const int n_base = xcd_tile(blockIdx.x, gridDim.x) * cols;
  const int m_base = blockIdx.y * 16 * MT;
  const Streams st = make_streams(a);
  int s0, s1;
  k_range(wave, waves, st.nsteps, &s0, &s1);
  const int gps = 128 >> st.log2g;
  const int xrows = min(16 * MT, a.m - m_base);  // rows staged by this workgroup
  const int xalloc = min(16 * MT, a.m);          // rows allocated per wave (same in every workgroup)
  const GemvLds L = gemv_lds_layout(win, st.log2g, cols, XLDS ? xalloc : 0);
  uint32_t* prm = lds + wave * L.wave_words;
  _Float16* xs = reinterpret_cast<_Float16*>(prm + L.pwords);
  const UnpackConsts uc = unpack_consts();
  const LaneStream<RT> ls_w(a, st, n_base, c, g, s1);

  const uint32_t* plane = prm + kParamWords * ((((g * 32) >> st.log2g) * cols) + c);
  const int pstep = kParamWords * gps * cols;
  const _Float16* xl[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = mt * 16 + c;
    xl[mt] = xs + (r < xrows ? r : 0) * L.xstride + g * 32;  // rows past M feed discarded outputs
  }
  // x streamed with the weights (block_k 64 variants): 64 bytes of row m per lane and step.
  uint32_t xoff[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = m_base + mt * 16 + c;
    xoff[mt] = m < a.m ? (uint32_t)(((int64_t)m * a.ldx + g * 32) * 2) : kOutOfRange;
  }

  f4 acc[MT][RT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[mt][rt] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  u4 ring[P][RT];
  u4 xring[XLDS ? 1 : P][XLDS ? 1 : MT][4];
  auto issue = [&](int p, int step) {
    ls_w.issue(ring[p], st, step);
    if (!XLDS) {
      const bool v = step < ls_w.lane_end;
#pragma unroll
      for (int mt = 0; mt < (XLDS ? 0 : MT); ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          xring[XLDS ? 0 : p][mt][j] =
              load_b128(st.x, v ? xoff[mt] + (uint32_t)step * 256u + 16u * j : kOutOfRange);
    }
  };
  // The first staging batch goes out ahead of the weight ring (see gemv_dot_kernel).
  const int srows = XLDS ? xrows : 0;
  Window win0 = make_window<RT>(st, n_base, s0, min(s1, s0 + win), win * gps, m_base, srows, L.xstride);
  StageBatch<kStageU> first;
  load_batch<RT, kStageU>(first, win0, a, st, 0, lane);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int p = 0; p < P; ++p) {
    issue(p, s0 + p);
    __builtin_amdgcn_sched_barrier(0);  // keep slot order: slot 0 must be the oldest ring load
  }
  store_batch<RT, kStageU>(prm, xs, first, win0, a, 0, lane);
  stage_rest<RT, kStageU>(prm, xs, win0, a, st, 64 * kStageU, lane);

  for (int w0 = s0; w0 < s1; w0 += win) {
    const int w1 = min(s1, w0 + win);
    if (w0 != s0)
      stage_rest<RT, kStageU>(prm, xs, make_window<RT>(st, n_base, w0, w1, win * gps, m_base, srows, L.xstride), a,
                             st, 0, lane);
    for (int s = w0; s < w1; s += P) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const int step = s + p;
        if (step < w1) {
          const int ls = step - w0;
          h8 xa[MT][4];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              xa[mt][j] = XLDS ? *reinterpret_cast<const h8*>(xl[mt] + ls * 128 + j * 8)
                               : __builtin_bit_cast(h8, xring[XLDS ? 0 : p][mt][j]);
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            const QuantParams qp = read_params(plane + ls * pstep + rt * 16 * kParamWords);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              h2 wd[4];
              dequant_word(ring[p][rt][j], qp, uc, wd);
              const h8 b = pack_h8(wd);
#pragma unroll
              for (int mt = 0; mt < MT; ++mt)
                acc[mt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[mt][j], b, acc[mt][rt], 0, 0, 0);
            }
          }
        }
        issue(p, step + P);
      }
    }
  }

  if (waves > 1) {
    float* red = reinterpret_cast<float*>(lds + waves * L.wave_words);  // [(waves - 1)][MT][RT][64][4]
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
    // Under SiLU*mul lanes c and c ^ 8 hold the gate and up columns of one output.
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int l = rt * 16 + c;
      const int n = phys_col(a, n_base, l);
      const bool valid = col_valid(a, n_base, l);
      const float b = (a.bias && valid) ? half_bits_to_float(a.bias[n]) : 0.0f;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m_base + mt * 16 + 4 * g + r;
          const float v = acc[mt][rt][r] * row_scale(a, m) + b;
          if (a.epilogue == TF_EPILOGUE_SILU_MUL) {
            const float u = __shfl_xor(v, 8);
            if (valid && !(l & 8) && m < a.m)
              a.out[(int64_t)m * a.ldo + silu_out_col(n_base, l)] = finish_silu_mul(v, u);
          } else if (valid && m < a.m) {
            store_out(a, m, n, v);
          }
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

// Staging window (in steps) and LDS bytes of a gemv launch. The window covers a wave's whole
// K range when that fits the device's LDS (one window, so its length is free); otherwise it is
// the largest multiple of the ring depth that fits. win = 0 when not even one ring's worth fits.
struct GemvPlan {
  int win;
  size_t lds;
};

GemvPlan plan_gemv(const LinearArgs& a, int waves, int rt, int depth, int x_rows, size_t red_per_wave) {
  const int nsteps = ((a.k >> 5) + 3) >> 2;
  const int steps = max_steps(nsteps, waves);
  const size_t cap = device_max_lds();
  auto bytes = [&](int win) {
    const GemvLds l = gemv_lds_layout(win, a.log2g, 16 * rt, x_rows);
    return (size_t)waves * (size_t)l.wave_words * 4 + (size_t)(waves - 1) * red_per_wave;
  };
  if (bytes(steps) <= cap) return GemvPlan{steps, bytes(steps)};
  int win = (steps - 1) / depth * depth;
  while (win > depth && bytes(win) > cap) win -= depth;
  if (win < depth || bytes(win) > cap) return GemvPlan{0, 0};
  return GemvPlan{win, bytes(win)};
}

template <int MAXM, int RT, int P, int MAXW>
int launch_dot(const LinearArgs& a, const tf_gemm_config& cfg, float*, hipStream_t stream) {
  if (a.m > MAXM) return fail(TF_EINVAL, "tf_w4a16_linear: gemv_dot variant needs m <= block_m");
  if (int rc = check_offsets(a)) return rc;
  const int waves = cfg.num_warps;
  const GemvPlan plan = plan_gemv(a, waves, RT, P, a.m < MAXM ? a.m : MAXM, (size_t)MAXM * RT * 16 * sizeof(float));
  if (plan.win == 0) return fail(TF_EINVAL, "tf_w4a16_linear: gemv_dot variant does not fit the device's LDS");
  if (int rc = reserve_lds(gemv_dot_kernel<MAXM, RT, P, MAXW>, plan.lds, "gemv_dot")) return rc;
  const dim3 grid((unsigned)cdiv(a.n, 16 * RT));
  gemv_dot_kernel<MAXM, RT, P, MAXW><<<grid, waves * 64, plan.lds, stream>>>(a, plan.win);
  return check_launch("tf_w4a16_linear(gemv_dot)");
}

template <int MT, int RT, int P, int MAXW, bool XLDS>
int launch_mfma(const LinearArgs& a, const tf_gemm_config& cfg, float*, hipStream_t stream) {
  if (int rc = check_offsets(a)) return rc;
  const int waves = cfg.num_warps;
  const GemvPlan plan = plan_gemv(a, waves, RT, P, XLDS ? (a.m < 16 * MT ? a.m : 16 * MT) : 0,
                                  (size_t)MT * RT * 64 * 4 * sizeof(float));
  if (plan.win == 0) return fail(TF_EINVAL, "tf_w4a16_linear: gemv_mfma variant does not fit the device's LDS");
  if (int rc = reserve_lds(gemv_mfma_kernel<MT, RT, P, MAXW, XLDS>, plan.lds, "gemv_mfma")) return rc;
  const dim3 grid((unsigned)cdiv(a.n, 16 * RT), (unsigned)cdiv(a.m, 16 * MT));
  gemv_mfma_kernel<MT, RT, P, MAXW, XLDS><<<grid, waves * 64, plan.lds, stream>>>(a, plan.win);
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
