// Decode-shaped W4A16 kernel (small M) on the gfx950 tile layout: stream the packed weights
// once, dequantize in registers (fp16(q - z) * s, one rounding), multiply on the matrix cores.
//
// Lane l = 16 g + c of a wave owns column c of a 16-row tile and K block g of every 128-wide K
// step: its 16 bytes of a step are chunk (c, g) of the tile layout, which sits at byte 16 l of
// the step's 1 KB block, so one 128-bit buffer load per wave reads one whole block (two full
// 128-byte lines per 16 lanes). Those 16 bytes (32 K values, one group for G >= 32) are exactly
// the B operand of v_mfma_f32_16x16x32_f16 for four MFMAs: MFMA j takes word j of every lane,
// K set {32 g + 8 j + e}; x rows are the A operand, read from LDS at the same K positions. The
// matrix core does the dot products and the VALU only unpacks and scales (13 instructions per
// packed word); rows m >= M of the A operand feed output rows that are never stored.
//
// Work split: a workgroup owns block_n = 16 * RT consecutive columns (RT tiles). block_k 128:
// its num_warps waves take disjoint, contiguous K ranges of those columns (on-chip split-K) and
// add their partial sums in wave order through LDS (bit-identical from run to run, no
// workspace, no atomics). block_k 256: the waves take different column sets over the whole K
// and share one copy of x staged cooperatively (one barrier, no reduction).
//
// Memory stream: every wave keeps a register ring of P steps in flight: per tile the 16 weight
// bytes, the scales word holding its column's scale and the qzeros word of its column and
// group. The loads of step s + P are issued as soon as step s has been consumed. Buffer loads
// return zeros past the end of a tensor (and for chunks past K), so ragged N and a partial last
// step need no branches. When every tile is full and K is a multiple of 128 ("uniform"), the
// step part of every offset is wave-uniform and rides in the loads' scalar offset.
//
// Before the loop each wave stages its slice of x in its own LDS region (no barrier: a wave
// reads only what it wrote); the first staging batch is issued ahead of the weight ring.
#include "linear.h"
#include "tile_layout.h"

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

// Buffer resources and per-launch constants.
struct Streams {
  __amdgpu_buffer_rsrc_t qw, sc, qz, x, x8;
  const void *qw_ptr, *sc_ptr, *qz_ptr;
  uint32_t qw_bytes, sc_bytes, qz_bytes;
  int q_total;  // K / 32: 16-byte chunks per row
  int nsteps;   // ceil(K / 128)
  int groups;   // K / G
  int log2g;
  int n;
};

__device__ __forceinline__ Streams make_streams(const LinearArgs& a) {
  Streams s;
  s.groups = a.k >> a.log2g;
  s.q_total = a.k >> 5;
  s.nsteps = (s.q_total + 3) >> 2;
  s.qw_bytes = (uint32_t)a.n * (uint32_t)(a.k >> 1);
  s.sc_bytes = (uint32_t)(s.groups * a.n * 2);
  s.qz_bytes = (uint32_t)(s.groups * (a.n >> 3) * 4);
  s.qw = make_rsrc(a.qw, s.qw_bytes);
  s.sc = make_rsrc(a.scales, s.sc_bytes);
  s.qz = make_rsrc(a.qz, s.qz_bytes);
  s.x = make_rsrc(a.x, (uint32_t)(((int64_t)(a.m - 1) * a.ldx + a.k) * 2));
  s.x8 = make_rsrc(a.x8, (uint32_t)((int64_t)(a.m - 1) * a.ldx8 + a.k));
  s.qw_ptr = a.qw;
  s.sc_ptr = a.scales;
  s.qz_ptr = a.qz;
  s.log2g = a.log2g;
  s.n = a.n;
  return s;
}

// Largest number of 128-wide K steps any wave gets.
__host__ __device__ __forceinline__ int max_steps(int nsteps, int waves) { return (nsteps + waves - 1) / waves; }

// Staging of one window of a wave's x slice into its LDS region: x[m0 + r][k0, k0 + kn) for
// r < rows, row stride xstride halfs, zero at k >= K (buffer loads past the tensor return zeros
// only at its very end, so the K bound is explicit). Work is split into batches of 64 U 16-byte
// chunks: load_batch issues a batch's loads into registers, store_batch writes them to LDS, so
// a batch costs one memory latency and the first batch can be issued ahead of the weight ring.
struct Window {
  int m0, rows, k0, chunks, xentries, xstride;
  float inv_chunks;
};

__device__ __forceinline__ Window make_window(int w0, int w1, int m0, int rows, int xstride) {
  Window w;
  w.m0 = m0;
  w.rows = rows;
  w.k0 = w0 * 128;
  w.chunks = (w1 - w0) * 16;  // 16-byte x chunks per row
  w.xentries = rows * w.chunks;
  w.xstride = xstride;
  w.inv_chunks = 1.0f / (float)(w.chunks > 0 ? w.chunks : 1);
  return w;
}

template <int U>
struct StageBatch {
  u4 xv[U];
  int xr[U], xq[U];
};

template <int U>
__device__ __forceinline__ void load_batch(StageBatch<U>& b, const Window& w, const LinearArgs& a,
                                           const Streams& st, int base, int lane) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int e = base + u * 64 + lane;
    // e = r * chunks + q; the float quotient is off by at most one for e < 2^24. One row (the
    // decode case) needs no division.
    int r = 0, q = e;
    if (w.rows > 1) {
      r = (int)((float)e * w.inv_chunks);
      q = e - r * w.chunks;
      if (q < 0) {
        r -= 1;
        q += w.chunks;
      } else if (q >= w.chunks) {
        r += 1;
        q -= w.chunks;
      }
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

template <int U>
__device__ __forceinline__ void store_batch(_Float16* xs, const StageBatch<U>& b, const Window& w,
                                            const LinearArgs& a, int base, int lane) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int e = base + u * 64 + lane;
    if (e < w.xentries)
      *reinterpret_cast<u4*>(xs + b.xr[u] * w.xstride + b.xq[u] * 8) =
          a.x8 != nullptr ? e4m3x8_to_f16(u2{b.xv[u][0], b.xv[u][1]}) : b.xv[u];
  }
}

// Stage the batches of a window from `first` on.
template <int U>
__device__ __forceinline__ void stage_rest(_Float16* xs, const Window& w, const LinearArgs& a, const Streams& st,
                                           int first, int lane) {
  for (int base = first; base < w.xentries; base += 64 * U) {
    StageBatch<U> b;
    load_batch<U>(b, w, a, st, base, lane);
    store_batch<U>(xs, b, w, a, base, lane);
  }
}

// One ring slot: per tile, the lane's 16 weight bytes, the scales word holding its column's
// scale (and its even/odd neighbour's) and the qzeros word of its column, for the lane's group.
// Whole words: no extension of a 16-bit load sits between a load and its use, where the
// compiler would wait for it early.
template <int RT>
struct Slot {
  u4 w[RT];
  uint32_t sw[RT], zw[RT];
};

// Per-lane view of the three streams in the tile layout. The lane reads chunk (column, K block
// g) of each of its RT tiles per step; its columns are local columns c + 16 rt of the set at
// n_base (phys_col). Offsets are those of step 0 (kOutOfRange past N, and still out of range
// after adding any step offset); *step are the per-step byte strides (for a full tile: 1 KB of
// weights, (128 / G) * 32 bytes of scales, (128 / G) * 8 bytes of zero words). lane_end is the
// first step whose chunk lies past K for this lane, or the wave's end.
//
// UNIFORM (every tile full, K a multiple of 128): the strides are the same in every lane and
// every chunk of the wave's range is inside K, so the step part of each offset is wave-uniform
// and goes into the loads' scalar offset. That part is not range-checked by the hardware; it
// never leaves the tensors because issued steps stay below the wave's end (steps past it go
// through resources with zero records) and the vector part addresses a valid chunk, scale and
// zero word (or is out of range, which stays out of range).
template <int RT, bool UNIFORM>
struct LaneStream {
  uint32_t woff[RT], soff[RT], zoff[RT], zsh[RT], ssel[RT];
  uint32_t wstep[RT], sstep[RT], zstep[RT];
  int lane_end;
  int wave_end;  // s1, wave-uniform

  __device__ __forceinline__ LaneStream(const LinearArgs& a, const Streams& st, int n_base, int l0, int g, int s1) {
    const uint32_t gl = (uint32_t)((g * 32) >> st.log2g);  // the lane's group inside a step
    const uint32_t gps = (uint32_t)(128 >> st.log2g);       // groups per step
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int l = l0 + rt * 16;
      const bool ok = col_valid(a, n_base, l);
      const uint32_t n = (uint32_t)phys_col(a, n_base, l);
      const uint32_t t = n >> 4, cc = n & 15u;
      const uint32_t rows = (uint32_t)tile_rows(st.n, t);
      woff[rt] = ok ? (t * (uint32_t)st.q_total * 16u + (uint32_t)g * rows + cc) * 16u : kOutOfRange;
      wstep[rt] = rows * 64u;
      const uint32_t e = t * 16u * (uint32_t)st.groups + gl * rows + cc;  // scale element index
      soff[rt] = ok ? (e & ~1u) * 2u : kOutOfRange;
      sstep[rt] = gps * rows * 2u;
      ssel[rt] = (cc & 1u) ? 0x03020302u : 0x01000100u;  // v_perm: this column's half in both halves
      zoff[rt] = ok ? (t * 2u * (uint32_t)st.groups + gl * (rows >> 3) + (cc >> 3)) * 4u : kOutOfRange;
      zstep[rt] = gps * (rows >> 3) * 4u;
      zsh[rt] = 4u * awq_nibble_of(n & 7u);
    }
    lane_end = min(s1, (st.q_total - g + 3) >> 2);
    wave_end = s1;
  }

  // Every call issues exactly 3 RT loads (zeros when the step is out of range), so the ring
  // has the same loads in flight on every path and the compiler's vmcnt waits stay exact
  // instead of draining the ring.
  __device__ __forceinline__ void issue(Slot<RT>& sl, const Streams& st, int step) const {
    if (UNIFORM) {
      // Steps past the wave's range read through resources with zero records: zeros, no traffic.
      // Every stride is a scalar here (full 16-row tiles): 1 KB of weights, (128 / G) 32-byte
      // groups of scales and (128 / G) 8-byte groups of zero words per step.
      const bool in = step < wave_end;
      const __amdgpu_buffer_rsrc_t rw = make_rsrc(st.qw_ptr, in ? st.qw_bytes : 0u);
      const __amdgpu_buffer_rsrc_t rs = make_rsrc(st.sc_ptr, in ? st.sc_bytes : 0u);
      const __amdgpu_buffer_rsrc_t rz = make_rsrc(st.qz_ptr, in ? st.qz_bytes : 0u);
      const int st_ = in ? step : 0;
      const int gps_step = st_ << (7 - st.log2g);  // groups before this step
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        sl.w[rt] = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)woff[rt], st_ * 1024, 0);
        sl.sw[rt] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)soff[rt], gps_step * 32, 0);
        sl.zw[rt] = __builtin_amdgcn_raw_buffer_load_b32(rz, (int)zoff[rt], gps_step * 8, 0);
      }
    } else {
      // Per-lane strides (a tile of 8 rows, or a partial last step); 24-bit products are exact
      // here (step < 2^16, strides <= 1 KB) and issue at the full VALU rate.
      const bool v = step < lane_end;
      const uint32_t us = (uint32_t)step;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        sl.w[rt] = load_b128(st.qw, v ? woff[rt] + __umul24(us, wstep[rt]) : kOutOfRange);
        sl.sw[rt] = load_b32(st.sc, v ? soff[rt] + __umul24(us, sstep[rt]) : kOutOfRange);
        sl.zw[rt] = load_b32(st.qz, v ? zoff[rt] + __umul24(us, zstep[rt]) : kOutOfRange);
      }
    }
  }

  // Dequantization operands of tile rt from a landed slot.
  __device__ __forceinline__ QuantParams params(const Slot<RT>& sl, int rt) const {
    const uint32_t z = (sl.zw[rt] >> zsh[rt]) & 0xFu;
    const uint32_t zz = z | (z << 16);
    QuantParams q;
    q.zlo = as_h2(zz | 0x64006400u);         // 1024 + z (see make_params)
    q.zhi = as_h2((zz << 4) | 0x54005400u);  // 64 + z
    q.s = as_h2(__builtin_amdgcn_perm(sl.sw[rt], sl.sw[rt], ssel[rt]));
    return q;
  }
};

// LDS carve-up of one launch. Each wave stages a window of `win` steps of its x slice; a wave
// whose range is longer re-stages per window. When a range takes several windows, each holds a
// multiple of the ring depth, so ring slot p always holds a step with (step - s0) % P == p.
struct GemvLds {
  int xstride;     // halfs per staged x row
  int wave_words;  // x words per wave
};

__host__ __device__ __forceinline__ GemvLds gemv_lds_layout(int win, int x_rows) {
  GemvLds l;
  l.xstride = win * 128 + 8;
  l.wave_words = (x_rows * l.xstride) / 2;
  return l;
}

constexpr int kStageU = 2;  // x staging chunks per lane and batch

// ------------------------------------------------------------------------ kernel

// DOTM == 0: the MFMA form (MT tiles of 16 rows). DOTM = 1, 2 or 4: the dot form for M <= DOTM
// (MT = 1): each lane multiplies its 32 K values of its column with v_dot2_f32_f16 for every
// row of x, and the four lanes of a column (K blocks g = 0..3) are added at the end in a fixed
// order. The dot form keeps the products on the VALU, next to the dequantization, instead of
// in the matrix core's dependent chain.
template <int MT, int RT, int P, int MAXW, bool UNIFORM, bool SPLITN, int DOTM = 0>
__global__ __launch_bounds__(MAXW * 64) void gemv_kernel(LinearArgs a, int win) {
  static_assert(DOTM == 0 || MT == 1, "the dot form serves one M tile");
  extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int waves = blockDim.x >> 6;
  const int c = lane & 15;
  const int g = lane >> 4;
  constexpr int cols = 16 * RT;
  const int n_base = SPLITN ? (xcd_tile(blockIdx.x, gridDim.x) * waves + wave) * cols
                            : xcd_tile(blockIdx.x, gridDim.x) * cols;
  const int m_base = blockIdx.y * 16 * MT;
  const Streams st = make_streams(a);
  int s0 = 0, s1 = st.nsteps;
  if (!SPLITN) k_range(wave, waves, st.nsteps, &s0, &s1);
  const int xrows = min(16 * MT, a.m - m_base);  // rows staged by this workgroup
  const int xalloc = min(16 * MT, a.m);          // rows allocated per wave (same in every workgroup)
  const GemvLds L = gemv_lds_layout(win, xalloc);
  _Float16* xs = reinterpret_cast<_Float16*>(lds + (SPLITN ? 0 : wave * L.wave_words));
  const UnpackConsts uc = unpack_consts();
  const LaneStream<RT, UNIFORM> ls_w(a, st, n_base, c, g, s1);

  // MFMA form: lane c reads row c of each M tile (the A operand); dot form: every lane reads
  // rows 0 .. DOTM - 1. Rows past M read a staged row and feed outputs that are never stored.
  constexpr int XP = DOTM ? DOTM : MT;
  const _Float16* xl[XP];
#pragma unroll
  for (int i = 0; i < XP; ++i) {
    const int r = DOTM ? i : i * 16 + c;
    xl[i] = xs + (r < xrows ? r : 0) * L.xstride + g * 32;
  }

  f4 acc[DOTM ? 1 : MT][RT];
  float dacc[DOTM ? DOTM : 1][RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
    for (int mt = 0; mt < (DOTM ? 1 : MT); ++mt) acc[mt][rt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int m = 0; m < (DOTM ? DOTM : 1); ++m) dacc[m][rt] = 0.0f;
  }

  // The first staging batch goes out ahead of the weight ring: every wave of the grid issues
  // its ring at once, and the x chunks that gate the first step must not queue behind it.
  // SPLITN: the waves stage the workgroup's one copy together, batch b by wave b % waves.
  Window win0 = make_window(s0, min(s1, s0 + win), m_base, xrows, L.xstride);
  const int first_base = SPLITN ? wave * 64 * kStageU : 0;
  const int batch_stride = SPLITN ? waves * 64 * kStageU : 64 * kStageU;
  StageBatch<kStageU> first;
  load_batch<kStageU>(first, win0, a, st, first_base, lane);
  __builtin_amdgcn_sched_barrier(0);
  Slot<RT> ring[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    ls_w.issue(ring[p], st, s0 + p);
    __builtin_amdgcn_sched_barrier(0);  // keep slot order: slot 0 must be the oldest ring load
  }
  store_batch<kStageU>(xs, first, win0, a, first_base, lane);
  for (int base = first_base + batch_stride; base < win0.xentries; base += batch_stride) {
    StageBatch<kStageU> b;
    load_batch<kStageU>(b, win0, a, st, base, lane);
    store_batch<kStageU>(xs, b, win0, a, base, lane);
  }
  if (SPLITN) __syncthreads();  // x is whole before any wave reads it (one window: win == s1)

  for (int w0 = s0; w0 < s1; w0 += win) {
    const int w1 = min(s1, w0 + win);
    if (w0 != s0) stage_rest<kStageU>(xs, make_window(w0, w1, m_base, xrows, L.xstride), a, st, 0, lane);
    for (int s = w0; s < w1; s += P) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const int step = s + p;
        const Slot<RT>& cur = ring[p];
        if (step < w1) {
          const int ls = step - w0;
          h8 xa[XP][4];
#pragma unroll
          for (int i = 0; i < XP; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) xa[i][j] = *reinterpret_cast<const h8*>(xl[i] + ls * 128 + j * 8);
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) {
            const QuantParams qp = ls_w.params(cur, rt);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              h2 wd[4];
              dequant_word(cur.w[rt][j], qp, uc, wd);
              if constexpr (DOTM == 0) {
                const h8 b = pack_h8(wd);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                  acc[mt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[mt][j], b, acc[mt][rt], 0, 0, 0);
              } else {
#pragma unroll
                for (int m = 0; m < DOTM; ++m) {
                  const u4 xv = __builtin_bit_cast(u4, xa[m][j]);
#pragma unroll
                  for (int e = 0; e < 4; ++e)
                    dacc[m][rt] = __builtin_amdgcn_fdot2(as_h2(xv[e]), wd[e], dacc[m][rt], false);
                }
              }
            }
          }
        }
        ls_w.issue(ring[p], st, step + P);
        // Slot boundary: keep the next slot's operand work (which waits for its loads) from
        // being hoisted above this point, where it would wait for more of the ring than needed.
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  if constexpr (DOTM != 0) {
    // The four K blocks of each column (lanes c, c + 16, c + 32, c + 48): one fixed tree, whose
    // result lane c (g == 0) stores.
#pragma unroll
    for (int m = 0; m < DOTM; ++m)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        dacc[m][rt] += __shfl_xor(dacc[m][rt], 16);
        dacc[m][rt] += __shfl_xor(dacc[m][rt], 32);
      }
  }

  if (!SPLITN && waves > 1) {
    float* red = reinterpret_cast<float*>(lds + waves * L.wave_words);
    if constexpr (DOTM == 0) {  // [(waves - 1)][MT][RT][64][4]
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
    } else {  // [(waves - 1)][DOTM][RT][16]
      if (wave > 0 && g == 0) {
#pragma unroll
        for (int m = 0; m < DOTM; ++m)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) red[(((wave - 1) * DOTM + m) * RT + rt) * 16 + c] = dacc[m][rt];
      }
      __syncthreads();
      if (wave == 0) {
        for (int w = 1; w < waves; ++w)
#pragma unroll
          for (int m = 0; m < DOTM; ++m)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) dacc[m][rt] += red[(((w - 1) * DOTM + m) * RT + rt) * 16 + c];
      }
    }
  }
  if (SPLITN || wave == 0) {
    // MFMA form, D layout of v_mfma_f32_16x16x32_f16: lane holds rows 4*(lane/16) + r, column
    // lane%16. Dot form: lane c (g == 0) holds column c of every row. Under SiLU*mul lanes c
    // and c ^ 8 hold the gate and up columns of one output.
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int l = rt * 16 + c;
      const int n = phys_col(a, n_base, l);
      const bool valid = col_valid(a, n_base, l) && (DOTM == 0 || g == 0);
      const float b = (a.bias && valid) ? half_bits_to_float(a.bias[n]) : 0.0f;
      constexpr int ROWS = DOTM ? DOTM : 4;
#pragma unroll
      for (int mt = 0; mt < (DOTM ? 1 : MT); ++mt)
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
          const int m = DOTM ? r : m_base + mt * 16 + 4 * g + r;
          const float sum = DOTM ? dacc[DOTM ? r : 0][rt] : acc[mt][rt][DOTM ? 0 : r];
          const float v = sum * row_scale(a, m) + b;
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

// Staging window (in steps) and LDS bytes of a gemv launch. The window covers a wave's whole
// K range when that fits the device's LDS (one window, so its length is free); otherwise it is
// the largest multiple of the ring depth that fits. win = 0 when not even one ring's worth fits.
struct GemvPlan {
  int win;
  size_t lds;
};

GemvPlan plan_gemv(const LinearArgs& a, int waves, int depth, int x_rows, size_t red_per_wave) {
  const int nsteps = ((a.k >> 5) + 3) >> 2;
  const int steps = max_steps(nsteps, waves);
  const size_t cap = device_max_lds();
  auto bytes = [&](int win) {
    const GemvLds l = gemv_lds_layout(win, x_rows);
    return (size_t)waves * (size_t)l.wave_words * 4 + (size_t)(waves - 1) * red_per_wave;
  };
  if (bytes(steps) <= cap) return GemvPlan{steps, bytes(steps)};
  int win = (steps - 1) / depth * depth;
  while (win > depth && bytes(win) > cap) win -= depth;
  if (win < depth || bytes(win) > cap) return GemvPlan{0, 0};
  return GemvPlan{win, bytes(win)};
}

// Every tile full and K a multiple of 128 selects the kernels that carry the step offsets in
// scalar registers.
bool uniform_steps(const LinearArgs& a) { return (a.k & 127) == 0 && (a.n & 15) == 0; }

// LDS bytes and staging window of a launch; win == 0 when it does not fit the device.
template <int MT, int RT, int P, bool SPLITN, int DOTM = 0>
GemvPlan gemv_plan(const LinearArgs& a, int waves) {
  const int xrows = a.m < 16 * MT ? a.m : 16 * MT;
  const size_t red_per_wave = DOTM ? (size_t)DOTM * RT * 16 * sizeof(float) : (size_t)MT * RT * 64 * 4 * sizeof(float);
  if (SPLITN) {  // one shared copy of all of x, no reduction buffer
    const int nsteps = ((a.k >> 5) + 3) >> 2;
    const GemvPlan p{nsteps, (size_t)gemv_lds_layout(nsteps, xrows).wave_words * 4};
    return p.lds <= device_max_lds() ? p : GemvPlan{0, 0};
  }
  return plan_gemv(a, waves, P, xrows, red_per_wave);
}

template <int MT, int RT, int P, int MAXW, bool SPLITN, int DOTM = 0>
int check_gemv(const LinearArgs& a, const tf_gemm_config& cfg) {
  if (DOTM != 0 && a.m > DOTM) return fail(TF_EINVAL, "tf_w4a16_linear: gemv_dot variant needs m <= block_m");
  if (int rc = check_offsets(a)) return rc;
  if (gemv_plan<MT, RT, P, SPLITN, DOTM>(a, cfg.num_warps).win == 0)
    return fail(TF_EINVAL, SPLITN ? "tf_w4a16_linear: gemv variant (block_k 256) needs x to fit the device's LDS"
                                  : "tf_w4a16_linear: gemv variant does not fit the device's LDS");
  return TF_OK;
}

template <int MT, int RT, int P, int MAXW, bool UNIFORM, bool SPLITN, int DOTM>
int launch_k(const LinearArgs& a, int waves, const GemvPlan& plan, hipStream_t stream) {
  auto kernel = gemv_kernel<MT, RT, P, MAXW, UNIFORM, SPLITN, DOTM>;
  if (int rc = reserve_lds(kernel, plan.lds, "gemv")) return rc;
  const int tiles = (int)cdiv(a.n, 16 * RT);
  const dim3 grid((unsigned)(SPLITN ? cdiv(tiles, waves) : tiles), (unsigned)cdiv(a.m, 16 * MT));
  kernel<<<grid, waves * 64, plan.lds, stream>>>(a, plan.win);
  return check_launch("tf_w4a16_linear(gemv)");
}

template <int MT, int RT, int P, int MAXW, bool SPLITN, int DOTM = 0>
int launch_gemv(const LinearArgs& a, const tf_gemm_config& cfg, float*, hipStream_t stream) {
  if (int rc = check_gemv<MT, RT, P, MAXW, SPLITN, DOTM>(a, cfg)) return rc;
  const GemvPlan plan = gemv_plan<MT, RT, P, SPLITN, DOTM>(a, cfg.num_warps);
  return uniform_steps(a) ? launch_k<MT, RT, P, MAXW, true, SPLITN, DOTM>(a, cfg.num_warps, plan, stream)
                          : launch_k<MT, RT, P, MAXW, false, SPLITN, DOTM>(a, cfg.num_warps, plan, stream);
}

// One table row per (variant, num_warps): num_warps ranges over 1..MAXW (powers of two).
#define TF_W1(K, BM, BN, BK, ST, FN, CK) {{K, BM, BN, BK, 1, 1, ST}, FN, no_workspace, CK}
#define TF_W2(K, BM, BN, BK, ST, FN, CK) TF_W1(K, BM, BN, BK, ST, FN, CK), {{K, BM, BN, BK, 1, 2, ST}, FN, no_workspace, CK}
#define TF_W4(K, BM, BN, BK, ST, FN, CK) TF_W2(K, BM, BN, BK, ST, FN, CK), {{K, BM, BN, BK, 1, 4, ST}, FN, no_workspace, CK}
#define TF_W8(K, BM, BN, BK, ST, FN, CK) TF_W4(K, BM, BN, BK, ST, FN, CK), {{K, BM, BN, BK, 1, 8, ST}, FN, no_workspace, CK}
#define TF_W16(K, BM, BN, BK, ST, FN, CK) TF_W8(K, BM, BN, BK, ST, FN, CK), {{K, BM, BN, BK, 1, 16, ST}, FN, no_workspace, CK}

// block_k = 128 marks the K split across the waves of a workgroup (x staged per wave), 256
// waves over column sets with one shared x (block_n is then the columns of one wave; a
// workgroup covers num_warps times as many).
#define TF_GEMV(MT, RT, P, MAXW) \
  TF_W##MAXW(TF_KERNEL_GEMV_MFMA, 16 * MT, 16 * RT, 128, P, (launch_gemv<MT, RT, P, MAXW, false>), \
             (check_gemv<MT, RT, P, MAXW, false>))
#define TF_GEMV_N(MT, RT, P, MAXW) \
  TF_W##MAXW(TF_KERNEL_GEMV_MFMA, 16 * MT, 16 * RT, 256, P, (launch_gemv<MT, RT, P, MAXW, true>), \
             (check_gemv<MT, RT, P, MAXW, true>))

#define TF_DOT(BM, RT, P, MAXW) \
  TF_W##MAXW(TF_KERNEL_GEMV_DOT, BM, 16 * RT, 128, P, (launch_gemv<1, RT, P, MAXW, false, BM>), \
             (check_gemv<1, RT, P, MAXW, false, BM>))
#define TF_DOT_N(BM, RT, P, MAXW) \
  TF_W##MAXW(TF_KERNEL_GEMV_DOT, BM, 16 * RT, 256, P, (launch_gemv<1, RT, P, MAXW, true, BM>), \
             (check_gemv<1, RT, P, MAXW, true, BM>))

const Variant kGemvVariants[] = {
    TF_DOT(1, 1, 2, 16), TF_DOT(1, 1, 4, 16), TF_DOT(1, 2, 2, 16), TF_DOT(2, 1, 2, 16), TF_DOT(4, 1, 2, 16),
    TF_DOT_N(1, 1, 2, 8), TF_DOT_N(1, 1, 4, 8), TF_DOT_N(2, 1, 4, 8), TF_DOT_N(4, 1, 4, 8),
    TF_GEMV(1, 1, 2, 16), TF_GEMV(1, 1, 4, 16), TF_GEMV(1, 1, 8, 16), TF_GEMV(1, 2, 2, 16),
    TF_GEMV(1, 2, 4, 8),  TF_GEMV(1, 4, 2, 8),  TF_GEMV(2, 1, 2, 16), TF_GEMV(2, 2, 2, 8),
    TF_GEMV_N(1, 1, 2, 8), TF_GEMV_N(1, 1, 4, 8), TF_GEMV_N(1, 1, 8, 8), TF_GEMV_N(1, 2, 2, 8),
    TF_GEMV_N(1, 2, 4, 8), TF_GEMV_N(2, 1, 2, 8),
};

}  // namespace

const Variant* gemv_variants(int* count) {
  *count = (int)(sizeof(kGemvVariants) / sizeof(kGemvVariants[0]));
  return kGemvVariants;
}

}  // namespace tf
