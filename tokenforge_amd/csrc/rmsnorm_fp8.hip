// Fused RMSNorm + OCP e4m3fn quantization: one HBM read of x, one write of the codes.
//
// Two forms, same bits. Row per workgroup (the default): up to 4 waves share a row; each wave
// reduces in registers (DPP lane exchanges, then four lane reads) and the waves meet in LDS
// behind a barrier. Row per wave: each wave owns one row and reduces it without LDS or a
// barrier; four independent rows per workgroup. Either way x and the weight are loaded up front
// and a row stays in registers between the two reductions (sum of squares, then absmax). x is
// loaded and the codes are stored non-temporally (each is touched once), which took the
// H = 3584, T = 4096 row per workgroup from ~14.5 to ~12 us on MI355X (compute alone: ~10 us,
// ~290 VALU instructions per wave). The two forms time alike at T = 4096 (~12 us); at T =
// 8192 the row per wave is ~5% faster. Giving a wave several rows, with the next row requested
// once the current row's data is in, was slower at every T (fewer waves per SIMD leave the
// latency of each row's dependent steps exposed), so each wave takes one row.
// The sum of squares is accumulated in fp64 (every x^2 of an fp16 x is exact) in the fixed
// order of norm_row.h, the same in both forms and in the decode GEMV's prologue, so a row's var
// does not depend on the form or the batch size; torch's fp32 `mean` (reference.py:37) can
// differ from it by an ulp of var on some rows.
//
// Quotient y / scale (reference.py:47-49) and the per-row divisions: exact forms in
// norm_row.h.
//
// Encoding: rows whose absmax and scale are finite (scale > 0) hold no NaN quotient, so they
// clamp with v_med3 and encode two values per v_cvt_pk_fp8_f32. That instruction rounds to
// nearest even onto e4m3fn exactly like e4m3_encode on every fp32 with |v| <= 448 (checked
// exhaustively on MI355X) but writes 0xFF for every NaN, where torch's cast keeps the sign
// (0x7F for +NaN); the remaining rows therefore clamp with NaN-preserving compares and use
// e4m3_encode.
#include "fp8.h"
#include "norm_row.h"
#include "tf_common.h"

namespace tf {
namespace {

typedef unsigned short us2 __attribute__((ext_vector_type(2)));

// Max of |y| as fp16 bit patterns: for non-NaN values the unsigned order of (bits & 0x7FFF)
// is the order of |y|, and every NaN pattern is above +inf, so a NaN anywhere wins (the NaN
// propagation of torch's amax). The result is wave-uniform.
template <int WAVES>
__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* red) {
  v = wave_max_u32(v);
  if (WAVES == 1) return v;
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  uint32_t t = red[0];
#pragma unroll
  for (int i = 1; i < WAVES; ++i) t = t > red[i] ? t : red[i];
  return t;
}

// Cache policy of the 16-byte loads: x is read once, so its loads are non-temporal (nt); the
// weight is read by every row and loads with the default policy.
constexpr int kLoadOnce = 2;  // nt
constexpr int kLoadReused = 0;

// One row's x (or the weight) into registers as fp16 pairs: pair j of chunk i holds elements
// 2j, 2j+1 of the chunk at (lane + i * threads) * 8. Chunks past h read as zeros. VEC: one
// 16-byte buffer load per chunk (cache policy AUX) through a resource bounded by the row, so
// chunks past h come back as zeros without a branch (h % 8 == 0 and 16-byte aligned rows);
// else element loads.
template <int CPT, int THREADS, bool VEC, int AUX>
__device__ __forceinline__ void load_row(const uint16_t* __restrict__ src, int tid, int h, h2 (&v)[CPT][4]) {
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(src, (uint32_t)h * 2u);
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int e0 = (tid + i * THREADS) * 8;
    if (VEC) {
      const u4 r = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)((uint32_t)e0 * 2u), 0, AUX);
#pragma unroll
      for (int j = 0; j < 4; ++j) v[i][j] = as_h2(r[j]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = e0 + 2 * j;
        const uint32_t a = e < h ? src[e] : 0u, b = e + 1 < h ? src[e + 1] : 0u;
        v[i][j] = as_h2(a | (b << 16));
      }
    }
  }
}

// Sum of squares of one row held in registers, over the WAVES waves that share it, in the fixed
// order of norm_row.h: thread tid's chunk i is chunk tid + 64 WAVES i of the row, its sum goes
// to sums[chunk] (CPT * 64 * WAVES entries, a power of two; chunks past h hold zeros), and after
// one barrier every wave adds them all. WAVES == 1 (a row of one wave, no barrier) orders the
// wave's own LDS writes before its reads with a wavefront fence.
template <int WAVES, int CPT>
__device__ __forceinline__ double row_sum_squares(const h2 (&xv)[CPT][4], double* sums, int tid) {
  constexpr int kThreads = WAVES * 64;
  constexpr int R = (CPT * WAVES) < 1 ? 1 : CPT * WAVES;
  static_assert((CPT & (CPT - 1)) == 0, "chunks per thread: a power of two");
#pragma unroll
  for (int i = 0; i < CPT; ++i) sums[tid + i * kThreads] = chunk_sum_squares(xv[i]);
  if (WAVES > 1)
    __syncthreads();
  else
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  return row_total_lds<R>(sums);
}

// Everything after the sum of squares (``total``) for one row held in registers (xv is
// overwritten with y): rstd -> y -> absmax -> scale -> codes (and dq). WAVES waves share the
// row (the absmax meets in red_u behind a barrier; WAVES == 1 reduces in the wave).
template <int WAVES, int CPT, bool VEC, bool DQ>
__device__ __forceinline__ void finish_row(h2 (&xv)[CPT][4], const h2 (&wv)[CPT][4], double total, int64_t row,
                                           int tid, uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale,
                                           int static_scale, float s_static, uint16_t* __restrict__ dq,
                                           int64_t lddq, int h, double inv_h, float eps, uint32_t* red_u) {
  constexpr int kThreads = WAVES * 64;

  // reference.py:37-38: var = mean(x^2) in fp32, rstd = 1 / sqrt(var + eps), IEEE ops (the
  // mean as an exact reciprocal product, inv_h = fp64(1 / h)).
  const float var = (float)((double)(float)total * inv_h);
  const float rstd = 1.0f / __builtin_sqrtf(var + eps);

  uint32_t amax_bits = 0;
  us2 amax_pk = {0, 0};
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int e0 = (tid + i * kThreads) * 8;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // reference.py:39: fp16(x * rstd) in fp32 then cast, times weight in fp16 (one rounding).
      h2 nrm;
      nrm[0] = mul_round_f32_then_f16((float)xv[i][j][0], rstd);
      nrm[1] = mul_round_f32_then_f16((float)xv[i][j][1], rstd);
      const h2 y = nrm * wv[i][j];
      xv[i][j] = y;  // the row is reused in place for y
      const uint32_t yb = as_u32(y) & 0x7FFF7FFFu;
      if (VEC) {
        // Whole 8-element chunks past h load x = 0 and weight = 0, so their y is fp16(0 * rstd) * 0:
        // 0 when rstd is finite, NaN only when rstd is inf or NaN, and then every y of the row is
        // NaN as well (0 * inf, x * NaN). No mask is needed; both halves go into one packed max.
        amax_pk = __builtin_elementwise_max(amax_pk, __builtin_bit_cast(us2, yb));
      } else {
        const uint32_t a0 = e0 + 2 * j < h ? (yb & 0xFFFFu) : 0u;
        const uint32_t a1 = e0 + 2 * j + 1 < h ? (yb >> 16) : 0u;
        const uint32_t am = a0 > a1 ? a0 : a1;
        amax_bits = amax_bits > am ? amax_bits : am;
      }
    }
  }
  if (VEC) amax_bits = amax_pk[0] > amax_pk[1] ? amax_pk[0] : amax_pk[1];
  const uint32_t m_bits = block_max_u32<WAVES>(amax_bits, red_u);
  const float amax = (float)__builtin_bit_cast(_Float16, (uint16_t)m_bits);

  float s;
  if (static_scale) {
    s = s_static;
  } else {
    s = dynamic_scale(amax);
    if (tid == 0) scale[row] = s;
  }
  const bool fast = __builtin_isfinite(amax) && __builtin_isfinite(s) && s > 0.0f;
  // Dynamic rows with a finite absmax take the fp32 quotient; static scales keep the fp64 one.
  const bool dynamic_fast = fast && !static_scale;
  const float r32 = dynamic_fast ? 1.0f / s : 0.0f;
  const double rcp = dynamic_fast ? 0.0 : 1.0 / (double)s;

  uint8_t* qr = q + row * ldq;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int e0 = (tid + i * kThreads) * 8;
    uint32_t lo, hi;
    if (dynamic_fast) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] = __builtin_amdgcn_fmed3f(quotient_dynamic<false>(xv[i][j], s, r32), -kFp8Max, kFp8Max);
        v[2 * j + 1] = __builtin_amdgcn_fmed3f(quotient_dynamic<true>(xv[i][j], s, r32), -kFp8Max, kFp8Max);
      }
      lo = encode4_clamped(v[0], v[1], v[2], v[3]);
      hi = encode4_clamped(v[4], v[5], v[6], v[7]);
    } else if (fast) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        v[j] = __builtin_amdgcn_fmed3f(quotient(xv[i][j >> 1][j & 1], rcp), -kFp8Max, kFp8Max);
      lo = encode4_clamped(v[0], v[1], v[2], v[3]);
      hi = encode4_clamped(v[4], v[5], v[6], v[7]);
    } else {
      uint8_t codes[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        codes[j] = encode_slow(xv[i][j >> 1][j & 1], rcp);
      }
      lo = hi = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lo |= (uint32_t)codes[j] << (8 * j);
        hi |= (uint32_t)codes[4 + j] << (8 * j);
      }
    }
    if (VEC) {
      // Non-temporal stores: the codes are written once and not read back by this kernel.
      if (e0 < h) __builtin_nontemporal_store(u2{lo, hi}, reinterpret_cast<u2*>(qr + e0));
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (e0 + j < h) qr[e0 + j] = (uint8_t)((j < 4 ? lo : hi) >> (8 * (j & 3)));
    }
    if (DQ) {
      const u2 a = dequant_codes4(lo, s), b = dequant_codes4(hi, s);
      uint16_t* dr = dq + row * lddq;
      if (VEC) {
        if (e0 < h) __builtin_nontemporal_store(u4{a[0], a[1], b[0], b[1]}, reinterpret_cast<u4*>(dr + e0));
      } else {
        const uint32_t words[4] = {a[0], a[1], b[0], b[1]};
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (e0 + j < h) dr[e0 + j] = (uint16_t)(words[j >> 1] >> (16 * (j & 1)));
      }
    }
  }
}

// Row per workgroup: WAVES waves share one row (blockIdx.x). CPT: 8-element chunks per thread.
// DQ: also write dq[T, H] fp16 = fp16(fp32(code) * scale) (16-byte stores when VEC).
template <int WAVES, int CPT, bool VEC, bool DQ>
__global__ __launch_bounds__(WAVES * 64) void rmsnorm_fp8_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ w,
    uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale, int static_scale,
    uint16_t* __restrict__ dq, int64_t lddq, int h, double inv_h, float eps) {
  __shared__ double sums[CPT * WAVES * 64];
  __shared__ uint32_t red_u[WAVES];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  // All inputs are requested before anything waits on any of them.
  const float s_static = static_scale ? scale[0] : 0.0f;
  h2 xv[CPT][4], wv[CPT][4];
  load_row<CPT, WAVES * 64, VEC, kLoadOnce>(x + row * ldx, tid, h, xv);
  load_row<CPT, WAVES * 64, VEC, kLoadReused>(w, tid, h, wv);
  const double total = row_sum_squares<WAVES, CPT>(xv, sums, tid);
  finish_row<WAVES, CPT, VEC, DQ>(xv, wv, total, row, tid, q, ldq, scale, static_scale, s_static, dq, lddq, h, inv_h,
                                  eps, red_u);
}

// Row per wave: wave g of the grid (4 per workgroup) takes row g. Needs VEC (16-byte rows).
template <int CPT, bool DQ>
__global__ __launch_bounds__(256) void rmsnorm_fp8_wave_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ w,
    uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale, int static_scale,
    uint16_t* __restrict__ dq, int64_t lddq, int64_t t, int h, double inv_h, float eps) {
  constexpr int CP = CPT <= 1 ? 1 : CPT <= 2 ? 2 : CPT <= 4 ? 4 : CPT <= 8 ? 8 : 16;  // power of two >= CPT
  __shared__ double sums[4][CP * 64];  // one region per wave
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= t) return;  // the whole wave: no row for it, and no barrier follows
  const float s_static = static_scale ? scale[0] : 0.0f;
  h2 xv[CPT][4], wv[CPT][4];
  load_row<CPT, 64, true, kLoadOnce>(x + row * ldx, lane, h, xv);
  load_row<CPT, 64, true, kLoadReused>(w, lane, h, wv);
  h2 xp[CP][4];  // the row's chunks padded to a power of two with zero chunks
#pragma unroll
  for (int i = 0; i < CP; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) xp[i][j] = i < CPT ? xv[i][j] : as_h2(0u);
  const double total = row_sum_squares<1, CP>(xp, sums[threadIdx.x >> 6], lane);
  finish_row<1, CPT, true, DQ>(xv, wv, total, row, lane, q, ldq, scale, static_scale, s_static, dq, lddq, h, inv_h,
                               eps, nullptr);
}

struct NormArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint16_t* w;
  uint8_t* q;
  int64_t ldq;
  float* scale;
  int static_scale;
  uint16_t* dq;  // nullptr: codes and scales only
  int64_t lddq;
  int64_t t;
  int h;
  double inv_h;  // fp64(1 / h)
  float eps;
};

template <int WAVES, int CPT, bool VEC>
int launch_vec(const NormArgs& n, hipStream_t stream) {
  if (n.dq)
    rmsnorm_fp8_kernel<WAVES, CPT, VEC, true><<<(unsigned)n.t, WAVES * 64, 0, stream>>>(
        n.x, n.ldx, n.w, n.q, n.ldq, n.scale, n.static_scale, n.dq, n.lddq, n.h, n.inv_h, n.eps);
  else
    rmsnorm_fp8_kernel<WAVES, CPT, VEC, false><<<(unsigned)n.t, WAVES * 64, 0, stream>>>(
        n.x, n.ldx, n.w, n.q, n.ldq, n.scale, n.static_scale, nullptr, 0, n.h, n.inv_h, n.eps);
  return check_launch("tf_rmsnorm_fp8_quant");
}

template <int WAVES, int CPT>
int launch_cpt(bool vec, const NormArgs& n, hipStream_t stream) {
  return vec ? launch_vec<WAVES, CPT, true>(n, stream) : launch_vec<WAVES, CPT, false>(n, stream);
}

template <int WAVES>
int launch_waves(int cpt, bool vec, const NormArgs& n, hipStream_t stream) {
  switch (cpt) {
    case 1: return launch_cpt<WAVES, 1>(vec, n, stream);
    case 2: return launch_cpt<WAVES, 2>(vec, n, stream);
    case 4: return launch_cpt<WAVES, 4>(vec, n, stream);
    case 8: return launch_cpt<WAVES, 8>(vec, n, stream);
    default: return launch_cpt<WAVES, 16>(vec, n, stream);
  }
}

// Row per wave: one wave per row, four per workgroup; cpt = 16-byte chunks per lane.
template <int CPT>
int launch_wave(const NormArgs& n, hipStream_t stream) {
  const unsigned grid = (unsigned)((n.t + 3) / 4);
  if (n.dq)
    rmsnorm_fp8_wave_kernel<CPT, true><<<grid, 256, 0, stream>>>(n.x, n.ldx, n.w, n.q, n.ldq, n.scale,
                                                                 n.static_scale, n.dq, n.lddq, n.t, n.h, n.inv_h, n.eps);
  else
    rmsnorm_fp8_wave_kernel<CPT, false><<<grid, 256, 0, stream>>>(n.x, n.ldx, n.w, n.q, n.ldq, n.scale,
                                                                  n.static_scale, nullptr, 0, n.t, n.h, n.inv_h, n.eps);
  return check_launch("tf_rmsnorm_fp8_quant");
}

int launch_row_per_wave(int cpt, const NormArgs& n, hipStream_t stream) {
  switch (cpt) {
    case 1: return launch_wave<1>(n, stream);
    case 2: return launch_wave<2>(n, stream);
    case 4: return launch_wave<4>(n, stream);
    case 7: return launch_wave<7>(n, stream);
    case 8: return launch_wave<8>(n, stream);
    default: return launch_wave<16>(n, stream);
  }
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace
}  // namespace tf

using namespace tf;

extern "C" int tf_rmsnorm_fp8_quant_ex(const uint16_t* x, int64_t ldx, const uint16_t* weight, uint8_t* q,
                                       int64_t ldq, float* scale, int32_t static_scale, uint16_t* dq, int64_t lddq,
                                       int64_t t, int64_t h, float eps, int32_t form, void* stream) {
  if (!x || !weight || !q || !scale) return fail(TF_EINVAL, "tf_rmsnorm_fp8_quant: null pointer");
  if (t < 0 || h <= 0) return fail(TF_EINVAL, "tf_rmsnorm_fp8_quant: need t >= 0 and h > 0");
  if (ldx < h || ldq < h) return fail(TF_EINVAL, "tf_rmsnorm_fp8_quant: row stride smaller than h");
  if (dq && lddq < h) return fail(TF_EINVAL, "tf_rmsnorm_fp8_quant_dq: dq row stride smaller than h");
  if (t > 0x7FFFFFFF) return fail(TF_EINVAL, "tf_rmsnorm_fp8_quant: too many rows");
  if (h > 16 * 8 * 256) return fail(TF_EINVAL, "tf_rmsnorm_fp8_quant: h above 32768 is not supported");
  if (form < TF_NORM_AUTO || form > TF_NORM_ROW_PER_WAVE)
    return fail(TF_EINVAL, "tf_rmsnorm_fp8_quant_ex: unknown form " + std::to_string(form));
  const int64_t chunks = cdiv(h, 8);
  const bool vec = (h % 8 == 0) && (ldx % 8 == 0) && (ldq % 8 == 0) && aligned(x, 16) &&
                   aligned(weight, 16) && aligned(q, 8) && (!dq || (lddq % 8 == 0 && aligned(dq, 16)));
  // Row per wave needs 16-byte accesses and at most 16 chunks per lane (h <= 8192).
  const bool wave_ok = vec && chunks <= 16 * 64;
  if (form == TF_NORM_ROW_PER_WAVE && !wave_ok)
    return fail(TF_EINVAL, "tf_rmsnorm_fp8_quant_ex: the row-per-wave form needs h % 8 == 0, 16-byte "
                           "aligned rows and h <= 8192");
  if (t == 0) return TF_OK;
  hipStream_t s = (hipStream_t)stream;
  const NormArgs n{x, ldx, weight, q, ldq, scale, static_scale, dq, lddq, t, (int)h, 1.0 / (double)h, eps};
  // Auto is the row per workgroup: it is as fast as the row per wave at long batches and faster
  // at short ones, where more lanes per row shorten each row's dependent steps.
  if (form == TF_NORM_ROW_PER_WAVE) {
    const int64_t per = cdiv(chunks, 64);
    const int cpt = per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : per == 7 ? 7 : per <= 8 ? 8 : 16;
    return launch_row_per_wave(cpt, n, s);
  }
  // Up to 4 waves per row, at most a few chunks per thread: short rows stay latency-bound,
  // and long ones keep the per-wave register footprint low enough for full occupancy. From
  // 2048 rows on, a row of up to 512 chunks takes 2 waves instead of 4: each wave repeats the
  // row's scalar steps (~120 of its ~290 instructions at 4 waves), and with enough rows in
  // flight the fewer, longer waves win (H = 3584 on MI355X: T = 4096 10.8 vs 11.6 us, T =
  // 8192 18.0-18.5 vs 19.1 us; T = 512 5.3 vs 4.7 us the other way).
  const bool long_batch = t >= 2048 && chunks <= 512;
  const int waves = chunks >= 256 ? (long_batch ? 2 : 4) : (chunks >= 128 ? 2 : 1);
  const int64_t per = cdiv(chunks, waves * 64);
  const int cpt = per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : per <= 8 ? 8 : 16;
  switch (waves) {
    case 1: return launch_waves<1>(cpt, vec, n, s);
    case 2: return launch_waves<2>(cpt, vec, n, s);
    default: return launch_waves<4>(cpt, vec, n, s);
  }
}

extern "C" int tf_rmsnorm_fp8_quant_dq(const uint16_t* x, int64_t ldx, const uint16_t* weight,
                                       uint8_t* q, int64_t ldq, float* scale, int32_t static_scale,
                                       uint16_t* dq, int64_t lddq, int64_t t, int64_t h, float eps,
                                       void* stream) {
  return tf_rmsnorm_fp8_quant_ex(x, ldx, weight, q, ldq, scale, static_scale, dq, lddq, t, h, eps, TF_NORM_AUTO,
                                 stream);
}

extern "C" int tf_rmsnorm_fp8_quant(const uint16_t* x, int64_t ldx, const uint16_t* weight,
                                    uint8_t* q, int64_t ldq, float* scale, int32_t static_scale,
                                    int64_t t, int64_t h, float eps, void* stream) {
  return tf_rmsnorm_fp8_quant_dq(x, ldx, weight, q, ldq, scale, static_scale, nullptr, 0, t, h, eps, stream);
}
