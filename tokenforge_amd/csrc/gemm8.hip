// W4A8 prefill GEMM on the fp8 matrix cores (v_mfma_scale_f32_16x16x128_f8f6f4 with neutral
// block scales):
//   y[m][n] = xscale[m] * sum_g s[g][n] * sum_{k in g} e4m3(x8[m][k]) * (q[n][k] - z[g][n]) + bias[n].
//
// The pipeline of the fp16 LDS-tile GEMM (one workgroup of 8 waves per BM x BN tile, x streamed
// into S LDS stages by buffer->LDS loads issued S - 1 blocks ahead, packed weights in a
// two-block register ring issued three blocks ahead, one barrier per block), with a block of
// K = 128, which is one quantization group (group_size 128):
//   * x stays in its e4m3 codes: a stage is [BM][128] bytes, so the LDS bytes per FLOP are half
//     the fp16 kernel's;
//   * the weights are dequantized once per workgroup to the e4m3 codes of (q - z), integers in
//     [-15, 15] that e4m3 holds exactly (magic-number unpack, exact fp16 subtraction, then
//     v_cvt_scalef32_pk_fp8_f16), into one of two [BN][128]-byte LDS buffers; the thread that
//     holds a column's first 32 K of the block also writes the column's group scale (fp32);
//   * each wave computes a (16 TM) x (16 TN) sub-tile: per block and 16-column fragment, one
//     MFMA per 16-row fragment into a zeroed accumulator, then acc += s[n] * that: the group
//     scale is applied exactly, in fp32, where the W4A16 path rounds (q - z) * s to fp16 first.
// Operand lanes (checked on MI355X): lane l gives row (A) or column (B) l % 16 and K bytes
// 32 (l / 16) .. +32 of the block; D lane l holds rows 4 (l / 16) + r, column l % 16.
//
// LDS rows hold 8 chunks of 16 bytes; chunk c of row r sits in slot c ^ s(r), with
// s(r) = 2 (r % 4) ^ ((r / 4) % 2). On gfx950 a 16-byte LDS read serves the wave in four phases
// of 16 lanes (the wave's halves, each split by the parity of lane bits 2-4) over 16 bank
// groups of 16 bytes, and a 16-byte write in eight phases of 8 consecutive lanes over 8 bank
// groups. Every 16-byte LDS access here has lane l at row l % 16 (of a 16-row fragment or
// weight-tile column group) and chunk 2 (l / 16) + j, j in {0, 1} (the fragment reads and the
// weight writes): under this s it is free of bank conflicts, where s(r) = (r / 2) % 8 costs
// four conflict cycles per read and eight per write (SQ_LDS_BANK_CONFLICT).
//
// Requirements (checked by the launch): group_size 128, K % 128 == 0, N % 16 == 0, x and
// qweight_t below 2 GiB. Split-K slices write fp32 partials to the caller's workspace and the
// fixed-order reduce of the other GEMMs finishes them.
#include <type_traits>

#include "linear.h"
#include "tile_layout.h"

namespace tf {

int64_t lds_gemm_workspace(const LinearArgs& a, int split);
int lds_gemm_finish(const LinearArgs& a, const float* ws, int split, hipStream_t stream);

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));

constexpr int kBK = 128;        // K per block = one group
constexpr int kRowChunks = 8;   // 16-byte chunks per 128-byte row
constexpr int kNeutralScale = 127;  // E8M0 2^0: the MFMA's block scales leave the product as is

__device__ __forceinline__ int slot_xor8(int row) { return ((row & 3) << 1) ^ ((row >> 2) & 1); }

__device__ __forceinline__ uint32_t swz8(int row, int chunk) {
  return (uint32_t)(row * kRowChunks + (chunk ^ slot_xor8(row))) * 16u;
}

template <int BM, int BN, int WM, int WN, int S>
struct G8 {
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int TM = BM / WM / 16;
  static constexpr int TN = BN / WN / 16;
  static constexpr int kAStage = BM * kBK;            // bytes of one x stage
  static constexpr int kBStage = BN * kBK;            // bytes of one fp8 weight buffer
  static constexpr int kScaleBytes = BN * 4;          // fp32 group scales of one buffer
  static constexpr int kADma = kAStage / 1024;        // 1 KB LDS-load instructions per stage
  static constexpr int kAPerWave = kADma / kWaves;
  static constexpr int kBChunks = BN * 4;             // 16-byte packed chunks (32 K of a column)
  static constexpr int kBPer = (kBChunks + kThreads - 1) / kThreads;
  static constexpr int kLds = S * kAStage + 2 * kBStage + 2 * kScaleBytes;
  static_assert(kWaves == 4 || kWaves == 8, "four or eight waves");
  static_assert(TM >= 1 && TN >= 1 && BM % (16 * WM) == 0 && BN % (16 * WN) == 0, "wave tile");
  static_assert(kADma % kWaves == 0, "x stage must split evenly over the waves");
  static_assert(S == 2 || S == 3, "x stages");
  // VMEM issued after x block kb (S - 1 iterations back) when iteration kb waits for it:
  // weights kb + 4 - S, then S - 2 whole iterations (x block, weights).
  static constexpr int kAfterA = 3 * kBPer + (S - 2) * (kAPerWave + 3 * kBPer);
};

// Block barrier at the top of an iteration: at most N vector-memory loads of this wave still
// in flight (its x-block loads into LDS and its LDS writes are done), then s_barrier.
template <int N>
__device__ __forceinline__ void block_barrier8() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// Eight exact (q - z) values of one packed word (K order) -> eight e4m3 codes (two words).
__device__ __forceinline__ u2 word_to_e4m3(uint32_t w, const QuantParams& p, const UnpackConsts& k) {
  const uint32_t w8 = w >> 8;
  const h2 d0 = as_h2((w & k.m_lo) | k.e_lo) - p.zlo;
  const h2 d1 = as_h2((w & k.m_hi) | k.e_hi) - p.zhi;
  const h2 d2 = as_h2((w8 & k.m_lo) | k.e_lo) - p.zlo;
  const h2 d3 = as_h2((w8 & k.m_hi) | k.e_hi) - p.zhi;
  typedef short s2 __attribute__((ext_vector_type(2)));
  s2 lo = {0, 0}, hi = {0, 0};
  lo = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(lo, d0, 1.0f, false);
  lo = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(lo, d1, 1.0f, true);
  hi = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(hi, d2, 1.0f, false);
  hi = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(hi, d3, 1.0f, true);
  return u2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
}

template <int BM, int BN, int WM, int WN, int S>
__global__ __launch_bounds__(64 * WM * WN) void gemm8_kernel(LinearArgs a, float* __restrict__ ws, int split_k,
                                                    int tiles_n, int tiles_m) {
  using C = G8<BM, BN, WM, WN, S>;
  constexpr int TM = C::TM, TN = C::TN, BP = C::kBPer;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* const a_lds = smem;
  uint8_t* const b_lds = smem + S * C::kAStage;
  float* const s_lds = reinterpret_cast<float*>(smem + S * C::kAStage + 2 * C::kBStage);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN;
  const int wn = wave % WN;

  const int per_split = tiles_n * tiles_m;
  const int t = xcd_tile(blockIdx.x, gridDim.x);
  const int z = t / per_split;
  const int r = t - z * per_split;
  const int m0 = (r % tiles_m) * BM;
  const int n0 = (r / tiles_m) * BN;

  const int nkb = a.k / kBK;
  const int kb0 = (int)(((int64_t)z * nkb) / split_k);
  const int kb1 = (int)(((int64_t)(z + 1) * nkb) / split_k);

  const int groups = a.k >> a.log2g;  // == nkb (group_size 128)
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x8, (uint32_t)((int64_t)(a.m - 1) * a.ldx8 + a.k));
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.qw, (uint32_t)((int64_t)a.n * (a.k >> 1)));
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.scales, (uint32_t)(groups * a.n * 2));
  const __amdgpu_buffer_rsrc_t rz = make_rsrc(a.qz, (uint32_t)(groups * (a.n >> 3) * 4));
  const UnpackConsts uc = unpack_consts();

  // ---- x block kb -> LDS stage st (lane l of instruction j writes 16-byte slot 64 j + l).
  uint32_t a_off[C::kAPerWave];
#pragma unroll
  for (int i = 0; i < C::kAPerWave; ++i) {
    const int p = (wave + C::kWaves * i) * 64 + lane;
    const int row = p >> 3;
    const int c = (p & 7) ^ slot_xor8(row);
    const int m = m0 + row;
    a_off[i] = m < a.m ? (uint32_t)((int64_t)m * a.ldx8 + c * 16) : kOutOfRange;
  }
  auto issue_a = [&](int kb, int st) {
    const bool ok = kb < kb1;
#pragma unroll
    for (int i = 0; i < C::kAPerWave; ++i) {
      const uint32_t off = ok ? a_off[i] + (uint32_t)kb * kBK : kOutOfRange;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rx, (__attribute__((address_space(3))) void*)(a_lds + st * C::kAStage + (wave + C::kWaves * i) * 1024), 16, off,
          0, 0, 0);
    }
  };

  // ---- packed weights of block kb -> register slot. Tile layout (N % 16 == 0, so every tile
  // has 16 rows): block kb of the 16-column tile t is the 1 KB at chunk 16 t Q + 64 kb, and
  // chunk 16 g + c of it holds K 32 g .. 32 g + 31 of column c. Chunk id takes chunk id % 64 of
  // tile id / 64, so 64 consecutive threads read one tile's 1 KB in order. Thread tid handles
  // chunks (tid + i * threads) % chunks: where the chunks do not divide evenly, a few threads
  // redo a chunk another thread also converts (same data to the same place), which keeps the
  // loop free of per-thread branches (a branch would split it into blocks the scheduler cannot
  // interleave with the MFMAs). The scale and zero word of column n, group kb: element
  // 16 t P + 16 kb + c, word 2 t P + 2 kb + c / 8.
  const uint32_t q_total = (uint32_t)(a.k >> 5);
  uint32_t b_off[BP], b_sbase[BP], b_zbase[BP];
  int b_col[BP], b_g[BP];
#pragma unroll
  for (int i = 0; i < BP; ++i) {
    const int id = (tid + i * C::kThreads) % C::kBChunks;
    const int col = ((id >> 6) << 4) | (id & 15);
    const int g = (id >> 4) & 3;
    const int n = n0 + col;
    b_col[i] = col;
    b_g[i] = g;
    const uint32_t tt = (uint32_t)n >> 4, cc = (uint32_t)n & 15u;
    const bool ok = n < a.n;
    b_off[i] = ok ? (tt * q_total * 16u + (uint32_t)g * 16u + cc) * 16u : kOutOfRange;
    b_sbase[i] = ok ? tt * 16u * (uint32_t)groups + cc : kOutOfRange;
    b_zbase[i] = ok ? tt * 2u * (uint32_t)groups + (cc >> 3) : kOutOfRange;
  }
  u4 braw[2][BP];
  uint32_t bsc[2][BP], bzw[2][BP];
  auto issue_b = [&](int kb, int slot) {
    const bool ok = kb < kb1;
#pragma unroll
    for (int i = 0; i < BP; ++i) {
      const bool v = ok && b_off[i] != kOutOfRange;
      braw[slot][i] = load_b128(rq, v ? b_off[i] + (uint32_t)kb * 1024u : kOutOfRange);
      bsc[slot][i] = load_b16(rs, v ? (b_sbase[i] + (uint32_t)kb * 16u) * 2u : kOutOfRange);
      bzw[slot][i] = load_b32(rz, v ? (b_zbase[i] + (uint32_t)kb * 2u) * 4u : kOutOfRange);
    }
  };
  // Half h (words 2 (h % 2), +1) of packed chunk h / 2 of a register slot -> one 16-byte chunk
  // of fp8 buffer `buf`; the first half also writes the column's group scale (fp32; the four
  // threads of a column write the same value). kHalves such pieces make a block; the iteration
  // spreads them over its column fragments so the conversion interleaves with the MFMAs.
  constexpr int kHalves = 2 * BP;
  auto store_b_half = [&](int slot, int buf, int h) {
    const int i = h >> 1, part = h & 1;
    const QuantParams qp = make_params(zero_of(bzw[slot][i], (uint32_t)(n0 + b_col[i])), bsc[slot][i]);
    const u2 lo = word_to_e4m3(braw[slot][i][2 * part], qp, uc);
    const u2 hi = word_to_e4m3(braw[slot][i][2 * part + 1], qp, uc);
    *reinterpret_cast<u4*>(b_lds + buf * C::kBStage + swz8(b_col[i], 2 * b_g[i] + part)) = u4{lo[0], lo[1], hi[0], hi[1]};
    if (part == 0) s_lds[buf * BN + b_col[i]] = half_bits_to_float((uint16_t)bsc[slot][i]);
  };
  auto store_b = [&](int slot, int buf) {
#pragma unroll
    for (int h = 0; h < kHalves; ++h) store_b_half(slot, buf, h);
  };

  f4 acc[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  const int a_row0 = wm * TM * 16 + (lane & 15);
  const int b_row0 = wn * TN * 16 + (lane & 15);
  const int kc = 2 * (lane >> 4);  // this lane's two chunks of the block
  auto frag = [&](const uint8_t* base, int row) {
    const u4 lo = *reinterpret_cast<const u4*>(base + swz8(row, kc));
    const u4 hi = *reinterpret_cast<const u4*>(base + swz8(row, kc + 1));
    return v8i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  };

  // ---- prologue: x blocks kb0 .. kb0 + S - 2 in flight; block kb0 dequantized into buffer 0;
  // the register slots hold blocks kb0 + 1 (slot 1) and kb0 + 2 (slot 0).
#pragma unroll
  for (int i = 0; i < S - 1; ++i) issue_a(kb0 + i, i);
  __builtin_amdgcn_sched_barrier(0);
  issue_b(kb0, 0);
  __builtin_amdgcn_sched_barrier(0);
  issue_b(kb0 + 1, 1);
  __builtin_amdgcn_sched_barrier(0);
  store_b(0, 0);
  __builtin_amdgcn_sched_barrier(0);
  issue_b(kb0 + 2, 0);
  __builtin_amdgcn_sched_barrier(0);

  constexpr int kAfterA = C::kAfterA;
  auto iteration = [&](int kb, int st, auto odd_tag) {
    constexpr int odd = decltype(odd_tag)::value;
    // Every wave's part of x block kb has landed in LDS and the fp8 buffer of block kb is
    // written; buffer odd ^ 1 and the stage read in the previous iteration are free.
    block_barrier8<kAfterA>();
    issue_a(kb + S - 1, (st + S - 1) % S);
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* A = a_lds + st * C::kAStage;
    const uint8_t* B = b_lds + odd * C::kBStage;
    v8i af[TM];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) af[tm] = frag(A, a_row0 + tm * 16);
    // The MFMAs take the weight fragment first: register q of lane l then holds column
    // 4 (l / 16) + q of the fragment, whose group scales are read as one 16-byte piece next to
    // the fragment's MFMAs.
    const float* const sc_row = s_lds + odd * BN + wn * TN * 16 + 4 * (lane >> 4);
    // One 16-column fragment at a time: its B operand, its TM MFMAs, then their scale FMAs.
    // The scheduling barriers keep the compiler from hoisting every fragment's MFMA results
    // ahead of the FMAs (TN x TM live accumulators of 4 registers each would spill); the
    // next fragment's LDS read is issued before this one's MFMAs.
    v8i bf[2];
    bf[0] = frag(B, b_row0);
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      if (tn + 1 < TN) bf[(tn + 1) & 1] = frag(B, b_row0 + (tn + 1) * 16);
      const f4 sc = *reinterpret_cast<const f4*>(sc_row + tn * 16);
      f4 d[TM];
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        d[tm] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[tn & 1], af[tm], f4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0,
                                                                   0, kNeutralScale, 0, kNeutralScale);
      __builtin_amdgcn_s_setprio(0);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[tm][tn][q] = __builtin_fmaf(sc[q], d[tm][q], acc[tm][tn][q]);
      // Part of block kb + 1's weights into the other buffer.
#pragma unroll
      for (int h = tn * kHalves / TN; h < (tn + 1) * kHalves / TN; ++h) store_b_half(odd ^ 1, odd ^ 1, h);
      __builtin_amdgcn_sched_barrier(0);
    }
    issue_b(kb + 3, odd ^ 1);
  };

  int kb = kb0;
  int st = 0;  // stage of block kb; with S = 2 it equals (kb - kb0) & 1
  for (; kb + 1 < kb1; kb += 2) {
    iteration(kb, S == 2 ? 0 : st, std::integral_constant<int, 0>{});
    st = (st + 1 == S) ? 0 : st + 1;
    iteration(kb + 1, S == 2 ? 1 : st, std::integral_constant<int, 1>{});
    st = (st + 1 == S) ? 0 : st + 1;
  }
  if (kb < kb1) iteration(kb, S == 2 ? 0 : st, std::integral_constant<int, 0>{});

  // ---- epilogue. The accumulators hold y transposed (weight fragment first): register q of
  // lane l is row (m) l % 16 and column (n) 4 (l / 16) + q of its tile, so a lane holds a run
  // of four consecutive columns of one row and stores it as one 8-byte piece (fp32 partials:
  // 16 bytes) straight from registers.
  const bool partials = split_k > 1;
  const bool stage_y = !partials && a.epilogue == TF_EPILOGUE_SILU_MUL;
  uint16_t* const dst = stage_y ? reinterpret_cast<uint16_t*>(ws) : a.out;
  const int64_t ldd = stage_y ? (int64_t)a.n : a.ldo;
  const bool residual = !stage_y && a.epilogue == TF_EPILOGUE_RESIDUAL;
  const bool vec = partials ? (a.n & 3) == 0 && (reinterpret_cast<uintptr_t>(ws) & 15) == 0
                            : run_store_ok(a, dst, ldd, residual);
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
    const int m = m0 + (wm * TM + tm) * 16 + (lane & 15);
    if (m >= a.m) continue;
    const float rs = row_scale(a, m);
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int n = n0 + (wn * TN + tn) * 16 + 4 * (lane >> 4);
      if (n >= a.n) continue;
      float v[4];
      if (partials) {
        float* const p = ws + ((int64_t)z * a.m + m) * a.n + n;
        if (vec) {
          *reinterpret_cast<f4*>(p) = acc[tm][tn];
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (n + j < a.n) p[j] = acc[tm][tn][j];
        }
        continue;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float b = (a.bias && n + j < a.n) ? half_bits_to_float(a.bias[n + j]) : 0.0f;
        v[j] = acc[tm][tn][j] * rs + b;
      }
      store_run4(a, dst, ldd, residual, m, n, v, vec);
    }
  }
}

// ------------------------------------------------------------------ producer / consumer form
//
// As gemm2.hip's producer / consumer form: WM x WN consumer waves read the x and weight
// fragments and run the fp8 MFMAs with the group-scale FMAs, four producer waves (one per SIMD)
// issue the x stages, load the packed weights and write their e4m3 (q - z) codes and group
// scales; both roles pass the same block barriers.
template <int BM, int BN, int WM, int WN, int S>
struct G8P {
  static constexpr int kCons = WM * WN;
  static constexpr int kProd = 4;
  static constexpr int kThreads = 64 * (kCons + kProd);
  static constexpr int kPThreads = 64 * kProd;
  static constexpr int TM = BM / WM / 16;
  static constexpr int TN = BN / WN / 16;
  static constexpr int kAStage = BM * kBK;
  static constexpr int kBStage = BN * kBK;
  static constexpr int kScaleBytes = BN * 4;
  static constexpr int kADma = kAStage / 1024;
  static constexpr int kAPerWave = kADma / kProd;
  static constexpr int kBChunks = BN * 4;
  static constexpr int kBPer = (kBChunks + kPThreads - 1) / kPThreads;
  static constexpr int kLds = S * kAStage + 2 * kBStage + 2 * kScaleBytes;
  static constexpr int kAfterA = 3 * kBPer + (S - 2) * (kAPerWave + 3 * kBPer);
  static_assert(kADma % kProd == 0, "x stage must split evenly over the producers");
  static_assert(S == 2, "x stages");
  static_assert(BM % (16 * WM) == 0 && BN % (16 * WN) == 0, "wave tile");
};

template <int BM, int BN, int WM, int WN, int S>
__global__ __launch_bounds__(64 * (WM * WN + 4), 1) void gemm8pc_kernel(LinearArgs a, float* __restrict__ ws,
                                                                         int split_k, int tiles_n, int tiles_m) {
  using C = G8P<BM, BN, WM, WN, S>;
  constexpr int TM = C::TM, TN = C::TN, BP = C::kBPer;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* const a_lds = smem;
  uint8_t* const b_lds = smem + S * C::kAStage;
  float* const s_lds = reinterpret_cast<float*>(smem + S * C::kAStage + 2 * C::kBStage);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool producer = wave >= C::kCons;  // wave-uniform
  const int pwave = wave - C::kCons;
  const int ptid = tid - 64 * C::kCons;
  const int wm = wave / WN;
  const int wn = wave % WN;

  const int per_split = tiles_n * tiles_m;
  const int t = xcd_tile(blockIdx.x, gridDim.x);
  const int z = t / per_split;
  const int r = t - z * per_split;
  const int m0 = (r % tiles_m) * BM;
  const int n0 = (r / tiles_m) * BN;
  const int nkb = a.k / kBK;
  const int kb0 = (int)(((int64_t)z * nkb) / split_k);
  const int kb1 = (int)(((int64_t)(z + 1) * nkb) / split_k);

  if (producer) {
    const int groups = a.k >> a.log2g;  // == nkb (group_size 128)
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x8, (uint32_t)((int64_t)(a.m - 1) * a.ldx8 + a.k));
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.qw, (uint32_t)((int64_t)a.n * (a.k >> 1)));
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.scales, (uint32_t)(groups * a.n * 2));
    const __amdgpu_buffer_rsrc_t rz = make_rsrc(a.qz, (uint32_t)(groups * (a.n >> 3) * 4));
    const UnpackConsts uc = unpack_consts();
    uint32_t a_off[C::kAPerWave];
#pragma unroll
    for (int i = 0; i < C::kAPerWave; ++i) {
      const int p = (pwave + C::kProd * i) * 64 + lane;
      const int row = p >> 3;
      const int c = (p & 7) ^ slot_xor8(row);
      const int m = m0 + row;
      a_off[i] = m < a.m ? (uint32_t)((int64_t)m * a.ldx8 + c * 16) : kOutOfRange;
    }
    auto issue_a = [&](int kb, int st) {
      const bool ok = kb < kb1;
#pragma unroll
      for (int i = 0; i < C::kAPerWave; ++i) {
        const uint32_t off = ok ? a_off[i] + (uint32_t)kb * kBK : kOutOfRange;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rx, (__attribute__((address_space(3))) void*)(a_lds + st * C::kAStage + (pwave + C::kProd * i) * 1024), 16,
            off, 0, 0, 0);
      }
    };
    // chunk (ptid + i * producers) % chunks, as gemm8_kernel assigns them (a few producer
    // threads redo a chunk another one converts: same data to the same place)
    const uint32_t q_total = (uint32_t)(a.k >> 5);
    uint32_t b_off[BP], b_sbase[BP], b_zbase[BP];
    int b_col[BP], b_g[BP];
#pragma unroll
    for (int i = 0; i < BP; ++i) {
      const int id = (ptid + i * C::kPThreads) % C::kBChunks;
      const int col = ((id >> 6) << 4) | (id & 15);
      const int g = (id >> 4) & 3;
      const int n = n0 + col;
      b_col[i] = col;
      b_g[i] = g;
      const uint32_t tt = (uint32_t)n >> 4, cc = (uint32_t)n & 15u;
      const bool ok = n < a.n;
      b_off[i] = ok ? (tt * q_total * 16u + (uint32_t)g * 16u + cc) * 16u : kOutOfRange;
      b_sbase[i] = ok ? tt * 16u * (uint32_t)groups + cc : kOutOfRange;
      b_zbase[i] = ok ? tt * 2u * (uint32_t)groups + (cc >> 3) : kOutOfRange;
    }
    u4 braw[2][BP];
    uint32_t bsc[2][BP], bzw[2][BP];
    auto issue_b = [&](int kb, int slot) {
      const bool ok = kb < kb1;
#pragma unroll
      for (int i = 0; i < BP; ++i) {
        const bool v = ok && b_off[i] != kOutOfRange;
        braw[slot][i] = load_b128(rq, v ? b_off[i] + (uint32_t)kb * 1024u : kOutOfRange);
        bsc[slot][i] = load_b16(rs, v ? (b_sbase[i] + (uint32_t)kb * 16u) * 2u : kOutOfRange);
        bzw[slot][i] = load_b32(rz, v ? (b_zbase[i] + (uint32_t)kb * 2u) * 4u : kOutOfRange);
      }
    };
    auto store_b = [&](int slot, int buf) {
#pragma unroll
      for (int i = 0; i < BP; ++i) {
        const QuantParams qp = make_params(zero_of(bzw[slot][i], (uint32_t)(n0 + b_col[i])), bsc[slot][i]);
#pragma unroll
        for (int part = 0; part < 2; ++part) {
          const u2 lo = word_to_e4m3(braw[slot][i][2 * part], qp, uc);
          const u2 hi = word_to_e4m3(braw[slot][i][2 * part + 1], qp, uc);
          *reinterpret_cast<u4*>(b_lds + buf * C::kBStage + swz8(b_col[i], 2 * b_g[i] + part)) =
              u4{lo[0], lo[1], hi[0], hi[1]};
        }
        s_lds[buf * BN + b_col[i]] = half_bits_to_float((uint16_t)bsc[slot][i]);
      }
    };
#pragma unroll
    for (int i = 0; i < S - 1; ++i) issue_a(kb0 + i, i);
    __builtin_amdgcn_sched_barrier(0);
    issue_b(kb0, 0);
    __builtin_amdgcn_sched_barrier(0);
    issue_b(kb0 + 1, 1);
    __builtin_amdgcn_sched_barrier(0);
    store_b(0, 0);
    __builtin_amdgcn_sched_barrier(0);
    issue_b(kb0 + 2, 0);
    __builtin_amdgcn_sched_barrier(0);
    auto iteration = [&](int kb, int st, auto odd_tag) {
      constexpr int odd = decltype(odd_tag)::value;
      block_barrier8<C::kAfterA>();
      issue_a(kb + S - 1, (st + S - 1) % S);
      __builtin_amdgcn_sched_barrier(0);
      store_b(odd ^ 1, odd ^ 1);
      __builtin_amdgcn_sched_barrier(0);
      issue_b(kb + 3, odd ^ 1);
    };
    int kb = kb0;
    for (; kb + 1 < kb1; kb += 2) {
      iteration(kb, 0, std::integral_constant<int, 0>{});
      iteration(kb + 1, 1, std::integral_constant<int, 1>{});
    }
    if (kb < kb1) iteration(kb, 0, std::integral_constant<int, 0>{});
    return;  // no barrier follows the main loop
  }

  // ---- consumers
  f4 acc[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  const int a_row0 = wm * TM * 16 + (lane & 15);
  const int b_row0 = wn * TN * 16 + (lane & 15);
  const int kc = 2 * (lane >> 4);
  auto frag = [&](const uint8_t* base, int row) {
    const u4 lo = *reinterpret_cast<const u4*>(base + swz8(row, kc));
    const u4 hi = *reinterpret_cast<const u4*>(base + swz8(row, kc + 1));
    return v8i{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  };
  auto iteration = [&](int kb, int st, auto odd_tag) {
    constexpr int odd = decltype(odd_tag)::value;
    block_barrier8<C::kAfterA>();
    const uint8_t* A = a_lds + st * C::kAStage;
    const uint8_t* B = b_lds + odd * C::kBStage;
    v8i af[TM];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) af[tm] = frag(A, a_row0 + tm * 16);
    const float* const sc_row = s_lds + odd * BN + wn * TN * 16 + 4 * (lane >> 4);
    v8i bf[2];
    bf[0] = frag(B, b_row0);
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      if (tn + 1 < TN) bf[(tn + 1) & 1] = frag(B, b_row0 + (tn + 1) * 16);
      const f4 sc = *reinterpret_cast<const f4*>(sc_row + tn * 16);
      f4 d[TM];
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        d[tm] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bf[tn & 1], af[tm], f4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0,
                                                                   0, kNeutralScale, 0, kNeutralScale);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[tm][tn][q] = __builtin_fmaf(sc[q], d[tm][q], acc[tm][tn][q]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  int kb = kb0;
  for (; kb + 1 < kb1; kb += 2) {
    iteration(kb, 0, std::integral_constant<int, 0>{});
    iteration(kb + 1, 1, std::integral_constant<int, 1>{});
  }
  if (kb < kb1) iteration(kb, 0, std::integral_constant<int, 0>{});

  // ---- epilogue (gemm8_kernel's)
  const bool partials = split_k > 1;
  const bool stage_y = !partials && a.epilogue == TF_EPILOGUE_SILU_MUL;
  uint16_t* const dst = stage_y ? reinterpret_cast<uint16_t*>(ws) : a.out;
  const int64_t ldd = stage_y ? (int64_t)a.n : a.ldo;
  const bool residual = !stage_y && a.epilogue == TF_EPILOGUE_RESIDUAL;
  const bool vec = partials ? (a.n & 3) == 0 && (reinterpret_cast<uintptr_t>(ws) & 15) == 0
                            : run_store_ok(a, dst, ldd, residual);
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
    const int m = m0 + (wm * TM + tm) * 16 + (lane & 15);
    if (m >= a.m) continue;
    const float rs = row_scale(a, m);
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int n = n0 + (wn * TN + tn) * 16 + 4 * (lane >> 4);
      if (n >= a.n) continue;
      float v[4];
      if (partials) {
        float* const p = ws + ((int64_t)z * a.m + m) * a.n + n;
        if (vec) {
          *reinterpret_cast<f4*>(p) = acc[tm][tn];
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (n + j < a.n) p[j] = acc[tm][tn][j];
        }
        continue;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float b = (a.bias && n + j < a.n) ? half_bits_to_float(a.bias[n + j]) : 0.0f;
        v[j] = acc[tm][tn][j] * rs + b;
      }
      store_run4(a, dst, ldd, residual, m, n, v, vec);
    }
  }
}

int effective_split8(const LinearArgs& a, const tf_gemm_config& cfg) {
  const int nkb = a.k / kBK;
  return cfg.split_k < nkb ? cfg.split_k : (nkb > 0 ? nkb : 1);
}

int64_t gemm8_workspace(const LinearArgs& a, const tf_gemm_config& cfg) {
  return lds_gemm_workspace(a, effective_split8(a, cfg));
}

// Everything the launch rejects, before anything is queued.
template <int BM, int BN, int WM, int WN, int S>
int check_gemm8(const LinearArgs& a, const tf_gemm_config& cfg) {
  if (a.x8 == nullptr)
    return fail(TF_EINVAL, "tf_w4a16_linear: the gemm_fp8 kernels take e4m3 activations (tf_w4a8_linear_ex)");
  if (a.log2g != 7) return fail(TF_EINVAL, "tf_w4a8_linear_ex: the gemm_fp8 kernels need group_size 128");
  if (a.k % kBK) return fail(TF_EINVAL, "tf_w4a8_linear_ex: the gemm_fp8 kernels need K to be a multiple of 128");
  if (a.n % 16) return fail(TF_EINVAL, "tf_w4a8_linear_ex: the gemm_fp8 kernels need N to be a multiple of 16");
  const int64_t x_bytes = (int64_t)(a.m - 1) * a.ldx8 + a.k;
  const int64_t w_bytes = (int64_t)a.n * (a.k / 2);
  if (x_bytes >= (int64_t)kOutOfRange || w_bytes >= (int64_t)kOutOfRange)
    return fail(TF_EINVAL, "tf_w4a8_linear_ex: the gemm_fp8 kernels need x and qweight_t below 2 GiB");
  if (cdiv(a.n, BN) * cdiv(a.m, BM) * effective_split8(a, cfg) > 0x7FFFFFFF)
    return fail(TF_EINVAL, "tf_w4a8_linear_ex: too many tiles");
  return TF_OK;
}

template <int BM, int BN, int WM, int WN, int S>
int launch_gemm8(const LinearArgs& a, const tf_gemm_config& cfg, float* ws, hipStream_t stream) {
  using C = G8<BM, BN, WM, WN, S>;
  if (int rc = check_gemm8<BM, BN, WM, WN, S>(a, cfg)) return rc;
  const int split = effective_split8(a, cfg);
  if (lds_gemm_workspace(a, split) > 0 && ws == nullptr)
    return fail(TF_EINVAL, "tf_w4a8_linear_ex: this config needs a workspace");
  const int tiles_n = (int)cdiv(a.n, BN);
  const int tiles_m = (int)cdiv(a.m, BM);
  const int64_t grid = (int64_t)tiles_n * tiles_m * split;
  auto kernel = gemm8_kernel<BM, BN, WM, WN, S>;
  if (C::kLds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          C::kLds) != hipSuccess)
    return fail(TF_ELAUNCH, "tf_w4a8_linear_ex: cannot reserve LDS for gemm_fp8");
  kernel<<<(unsigned)grid, C::kThreads, C::kLds, stream>>>(a, ws, split, tiles_n, tiles_m);
  if (int rc = check_launch("tf_w4a8_linear_ex(gemm_fp8)")) return rc;
  return lds_gemm_finish(a, ws, split, stream);
}

template <int BM, int BN, int WM, int WN>
int launch_gemm8pc(const LinearArgs& a, const tf_gemm_config& cfg, float* ws, hipStream_t stream) {
  using C = G8P<BM, BN, WM, WN, 2>;
  if (int rc = check_gemm8<BM, BN, WM, WN, 2>(a, cfg)) return rc;
  const int split = effective_split8(a, cfg);
  if (lds_gemm_workspace(a, split) > 0 && ws == nullptr)
    return fail(TF_EINVAL, "tf_w4a8_linear_ex: this config needs a workspace");
  const int tiles_n = (int)cdiv(a.n, BN);
  const int tiles_m = (int)cdiv(a.m, BM);
  const int64_t grid = (int64_t)tiles_n * tiles_m * split;
  auto kernel = gemm8pc_kernel<BM, BN, WM, WN, 2>;
  if (C::kLds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          C::kLds) != hipSuccess)
    return fail(TF_ELAUNCH, "tf_w4a8_linear_ex: cannot reserve LDS for gemm_fp8");
  kernel<<<(unsigned)grid, C::kThreads, C::kLds, stream>>>(a, ws, split, tiles_n, tiles_m);
  if (int rc = check_launch("tf_w4a8_linear_ex(gemm_fp8)")) return rc;
  return lds_gemm_finish(a, ws, split, stream);
}

// block_k 128 (one group per block); num_stages = S + 1, as the fp16 pipelined GEMM counts them.
#define TF_GEMM8(BM, BN, WM, WN, S)                                                                         \
  {{TF_KERNEL_GEMM_FP8, BM, BN, 128, 1, WM * WN, S + 1}, (launch_gemm8<BM, BN, WM, WN, S>), gemm8_workspace, \
   (check_gemm8<BM, BN, WM, WN, S>)}

// num_stages 8: the producer / consumer form (two x stages); num_warps counts the consumer waves.
#define TF_GEMM8PC(BM, BN, WM, WN)                                                                          \
  {{TF_KERNEL_GEMM_FP8, BM, BN, 128, 1, WM * WN, 8}, (launch_gemm8pc<BM, BN, WM, WN>), gemm8_workspace, \
   (check_gemm8<BM, BN, WM, WN, 2>)}

const Variant kGemm8Variants[] = {
    TF_GEMM8(256, 192, 4, 2, 2), TF_GEMM8(256, 128, 4, 2, 2), TF_GEMM8(128, 256, 2, 4, 2),
    TF_GEMM8(256, 160, 4, 2, 2), TF_GEMM8(128, 128, 2, 4, 2), TF_GEMM8(256, 192, 4, 2, 3),
    TF_GEMM8PC(256, 160, 4, 2), TF_GEMM8PC(256, 128, 4, 2), TF_GEMM8PC(128, 256, 2, 4), TF_GEMM8PC(128, 128, 2, 4),
};

}  // namespace

const Variant* gemm8_variants(int* count) {
  *count = (int)(sizeof(kGemm8Variants) / sizeof(kGemm8Variants[0]));
  return kGemm8Variants;
}

}  // namespace tf
