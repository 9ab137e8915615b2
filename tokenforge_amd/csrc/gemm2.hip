// Prefill-shaped W4A16 GEMM, pipelined form (M >= 64, group size 64 or 128).
//
// A workgroup of 4, 8 or 16 waves (WM x WN) computes a BM x BN tile of y = x W^T with
// v_mfma_f32_32x32x16_f16, K in blocks of 64. With 8 waves two waves share each SIMD, so one
// wave's MFMAs overlap the other's dequantization, LDS traffic and waits; with 16 (four per
// SIMD, 32-row wave tiles) the other waves also cover the LDS latency of the fragment reads,
// at the cost of more of them (gate_up at M = 256: 7% faster than 8 waves). Per block:
//   * the x tile [BM][64] fp16 streams from global memory straight into LDS (buffer loads
//     with the LDS destination, 16 bytes per lane, no registers), S stages deep;
//   * the packed weight tile [BN][64/8] and its scales / zero points are loaded into a
//     two-block register ring, dequantized once per workgroup (fp16(q - z) * s, one rounding)
//     and written to one of two fp16 LDS buffers;
//   * each wave reads F x 16 (F = 32) or F x 32 (F = 16) operand fragments, 8 consecutive K
//     per lane, the layouts of v_mfma_f32_32x32x16_f16 and v_mfma_f32_16x16x32_f16, and
//     accumulates a (BM/WM) x (BN/WN) sub-tile in fp32. The 16-wide form gives the wave tile a
//     16-column granularity: 256 x 160 tiles (8 waves, 64 x 80 wave tiles) cover gate_up at
//     M = 256 in 237 workgroups instead of the 198 of 256 x 192 on the 256 CUs, and
//     256 x 224 tiles fit gate_up and down at M >= 1024 in fewer rounds.
// Iteration kb waits for x block kb (issued S - 1 iterations earlier), issues x block
// kb + S - 1, multiplies block kb, dequantizes block kb + 1 into the other B buffer, then issues
// the weights of block kb + 3: weight latency is covered by two blocks of MFMA work (x comes
// from L2 and is covered by S - 1 blocks), and there is one barrier per block. With S = 2 the
// stage of a block is a compile-time value of the two-iteration loop body. The loop body is
// straight-line (loads past the K range are issued with out-of-range offsets and return
// zeros), so the count of loads in flight is the same on every path and the waits stay exact.
//
// LDS rows hold 8 chunks of 16 bytes; chunk c of row r sits in slot c ^ s(r), with
// s(r) = (r % 8) ^ ((r / 16) % 2). On gfx950 a 16-byte LDS read serves the wave in four phases
// of 16 lanes (the wave's halves, each split by the parity of lane bits 2-4) over 16 bank
// groups of 16 bytes (a 256-byte line), and a 16-byte write in eight phases of 8 consecutive
// lanes over 8 bank groups (a 128-byte line). Under this s both patterns here are free of
// bank conflicts: the fragment reads (lane l at row l % 32, chunk l / 32 + 2 kk) and the weight
// writes (lane l at row 16 (l / 32) + l % 16, chunk 4 ((l / 16) % 2) + j), and the 16x16
// fragment reads (lane l at row l % 16, chunk l / 16 + 4 kk) too. With s(r) = (r / 2) % 8
// the writes cost eight conflict cycles each (SQ_LDS_BANK_CONFLICT).
//
// Tile order: the grid is one-dimensional; workgroups are numbered XCD by XCD (xcd_tile) and
// within an XCD the M tiles of one N tile are adjacent, so a weight panel is fetched into one
// L2 and reused there by every M tile.
//
// Split-K (split_k > 1): each K slice writes fp32 partials [split][M][N] to the caller's
// workspace; splitk_reduce (gemm.hip) sums them in split order, adds the bias and rounds once.
#include <type_traits>

#include "linear.h"
#include "tile_layout.h"

namespace tf {

int splitk_reduce(const LinearArgs& a, const float* ws, int split, hipStream_t stream);
int64_t lds_gemm_workspace(const LinearArgs& a, int split);
int lds_gemm_finish(const LinearArgs& a, const float* ws, int split, hipStream_t stream);

namespace {

constexpr int kBK = 64;           // K per block
constexpr int kRowChunks = 8;     // 16-byte chunks per 64-wide fp16 row
constexpr uint32_t kChunkBytes = 16;

__device__ __forceinline__ int slot_xor(int row) { return (row & 7) ^ ((row >> 4) & 1); }

__device__ __forceinline__ uint32_t swz(int row, int chunk) {
  return (uint32_t)(row * kRowChunks + (chunk ^ slot_xor(row))) * kChunkBytes;
}

template <int BM, int BN, int WM, int WN, int S, int F>
struct G2 {
  static_assert(F == 32 || F == 16, "fragment edge");
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int TM = BM / WM / F;
  static constexpr int TN = BN / WN / F;
  static constexpr int kSteps = kBK / (F == 32 ? 16 : 32);  // MFMA K steps per block
  static constexpr int kAccRegs = F == 32 ? 16 : 4;         // fp32 accumulators per lane and MFMA tile
  static constexpr int kAStage = BM * kBK * 2;       // bytes of one x stage
  static constexpr int kBStage = BN * kBK * 2;       // bytes of one fp16 weight buffer
  static constexpr int kADma = kAStage / 1024;       // 1 KB LDS-load instructions per stage
  static constexpr int kAPerWave = kADma / kWaves;
  static constexpr int kBChunks = BN * kBK / 32;     // 16-byte packed chunks (32 K of a column)
  static constexpr int kBPer = (kBChunks + kThreads - 1) / kThreads;
  static constexpr int kLds = S * kAStage + 2 * kBStage;
  static_assert(kWaves == 4 || kWaves == 8 || kWaves == 16, "four, eight or sixteen waves");
  static_assert(TM >= 1 && TN >= 1 && BM % (F * WM) == 0 && BN % (F * WN) == 0, "wave tile");
  static_assert(kADma % kWaves == 0, "x stage must split evenly over the waves");
  static_assert(S == 2 || S == 3, "x stages");
  // VMEM issued after x block kb (S - 1 iterations back) when iteration kb waits for it:
  // weights kb + 4 - S, then S - 2 whole iterations (x block, weights).
  static constexpr int kAfterA = 3 * kBPer + (S - 2) * (kAPerWave + 3 * kBPer);
  // K steps whose operand fragments are in flight ahead of the MFMAs: with F = 32 (16-wide
  // steps) two where the registers allow it without lowering occupancy (LDS latency is the
  // exposed cost), else one; with F = 16 (32-wide steps, two per block) one; none with 16
  // waves, where the SIMD's other three waves cover the LDS latency and the 128 registers a
  // wave has at that occupancy hold no second step.
  // 16x16 fragments with sixteen waves (128 registers a wave) or more than 24 MFMA tiles a
  // wave: B fragments streamed one at a time (no spills), not a whole step's set.
  static constexpr bool kStreamB = F == 16 && (kWaves == 16 || TM * TN > 24);
  static constexpr int kAhead = kWaves == 16 ? 0
                                : F == 16    ? 1
                                : (kWaves == 8 && TM * TN <= 6) || (kWaves == 4 && TM * TN <= 8) ? 2
                                                                                                 : 1;
};

// Block barrier at the top of an iteration: at most N vector-memory loads of this wave still
// in flight (s_waitcnt vmcnt(N) lgkmcnt(0): its x-block loads into LDS and its LDS writes
// are done), then s_barrier. Written out instead of __syncthreads so that no wider wait than
// vmcnt(N) is added; the scheduling barriers keep every LDS access on its side.
template <int N>
__device__ __forceinline__ void block_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// Four-wave 16x16-fragment tiles are compiled for two workgroups per CU (256 registers a
// wave): their LDS (two x stages, two weight buffers) fits twice, and the two workgroups'
// barriers then fall at different times.
template <int BM, int BN, int WM, int WN, int S, int F>
__global__ __launch_bounds__(64 * WM * WN, (WM * WN == 4 && F == 16) ? 2 : 1) void gemm2_kernel(LinearArgs a, float* __restrict__ ws, int split_k,
                                                    int tiles_n, int tiles_m) {
  using C = G2<BM, BN, WM, WN, S, F>;
  constexpr int TM = C::TM, TN = C::TN, BP = C::kBPer;
  constexpr bool kEvenB = C::kBChunks % C::kThreads == 0;  // every thread holds BP chunks
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* const a_lds = smem;
  uint8_t* const b_lds = smem + S * C::kAStage;

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

  const uint32_t row_bytes = (uint32_t)(a.k >> 1);
  const int groups = a.k >> a.log2g;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)(((int64_t)(a.m - 1) * a.ldx + a.k) * 2));
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.qw, (uint32_t)a.n * row_bytes);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.scales, (uint32_t)(groups * a.n * 2));
  const __amdgpu_buffer_rsrc_t rz = make_rsrc(a.qz, (uint32_t)(groups * (a.n >> 3) * 4));
  const UnpackConsts uc = unpack_consts();

  // ---- x block kb -> LDS stage st (LDS-destination loads; lane l of instruction j writes
  // 16-byte slot 64 j + l of the stage).
  uint32_t a_off[C::kAPerWave];  // byte offset of this lane's chunk in block 0 (or out of range)
#pragma unroll
  for (int i = 0; i < C::kAPerWave; ++i) {
    const int p = (wave + C::kWaves * i) * 64 + lane;
    const int row = p >> 3;
    const int c = (p & 7) ^ slot_xor(row);
    const int m = m0 + row;
    a_off[i] = m < a.m ? (uint32_t)(((int64_t)m * a.ldx + c * 8) * 2) : kOutOfRange;
  }
  auto issue_a = [&](int kb, int st) {
    const bool ok = kb < kb1;
#pragma unroll
    for (int i = 0; i < C::kAPerWave; ++i) {
      const uint32_t off = ok ? a_off[i] + (uint32_t)kb * (kBK * 2) : kOutOfRange;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rx, (__attribute__((address_space(3))) void*)(a_lds + st * C::kAStage + (wave + C::kWaves * i) * 1024), 16, off,
          0, 0, 0);
    }
  };

  // ---- packed weights of block kb -> register slot. Tile layout: block kb of column n is
  // chunks q = 2 kb + half (half = 0, 1) at chunk index 16 t Q + half rows + cc + 2 kb rows
  // (t = n / 16, cc = n % 16, rows = the tile's row count), i.e. each 16-column tile's block is
  // 512 contiguous bytes. Thread id takes half (id / 16) % 2 of column 16 (id / 32) + id % 16,
  // so 32 consecutive threads read one tile's 512 bytes in order. Scale and zero word of
  // column n, group grp: element 16 t P + grp rows + cc, word 2 t P + grp (rows / 8) + cc / 8.
  // Where the chunks divide evenly over the threads (kEvenB) no thread checks its chunk id, so
  // the loop has no per-thread branch (a branch splits it into blocks the scheduler cannot
  // interleave with the MFMAs); otherwise the threads past the last chunk skip the
  // conversion (measured faster than having them redo other threads' chunks).
  const uint32_t q_total = (uint32_t)(a.k >> 5);
  uint32_t b_off[BP], b_step[BP], b_sbase[BP], b_zbase[BP], b_rows[BP];
  int b_col[BP], b_half[BP];
#pragma unroll
  for (int i = 0; i < BP; ++i) {
    const int id = tid + i * C::kThreads;
    const int col = ((id >> 5) << 4) | (id & 15);
    const int half = (id >> 4) & 1;
    const int n = n0 + col;
    b_col[i] = col;
    b_half[i] = half;
    const uint32_t tt = (uint32_t)n >> 4, cc = (uint32_t)n & 15u;
    const uint32_t rows = (uint32_t)tile_rows(a.n, tt);
    b_rows[i] = rows;
    b_off[i] = ((kEvenB || id < C::kBChunks) && n < a.n) ? (tt * q_total * 16u + (uint32_t)half * rows + cc) * 16u
                                                          : kOutOfRange;
    b_step[i] = rows * 32u;
    b_sbase[i] = tt * 16u * (uint32_t)groups + cc;
    b_zbase[i] = tt * 2u * (uint32_t)groups + (cc >> 3);
  }
  u4 braw[2][BP];
  uint32_t bsc[2][BP], bzw[2][BP];
  auto issue_b = [&](int kb, int slot) {
    const bool ok = kb < kb1;
    const uint32_t grp = (uint32_t)((kb * kBK) >> a.log2g);
#pragma unroll
    for (int i = 0; i < BP; ++i) {
      // Offsets computed unconditionally, then selected (a conditional arm holding a multiply
      // becomes a per-lane branch around each load).
      const bool v = ok && b_off[i] != kOutOfRange;
      const uint32_t wo = b_off[i] + (uint32_t)kb * b_step[i];
      const uint32_t so = (b_sbase[i] + grp * b_rows[i]) * 2u;
      const uint32_t zo = (b_zbase[i] + grp * (b_rows[i] >> 3)) * 4u;
      braw[slot][i] = load_b128(rq, v ? wo : kOutOfRange);
      bsc[slot][i] = load_b16(rs, v ? so : kOutOfRange);
      bzw[slot][i] = load_b32(rz, v ? zo : kOutOfRange);
    }
  };
  // Dequantization operands of a register slot, one per packed chunk.
  auto slot_params = [&](int slot, QuantParams (&qp)[BP]) {
#pragma unroll
    for (int i = 0; i < BP; ++i) qp[i] = make_params(zero_of(bzw[slot][i], (uint32_t)(n0 + b_col[i])), bsc[slot][i]);
  };
  // Word j of every chunk of a register slot -> fp16 buffer `buf` (chunk h*4 + j of the
  // column's row); the four words of a block are spread over its four 16-wide K steps.
  auto store_b_word = [&](int slot, int buf, int j, const QuantParams (&qp)[BP]) {
#pragma unroll
    for (int i = 0; i < BP; ++i) {
      if (kEvenB || tid + i * C::kThreads < C::kBChunks) {
        h2 d[4];
        dequant_word(braw[slot][i][j], qp[i], uc, d);
        *reinterpret_cast<u4*>(b_lds + buf * C::kBStage + swz(b_col[i], b_half[i] * 4 + j)) =
            u4{as_u32(d[0]), as_u32(d[1]), as_u32(d[2]), as_u32(d[3])};
      }
    }
  };
  auto store_b = [&](int slot, int buf) {
    QuantParams qp[BP];
    slot_params(slot, qp);
#pragma unroll
    for (int j = 0; j < 4; ++j) store_b_word(slot, buf, j, qp);
  };

  using Acc = std::conditional_t<F == 32, f16v, f4>;
  constexpr int AR = C::kAccRegs;
  Acc acc[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int q = 0; q < AR; ++q) acc[tm][tn][q] = 0.0f;

  const int a_row0 = wm * TM * F + (lane & (F - 1));
  const int b_row0 = wn * TN * F + (lane & (F - 1));
  // Operand fragments of the kk-th MFMA K step: lane l holds row / column l % F and the 8 K
  // values of chunk 2 kk + l / 32 (F = 32, 16-wide steps) or 4 kk + l / 16 (F = 16, 32-wide).
  auto read_frags = [&](const uint8_t* A, const uint8_t* B, int kk, h8 (&af)[TM], h8 (&bf)[TN]) {
    const int c = F == 32 ? 2 * kk + (lane >> 5) : 4 * kk + (lane >> 4);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) af[tm] = *reinterpret_cast<const h8*>(A + swz(a_row0 + tm * F, c));
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) bf[tn] = *reinterpret_cast<const h8*>(B + swz(b_row0 + tn * F, c));
  };
  auto mfmas = [&](const h8 (&af)[TM], const h8 (&bf)[TN]) {
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        if constexpr (F == 32)
          acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[tn], af[tm], acc[tm][tn], 0, 0, 0);
        else
          acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[tn], af[tm], acc[tm][tn], 0, 0, 0);
      }
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

  // One iteration; `odd` is (kb - kb0) & 1, compile-time so the register slots are static.
  constexpr int kAfterA = C::kAfterA;
  auto iteration = [&](int kb, int st, auto odd_tag) {
    constexpr int odd = decltype(odd_tag)::value;
    // Every wave's part of x block kb has landed in LDS and the B buffer of block kb is
    // written; buffer odd ^ 1 and the stage read in the previous iteration are free.
    block_barrier<kAfterA>();
    issue_a(kb + S - 1, (st + S - 1) % S);
    // The waits count the loads issued after each x block: no later load may move above it.
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* A = a_lds + st * C::kAStage;
    const uint8_t* B = b_lds + odd * C::kBStage;
    // Fragments of step kk + D are read while the MFMAs of step kk run (D = kAhead steps in
    // flight); one word of each chunk of block kb + 1 is dequantized into the other buffer per
    // step.
    constexpr int KS = C::kSteps;
    QuantParams qp[BP];
    if constexpr (C::kStreamB) {
      // 16x16 fragments where the registers hold no whole step of fragments next to the
      // accumulators: per step the A fragments, then one 16-column B fragment at a time (the
      // next one read before this one's MFMAs).
      slot_params(odd ^ 1, qp);
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const int c = 4 * kk + (lane >> 4);
        h8 af[TM], bq[2];
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) af[tm] = *reinterpret_cast<const h8*>(A + swz(a_row0 + tm * F, c));
        bq[0] = *reinterpret_cast<const h8*>(B + swz(b_row0, c));
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
          if (tn + 1 < TN) bq[(tn + 1) & 1] = *reinterpret_cast<const h8*>(B + swz(b_row0 + (tn + 1) * F, c));
          __builtin_amdgcn_s_setprio(1);
#pragma unroll
          for (int tm = 0; tm < TM; ++tm)
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bq[tn & 1], af[tm], acc[tm][tn], 0, 0, 0);
          __builtin_amdgcn_s_setprio(0);
        }
#pragma unroll
        for (int j = kk * 4 / KS; j < (kk + 1) * 4 / KS; ++j) store_b_word(odd ^ 1, odd ^ 1, j, qp);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      constexpr int D = C::kAhead;
      h8 af[KS][TM], bf[KS][TN];
#pragma unroll
      for (int kk = 0; kk < D; ++kk) read_frags(A, B, kk, af[kk], bf[kk]);
      slot_params(odd ^ 1, qp);
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        if (kk + D < KS) read_frags(A, B, kk + D, af[kk + D], bf[kk + D]);
        // Raised priority while this wave queues its MFMAs: the SIMD's other wave then runs
        // its LDS reads and dequantization in the shadow of these MFMAs instead of competing
        // for issue slots with them (measured 6-8% on the M = 256 gate_up shape).
        __builtin_amdgcn_s_setprio(1);
        mfmas(af[kk], bf[kk]);
        __builtin_amdgcn_s_setprio(0);
        // Block kb + 1: the four words of each chunk, spread over the block's MFMA steps.
#pragma unroll
        for (int j = kk * 4 / KS; j < (kk + 1) * 4 / KS; ++j) store_b_word(odd ^ 1, odd ^ 1, j, qp);
      }
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

  // ---- epilogue. The MFMAs take the weight fragment as their first operand, so each
  // accumulator tile is y transposed: register q of lane l is row (m) l % F of the tile and
  // column (n) 4 (l / 16) + q (16x16) or 8 (q / 4) + 4 (l / 32) + q % 4 (32x32). A lane thus
  // holds runs of four consecutive columns of one row and stores each straight from registers
  // as one 8-byte piece (fp32 partials: 16 bytes). A SiLU*mul epilogue pairs columns of
  // different tiles: without split-K the fp16 y goes to the workspace for the SiLU*mul
  // kernel, with split-K the fp32 partials go to the reduce kernel.
  const bool partials = split_k > 1;
  const bool stage_y = !partials && a.epilogue == TF_EPILOGUE_SILU_MUL;
  uint16_t* const dst = stage_y ? reinterpret_cast<uint16_t*>(ws) : a.out;
  const int64_t ldd = stage_y ? (int64_t)a.n : a.ldo;
  const bool residual = !stage_y && a.epilogue == TF_EPILOGUE_RESIDUAL;
  const bool vec = partials ? (a.n & 3) == 0 && (reinterpret_cast<uintptr_t>(ws) & 15) == 0
                           : run_store_ok(a, dst, ldd, residual);
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
    const int m = m0 + (wm * TM + tm) * F + (lane & (F - 1));
    if (m >= a.m) continue;
    const float rs = row_scale(a, m);
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int g = 0; g < AR / 4; ++g) {
        const int n = n0 + (wn * TN + tn) * F + (F == 32 ? 8 * g + 4 * (lane >> 5) : 4 * (lane >> 4));
        if (n >= a.n) continue;
        float v[4];
        if (partials) {
#pragma unroll
          for (int j = 0; j < 4; ++j) v[j] = acc[tm][tn][4 * g + j];
          float* const p = ws + ((int64_t)z * a.m + m) * a.n + n;
          if (vec) {
            *reinterpret_cast<f4*>(p) = f4{v[0], v[1], v[2], v[3]};
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (n + j < a.n) p[j] = v[j];
          }
          continue;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float b = (a.bias && n + j < a.n) ? half_bits_to_float(a.bias[n + j]) : 0.0f;
          v[j] = acc[tm][tn][4 * g + j] * rs + b;
        }
        store_run4(a, dst, ldd, residual, m, n, v, vec);
      }
  }
}

// ------------------------------------------------------------------ producer / consumer form
//
// The same pipeline with the roles split between waves: WM x WN consumer waves only read
// operand fragments and run v_mfma_f32_16x16x32_f16 on a BM x BN tile, and kProd producer waves
// (one per SIMD) issue the x stages, load the packed weights and dequantize them into the LDS
// buffers. Consumers then issue no conversion work between their MFMAs, and the conversion is
// spread over the four SIMDs. Both roles pass the same block barriers: iteration kb, after the
// barrier, consumers multiply block kb while producers issue x block kb + S - 1, dequantize
// block kb + 1 into the other buffer and issue the weights of block kb + 3; the producers'
// vmcnt wait before the barrier covers the x stage of the next block (consumers issue no loads).
template <int BM, int BN, int WM, int WN, int S>
struct G2P {
  static constexpr int kCons = WM * WN;
  static constexpr int kProd = 4;
  static constexpr int kThreads = 64 * (kCons + kProd);
  static constexpr int kPThreads = 64 * kProd;
  static constexpr int TM = BM / WM / 16;
  static constexpr int TN = BN / WN / 16;
  static constexpr int kAStage = BM * kBK * 2;
  static constexpr int kBStage = BN * kBK * 2;
  static constexpr int kADma = kAStage / 1024;
  static constexpr int kAPerWave = kADma / kProd;
  static constexpr int kBChunks = BN * kBK / 32;
  static constexpr int kBPer = (kBChunks + kPThreads - 1) / kPThreads;
  static constexpr int kLds = S * kAStage + 2 * kBStage;
  static constexpr int kAfterA = 3 * kBPer + (S - 2) * (kAPerWave + 3 * kBPer);
  static_assert(kADma % kProd == 0, "x stage must split evenly over the producers");
  static_assert(S == 2 || S == 3, "x stages");
  static_assert(BM % (16 * WM) == 0 && BN % (16 * WN) == 0, "wave tile");
  // More than 20 MFMA tiles a consumer: its weight fragments are read one 16-column fragment at
  // a time (the registers of 12 waves a CU hold no two whole steps of fragments beside them).
  static constexpr bool kStreamB = TM * TN > 20;
};

template <int BM, int BN, int WM, int WN, int S>
__global__ __launch_bounds__(64 * (WM * WN + 4), 1) void gemm2pc_kernel(
    LinearArgs a, float* __restrict__ ws, int split_k, int tiles_n, int tiles_m) {
  using C = G2P<BM, BN, WM, WN, S>;
  constexpr int TM = C::TM, TN = C::TN, BP = C::kBPer;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* const a_lds = smem;
  uint8_t* const b_lds = smem + S * C::kAStage;

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
    const uint32_t row_bytes = (uint32_t)(a.k >> 1);
    const int groups = a.k >> a.log2g;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)(((int64_t)(a.m - 1) * a.ldx + a.k) * 2));
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.qw, (uint32_t)a.n * row_bytes);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.scales, (uint32_t)(groups * a.n * 2));
    const __amdgpu_buffer_rsrc_t rz = make_rsrc(a.qz, (uint32_t)(groups * (a.n >> 3) * 4));
    const UnpackConsts uc = unpack_consts();
    uint32_t a_off[C::kAPerWave];
#pragma unroll
    for (int i = 0; i < C::kAPerWave; ++i) {
      const int p = (pwave + C::kProd * i) * 64 + lane;
      const int row = p >> 3;
      const int c = (p & 7) ^ slot_xor(row);
      const int m = m0 + row;
      a_off[i] = m < a.m ? (uint32_t)(((int64_t)m * a.ldx + c * 8) * 2) : kOutOfRange;
    }
    auto issue_a = [&](int kb, int st) {
      const bool ok = kb < kb1;
#pragma unroll
      for (int i = 0; i < C::kAPerWave; ++i) {
        const uint32_t off = ok ? a_off[i] + (uint32_t)kb * (kBK * 2) : kOutOfRange;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rx, (__attribute__((address_space(3))) void*)(a_lds + st * C::kAStage + (pwave + C::kProd * i) * 1024), 16,
            off, 0, 0, 0);
      }
    };
    const uint32_t q_total = (uint32_t)(a.k >> 5);
    uint32_t b_off[BP], b_step[BP], b_sbase[BP], b_zbase[BP], b_rows[BP];
    int b_col[BP], b_half[BP];
    bool b_act[BP];
#pragma unroll
    for (int i = 0; i < BP; ++i) {
      const int id = ptid + i * C::kPThreads;
      const int col = ((id >> 5) << 4) | (id & 15);
      const int half = (id >> 4) & 1;
      const int n = n0 + col;
      b_act[i] = id < C::kBChunks;
      b_col[i] = b_act[i] ? col : 0;
      b_half[i] = half;
      const uint32_t tt = (uint32_t)n >> 4, cc = (uint32_t)n & 15u;
      const uint32_t rows = (uint32_t)tile_rows(a.n, tt);
      b_rows[i] = rows;
      b_off[i] = (b_act[i] && n < a.n) ? (tt * q_total * 16u + (uint32_t)half * rows + cc) * 16u : kOutOfRange;
      b_step[i] = rows * 32u;
      b_sbase[i] = tt * 16u * (uint32_t)groups + cc;
      b_zbase[i] = tt * 2u * (uint32_t)groups + (cc >> 3);
    }
    u4 braw[2][BP];
    uint32_t bsc[2][BP], bzw[2][BP];
    auto issue_b = [&](int kb, int slot) {
      const bool ok = kb < kb1;
      const uint32_t grp = (uint32_t)((kb * kBK) >> a.log2g);
#pragma unroll
      for (int i = 0; i < BP; ++i) {
        const bool v = ok && b_off[i] != kOutOfRange;
        const uint32_t wo = b_off[i] + (uint32_t)kb * b_step[i];
        const uint32_t so = (b_sbase[i] + grp * b_rows[i]) * 2u;
        const uint32_t zo = (b_zbase[i] + grp * (b_rows[i] >> 3)) * 4u;
        braw[slot][i] = load_b128(rq, v ? wo : kOutOfRange);
        bsc[slot][i] = load_b16(rs, v ? so : kOutOfRange);
        bzw[slot][i] = load_b32(rz, v ? zo : kOutOfRange);
      }
    };
    auto store_b = [&](int slot, int buf) {
#pragma unroll
      for (int i = 0; i < BP; ++i) {
        if (!b_act[i]) continue;
        const QuantParams qp = make_params(zero_of(bzw[slot][i], (uint32_t)(n0 + b_col[i])), bsc[slot][i]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          h2 d[4];
          dequant_word(braw[slot][i][j], qp, uc, d);
          *reinterpret_cast<u4*>(b_lds + buf * C::kBStage + swz(b_col[i], b_half[i] * 4 + j)) =
              u4{as_u32(d[0]), as_u32(d[1]), as_u32(d[2]), as_u32(d[3])};
        }
      }
    };
    // prologue: x blocks kb0 .. kb0 + S - 2 in flight; block kb0 dequantized into buffer 0; the
    // register slots hold blocks kb0 + 1 (slot 1) and kb0 + 2 (slot 0).
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
      block_barrier<C::kAfterA>();
      issue_a(kb + S - 1, (st + S - 1) % S);
      __builtin_amdgcn_sched_barrier(0);
      store_b(odd ^ 1, odd ^ 1);
      __builtin_amdgcn_sched_barrier(0);
      issue_b(kb + 3, odd ^ 1);
    };
    int kb = kb0, st = 0;
    for (; kb + 1 < kb1; kb += 2) {
      iteration(kb, S == 2 ? 0 : st, std::integral_constant<int, 0>{});
      st = (st + 1 == S) ? 0 : st + 1;
      iteration(kb + 1, S == 2 ? 1 : st, std::integral_constant<int, 1>{});
      st = (st + 1 == S) ? 0 : st + 1;
    }
    if (kb < kb1) iteration(kb, S == 2 ? 0 : st, std::integral_constant<int, 0>{});
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
  auto read_frags = [&](const uint8_t* A, const uint8_t* B, int kk, h8 (&af)[TM], h8 (&bf)[TN]) {
    const int c = 4 * kk + (lane >> 4);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) af[tm] = *reinterpret_cast<const h8*>(A + swz(a_row0 + tm * 16, c));
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) bf[tn] = *reinterpret_cast<const h8*>(B + swz(b_row0 + tn * 16, c));
  };
  auto iteration = [&](int kb, int st, auto odd_tag) {
    constexpr int odd = decltype(odd_tag)::value;
    block_barrier<C::kAfterA>();
    const uint8_t* A = a_lds + st * C::kAStage;
    const uint8_t* B = b_lds + odd * C::kBStage;
    if constexpr (C::kStreamB) {
      // per step the A fragments, then one B fragment at a time (the next read before this
      // one's MFMAs)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int c = 4 * kk + (lane >> 4);
        h8 af[TM], bq[2];
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) af[tm] = *reinterpret_cast<const h8*>(A + swz(a_row0 + tm * 16, c));
        bq[0] = *reinterpret_cast<const h8*>(B + swz(b_row0, c));
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
          if (tn + 1 < TN) bq[(tn + 1) & 1] = *reinterpret_cast<const h8*>(B + swz(b_row0 + (tn + 1) * 16, c));
#pragma unroll
          for (int tm = 0; tm < TM; ++tm)
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bq[tn & 1], af[tm], acc[tm][tn], 0, 0, 0);
        }
      }
      return;
    }
    h8 af[2][TM], bf[2][TN];
    read_frags(A, B, 0, af[0], bf[0]);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      if (kk + 1 < 2) read_frags(A, B, kk + 1, af[kk + 1], bf[kk + 1]);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
          acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[kk][tn], af[kk][tm], acc[tm][tn], 0, 0, 0);
    }
  };
  int kb = kb0, st = 0;
  for (; kb + 1 < kb1; kb += 2) {
    iteration(kb, S == 2 ? 0 : st, std::integral_constant<int, 0>{});
    st = (st + 1 == S) ? 0 : st + 1;
    iteration(kb + 1, S == 2 ? 1 : st, std::integral_constant<int, 1>{});
    st = (st + 1 == S) ? 0 : st + 1;
  }
  if (kb < kb1) iteration(kb, S == 2 ? 0 : st, std::integral_constant<int, 0>{});

  // ---- epilogue (the 16x16 form's, transposed accumulators: see gemm2_kernel)
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

int effective_split2(const LinearArgs& a, const tf_gemm_config& cfg) {
  const int nkb = a.k / kBK;
  return cfg.split_k < nkb ? cfg.split_k : (nkb > 0 ? nkb : 1);
}

int64_t gemm2_workspace(const LinearArgs& a, const tf_gemm_config& cfg) {
  return lds_gemm_workspace(a, effective_split2(a, cfg));
}

template <int BM, int BN, int WM, int WN, int S, int F>
int launch_gemm2(const LinearArgs& a, const tf_gemm_config& cfg, float* ws, hipStream_t stream) {
  using C = G2<BM, BN, WM, WN, S, F>;
  if ((1 << a.log2g) < kBK)
    return fail(TF_EINVAL, "tf_w4a16_linear: this gemm_mfma variant needs group_size >= 64 (block_k 64)");
  const int64_t x_bytes = ((int64_t)(a.m - 1) * a.ldx + a.k) * 2;
  const int64_t w_bytes = (int64_t)a.n * (a.k / 2);
  if (x_bytes >= (int64_t)kOutOfRange || w_bytes >= (int64_t)kOutOfRange)
    return fail(TF_EINVAL, "tf_w4a16_linear: this gemm_mfma variant needs x and qweight_t below 2 GiB");
  const int split = effective_split2(a, cfg);
  if (lds_gemm_workspace(a, split) > 0 && ws == nullptr)
    return fail(TF_EINVAL, "tf_w4a16_linear: this config needs a workspace");
  const int tiles_n = (int)cdiv(a.n, BN);
  const int tiles_m = (int)cdiv(a.m, BM);
  const int64_t grid = (int64_t)tiles_n * tiles_m * split;
  if (grid > 0x7FFFFFFF) return fail(TF_EINVAL, "tf_w4a16_linear: too many tiles");
  auto kernel = gemm2_kernel<BM, BN, WM, WN, S, F>;
  if (C::kLds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          C::kLds) != hipSuccess)
    return fail(TF_ELAUNCH, "tf_w4a16_linear: cannot reserve LDS for gemm_mfma");
  kernel<<<(unsigned)grid, C::kThreads, C::kLds, stream>>>(a, ws, split, tiles_n, tiles_m);
  if (int rc = check_launch("tf_w4a16_linear(gemm_mfma)")) return rc;
  return lds_gemm_finish(a, ws, split, stream);
  return TF_OK;
}

template <int BM, int BN, int WM, int WN, int S>
int launch_gemm2pc(const LinearArgs& a, const tf_gemm_config& cfg, float* ws, hipStream_t stream) {
  using C = G2P<BM, BN, WM, WN, S>;
  if ((1 << a.log2g) < kBK)
    return fail(TF_EINVAL, "tf_w4a16_linear: this gemm_mfma variant needs group_size >= 64 (block_k 64)");
  const int64_t x_bytes = ((int64_t)(a.m - 1) * a.ldx + a.k) * 2;
  const int64_t w_bytes = (int64_t)a.n * (a.k / 2);
  if (x_bytes >= (int64_t)kOutOfRange || w_bytes >= (int64_t)kOutOfRange)
    return fail(TF_EINVAL, "tf_w4a16_linear: this gemm_mfma variant needs x and qweight_t below 2 GiB");
  const int split = effective_split2(a, cfg);
  if (lds_gemm_workspace(a, split) > 0 && ws == nullptr)
    return fail(TF_EINVAL, "tf_w4a16_linear: this config needs a workspace");
  const int tiles_n = (int)cdiv(a.n, BN);
  const int tiles_m = (int)cdiv(a.m, BM);
  const int64_t grid = (int64_t)tiles_n * tiles_m * split;
  if (grid > 0x7FFFFFFF) return fail(TF_EINVAL, "tf_w4a16_linear: too many tiles");
  auto kernel = gemm2pc_kernel<BM, BN, WM, WN, S>;
  if (C::kLds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          C::kLds) != hipSuccess)
    return fail(TF_ELAUNCH, "tf_w4a16_linear: cannot reserve LDS for gemm_mfma");
  kernel<<<(unsigned)grid, C::kThreads, C::kLds, stream>>>(a, ws, split, tiles_n, tiles_m);
  if (int rc = check_launch("tf_w4a16_linear(gemm_mfma)")) return rc;
  return lds_gemm_finish(a, ws, split, stream);
}

// num_stages = S + 1 (3: two x stages, 4: three) tells these variants apart from the
// two-buffer kernel (num_stages 2), S + 4 (6, 7) the 16x16 fragment form; num_warps = WM * WN.
#define TF_GEMM2(BM, BN, WM, WN, S) \
  {{TF_KERNEL_GEMM_MFMA, BM, BN, 64, 1, WM * WN, S + 1}, (launch_gemm2<BM, BN, WM, WN, S, 32>), gemm2_workspace}
// num_stages 8: the producer / consumer form (two x stages); num_warps counts the consumer waves.
#define TF_GEMM2PC(BM, BN, WM, WN) \
  {{TF_KERNEL_GEMM_MFMA, BM, BN, 64, 1, WM * WN, 8}, (launch_gemm2pc<BM, BN, WM, WN, 2>), gemm2_workspace}
#define TF_GEMM2F16(BM, BN, WM, WN, S) \
  {{TF_KERNEL_GEMM_MFMA, BM, BN, 64, 1, WM * WN, S + 4}, (launch_gemm2<BM, BN, WM, WN, S, 16>), gemm2_workspace}

const Variant kGemm2Variants[] = {
    // four waves, three x stages
    TF_GEMM2(256, 160, 4, 1, 3), TF_GEMM2(256, 128, 2, 2, 3), TF_GEMM2(128, 256, 2, 2, 3),
    TF_GEMM2(128, 128, 2, 2, 3), TF_GEMM2(256, 192, 2, 2, 3), TF_GEMM2(256, 96, 4, 1, 3),
    TF_GEMM2(64, 256, 1, 4, 3),  TF_GEMM2(128, 192, 2, 2, 3),
    // eight waves (two per SIMD)
    TF_GEMM2(256, 256, 4, 2, 2), TF_GEMM2(256, 192, 4, 2, 2), TF_GEMM2(256, 192, 4, 2, 3),
    TF_GEMM2(256, 128, 4, 2, 2), TF_GEMM2(128, 256, 2, 4, 2), TF_GEMM2(256, 160, 8, 1, 2),
    // sixteen waves (four per SIMD): 32-row wave tiles
    TF_GEMM2(256, 192, 8, 2, 2), TF_GEMM2(256, 192, 8, 2, 3), TF_GEMM2(256, 128, 8, 2, 2),
    // 16x16 fragments: sixteen waves (32-row wave tiles, 16-column granularity), eight waves
    TF_GEMM2F16(256, 160, 8, 2, 2), TF_GEMM2F16(256, 160, 8, 2, 3), TF_GEMM2F16(256, 160, 4, 2, 2),
    TF_GEMM2F16(256, 160, 4, 2, 3), TF_GEMM2F16(256, 192, 4, 2, 2), TF_GEMM2F16(256, 224, 4, 2, 2),
    TF_GEMM2F16(256, 128, 4, 2, 2), TF_GEMM2F16(256, 256, 4, 2, 2), TF_GEMM2F16(128, 160, 2, 2, 2),
    TF_GEMM2F16(128, 128, 2, 2, 2), TF_GEMM2F16(128, 256, 2, 4, 2),
    // producer / consumer form
    TF_GEMM2PC(256, 160, 4, 2), TF_GEMM2PC(256, 128, 4, 2), TF_GEMM2PC(128, 256, 2, 4), TF_GEMM2PC(128, 128, 2, 2),
    TF_GEMM2PC(256, 192, 4, 2),
};

}  // namespace

const Variant* gemm2_variants(int* count) {
  *count = (int)(sizeof(kGemm2Variants) / sizeof(kGemm2Variants[0]));
  return kGemm2Variants;
}

}  // namespace tf
