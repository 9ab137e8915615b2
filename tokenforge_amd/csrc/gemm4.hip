// Wave-tile register-streamed W4A16 GEMM for prefill M (M >= 128, gfx950).
//
// One wave per SIMD, each owning a large output tile, so that no operand but x passes through
// LDS and each dequantized weight word feeds many MFMAs:
//   * a workgroup of 4 waves (WM along M, WN = 4 / WM along N) covers BM = 16 MT WM rows and
//     BN = 16 RT WN columns; wave (wm, wn) owns 16 MT rows x 16 RT columns and keeps their fp32
//     accumulators (MT RT / 4 x 16 registers, in the accumulation registers);
//   * the wave streams the packed weights, scales and zero points of its columns from memory
//     into a register ring P steps (of 128 K) deep and dequantizes each packed word
//     (fp16(q - z) * s, one rounding) straight into the B operand of v_mfma_f32_16x16x32_f16,
//     where it meets MT row tiles of x: a word is dequantized by the WM waves of its column
//     set and by nobody else;
//   * x streams from memory into two LDS stages of [BM][128] fp16 through buffer loads with the
//     LDS destination (no registers), one step ahead, with one barrier per step.
// Inside a step the A fragments and B operands of K block j + 1 are read and dequantized while
// the MFMAs of block j run, so the wave's LDS latency and VALU work sit in the shadow of its own
// matrix work.
//
// Lane (c = lane % 16, g = lane / 16) holds chunk g (32 consecutive K) of column c of a 16-column
// tile: the tile layout's 1 KB step block, one 16-byte load per lane. MFMA j of a step takes word
// j of every lane's chunk, so its K set is {32 g + 8 j + e}, and the A fragment of row tile mt
// reads x at the same positions (row 16 mt + c, 16 bytes). LDS rows hold 16 chunks of 16 bytes
// (one 256-byte bank line); chunk c of row r sits in slot c ^ (r & 11). A 16-byte LDS read on
// gfx950 serves the wave in four phases of 16 lanes (the wave's halves, each split by the
// parity of lane bits 2-4), and under this slot map each phase of the fragment read (lane
// 16 g + c at row c, chunk 4 g + j) hits 16 distinct bank groups; c ^ (r % 16) costs four
// conflict cycles per read.
//
// The weight ring's slot of a step is a compile-time value of the step loop, unrolled P times.
// Loads past the workgroup's K range are issued through an empty buffer resource (they
// return zeros), so the count of loads in flight is the same on every path and the barrier's
// wait stays exact. Shapes: N % 16 == 0 and K % 128 == 0 (checked before the launch), so every
// per-step address part is a wave-uniform soffset and only the lane part needs a register.
//
// Split-K (split_k > 1): K slices write fp32 partials [split][M][N] to the caller's workspace
// and splitk_reduce (gemm.hip) sums them in split order, adds the bias and rounds once.
#include <type_traits>

#include "linear.h"
#include "tile_layout.h"

namespace tf {

int splitk_reduce(const LinearArgs& a, const float* ws, int split, hipStream_t stream);

namespace {

constexpr int kStepK = 128;

__device__ __forceinline__ uint32_t xslot(int row, int chunk) {
  return (uint32_t)(row * 16 + (chunk ^ (row & 11))) * 16u;
}

template <int MT, int RT, int WM, int S, int P>
struct G4 {
  static constexpr int kThreads = 256;
  static constexpr int WN = 4 / WM;
  static constexpr int BM = 16 * MT * WM;
  static constexpr int BN = 16 * RT * WN;
  static constexpr int kStage = BM * kStepK * 2;    // bytes of one x stage
  static constexpr int kDmaPerWave = kStage / 4096;  // 1 KB LDS-load instructions per wave and step
  static constexpr int kLds = S * kStage;
  // VMEM loads issued after x step s + 1 when iteration s waits for it before its last K block
  // (x step s + 1 was issued before the last block of iteration s + 2 - S): the weights issued at
  // the end of that iteration, then S - 3 whole iterations. Where more loads have been issued
  // after it (the first iterations, after the prologue's loads) the wait is longer, never short.
  static constexpr int kAfterX = 3 * RT + (S - 3) * (kDmaPerWave + 3 * RT);
  // The prologue's wait for x step s0: the other S - 2 x steps and P steps of weights.
  static constexpr int kFirstWait = (S - 2) * kDmaPerWave + 3 * RT * P;
  static_assert(WM == 1 || WM == 2 || WM == 4, "waves along M");
  static_assert(kDmaPerWave >= 1 && kStage % 4096 == 0, "x stage must split evenly over the waves");
  static_assert(S == 3 || S == 4, "three or four x stages (x step s + S - 1 goes into the stage of step s - 1)");
  static_assert(P >= 2 && P <= 4, "weight ring of two to four steps");
  static_assert(kLds <= 160 * 1024, "x stages exceed the LDS");
  static_assert(kAfterX < 64 && kFirstWait < 64, "vmcnt range");
};

template <int N>
__device__ __forceinline__ void step_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

template <int MT, int RT, int WM, int S, int P>
__global__ __launch_bounds__(256) void gemm4_kernel(LinearArgs a, float* __restrict__ ws, int split_k, int tiles_n,
                                                    int tiles_m) {
  using C = G4<MT, RT, WM, S, P>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;
  const int wm = wave / C::WN;
  const int wn = wave % C::WN;

  const int per_split = tiles_n * tiles_m;
  const int t = xcd_tile(blockIdx.x, gridDim.x);
  const int z = t / per_split;
  const int r = t - z * per_split;
  const int m0 = (r % tiles_m) * C::BM;
  const int n_base = (r / tiles_m) * C::BN;  // the tile's first column
  const int wl = wn * 16 * RT;                 // this wave's first column in the tile
  const int wrow = wm * 16 * MT;               // this wave's first row in the tile

  const int nchunks = a.k >> 5;
  const int nsteps = (nchunks + 3) >> 2;
  const int s0 = (int)(((int64_t)z * nsteps) / split_k);
  const int s1 = (int)(((int64_t)(z + 1) * nsteps) / split_k);

  const int groups = a.k >> a.log2g;
  // The K range of this workgroup as buffer sizes: a step outside it reads zeros through an
  // empty resource (wave-uniform), so the loop issues the same loads on every path.
  const uint32_t x_bytes = (uint32_t)(((int64_t)(a.m - 1) * a.ldx + a.k) * 2);
  const uint32_t q_bytes = (uint32_t)a.n * (uint32_t)(a.k >> 1);
  const uint32_t s_bytes = (uint32_t)(groups * a.n * 2);
  const uint32_t z_bytes = (uint32_t)(groups * (a.n >> 3) * 4);
  const UnpackConsts uc = unpack_consts();

  // ---- x step s -> LDS stage st: instruction i of this wave fills 1 KB at
  // (wave * kDmaPerWave + i) KB of the stage, rows 4 (wave * kDmaPerWave + i) + lane / 16, lane l
  // writing 16-byte slot l of it (chunk (l % 16) ^ (row & 11) of its row; row % 16 depends on i % 4
  // only). The lane's byte offset in the wave's first row is a register, the row offset of
  // instruction i and the step's K offset a wave-uniform running sum added to it. When the M tile
  // is not full, rows past M take an out-of-range offset instead, so nothing past x is read.
  const int x_row0 = 4 * wave * C::kDmaPerWave + g;  // the lane's row for instruction 0
  uint32_t x_lane[4];                                 // by i % 4
#pragma unroll
  for (int i = 0; i < 4; ++i) x_lane[i] = (uint32_t)(((int64_t)(m0 + x_row0) * a.ldx + ((c ^ ((4 * i + g) & 11)) * 8)) * 2);
  const bool x_full = m0 + C::BM <= a.m;  // wave-uniform
  const uint32_t x_istride = (uint32_t)(8 * a.ldx);  // bytes between the rows of instructions i and i + 1
  auto issue_x = [&](int s, int st) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, s < s1 ? x_bytes : 0u);
    // Running scalar offsets, opaque to the compiler at each instruction: otherwise it
    // precomputes every instruction's row offset and LDS address for both stages and keeps them
    // all in scalar registers (spilled).
    uint32_t soff = (uint32_t)s * (kStepK * 2);
    uint32_t lds = (uint32_t)(uintptr_t)smem + (uint32_t)(st * C::kStage + wave * C::kDmaPerWave * 1024);
    int row = m0 + x_row0;
#pragma unroll
    for (int i = 0; i < C::kDmaPerWave; ++i) {
      __asm__ volatile("" : "+s"(soff), "+s"(lds));
      // The whole offset goes into the register operand (the scalar one is 0): the range check
      // and the LDS destination then see exactly the address of the chunk.
      uint32_t voff = x_lane[i & 3] + soff;
      if (!x_full) voff = row < a.m ? voff : kOutOfRange;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (__attribute__((address_space(3))) void*)(uintptr_t)lds, 16, voff,
                                               0, 0, 0);
      soff += x_istride;
      lds += 1024;
      row += 4;
    }
  };

  // ---- weights of step s (N % 16 == 0: every 16-column tile is full). Tile layout: the lane's
  // chunk (column n, K block g) of step s sits at chunk 16 t Q + 64 s + 16 g + cc (t = n / 16,
  // cc = n % 16), its scale at element 16 t P + 16 grp + cc and its zero word at
  // 2 t P + 2 grp + cc / 8, with grp = s (128 / G) + (32 g) / G. The lane parts are registers
  // (kOutOfRange for a column past N), the step parts wave-uniform soffsets.
  const uint32_t gps = (uint32_t)(kStepK >> a.log2g);          // groups per step
  const uint32_t gl = (uint32_t)((g * 32) >> a.log2g);         // the lane's group inside a step
  uint32_t w_off[RT], s_off[RT], z_off[RT], zsh[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int l = wl + rt * 16 + c;
    const int n = phys_col(a, n_base, l);
    const bool valid = col_valid(a, n_base, l);
    const uint32_t tt = (uint32_t)n >> 4, cc = (uint32_t)n & 15u;
    w_off[rt] = valid ? (tt * (uint32_t)nchunks * 16u + (uint32_t)g * 16u + cc) * 16u : kOutOfRange;
    s_off[rt] = valid ? (tt * 16u * (uint32_t)groups + 16u * gl + cc) * 2u : kOutOfRange;
    z_off[rt] = valid ? (tt * 2u * (uint32_t)groups + 2u * gl + (cc >> 3)) * 4u : kOutOfRange;
    zsh[rt] = 4u * awq_nibble_of((uint32_t)n & 7u);
  }
  u4 wraw[P][RT];
  uint32_t wsc[P][RT], wzw[P][RT];
  auto issue_w = [&](int s, int slot) __attribute__((always_inline)) {
    const bool ok = s < s1;
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.qw, ok ? q_bytes : 0u);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.scales, ok ? s_bytes : 0u);
    const __amdgpu_buffer_rsrc_t rz = make_rsrc(a.qz, ok ? z_bytes : 0u);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      wraw[slot][rt] = __builtin_amdgcn_raw_buffer_load_b128(rq, (int)w_off[rt], s * 1024, 0);
      wsc[slot][rt] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)s_off[rt], (int)(s * gps * 32u), 0);
      wzw[slot][rt] = __builtin_amdgcn_raw_buffer_load_b32(rz, (int)z_off[rt], (int)(s * gps * 8u), 0);
    }
  };

  f4 acc[MT][RT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[mt][rt] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  // A fragments of K block j of the stage at X, and the B operands of word j of a ring slot.
  auto read_a = [&](const uint8_t* X, int j, h8 (&af)[MT]) __attribute__((always_inline)) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) af[mt] = *reinterpret_cast<const h8*>(X + xslot(wrow + mt * 16 + c, g * 4 + j));
  };
  auto dequant_b = [&](int slot, int j, const QuantParams (&qp)[RT], h8 (&bf)[RT]) __attribute__((always_inline)) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      h2 wd[4];
      dequant_word(wraw[slot][rt][j], qp[rt], uc, wd);
      bf[rt] = pack_h8(wd);
    }
  };

  // Interleave hint for one K block: each MFMA followed by two VALU instructions (the
  // dequantization of the next block), an LDS read after every RT MFMAs.
  auto interleave = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);    // LDS read
    }
  };

  // ---- prologue: x steps s0 .. s0 + S - 2 in flight, weights of s0 + i in slot i (i < P);
  // once x step s0 is in, block 0 of step s0: its A fragments and dequantized B operands.
#pragma unroll
  for (int i = 0; i < S - 1; ++i) issue_x(s0 + i, i);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < P; ++i) {
    issue_w(s0 + i, i);
    __builtin_amdgcn_sched_barrier(0);
  }
  h8 af[MT], bf[2][RT];
  step_barrier<C::kFirstWait>();
  {
    QuantParams qp[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) qp[rt] = make_params((wzw[0][rt] >> zsh[rt]) & 0xFu, wsc[0][rt]);
    read_a(smem, 0, af);
    dequant_b(0, 0, qp, bf[0]);
  }

  // Iteration s (slot = (s - s0) % P, compile-time; stage st): block 0 of step s is in af and
  // bf[0]. Blocks j = 0..3: the MFMAs of block j while the operands of block j + 1 are read and
  // dequantized; before block 3 the workgroup meets at the barrier for x step s + 1, issues x
  // step s + S - 1 into the stage of step s - 1, and block 3 runs in the shadow of block 0 of
  // step s + 1. Then the weights of step s + P go into the freed slot.
  // In the tail (fewer than P steps left) the weights an iteration issues are never read, so the
  // compiler drops those loads and the count after x step s + 1 is smaller than kAfterX: the
  // tail's barriers wait for every load instead.
  auto iteration = [&](int s, int st, auto slot_tag, auto tail_tag) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_tag)::value;
    constexpr bool tail = decltype(tail_tag)::value;
    constexpr int nslot = (slot + 1) % P;
    const int st_next = st + 1 == S ? 0 : st + 1;
    const uint8_t* X = smem + st * C::kStage;
    const uint8_t* Xn = smem + st_next * C::kStage;
    QuantParams qp[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) qp[rt] = make_params((wzw[slot][rt] >> zsh[rt]) & 0xFu, wsc[slot][rt]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int cur = j & 1;
      __builtin_amdgcn_sched_barrier(0);
      if (j < 3) {
        dequant_b(slot, j + 1, qp, bf[cur ^ 1]);
      } else {
        // x step s + 1 has landed in every wave's part of its stage, and every wave is past
        // step s - 1: its stage is free.
        step_barrier<tail ? 0 : C::kAfterX>();
        issue_x(s + S - 1, st == 0 ? S - 1 : st - 1);
        // The wait above counts the loads issued after each x step: no later load moves above it.
        __builtin_amdgcn_sched_barrier(0);
        QuantParams qn[RT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) qn[rt] = make_params((wzw[nslot][rt] >> zsh[rt]) & 0xFu, wsc[nslot][rt]);
        dequant_b(nslot, 0, qn, bf[0]);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
          acc[mt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[mt], bf[cur][rt], acc[mt][rt], 0, 0, 0);
        // Fragment mt of the next block, as soon as this block's MFMAs that read it are issued.
        af[mt] = *reinterpret_cast<const h8*>((j < 3 ? X : Xn) + xslot(wrow + mt * 16 + c, g * 4 + ((j + 1) & 3)));
      }
      interleave();
    }
    __builtin_amdgcn_sched_barrier(0);
    issue_w(s + P, slot);
  };

  auto next = [](int st) { return st + 1 == S ? 0 : st + 1; };
  using Loop = std::false_type;
  using Tail = std::true_type;
  int s = s0;
  int st = 0;  // stage of step s
  for (; s + P - 1 < s1; s += P) {
    iteration(s, st, std::integral_constant<int, 0>{}, Loop{});
    st = next(st);
    iteration(s + 1, st, std::integral_constant<int, 1>{}, Loop{});
    st = next(st);
    if constexpr (P > 2) {
      iteration(s + 2, st, std::integral_constant<int, 2>{}, Loop{});
      st = next(st);
    }
    if constexpr (P > 3) {
      iteration(s + 3, st, std::integral_constant<int, 3>{}, Loop{});
      st = next(st);
    }
  }
  // Fewer than P steps remain.
  if (s < s1) {
    iteration(s, st, std::integral_constant<int, 0>{}, Tail{});
    st = next(st);
  }
  if constexpr (P > 2) {
    if (s + 1 < s1) {
      iteration(s + 1, st, std::integral_constant<int, 1>{}, Tail{});
      st = next(st);
    }
  }
  if constexpr (P > 3) {
    if (s + 2 < s1) iteration(s + 2, st, std::integral_constant<int, 2>{}, Tail{});
  }

  // ---- epilogue. D layout of v_mfma_f32_16x16x32_f16: lane holds rows 4 (lane / 16) + q,
  // column lane % 16. Under SiLU*mul, lanes c and c ^ 8 hold the gate and up columns of one
  // output column (phys_col); the partner value comes over with a lane shuffle that every lane
  // executes, before any per-lane branch.
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int l = wl + rt * 16 + c;
    const int n = phys_col(a, n_base, l);
    const bool valid = col_valid(a, n_base, l);
    const float b = (split_k == 1 && a.bias && valid) ? half_bits_to_float(a.bias[n]) : 0.0f;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = m0 + wrow + mt * 16 + 4 * g + q;
        const float v = acc[mt][rt][q] * row_scale(a, m) + b;
        if (split_k == 1 && a.epilogue == TF_EPILOGUE_SILU_MUL) {
          const float u = __shfl_xor(v, 8);
          if (valid && !(l & 8) && m < a.m)
            a.out[(int64_t)m * a.ldo + silu_out_col(n_base, l)] = finish_silu_mul(v, u);
        } else if (valid && m < a.m) {
          if (split_k == 1)
            store_out(a, m, n, v);
          else
            ws[((int64_t)z * a.m + m) * a.n + n] = acc[mt][rt][q];
        }
      }
  }
}

int effective_split4(const LinearArgs& a, const tf_gemm_config& cfg) {
  const int nsteps = ((a.k >> 5) + 3) >> 2;
  return cfg.split_k < nsteps ? cfg.split_k : (nsteps > 0 ? nsteps : 1);
}

int64_t gemm4_workspace(const LinearArgs& a, const tf_gemm_config& cfg) {
  const int s = effective_split4(a, cfg);
  return s > 1 ? (int64_t)s * a.m * a.n * (int64_t)sizeof(float) : 0;
}

template <int MT, int RT, int WM, int S, int P>
int launch_gemm4(const LinearArgs& a, const tf_gemm_config& cfg, float* ws, hipStream_t stream) {
  using C = G4<MT, RT, WM, S, P>;
  if ((a.n & 15) || (a.k & 127))
    return fail(TF_EINVAL, "tf_w4a16_linear: this gemm_mfma variant needs N % 16 == 0 and K % 128 == 0");
  const int64_t x_bytes = ((int64_t)(a.m - 1) * a.ldx + a.k) * 2;
  const int64_t w_bytes = (int64_t)a.n * (a.k / 2);
  if (x_bytes >= (int64_t)kOutOfRange || w_bytes >= (int64_t)kOutOfRange)
    return fail(TF_EINVAL, "tf_w4a16_linear: this gemm_mfma variant needs x and qweight_t below 2 GiB");
  const int split = effective_split4(a, cfg);
  if (split > 1 && ws == nullptr) return fail(TF_EINVAL, "tf_w4a16_linear: split-K needs a workspace");
  const int tiles_n = (int)cdiv(a.n, C::BN);
  const int tiles_m = (int)cdiv(a.m, C::BM);
  const int64_t grid = (int64_t)tiles_n * tiles_m * split;
  if (grid > 0x7FFFFFFF) return fail(TF_EINVAL, "tf_w4a16_linear: too many tiles");
  auto kernel = gemm4_kernel<MT, RT, WM, S, P>;
  if (int rc = reserve_lds(kernel, C::kLds, "gemm_mfma")) return rc;
  kernel<<<(unsigned)grid, C::kThreads, C::kLds, stream>>>(a, ws, split, tiles_n, tiles_m);
  if (int rc = check_launch("tf_w4a16_linear(gemm_mfma)")) return rc;
  if (split > 1) return splitk_reduce(a, ws, split, stream);
  return TF_OK;
}

// block_k 128 with num_stages 4 + S (S = 3 or 4 x stages) marks these variants: the
// register-streamed family (block_k 128) with S x stages (x issued S - 1 steps ahead) and the
// weights three steps ahead; block_m = 16 MT WM, block_n = 16 RT (4 / WM), num_warps 4.
#define TF_GEMM4(MT, RT, WM, S)                                                                       \
  {{TF_KERNEL_GEMM_MFMA, 16 * MT * WM, 16 * RT * (4 / WM), 128, 1, 4, 4 + S},                          \
   (launch_gemm4<MT, RT, WM, S, 3>), gemm4_workspace}

const Variant kGemm4Variants[] = {
    TF_GEMM4(8, 5, 1, 3), TF_GEMM4(8, 4, 1, 4), TF_GEMM4(8, 3, 1, 4), TF_GEMM4(8, 2, 1, 4),
};

}  // namespace

const Variant* gemm4_variants(int* count) {
  *count = (int)(sizeof(kGemm4Variants) / sizeof(kGemm4Variants[0]));
  return kGemm4Variants;
}

}  // namespace tf
