// Register-streamed W4A16 GEMM: weights go straight from memory into MFMA operand registers.
//
// For small M the weight stream is the cost, so the kernel is shaped like the decode GEMV
// rather than like a tiled GEMM; with waves along M the same structure serves larger M
// without the dequantized-weight LDS buffer of the LDS-tile kernels:
//   * a workgroup of 4 waves, WM along M and WN = 4 / WM along N, covers BM = WM * 16 * MT
//     rows and BN = WN * 16 * RT columns; each wave owns 16 * MT rows and 16 * RT columns and
//     streams the packed weights, scales and zero points of its columns into a register ring
//     (P steps of 128 K ahead), dequantizes each packed word (fp16(q - z) * s, one rounding)
//     straight into the B operand of v_mfma_f32_16x16x32_f16 and reuses it for its MT row
//     tiles (the WM waves of a column set load and dequantize the same words);
//   * the x tile [BM][128] of each step is shared by the 4 waves: it streams from global
//     memory into S LDS stages through buffer loads with the LDS destination, issued S - 1
//     steps ahead, with one barrier per step;
//   * lane (c = lane % 16, g = lane / 16) holds 32 consecutive K values (chunk g) of column c,
//     the B layout of the 16x16x32 MFMA; MFMA j takes word j of every lane group, so its K set
//     is {g * 32 + j * 8 + e}, and the A fragments read x at the same K positions. In the tile
//     layout the 64 lanes of a 16-column tile read one contiguous 1 KB block per step.
// Rows of a stage hold 16 chunks of 16 bytes (one 256-byte LDS bank line); chunk c of row r
// sits in slot c ^ (r & 11). A 16-byte LDS read on gfx950 serves the wave in four phases of
// 16 lanes (the wave's halves, each split by the parity of lane bits 2-4): the fragment read
// (lane 16 g + c at row c, chunk 4 g + j) then gives each phase's 16 lanes 16 distinct slots,
// where c ^ (r % 16) costs four conflict cycles per read.
// K may end in a partial 128-wide step: chunks past K read as zeros (per-lane bounds). Loads
// past the K range of the workgroup are issued with out-of-range offsets, so the count of
// loads in flight is the same on every path and the waits stay exact.
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
constexpr int kStageRowChunks = 16;  // 16-byte chunks per 128-wide fp16 row

__device__ __forceinline__ uint32_t swz16(int row, int chunk) {
  return (uint32_t)(row * kStageRowChunks + (chunk ^ (row & 11))) * 16u;
}

template <int MT, int RT, int WM, int P, int S>
struct G3 {
  static constexpr int kThreads = 256;
  static constexpr int WN = 4 / WM;
  static constexpr int BM = 16 * MT * WM;
  static constexpr int BN = 16 * RT * WN;
  static constexpr int kStage = BM * kStepK * 2;  // bytes of one x stage
  static constexpr int kDmaPerWave = kStage / 1024 / 4;
  static constexpr int kLds = S * kStage;
  // VMEM issued after x step s (S - 1 iterations back) when iteration s waits for it:
  // weights of step s - S + 1 + P, then S - 2 whole iterations (x step, weights). (The first
  // iteration may have more in flight; its wait is then longer, never too short.)
  static constexpr int kAfterA = 3 * RT + (S - 2) * (kDmaPerWave + 3 * RT);
  static_assert(WM == 1 || WM == 2 || WM == 4, "waves along M");
  static_assert(kDmaPerWave >= 1 && kStage % 4096 == 0, "x stage must split evenly over the waves");
  static_assert(S == 2 || S == 3, "x stages");
  static_assert(P >= 2 && P <= 4, "register ring of two to four steps");
  static_assert(kLds <= 160 * 1024, "x stages exceed the LDS");
  static_assert(kAfterA < 64, "vmcnt range");
};

template <int N>
__device__ __forceinline__ void step_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

template <int MT, int RT, int WM, int P, int S>
__global__ __launch_bounds__(256) void gemm3_kernel(LinearArgs a, float* __restrict__ ws, int split_k,
                                                    int tiles_n, int tiles_m) {
  using C = G3<MT, RT, WM, P, S>;
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
  const int wrow = wm * 16 * MT;                          // this wave's first row in the tile

  const int nchunks = a.k >> 5;
  const int nsteps = (nchunks + 3) >> 2;
  const int s0 = (int)(((int64_t)z * nsteps) / split_k);
  const int s1 = (int)(((int64_t)(z + 1) * nsteps) / split_k);

  const uint32_t row_bytes = (uint32_t)(a.k >> 1);
  const int groups = a.k >> a.log2g;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)(((int64_t)(a.m - 1) * a.ldx + a.k) * 2));
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.qw, (uint32_t)a.n * row_bytes);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.scales, (uint32_t)(groups * a.n * 2));
  const __amdgpu_buffer_rsrc_t rz = make_rsrc(a.qz, (uint32_t)(groups * (a.n >> 3) * 4));
  const UnpackConsts uc = unpack_consts();

  // ---- x step s -> LDS stage st. Instruction i of this wave writes 1 KB at
  // (wave * kDmaPerWave + i) KB of the stage; lane l of it fills 16-byte slot 64 j + l.
  uint32_t x_off[C::kDmaPerWave];  // byte offset of the chunk in step 0; kOutOfRange if none
  int x_k[C::kDmaPerWave];         // K index of the chunk in step 0
#pragma unroll
  for (int i = 0; i < C::kDmaPerWave; ++i) {
    const int p = (wave * C::kDmaPerWave + i) * 64 + lane;
    const int row = p >> 4;
    const int ch = (p & 15) ^ (row & 11);
    const int m = m0 + row;
    x_k[i] = ch * 8;
    x_off[i] = m < a.m ? (uint32_t)(((int64_t)m * a.ldx + ch * 8) * 2) : kOutOfRange;
  }
  auto issue_x = [&](int s, int st) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < C::kDmaPerWave; ++i) {
      const bool ok = s < s1 && s * kStepK + x_k[i] < a.k;
      const uint32_t off = ok ? x_off[i] + (uint32_t)s * (kStepK * 2) : kOutOfRange;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rx, (__attribute__((address_space(3))) void*)(smem + st * C::kStage + (wave * C::kDmaPerWave + i) * 1024),
          16, off, 0, 0, 0);
    }
  };

  // ---- weights, scales and zero points of step s -> register slot. Tile layout: the lane's
  // chunk (column n, K block g) of step s sits at chunk 16 t Q + 4 rows s + g rows + cc
  // (t = n / 16, cc = n % 16, rows = the tile's row count), its scale at element
  // 16 t P + grp rows + cc and its zero word at 2 t P + grp (rows / 8) + cc / 8.
  const uint32_t q_total = (uint32_t)nchunks;
  uint32_t w_off[RT], w_step[RT], s_base[RT], z_base[RT], t_rows[RT];
  uint32_t col[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int l = wl + rt * 16 + c;
    const int n = phys_col(a, n_base, l);
    col[rt] = (uint32_t)n;
    const uint32_t t = (uint32_t)n >> 4, cc = (uint32_t)n & 15u;
    const uint32_t rows = (uint32_t)tile_rows(a.n, t);
    t_rows[rt] = rows;
    w_off[rt] = col_valid(a, n_base, l) ? (t * q_total * 16u + (uint32_t)g * rows + cc) * 16u : kOutOfRange;
    w_step[rt] = rows * 64u;
    s_base[rt] = t * 16u * (uint32_t)groups + cc;
    z_base[rt] = t * 2u * (uint32_t)groups + (cc >> 3);
  }
  const int lane_end = min(s1, (nchunks - g + 3) >> 2);  // steps whose chunk g lies inside K
  u4 wraw[P][RT];
  uint32_t wsc[P][RT], wzw[P][RT];
  auto issue_w = [&](int s, int slot) __attribute__((always_inline)) {
    const bool ok = s < lane_end;
    const uint32_t grp = (uint32_t)((s * kStepK + g * 32) >> a.log2g);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      // Offsets are computed unconditionally and then selected: a conditional arm holding a
      // multiply is compiled as a per-lane branch around each load, which splits the loop
      // into scheduling regions and forces a full vmcnt drain where the branches rejoin.
      const bool v = ok && w_off[rt] != kOutOfRange;
      const uint32_t wo = w_off[rt] + (uint32_t)s * w_step[rt];
      const uint32_t so = (s_base[rt] + grp * t_rows[rt]) * 2u;
      const uint32_t zo = (z_base[rt] + grp * (t_rows[rt] >> 3)) * 4u;
      wraw[slot][rt] = load_b128(rq, v ? wo : kOutOfRange);
      wsc[slot][rt] = load_b16(rs, v ? so : kOutOfRange);
      wzw[slot][rt] = load_b32(rz, v ? zo : kOutOfRange);
    }
  };

  f4 acc[MT][RT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[mt][rt] = f4{0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](int st, int slot) __attribute__((always_inline)) {
    const uint8_t* X = smem + st * C::kStage;
    QuantParams qp[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) qp[rt] = make_params(zero_of(wzw[slot][rt], col[rt]), wsc[slot][rt]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h8 xa[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) xa[mt] = *reinterpret_cast<const h8*>(X + swz16(wrow + mt * 16 + c, g * 4 + j));
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        h2 wd[4];
        dequant_word(wraw[slot][rt][j], qp[rt], uc, wd);
        const h8 b = pack_h8(wd);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[mt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[mt], b, acc[mt][rt], 0, 0, 0);
      }
    }
  };

  // ---- prologue: x steps s0 .. s0 + S - 2 in flight, weights of s0 + i in slot i (i < P)
#pragma unroll
  for (int i = 0; i < S - 1; ++i) issue_x(s0 + i, i);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < P; ++i) {
    issue_w(s0 + i, i);
    __builtin_amdgcn_sched_barrier(0);
  }

  // Iteration s (slot = (s - s0) % P, compile-time): wait for x step s, issue x step
  // s + S - 1, multiply step s, issue the weights of step s + P into the freed slot.
  auto iteration = [&](int s, int st, auto slot_tag) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_tag)::value;
    step_barrier<C::kAfterA>();
    issue_x(s + S - 1, (st + S - 1) % S);
    // The waits count the loads issued after each x step: no later load may move above it.
    __builtin_amdgcn_sched_barrier(0);
    compute(st, slot);
    issue_w(s + P, slot);
  };
  auto next_stage = [](int st) { return st + 1 == S ? 0 : st + 1; };

  int s = s0;
  int st = 0;  // stage of step s
  for (; s + P - 1 < s1; s += P) {
    iteration(s, st, std::integral_constant<int, 0>{});
    st = next_stage(st);
    iteration(s + 1, st, std::integral_constant<int, 1>{});
    st = next_stage(st);
    if constexpr (P > 2) {
      iteration(s + 2, st, std::integral_constant<int, 2>{});
      st = next_stage(st);
    }
    if constexpr (P > 3) {
      iteration(s + 3, st, std::integral_constant<int, 3>{});
      st = next_stage(st);
    }
  }
  // Fewer than P steps remain.
  if (s < s1) {
    iteration(s, st, std::integral_constant<int, 0>{});
    st = next_stage(st);
  }
  if constexpr (P > 2) {
    if (s + 1 < s1) {
      iteration(s + 1, st, std::integral_constant<int, 1>{});
      st = next_stage(st);
    }
  }
  if constexpr (P > 3) {
    if (s + 2 < s1) iteration(s + 2, st, std::integral_constant<int, 2>{});
  }

  // ---- epilogue. D layout of v_mfma_f32_16x16x32_f16: lane holds rows 4 (lane / 16) + r,
  // column lane % 16. Under SiLU*mul, lanes c and c ^ 8 hold the gate and up columns of one
  // output column (phys_col); the partner value comes over with a lane shuffle that every
  // lane executes, before any per-lane branch.
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int l = wl + rt * 16 + c;
    const int n = (int)col[rt];
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

int effective_split3(const LinearArgs& a, const tf_gemm_config& cfg) {
  const int nsteps = ((a.k >> 5) + 3) >> 2;
  return cfg.split_k < nsteps ? cfg.split_k : (nsteps > 0 ? nsteps : 1);
}

int64_t gemm3_workspace(const LinearArgs& a, const tf_gemm_config& cfg) {
  const int s = effective_split3(a, cfg);
  return s > 1 ? (int64_t)s * a.m * a.n * (int64_t)sizeof(float) : 0;
}

template <int MT, int RT, int WM, int P, int S>
int launch_gemm3(const LinearArgs& a, const tf_gemm_config& cfg, float* ws, hipStream_t stream) {
  using C = G3<MT, RT, WM, P, S>;
  const int64_t x_bytes = ((int64_t)(a.m - 1) * a.ldx + a.k) * 2;
  const int64_t w_bytes = (int64_t)a.n * (a.k / 2);
  if (x_bytes >= (int64_t)kOutOfRange || w_bytes >= (int64_t)kOutOfRange)
    return fail(TF_EINVAL, "tf_w4a16_linear: this gemm_mfma variant needs x and qweight_t below 2 GiB");
  const int split = effective_split3(a, cfg);
  if (split > 1 && ws == nullptr) return fail(TF_EINVAL, "tf_w4a16_linear: split-K needs a workspace");
  const int tiles_n = (int)cdiv(a.n, C::BN);
  const int tiles_m = (int)cdiv(a.m, C::BM);
  const int64_t grid = (int64_t)tiles_n * tiles_m * split;
  if (grid > 0x7FFFFFFF) return fail(TF_EINVAL, "tf_w4a16_linear: too many tiles");
  auto kernel = gemm3_kernel<MT, RT, WM, P, S>;
  if (C::kLds > 64 * 1024 &&
      hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          C::kLds) != hipSuccess)
    return fail(TF_ELAUNCH, "tf_w4a16_linear: cannot reserve LDS for gemm_mfma");
  kernel<<<(unsigned)grid, C::kThreads, C::kLds, stream>>>(a, ws, split, tiles_n, tiles_m);
  if (int rc = check_launch("tf_w4a16_linear(gemm_mfma)")) return rc;
  if (split > 1) return splitk_reduce(a, ws, split, stream);
  return TF_OK;
}

// block_k 128 (one 128-wide step per barrier) tells these variants apart from the LDS-tile
// kernels; num_stages = S (x stages). TF_GEMM3: one wave along M; TF_GEMM3W: WM waves along
// M (its tile shapes do not occur among the one-wave variants).
#define TF_GEMM3(MT, RT, S) \
  {{TF_KERNEL_GEMM_MFMA, 16 * MT, 64 * RT, 128, 1, 4, S}, (launch_gemm3<MT, RT, 1, 2, S>), gemm3_workspace}
#define TF_GEMM3W(MT, RT, WM, S)                                                                  \
  {{TF_KERNEL_GEMM_MFMA, 16 * MT * WM, 16 * RT * (4 / WM), 128, 1, 4, S}, (launch_gemm3<MT, RT, WM, 2, S>), \
   gemm3_workspace}

const Variant kGemm3Variants[] = {
    TF_GEMM3(1, 1, 3), TF_GEMM3(1, 2, 3), TF_GEMM3(1, 4, 3), TF_GEMM3(2, 1, 3), TF_GEMM3(2, 2, 3),
    TF_GEMM3(2, 4, 3), TF_GEMM3(4, 1, 3), TF_GEMM3(4, 2, 3), TF_GEMM3(4, 4, 3), TF_GEMM3(8, 1, 3),
    TF_GEMM3(8, 2, 3), TF_GEMM3(2, 2, 2), TF_GEMM3(4, 2, 2), TF_GEMM3W(8, 5, 2, 2),
};

}  // namespace

const Variant* gemm3_variants(int* count) {
  *count = (int)(sizeof(kGemm3Variants) / sizeof(kGemm3Variants[0]));
  return kGemm3Variants;
}

}  // namespace tf
