// Load-time layout kernels: int4 pack/unpack, AWQ <-> TokenForge repack, full dequant.
//
// Repack is an 8x8 transpose of 4-bit values: the eight AWQ words qweight[8*kb + i][nb]
// (i = 0..7) hold exactly the same 64 values as the eight TokenForge words
// qweight_t[8*nb + j][kb] (j = 0..7). Each thread moves whole 8x8 blocks in registers
// (three masked-swap stages) and the tile is staged through LDS so that both the reads
// and the writes are 128-byte coalesced rows.
//
// pack_awq's layout is the gfx950 tile layout (tile_layout.h): the tile kernels move 16-byte
// weight chunks, scales and zero-point words between the reference's TokenForge layout and
// it, one thread per destination element. awq_quantize (the test and benchmark fixture
// generator) quantizes an fp32 [N, K] weight straight into AWQ format.
#include "tf_common.h"
#include "tile_layout.h"

namespace tf {

int log2_group(int32_t g);
int check_group_size(int32_t group_size, int64_t k, const char* name);

namespace {

// AWQ_ORDER[i]: offset held by nibble i (pack.py:32).
__host__ __device__ constexpr uint32_t awq_order(uint32_t i) {
  return (i < 4) ? 2 * i : 2 * (i - 4) + 1;
}

// In-place transpose of an 8x8 matrix of nibbles: row r = word r, column c = nibble c.
// After the call, nibble c of word r holds what nibble r of word c held before.
__device__ __forceinline__ void transpose_nibbles(uint32_t w[8]) {
#pragma unroll
  for (int r = 0; r < 8; r += 2) {  // 1x1 blocks, 1 row apart
    const uint32_t t = ((w[r] >> 4) ^ w[r + 1]) & 0x0F0F0F0Fu;
    w[r + 1] ^= t;
    w[r] ^= t << 4;
  }
  constexpr int kStage2Rows[4] = {0, 1, 4, 5};  // 2x2 blocks, 2 rows apart
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = kStage2Rows[i];
    const uint32_t t = ((w[r] >> 8) ^ w[r + 2]) & 0x00FF00FFu;
    w[r + 2] ^= t;
    w[r] ^= t << 8;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {  // 4x4 blocks, 4 rows apart
    const uint32_t t = ((w[r] >> 16) ^ w[r + 4]) & 0x0000FFFFu;
    w[r + 4] ^= t;
    w[r] ^= t << 16;
  }
}

// Logical 8x8 block transpose in the AWQ nibble order: in[r] nibble p(c) holds element
// (r, c); returns out[c] with nibble p(r) holding element (r, c), p = AWQ_REVERSE_ORDER.
// Reordering the input words by AWQ_ORDER turns it into a plain nibble transpose whose
// word x is the output word c with p(c) = x.
__device__ __forceinline__ void awq_block_transpose(const uint32_t in[8], uint32_t out[8]) {
  uint32_t w[8];
#pragma unroll
  for (int y = 0; y < 8; ++y) w[y] = in[awq_order(y)];
  transpose_nibbles(w);
#pragma unroll
  for (int c = 0; c < 8; ++c) out[c] = w[awq_nibble_of(c)];
}

constexpr int kTileBlocks = 32;  // 32 x 32 blocks of 8x8 nibbles per workgroup
constexpr int kRepackThreads = 256;

// src int32 [rows_a, cols_b / 8] -> dst int32 [cols_b, rows_a / 8] where src word
// (a, b/8) nibble p(b%8) and dst word (b, a/8) nibble p(a%8) hold the same element.
// AWQ -> TokenForge is (a, b) = (k, n); the inverse is (a, b) = (n, k).
__global__ __launch_bounds__(kRepackThreads) void repack_kernel(const uint32_t* __restrict__ src,
                                                               uint32_t* __restrict__ dst,
                                                               int64_t rows_a, int64_t cols_b) {
  // LDS tile of output words: 256 output rows (8 * 32 b-blocks) x 32 a-blocks.
  // Column index is XOR-swizzled with the b-block so that the block-wise writes spread
  // over the banks; rows are read back word by word.
  __shared__ uint32_t tile[8 * kTileBlocks][kTileBlocks];

  const int64_t a_blocks = rows_a / 8;   // words per dst row
  const int64_t b_blocks = cols_b / 8;   // words per src row
  const int64_t ab0 = (int64_t)blockIdx.y * kTileBlocks;
  const int64_t bb0 = (int64_t)blockIdx.x * kTileBlocks;
  const int tid = threadIdx.x;

#pragma unroll
  for (int r = 0; r < (kTileBlocks * kTileBlocks) / kRepackThreads; ++r) {
    const int blk = tid + r * kRepackThreads;
    const int bbi = blk % kTileBlocks;
    const int abi = blk / kTileBlocks;
    const int64_t ab = ab0 + abi;
    const int64_t bb = bb0 + bbi;
    uint32_t in[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (ab < a_blocks && bb < b_blocks) {
#pragma unroll
      for (int i = 0; i < 8; ++i) in[i] = src[(ab * 8 + i) * b_blocks + bb];
    }
    uint32_t out[8];
    awq_block_transpose(in, out);
#pragma unroll
    for (int j = 0; j < 8; ++j) tile[bbi * 8 + j][abi ^ bbi] = out[j];
  }
  __syncthreads();

  // Write back: 32 consecutive threads write one 128-byte dst row segment.
#pragma unroll 4
  for (int idx = tid; idx < 8 * kTileBlocks * kTileBlocks; idx += kRepackThreads) {
    const int row = idx / kTileBlocks;   // 0..255 -> b = 8*bb0 + row
    const int abi = idx % kTileBlocks;
    const int bbi = row / 8;
    const int64_t b = bb0 * 8 + row;
    const int64_t ab = ab0 + abi;
    if (b < cols_b && ab < a_blocks) dst[b * a_blocks + ab] = tile[row][abi ^ bbi];
  }
}

// values int32 [rows, n] -> packed [rows, n/8]; one thread per output word.
__global__ void pack_int4_kernel(const int32_t* __restrict__ values, int32_t* __restrict__ packed,
                                 int64_t words, int32_t* __restrict__ range_flag) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= words) return;
  const int32_t* v = values + i * 8;
  uint32_t word = 0;
  bool bad = false;
#pragma unroll
  for (int nib = 0; nib < 8; ++nib) {
    const int32_t x = v[awq_order(nib)];
    bad |= (x < 0) | (x > 15);
    word |= ((uint32_t)x & 0xFu) << (4 * nib);
  }
  packed[i] = (int32_t)word;
  if (bad && range_flag != nullptr) range_flag[0] = 1;
}

// packed [rows, words] -> values [rows, 8*words]; one thread per input word.
__global__ void unpack_int4_kernel(const int32_t* __restrict__ packed, int32_t* __restrict__ values,
                                   int64_t words) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= words) return;
  const uint32_t w = (uint32_t)packed[i];
  int32_t* v = values + i * 8;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = (int32_t)((w >> (4 * awq_nibble_of(j))) & 0xFu);
}

// Tile-layout weights -> out fp16 [n, k] (nn.Linear layout); one thread per 16-byte chunk (32
// values of one row), threads in row-major chunk order so the 64-byte stores are contiguous.
__global__ void dequant_kernel(const uint32_t* __restrict__ qw, const uint16_t* __restrict__ scales,
                               const uint32_t* __restrict__ qzeros, uint16_t* __restrict__ out,
                               int64_t n, int64_t k, int log2_group) {
  const int64_t q_total = k / 32;
  const int64_t p_total = k >> log2_group;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * q_total) return;
  const int64_t row = i / q_total;
  const int64_t q = i % q_total;
  const u4 words = *reinterpret_cast<const u4*>(qw + tile_chunk(row, q, n, q_total) * 4);
  const int64_t grp = (q * 32) >> log2_group;
  const uint32_t zw = qzeros[tile_zero(grp, row >> 3, n, p_total)];
  const QuantParams p = make_params(zero_of(zw, (uint32_t)row), scales[tile_scale(grp, row, n, p_total)]);
  u4* dst = reinterpret_cast<u4*>(out + row * k + q * 32);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h2 v[4];
    dequant_word(words[j], p, v);
    u4 o;
    o[0] = as_u32(v[0]);
    o[1] = as_u32(v[1]);
    o[2] = as_u32(v[2]);
    o[3] = as_u32(v[3]);
    dst[j] = o;
  }
}

// One of the three tensors of a layer, moved between the TokenForge layout ("natural" index)
// and the tile layout; TO_TILE gathers destination index i of the tile layout from its
// natural source, the other direction gathers natural index i from its tile position.
enum TileTensor { kTileWeights = 0, kTileScales = 1, kTileZeros = 2 };

template <typename T, int KIND, bool TO_TILE>
__global__ void tile_permute_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t count,
                                    int64_t n, int64_t k, int log2_group) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  const int64_t q_total = k / 32;
  const int64_t p_total = k >> log2_group;
  int64_t from;
  if (KIND == kTileWeights) {
    if (TO_TILE) {
      int64_t row, q;
      tile_chunk_source(i, n, q_total, &row, &q);
      from = row * q_total + q;
    } else {
      from = tile_chunk(i / q_total, i % q_total, n, q_total);
    }
  } else if (KIND == kTileScales) {
    if (TO_TILE) {
      int64_t grp, row;
      tile_scale_source(i, n, p_total, &grp, &row);
      from = grp * n + row;
    } else {
      from = tile_scale(i / n, i % n, n, p_total);
    }
  } else {
    const int64_t words = n / 8;
    if (TO_TILE) {
      int64_t grp, w;
      tile_zero_source(i, n, p_total, &grp, &w);
      from = grp * words + w;
    } else {
      from = tile_zero(i / words, i % words, n, p_total);
    }
  }
  dst[i] = src[from];
}

template <bool TO_TILE>
int launch_tile(const int32_t* qw, const uint16_t* sc, const int32_t* qz, int32_t* qw_out, uint16_t* sc_out,
                int32_t* qz_out, int64_t n, int64_t k, int32_t group_size, hipStream_t stream, const char* name) {
  const int lg = log2_group(group_size);
  const int64_t chunks = n * (k / 32);
  const int64_t groups = k / group_size;
  if (chunks > 0)
    tile_permute_kernel<u4, kTileWeights, TO_TILE><<<(unsigned)cdiv(chunks, 256), 256, 0, stream>>>(
        reinterpret_cast<const u4*>(qw), reinterpret_cast<u4*>(qw_out), chunks, n, k, lg);
  if (groups * n > 0)
    tile_permute_kernel<uint16_t, kTileScales, TO_TILE><<<(unsigned)cdiv(groups * n, 256), 256, 0, stream>>>(
        sc, sc_out, groups * n, n, k, lg);
  if (groups * (n / 8) > 0)
    tile_permute_kernel<uint32_t, kTileZeros, TO_TILE><<<(unsigned)cdiv(groups * (n / 8), 256), 256, 0, stream>>>(
        reinterpret_cast<const uint32_t*>(qz), reinterpret_cast<uint32_t*>(qz_out), groups * (n / 8), n, k, lg);
  return check_launch(name);
}

// AWQ min-max quantization of fp32 weight [n, k] (pack.py:83-107), one thread per (group p,
// eight rows 8o..8o+7): the eight rows' statistics over the group, then the group's k words of
// AWQ qweight [k, n/8] (word o of each row k), its qzeros word and its eight scales.
//   scale = fp16(max(max - min, 1e-5) / 15), zero = clamp(-rint(min / scale), 0, 15),
//   q = clamp(rint(w / scale) + zero, 0, 15); fp32 IEEE division, rint = round half to even.
__global__ void awq_quantize_kernel(const float* __restrict__ w, int64_t n, int64_t k, int group,
                                    uint32_t* __restrict__ qweight, uint32_t* __restrict__ qzeros,
                                    uint16_t* __restrict__ scales) {
  const int64_t octets = n / 8;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= octets * (k / group)) return;
  const int64_t o = i % octets;  // consecutive threads: consecutive words of one qweight row
  const int64_t p = i / octets;
  float s[8], z[8];
  uint32_t zword = 0;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const float* row = w + (o * 8 + r) * k + p * group;
    float lo = row[0], hi = row[0];
    for (int e = 1; e < group; ++e) {
      lo = fminf(lo, row[e]);
      hi = fmaxf(hi, row[e]);
    }
    const _Float16 s16 = (_Float16)(fmaxf(hi - lo, 1e-5f) / 15.0f);
    s[r] = (float)s16;
    z[r] = fminf(fmaxf(-__builtin_rintf(lo / s[r]), 0.0f), 15.0f);
    scales[p * n + o * 8 + r] = __builtin_bit_cast(uint16_t, s16);
    zword |= (uint32_t)z[r] << (4 * awq_nibble_of((uint32_t)r));
  }
  qzeros[p * octets + o] = zword;
  for (int e = 0; e < group; ++e) {
    uint32_t word = 0;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const float v = w[(o * 8 + r) * k + p * group + e];
      const float q = fminf(fmaxf(__builtin_rintf(v / s[r]) + z[r], 0.0f), 15.0f);
      word |= (uint32_t)q << (4 * awq_nibble_of((uint32_t)r));
    }
    qweight[(p * group + e) * octets + o] = word;
  }
}

int log2_exact(int v) {
  int l = 0;
  while ((1 << l) < v) ++l;
  return ((1 << l) == v) ? l : -1;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int launch_repack(const int32_t* src, int32_t* dst, int64_t rows_a, int64_t cols_b, void* stream,
                  const char* name) {
  if (src == nullptr || dst == nullptr) return fail(TF_EINVAL, std::string(name) + ": null pointer");
  if (rows_a < 0 || cols_b < 0 || rows_a % 8 || cols_b % 8)
    return fail(TF_EINVAL, std::string(name) + ": both dimensions must be non-negative multiples of 8");
  if (rows_a == 0 || cols_b == 0) return TF_OK;
  const dim3 grid((unsigned)cdiv(cols_b / 8, kTileBlocks), (unsigned)cdiv(rows_a / 8, kTileBlocks));
  if (grid.y > 65535u) return fail(TF_EINVAL, std::string(name) + ": too many rows");
  repack_kernel<<<grid, kRepackThreads, 0, (hipStream_t)stream>>>(
      reinterpret_cast<const uint32_t*>(src), reinterpret_cast<uint32_t*>(dst), rows_a, cols_b);
  return check_launch(name);
}

}  // namespace

int check_group_size(int32_t group_size, int64_t k, const char* name) {
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(TF_EINVAL, std::string(name) + ": group_size must be 32, 64 or 128");
  if (k % group_size != 0)
    return fail(TF_EINVAL, std::string(name) + ": K is not a multiple of group_size");
  return TF_OK;
}

int log2_group(int32_t g) { return log2_exact(g); }

}  // namespace tf

using namespace tf;

extern "C" int tf_pack_int4(const int32_t* values, int32_t* packed, int64_t rows, int64_t n,
                            int32_t* range_flag, void* stream) {
  if (values == nullptr || packed == nullptr) return fail(TF_EINVAL, "tf_pack_int4: null pointer");
  if (rows < 0 || n < 0 || n % 8) return fail(TF_EINVAL, "tf_pack_int4: n must be a multiple of 8");
  const int64_t words = rows * (n / 8);
  if (words == 0) return TF_OK;
  pack_int4_kernel<<<(unsigned)cdiv(words, 256), 256, 0, (hipStream_t)stream>>>(values, packed, words,
                                                                                range_flag);
  return check_launch("tf_pack_int4");
}

extern "C" int tf_unpack_int4(const int32_t* packed, int32_t* values, int64_t rows, int64_t words,
                              void* stream) {
  if (values == nullptr || packed == nullptr) return fail(TF_EINVAL, "tf_unpack_int4: null pointer");
  if (rows < 0 || words < 0) return fail(TF_EINVAL, "tf_unpack_int4: negative size");
  const int64_t total = rows * words;
  if (total == 0) return TF_OK;
  unpack_int4_kernel<<<(unsigned)cdiv(total, 256), 256, 0, (hipStream_t)stream>>>(packed, values,
                                                                                 total);
  return check_launch("tf_unpack_int4");
}

extern "C" int tf_awq_to_tf(const int32_t* qweight, int32_t* qweight_t, int64_t k, int64_t n,
                            void* stream) {
  return launch_repack(qweight, qweight_t, k, n, stream, "tf_awq_to_tf");
}

extern "C" int tf_tf_to_awq(const int32_t* qweight_t, int32_t* qweight, int64_t n, int64_t k,
                            void* stream) {
  return launch_repack(qweight_t, qweight, n, k, stream, "tf_tf_to_awq");
}

extern "C" int tf_w4a16_dequant(const int32_t* qweight_t, const uint16_t* scales,
                                const int32_t* qzeros, uint16_t* out, int64_t n, int64_t k,
                                int32_t group_size, void* stream) {
  if (!qweight_t || !scales || !qzeros || !out) return fail(TF_EINVAL, "tf_w4a16_dequant: null pointer");
  if (n < 0 || k < 0 || n % 8) return fail(TF_EINVAL, "tf_w4a16_dequant: N must be a multiple of 8");
  if (int rc = check_group_size(group_size, k, "tf_w4a16_dequant")) return rc;
  if (!aligned16(qweight_t) || !aligned16(out))
    return fail(TF_EINVAL, "tf_w4a16_dequant: qweight_t and out must be 16-byte aligned");
  const int64_t total = n * (k / 32);
  if (total == 0) return TF_OK;
  dequant_kernel<<<(unsigned)cdiv(total, 256), 256, 0, (hipStream_t)stream>>>(
      reinterpret_cast<const uint32_t*>(qweight_t), scales, reinterpret_cast<const uint32_t*>(qzeros),
      out, n, k, log2_group(group_size));
  return check_launch("tf_w4a16_dequant");
}

static int check_tile_args(const void* a, const void* b, const void* c, const void* d, const void* e,
                           const void* f, int64_t n, int64_t k, int32_t group_size, const char* name) {
  if (!a || !b || !c || !d || !e || !f) return fail(TF_EINVAL, std::string(name) + ": null pointer");
  if (n < 0 || k < 0 || n % 8) return fail(TF_EINVAL, std::string(name) + ": N must be a multiple of 8");
  if (int rc = check_group_size(group_size, k, name)) return rc;
  if (!aligned16(a) || !aligned16(d)) return fail(TF_EINVAL, std::string(name) + ": qweight must be 16-byte aligned");
  return TF_OK;
}

extern "C" int tf_tile_pack(const int32_t* qweight_t, const uint16_t* scales, const int32_t* qzeros,
                            int32_t* qweight_tile, uint16_t* scales_tile, int32_t* qzeros_tile, int64_t n,
                            int64_t k, int32_t group_size, void* stream) {
  if (int rc = check_tile_args(qweight_t, scales, qzeros, qweight_tile, scales_tile, qzeros_tile, n, k,
                               group_size, "tf_tile_pack"))
    return rc;
  return launch_tile<true>(qweight_t, scales, qzeros, qweight_tile, scales_tile, qzeros_tile, n, k, group_size,
                           (hipStream_t)stream, "tf_tile_pack");
}

extern "C" int tf_tile_unpack(const int32_t* qweight_tile, const uint16_t* scales_tile, const int32_t* qzeros_tile,
                              int32_t* qweight_t, uint16_t* scales, int32_t* qzeros, int64_t n, int64_t k,
                              int32_t group_size, void* stream) {
  if (int rc = check_tile_args(qweight_tile, scales_tile, qzeros_tile, qweight_t, scales, qzeros, n, k,
                               group_size, "tf_tile_unpack"))
    return rc;
  return launch_tile<false>(qweight_tile, scales_tile, qzeros_tile, qweight_t, scales, qzeros, n, k, group_size,
                            (hipStream_t)stream, "tf_tile_unpack");
}

extern "C" int tf_awq_quantize(const float* weight, int64_t n, int64_t k, int32_t group_size, int32_t* qweight,
                               int32_t* qzeros, uint16_t* scales, void* stream) {
  if (!weight || !qweight || !qzeros || !scales) return fail(TF_EINVAL, "tf_awq_quantize: null pointer");
  if (n < 0 || k < 0 || n % 8) return fail(TF_EINVAL, "tf_awq_quantize: N must be a multiple of 8");
  if (group_size <= 0 || k % group_size)
    return fail(TF_EINVAL, "tf_awq_quantize: K is not a multiple of group_size");
  const int64_t threads = (n / 8) * (k / group_size);
  if (threads == 0) return TF_OK;
  awq_quantize_kernel<<<(unsigned)cdiv(threads, 256), 256, 0, (hipStream_t)stream>>>(
      weight, n, k, group_size, reinterpret_cast<uint32_t*>(qweight), reinterpret_cast<uint32_t*>(qzeros), scales);
  return check_launch("tf_awq_quantize");
}
