// Load-time layout kernels: int4 pack/unpack, AWQ <-> TokenForge repack, full dequant.
//
// Repack is an 8x8 transpose of 4-bit values: the eight AWQ words qweight[8*kb + i][nb]
// (i = 0..7) hold exactly the same 64 values as the eight TokenForge words
// qweight_t[8*nb + j][kb] (j = 0..7). Each thread moves whole 8x8 blocks in registers
// (three masked-swap stages) and the tile is staged through LDS so that both the reads
// and the writes are 128-byte coalesced rows.
#include "tf_common.h"

namespace tf {
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

// qweight_t [n, k/8] -> out fp16 [n, k]; one thread per 4 packed words (32 values).
__global__ void dequant_kernel(const uint32_t* __restrict__ qw, const uint16_t* __restrict__ scales,
                               const uint32_t* __restrict__ qzeros, uint16_t* __restrict__ out,
                               int64_t n, int64_t k, int log2_group) {
  const int64_t chunks_per_row = k / 32;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * chunks_per_row) return;
  const int64_t row = i / chunks_per_row;
  const int64_t ch = i % chunks_per_row;
  const u4 words = *reinterpret_cast<const u4*>(qw + row * (k / 8) + ch * 4);
  const int64_t grp = (ch * 32) >> log2_group;
  const uint32_t zw = qzeros[grp * (n / 8) + row / 8];
  const QuantParams p = make_params(zero_of(zw, (uint32_t)row), scales[grp * n + row]);
  u4* dst = reinterpret_cast<u4*>(out + row * k + ch * 32);
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
