// The gfx950 tile layout of a W4A16 layer: where pack_awq puts qweight_t, scales and qzeros.
//
// Every tensor keeps the shape and dtype of the reference's TokenForge layout (qweight_t
// int32 [N, K/8], scales fp16 [K/G, N], qzeros int32 [K/G, N/8]); only element positions
// change. Rows (output columns) are grouped in tiles of 16: tile t holds rows 16t..16t+r_t-1,
// r_t = min(16, N - 16t) (16, or 8 for a last tile of an N that is 8 mod 16).
//
// qweight_t is moved in 16-byte chunks. Chunk (n, q) is the reference layout's words
// 4q..4q+3 of row n: 32 consecutive K values (K offsets 32q..32q+31, AWQ nibble order inside
// each word, words in K order), unchanged. With Q = K/32 chunks per row, j = q / 4 (the
// 128-wide K step) and g = q % 4 (the chunk inside the step), chunk (n, q) sits at chunk index
//
//     16 t Q  +  4 r_t j  +  g r_t  +  c          (t = n / 16, c = n % 16)
//
// i.e. a tile keeps its rows' region of the reference layout, and inside it each 128-wide K
// step is one contiguous block (1 KB for a full tile) ordered chunk-major. Lane l = 16 g + c of
// a wave therefore reads bytes 16 l .. 16 l + 15 of a step block: one wave instruction reads
// one whole 1 KB block (two full 128-byte lines per 16 lanes), and each lane's 16 bytes are
// exactly the B operand of four v_mfma_f32_16x16x32_f16 (lane = column c % 16, K block g).
// A last step shorter than 128 (K = 32, 64 or 96 mod 128) has n_g = Q - 4j chunks per row,
// ordered the same way (block of r_t n_g chunks).
//
// scales: element (p, n) (group p, row n) sits at  16 t P + p r_t + c   (P = K/G groups):
// tile-major, each group's r_t scales contiguous, the tile's groups consecutive.
// qzeros: word (p, w) (group p, rows 8w..8w+7, AWQ nibble order, content unchanged) sits at
// 2 t P + p (r_t / 8) + (w - 2t)   with t = w / 2.
//
// Each map is a bijection on its tensor's index range (the inverse functions below).
#pragma once

#include <stdint.h>

namespace tf {

__host__ __device__ __forceinline__ int64_t tile_rows(int64_t n_total, int64_t t) {
  const int64_t r = n_total - 16 * t;
  return r < 16 ? r : 16;
}

// Chunk index of chunk q (K offsets 32q..32q+31) of row n; q_total = K / 32.
__host__ __device__ __forceinline__ int64_t tile_chunk(int64_t n, int64_t q, int64_t n_total, int64_t q_total) {
  const int64_t t = n >> 4, c = n & 15, rt = tile_rows(n_total, t);
  const int64_t j = q >> 2, g = q & 3;
  return 16 * t * q_total + 4 * rt * j + g * rt + c;
}

// Inverse of tile_chunk: the (row, chunk) stored at chunk index pos.
__host__ __device__ __forceinline__ void tile_chunk_source(int64_t pos, int64_t n_total, int64_t q_total,
                                                           int64_t* n, int64_t* q) {
  const int64_t t = pos / (16 * q_total);
  const int64_t rt = tile_rows(n_total, t);
  const int64_t e = pos - 16 * t * q_total;
  const int64_t j = e / (4 * rt);
  const int64_t f = e - 4 * rt * j;
  const int64_t g = f / rt;
  *n = 16 * t + (f - g * rt);
  *q = 4 * j + g;
}

// Element index of scale (group p, row n); p_total = K / G.
__host__ __device__ __forceinline__ int64_t tile_scale(int64_t p, int64_t n, int64_t n_total, int64_t p_total) {
  const int64_t t = n >> 4;
  return 16 * t * p_total + p * tile_rows(n_total, t) + (n & 15);
}

__host__ __device__ __forceinline__ void tile_scale_source(int64_t pos, int64_t n_total, int64_t p_total,
                                                           int64_t* p, int64_t* n) {
  const int64_t t = pos / (16 * p_total);
  const int64_t rt = tile_rows(n_total, t);
  const int64_t e = pos - 16 * t * p_total;
  *p = e / rt;
  *n = 16 * t + (e - *p * rt);
}

// Word index of zero-point word (group p, word w = rows 8w..8w+7).
__host__ __device__ __forceinline__ int64_t tile_zero(int64_t p, int64_t w, int64_t n_total, int64_t p_total) {
  const int64_t t = w >> 1;
  const int64_t words = tile_rows(n_total, t) >> 3;
  return 2 * t * p_total + p * words + (w - 2 * t);
}

__host__ __device__ __forceinline__ void tile_zero_source(int64_t pos, int64_t n_total, int64_t p_total,
                                                          int64_t* p, int64_t* w) {
  const int64_t t = pos / (2 * p_total);
  const int64_t words = tile_rows(n_total, t) >> 3;
  const int64_t e = pos - 2 * t * p_total;
  *p = e / words;
  *w = 2 * t + (e - *p * words);
}

}  // namespace tf
