// Memory-system probes behind the GEMV's cost model (bench.py --probe): pure-read kernels with
// the decode GEMV's grid, wave split, ring depth and access pattern, and no arithmetic, so
// their time is the floor the memory system sets for that pattern. Built into a library of its
// own (bench_probes/lib/libtokenforge_read_probes.so); the product library never contains or
// calls them.
//
// Patterns (all loads are 128-bit buffer loads; a lane XORs what it loads and writes one word):
//   0 tile:    tile layout. A workgroup owns one 16-row tile, its waves split the tile's
//              128-wide K steps; a wave step reads the step's contiguous 1 KB (lane l at 16 l).
//   1 tile+meta: as 0, plus per step the 32-bit scales word and zero-point word of the lane's
//              column in the tile layout (the GEMV's three loads per step).
//   2 rows:    the TokenForge layout: lane (row l / 4, chunk l % 4) reads 16 bytes of each of the
//              tile's 16 rows per step (16 runs of 64 bytes per instruction).
//   3 stream:  a plain grid-stride read of the whole buffer, 16 bytes per lane per load.
//   4 wave:    the weights as the linear sequence of 1 KB step blocks they are in the tile layout
//              (tile-major, step-minor; full tiles), each wave streaming its own contiguous range;
//   5 group:   each workgroup owns a contiguous range of blocks and its waves take them round
//              robin (neighbouring blocks in flight: the GEMV stream form's pattern);
//   6 grid:    the whole grid takes the blocks round robin.
//   Patterns 4-6 also read each block's 32-byte scale group and 8-byte zero group as the GEMV
//   does (a 32-bit word per lane), on a grid of their own (workgroups x waves x ring depth).
// The empty kernel measures the fixed cost of one launch inside a graph.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__global__ void empty_kernel() {}

template <int P, int PATTERN>
__global__ __launch_bounds__(1024) void tile_read_kernel(const void* w, uint32_t w_bytes, const void* sc,
                                                         uint32_t sc_bytes, const void* qz, uint32_t qz_bytes,
                                                         int q_total, int groups, uint32_t* out) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int waves = blockDim.x >> 6;
  // Workgroup b runs on XCD b % 8: give each XCD a contiguous range of tiles, as the GEMV does.
  const int nb = gridDim.x, b = blockIdx.x, q = nb / 8, r = nb % 8, x = b % 8;
  const int t = x * q + (x < r ? x : r) + b / 8;
  const int nsteps = (q_total + 3) >> 2;
  const int s0 = (wave * nsteps) / waves, s1 = ((wave + 1) * nsteps) / waves;
  const __amdgpu_buffer_rsrc_t rw = rsrc(w, w_bytes), rs = rsrc(sc, sc_bytes), rz = rsrc(qz, qz_bytes);
  const int c = lane & 15, g = lane >> 4;
  uint32_t base;
  if (PATTERN == 2)  // row (lane / 4) of the tile, chunk lane % 4
    base = (uint32_t)((16 * t + (lane >> 2)) * q_total + (lane & 3)) * 16u;
  else
    base = (uint32_t)(t * q_total * 16) * 16u + (uint32_t)lane * 16u;
  const uint32_t step_bytes = PATTERN == 2 ? 64u : 1024u;
  const uint32_t soff = (uint32_t)(t * 16 * groups + (c & ~1)) * 2u;
  const uint32_t zoff = (uint32_t)(t * 2 * groups + (c >> 3)) * 4u;
  (void)g;
  u4 acc = {0u, 0u, 0u, 0u};
  u4 ring[P];
  uint32_t sring[P], zring[P];
  auto issue = [&](int p, int s) {
    const bool in = s < s1;
    ring[p] = __builtin_amdgcn_raw_buffer_load_b128(rw, in ? (int)(base + (uint32_t)s * step_bytes) : (int)0x80000000, 0, 0);
    if (PATTERN == 1) {
      sring[p] = __builtin_amdgcn_raw_buffer_load_b32(rs, in ? (int)(soff + (uint32_t)s * 32u) : (int)0x80000000, 0, 0);
      zring[p] = __builtin_amdgcn_raw_buffer_load_b32(rz, in ? (int)(zoff + (uint32_t)s * 8u) : (int)0x80000000, 0, 0);
    }
  };
#pragma unroll
  for (int p = 0; p < P; ++p) issue(p, s0 + p);
  for (int s = s0; s < s1; s += P) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      acc ^= ring[p];
      if (PATTERN == 1) acc[0] ^= sring[p] ^ zring[p];
      issue(p, s + p + P);
    }
  }
  out[(size_t)b * blockDim.x + threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

__global__ __launch_bounds__(256) void stream_read_kernel(const u4* __restrict__ w, size_t chunks, uint32_t* out) {
  u4 acc = {0u, 0u, 0u, 0u};
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < chunks; i += stride) acc ^= w[i];
  out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

// Patterns 4-6 over nblk 1 KB blocks (plus 32-byte scale and 8-byte zero groups per block).
template <int P, int MODE>
__global__ __launch_bounds__(1024) void block_read_kernel(const void* w, const void* sc, const void* qz, int nblk,
                                                          uint32_t* out) {
  const int lane = threadIdx.x & 63;
  const int W = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int V = gridDim.x * W;
  const int v = blockIdx.x * W + wave;
  int i0, i1, di;
  if (MODE == 0) {  // each wave its own contiguous range
    i0 = (int)((int64_t)nblk * v / V);
    i1 = (int)((int64_t)nblk * (v + 1) / V);
    di = 1;
  } else if (MODE == 1) {  // workgroup range, waves round robin inside it
    i0 = (int)((int64_t)nblk * blockIdx.x / gridDim.x) + wave;
    i1 = (int)((int64_t)nblk * (blockIdx.x + 1) / gridDim.x);
    di = W;
  } else {  // whole grid round robin
    i0 = v;
    i1 = nblk;
    di = V;
  }
  const uint32_t wb = (uint32_t)nblk * 1024u, sb = (uint32_t)nblk * 32u, zb = (uint32_t)nblk * 8u;
  const int c = lane & 15;
  u4 acc = {0u, 0u, 0u, 0u};
  u4 rw[P];
  uint32_t rs[P], rz[P];
  auto issue = [&](int p, int i) {
    const bool in = i < i1;
    const int ii = in ? i : 0;
    rw[p] = __builtin_amdgcn_raw_buffer_load_b128(rsrc(w, in ? wb : 0u), lane * 16, ii * 1024, 0);
    rs[p] = __builtin_amdgcn_raw_buffer_load_b32(rsrc(sc, in ? sb : 0u), (c & ~1) * 2, ii * 32, 0);
    rz[p] = __builtin_amdgcn_raw_buffer_load_b32(rsrc(qz, in ? zb : 0u), (c >> 3) * 4, ii * 8, 0);
  };
#pragma unroll
  for (int p = 0; p < P; ++p) issue(p, i0 + p * di);
  for (int s = i0; s < i1; s += P * di) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      acc ^= rw[p];
      acc[0] ^= rs[p] ^ rz[p];
      issue(p, s + (p + P) * di);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

template <int P, int PATTERN>
int launch_tile(const void* w, int64_t n, int64_t k, int64_t groups, const void* sc, const void* qz, int waves,
                uint32_t* out, hipStream_t stream) {
  const int tiles = (int)(n / 16);
  tile_read_kernel<P, PATTERN><<<tiles, waves * 64, 0, stream>>>(
      w, (uint32_t)(n * k / 2), sc, (uint32_t)(groups * n * 2), qz, (uint32_t)(groups * n / 2), (int)(k / 32),
      (int)groups, out);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // namespace

// Bytes of `out` a tile-pattern launch writes: one word per thread.
extern "C" int64_t tfp_out_words(int64_t n, int waves) { return (n / 16) * waves * 64; }

// Pure-read probe. pattern: 0 tile, 1 tile + scales/zeros, 2 rows (TokenForge layout),
// 3 grid-stride stream (waves = workgroups of 256 threads, depth unused). n % 16 == 0,
// k % 128 == 0 for patterns 0-2; the buffers hold n * k / 2 bytes of weights, k / 128 * n fp16
// scales and k / 128 * n / 8 zero words. out: tfp_out_words(n, waves) words (pattern 3:
// waves * 256 words). Returns 0, 1 (bad arguments) or 2 (launch error).
extern "C" int tfp_read(int pattern, const void* w, const void* sc, const void* qz, int64_t n, int64_t k,
                        int waves, int depth, uint32_t* out, void* stream) {
  const hipStream_t s = (hipStream_t)stream;
  if (!w || !out || n <= 0 || k <= 0) return 1;
  if (pattern == 3) {
    stream_read_kernel<<<waves, 256, 0, s>>>(reinterpret_cast<const u4*>(w), (size_t)(n * k / 32), out);
    return hipGetLastError() == hipSuccess ? 0 : 2;
  }
  if (n % 16 || k % 128 || waves < 1 || waves > 16 || !sc || !qz) return 1;
  const int64_t groups = k / 128;
  switch (pattern * 16 + depth) {
    case 0 * 16 + 2: return launch_tile<2, 0>(w, n, k, groups, sc, qz, waves, out, s);
    case 0 * 16 + 4: return launch_tile<4, 0>(w, n, k, groups, sc, qz, waves, out, s);
    case 0 * 16 + 8: return launch_tile<8, 0>(w, n, k, groups, sc, qz, waves, out, s);
    case 1 * 16 + 2: return launch_tile<2, 1>(w, n, k, groups, sc, qz, waves, out, s);
    case 1 * 16 + 4: return launch_tile<4, 1>(w, n, k, groups, sc, qz, waves, out, s);
    case 1 * 16 + 8: return launch_tile<8, 1>(w, n, k, groups, sc, qz, waves, out, s);
    case 2 * 16 + 2: return launch_tile<2, 2>(w, n, k, groups, sc, qz, waves, out, s);
    case 2 * 16 + 4: return launch_tile<4, 2>(w, n, k, groups, sc, qz, waves, out, s);
    case 2 * 16 + 8: return launch_tile<8, 2>(w, n, k, groups, sc, qz, waves, out, s);
    default: return 1;
  }
}

// One empty kernel launch (grid x 64 threads): the fixed cost of a launch.
extern "C" int tfp_empty(int grid, void* stream) {
  empty_kernel<<<grid, 64, 0, (hipStream_t)stream>>>();
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Patterns 4-6 (see above) on a grid of `grid` workgroups of `waves` waves with a ring of
// `depth` blocks (2 or 4). n % 16 == 0, k % 128 == 0; the buffers as for tfp_read. out:
// grid * waves * 64 words. Returns 0, 1 (bad arguments) or 2 (launch error).
extern "C" int tfp_read_blocks(int pattern, const void* w, const void* sc, const void* qz, int64_t n, int64_t k,
                               int grid, int waves, int depth, uint32_t* out, void* stream) {
  const hipStream_t s = (hipStream_t)stream;
  if (!w || !sc || !qz || !out || n <= 0 || k <= 0 || n % 16 || k % 128 || grid < 1 || waves < 1 || waves > 16)
    return 1;
  const int nblk = (int)(n / 16 * (k / 128));
  const dim3 g(grid), b(waves * 64);
  switch (pattern * 16 + depth) {
    case 4 * 16 + 2: block_read_kernel<2, 0><<<g, b, 0, s>>>(w, sc, qz, nblk, out); break;
    case 4 * 16 + 4: block_read_kernel<4, 0><<<g, b, 0, s>>>(w, sc, qz, nblk, out); break;
    case 5 * 16 + 2: block_read_kernel<2, 1><<<g, b, 0, s>>>(w, sc, qz, nblk, out); break;
    case 5 * 16 + 4: block_read_kernel<4, 1><<<g, b, 0, s>>>(w, sc, qz, nblk, out); break;
    case 6 * 16 + 2: block_read_kernel<2, 2><<<g, b, 0, s>>>(w, sc, qz, nblk, out); break;
    case 6 * 16 + 4: block_read_kernel<4, 2><<<g, b, 0, s>>>(w, sc, qz, nblk, out); break;
    default: return 1;
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
