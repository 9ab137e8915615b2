// LDS bank-conflict probe (measurement only, not part of the library): pattern p gives each of
// the 64 lanes of one wave a 16-byte-aligned address in a 16 KB LDS region; dispatch p reads
// (mode 0) or writes (mode 1) 16 bytes per lane at those addresses 16 times. The patterns come
// from a binary file of uint32 records (mode, a[0..63]) that bench_probes/lds_bank_probe.py
// writes; every address is masked into the region, so no access leaves it. Run under
// rocprofv3 --pmc SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT, one dispatch per pattern in file order.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <vector>

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kReps = 16;

__global__ __launch_bounds__(64) void lds_pattern(const uint32_t* __restrict__ addrs, int mode,
                                                  uint32_t* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) uint32_t lds[4096];  // 16 KB
  for (int i = threadIdx.x; i < 4096; i += 64) lds[i] = i * 2654435761u;
  __syncthreads();
  const int l = threadIdx.x;
  const uint32_t a = addrs[l] & 16368u;  // 16-byte aligned, inside the 16 KB
  u4* p = reinterpret_cast<u4*>(reinterpret_cast<uint8_t*>(lds) + a);
  u4 acc = {(uint32_t)l, 1u, 2u, 3u};
  if (mode == 0) {
    for (int rep = 0; rep < kReps; ++rep) {
      acc ^= *p;
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): one LDS access in flight
    }
  } else {
    for (int rep = 0; rep < kReps; ++rep) {
      *p = acc;
      acc += u4{1u, 1u, 1u, 1u};
      __builtin_amdgcn_s_waitcnt(0xC07F);
    }
  }
  __syncthreads();
  out[l] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3] ^ lds[l];
}

int main(int argc, char** argv) {
  if (argc < 2) {
    std::printf("usage: lds_bank_probe PATTERNS.bin\n");
    return 1;
  }
  FILE* f = std::fopen(argv[1], "rb");
  if (!f) {
    std::printf("cannot open %s\n", argv[1]);
    return 1;
  }
  std::vector<uint32_t> rec(65);
  std::vector<std::vector<uint32_t>> pats;
  while (std::fread(rec.data(), 4, 65, f) == 65) pats.push_back(rec);
  std::fclose(f);
  if (pats.empty()) return 1;
  uint32_t *d_addr = nullptr, *d_out = nullptr;
  if (hipMalloc(&d_addr, pats.size() * 64 * 4) != hipSuccess || hipMalloc(&d_out, 64 * 4) != hipSuccess) return 2;
  for (size_t i = 0; i < pats.size(); ++i)
    if (hipMemcpy(d_addr + i * 64, pats[i].data() + 1, 64 * 4, hipMemcpyHostToDevice) != hipSuccess) return 3;
  for (size_t i = 0; i < pats.size(); ++i) lds_pattern<<<1, 64>>>(d_addr + i * 64, (int)pats[i][0], d_out);
  if (hipDeviceSynchronize() != hipSuccess) return 4;
  std::printf("lds_bank_probe: %zu patterns\n", pats.size());
  return 0;
}
