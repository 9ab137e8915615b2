// tf_w4a16_linear_ex_noalloc: tf_w4a16_linear_ex for callers that cannot allocate.
//
// The kernels that need a workspace (split-K partials of the GEMMs, the fp32 rows the LDS-tile
// GEMMs reduce a SiLU*mul epilogue through) get it from `scratch`, a fixed device array of
// kScratchBytes that every GPU the library runs on holds until the process ends. Nothing here
// calls hipMalloc, hipFree or any allocating routine. The array's device address is looked up
// once per device (hipGetSymbolAddress, with that device current) on the entry point's first
// call there and kept per device; host code only ever passes that address, never the array's
// name (which on the host is a stand-in, not a device address).
//
// The kernels write every workspace element they later read, so nothing has to be cleared
// between calls. All calls on one GPU share its array: calls that overlap in time on one GPU
// (different streams, or a second host thread) race and must be serialized by the caller.
#include <mutex>

#include "linear.h"

namespace {

constexpr int64_t kScratchBytes = int64_t(32) << 20;  // 32 MiB per device

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up once per device).
int scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return tf::fail(TF_ELAUNCH, "tf_w4a16_linear_ex_noalloc: no current HIP device");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (rc != hipSuccess || p == nullptr)
      return tf::fail(TF_ELAUNCH, std::string("tf_w4a16_linear_ex_noalloc: hipGetSymbolAddress(scratch) failed: ") +
                                      hipGetErrorString(rc));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TF_OK;
}

}  // namespace

extern "C" int64_t tf_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" int tf_w4a16_linear_ex_noalloc(const uint16_t* x, int64_t ldx, const int32_t* qweight_t,
                                          const uint16_t* scales, const int32_t* qzeros, const uint16_t* bias,
                                          uint16_t* out, int64_t ldo, int64_t m, int64_t n, int64_t k,
                                          int32_t group_size, const tf_gemm_config* cfg, int32_t epilogue,
                                          const uint16_t* residual, int64_t ldr, void* stream) {
  if (cfg == nullptr) return tf::fail(TF_EINVAL, "tf_w4a16_linear_ex_noalloc: null config");
  const int64_t need = tf_w4a16_workspace_bytes_ex(m, n, k, group_size, cfg, epilogue);
  if (need > kScratchBytes)
    return tf::fail(TF_EINVAL, "tf_w4a16_linear_ex_noalloc: this call needs " + std::to_string(need) +
                                   " bytes of workspace, above the fixed " + std::to_string(kScratchBytes) +
                                   " (use tf_w4a16_linear_ex with a caller workspace, or a smaller split_k)");
  void* ws = nullptr;
  if (need > 0)
    if (int rc = scratch_address(&ws)) return rc;
  return tf_w4a16_linear_ex(x, ldx, qweight_t, scales, qzeros, bias, out, ldo, m, n, k, group_size, cfg, epilogue,
                            residual, ldr, static_cast<float*>(ws), need, stream);
}
