// ABI version, thread-local error reporting and the e4m3 encoder test hook.
#include <string>

#include "fp8.h"
#include "tf_common.h"

namespace tf {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return fail(TF_ELAUNCH, std::string(what) + ": " + hipGetErrorString(err));
  return TF_OK;
}

namespace {
__global__ void e4m3_encode_kernel(const float* __restrict__ in, uint8_t* __restrict__ out,
                                   int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) out[i] = e4m3_encode_hw(in[i]);
}
}  // namespace

}  // namespace tf

using namespace tf;

extern "C" int tf_abi_version(void) { return 7; }

extern "C" const char* tf_last_error(void) { return g_last_error.c_str(); }

extern "C" int tf_e4m3_encode(const float* in, uint8_t* out, int64_t count, void* stream) {
  if (in == nullptr || out == nullptr) return fail(TF_EINVAL, "tf_e4m3_encode: null pointer");
  if (count < 0) return fail(TF_EINVAL, "tf_e4m3_encode: negative count");
  if (count == 0) return TF_OK;
  e4m3_encode_kernel<<<(unsigned)cdiv(count, 256), 256, 0, (hipStream_t)stream>>>(in, out, count);
  return check_launch("tf_e4m3_encode");
}
