// The GPU kernels of the torch.ops.tokenforge operators, registered with the PyTorch
// dispatcher in C++: the launch path of a call costs a few microseconds of host time instead
// of the tens that a Python operator body, its checks and a ctypes call cost.
//
// Schemas are those of the reference's ops (ops.py:48-156) and of this build's fused forms.
// Each CUDA (HIP) kernel here is a fast path for the calls that need nothing but a launch:
//
//   * the call's shape, dtypes, devices and layout are the ones the kernels take directly
//     (anything else -- a bad argument to report, a tensor to copy, an empty input -- goes to
//     the operator's Python body, registered as tokenforge::_py_<op>, which raises the
//     reference's exceptions or handles the case and launches the same kernels);
//   * the launch config of (op, epilogue, M, N, K, group size, device) is resolved once by the
//     Python resolver tokenforge::_resolve_launch (bucket, autotune lookup, the per-M rules of
//     the dispatch, the device check) and kept here until the autotune cache changes
//     (tokenforge::_clear_launch_cache);
//   * the dispatch counter (tokenforge_kernel_calls_total{kernel,bucket}) is counted here,
//     atomically, and folded into the Python counter when that is read.
//
// The kernels are the C ABI of libtokenforge_hip.so, bound at run time by
// tokenforge::_bind_library(path) to the library the Python side loaded (one copy per process).

#include <ATen/ATen.h>
#include <ATen/core/dispatch/Dispatcher.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <dlfcn.h>
#include <torch/library.h>

#include <array>
#include <atomic>
#include <cstdint>
#include <mutex>
#include <shared_mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/tokenforge_hip.h"

namespace {

// ----------------------------------------------------------------------------- the C ABI

struct Api {
  decltype(&tf_w4a16_linear_ex) linear = nullptr;
  decltype(&tf_w4a8_linear_ex) w4a8 = nullptr;
  decltype(&tf_rmsnorm_fp8_quant_ex) norm = nullptr;
  decltype(&tf_rmsnorm_fp8_w4a16_linear) norm_linear = nullptr;
  decltype(&tf_last_error) last_error = nullptr;
};

std::mutex g_bind_mutex;
Api g_api;
std::atomic<bool> g_bound{false};

template <typename F>
void bind_symbol(void* handle, const char* name, F& slot) {
  void* p = dlsym(handle, name);
  TORCH_CHECK(p != nullptr, "tokenforge: the kernel library has no symbol ", name);
  slot = reinterpret_cast<F>(p);
}

void bind_library(c10::string_view path) {
  std::lock_guard<std::mutex> lock(g_bind_mutex);
  const std::string p(path);
  void* handle = dlopen(p.c_str(), RTLD_NOW | RTLD_LOCAL);
  TORCH_CHECK(handle != nullptr, "tokenforge: cannot load ", p, ": ", dlerror());
  Api api;
  bind_symbol(handle, "tf_w4a16_linear_ex", api.linear);
  bind_symbol(handle, "tf_w4a8_linear_ex", api.w4a8);
  bind_symbol(handle, "tf_rmsnorm_fp8_quant_ex", api.norm);
  bind_symbol(handle, "tf_rmsnorm_fp8_w4a16_linear", api.norm_linear);
  bind_symbol(handle, "tf_last_error", api.last_error);
  g_api = api;
  g_bound.store(true, std::memory_order_release);
}

const Api& api() {
  TORCH_CHECK(g_bound.load(std::memory_order_acquire),
              "tokenforge: the kernel library is not bound (import tokenforge.kernels.ops)");
  return g_api;
}

// A tf_* status as the exception the Python launchers raise for it.
void check(int rc, const char* what) {
  if (rc == TF_OK) return;
  const char* msg = api().last_error();
  const std::string text = (msg != nullptr && msg[0] != '\0') ? std::string(msg) : std::string(what);
  if (rc == TF_EINVAL || rc == TF_ERANGE) TORCH_CHECK_VALUE(false, text);
  TORCH_CHECK(false, text);
}

// ----------------------------------------------------------------------------- launch configs

enum Kind : int64_t { kLinear = 0, kW4A8 = 1, kNormLinear = 2 };

struct Key {
  int64_t kind, epilogue, m, n, k, group, device;
  bool operator==(const Key& o) const {
    return kind == o.kind && epilogue == o.epilogue && m == o.m && n == o.n && k == o.k && group == o.group &&
           device == o.device;
  }
};

struct KeyHash {
  size_t operator()(const Key& key) const {
    uint64_t h = 1469598103934665603ull;
    for (int64_t v : {key.kind, key.epilogue, key.m, key.n, key.k, key.group, key.device}) {
      h ^= static_cast<uint64_t>(v);
      h *= 1099511628211ull;
    }
    return static_cast<size_t>(h);
  }
};

// What the resolver decided for one key (the order of its int[] result).
struct Launch {
  tf_gemm_config cfg;
  int64_t family;  // counter label: 0 hip_gemv, 1 hip_gemm
  int64_t bucket;  // index of the counter's bucket label
  int64_t need;    // workspace bytes
  int64_t fused;   // kNormLinear: 1 when the GEMV's prologue runs the norm (one launch)
};
constexpr size_t kLaunchFields = 11;

std::shared_mutex g_cache_mutex;
std::unordered_map<Key, Launch, KeyHash> g_cache;

constexpr int kFamilies = 2;
constexpr int kBuckets = 64;
std::array<std::atomic<int64_t>, kFamilies * kBuckets> g_calls{};

Launch resolve(const Key& key) {
  {
    std::shared_lock<std::shared_mutex> lock(g_cache_mutex);
    auto it = g_cache.find(key);
    if (it != g_cache.end()) return it->second;
  }
  static auto op = c10::Dispatcher::singleton()
                       .findSchemaOrThrow("tokenforge::_resolve_launch", "")
                       .typed<std::vector<int64_t>(int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t)>();
  const std::vector<int64_t> r = op.call(key.kind, key.epilogue, key.m, key.n, key.k, key.group, key.device);
  TORCH_CHECK(r.size() == kLaunchFields, "tokenforge::_resolve_launch returned ", r.size(), " fields");
  Launch l;
  l.cfg = tf_gemm_config{static_cast<int32_t>(r[0]), static_cast<int32_t>(r[1]), static_cast<int32_t>(r[2]),
                         static_cast<int32_t>(r[3]), static_cast<int32_t>(r[4]), static_cast<int32_t>(r[5]),
                         static_cast<int32_t>(r[6])};
  l.family = r[7];
  l.bucket = r[8];
  l.need = r[9];
  l.fused = r[10];
  TORCH_CHECK(l.family >= 0 && l.family < kFamilies && l.bucket >= 0 && l.bucket < kBuckets,
              "tokenforge::_resolve_launch: counter label out of range");
  std::unique_lock<std::shared_mutex> lock(g_cache_mutex);
  g_cache.emplace(key, l);
  return l;
}

void count(const Launch& l) { g_calls[l.family * kBuckets + l.bucket].fetch_add(1, std::memory_order_relaxed); }

std::vector<int64_t> native_calls() {
  std::vector<int64_t> out(g_calls.size());
  for (size_t i = 0; i < g_calls.size(); ++i) out[i] = g_calls[i].load(std::memory_order_relaxed);
  return out;
}

void clear_launch_cache() {
  std::unique_lock<std::shared_mutex> lock(g_cache_mutex);
  g_cache.clear();
}

// ----------------------------------------------------------------------------- fast-path checks

bool backend_ok(c10::string_view b) { return b == "hip" || b == "triton" || b == "cuda"; }

int64_t epilogue_code(c10::string_view e) {
  if (e == "none") return TF_EPILOGUE_NONE;
  if (e == "residual") return TF_EPILOGUE_RESIDUAL;
  if (e == "silu_mul") return TF_EPILOGUE_SILU_MUL;
  return -1;
}

bool on(const at::Tensor& t, const c10::Device& dev) { return t.device() == dev; }

// The weights as the kernels read them: int32 qweight_t [N, K/8], fp16 scales [K/G, N], int32
// qzeros [K/G, N/8], all contiguous, on the device, K a multiple of G.
bool weights_ok(const at::Tensor& qw, const at::Tensor& sc, const at::Tensor& qz, int64_t k, int64_t g,
                const c10::Device& dev) {
  if (g <= 0 || qw.dim() != 2 || sc.dim() != 2 || qz.dim() != 2) return false;
  const int64_t n = qw.size(0);
  if (qw.size(1) * 8 != k || k % g != 0 || n % 8 != 0) return false;
  if (sc.size(0) != k / g || sc.size(1) != n || qz.size(0) != k / g || qz.size(1) != n / 8) return false;
  if (qw.scalar_type() != at::kInt || qz.scalar_type() != at::kInt || sc.scalar_type() != at::kHalf) return false;
  if (!qw.is_contiguous() || !sc.is_contiguous() || !qz.is_contiguous()) return false;
  return on(qw, dev) && on(sc, dev) && on(qz, dev);
}

bool bias_ok(const std::optional<at::Tensor>& bias, int64_t n, const c10::Device& dev) {
  if (!bias.has_value()) return true;
  const at::Tensor& b = *bias;
  return b.dim() == 1 && b.size(0) == n && b.scalar_type() == at::kHalf && b.is_contiguous() && on(b, dev);
}

// x with 16-byte aligned rows (the kernels use 128-bit loads); a copy only when needed.
at::Tensor aligned_rows(const at::Tensor& x) {
  const auto addr = reinterpret_cast<uintptr_t>(x.data_ptr());
  if (addr % 16 == 0 && (x.size(0) <= 1 || x.stride(0) % 8 == 0)) return x;
  return x.clone(at::MemoryFormat::Contiguous);
}

const void* ptr_or_null(const std::optional<at::Tensor>& t) { return t.has_value() ? t->data_ptr() : nullptr; }

template <typename T>
T* data(const at::Tensor& t) {
  return static_cast<T*>(t.data_ptr());
}

std::vector<int64_t> with_last(at::IntArrayRef lead, int64_t last) {
  std::vector<int64_t> s(lead.begin(), lead.end());
  s.push_back(last);
  return s;
}

// The operator's Python body (tokenforge::_py_<name>, same schema), for every call the fast path
// does not take. F is the operator's C++ signature.
template <typename F, typename... Args>
decltype(auto) python_body(const char* name, Args&&... args) {
  static thread_local std::unordered_map<std::string, c10::TypedOperatorHandle<F>> ops;
  auto it = ops.find(name);
  if (it == ops.end())
    it = ops.emplace(name, c10::Dispatcher::singleton().findSchemaOrThrow(name, "").typed<F>()).first;
  return it->second.call(std::forward<Args>(args)...);
}

using LinearFn = at::Tensor(const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                            const std::optional<at::Tensor>&, c10::SymInt, c10::string_view);
using ResidualFn = at::Tensor(const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                              const std::optional<at::Tensor>&, const at::Tensor&, c10::SymInt, c10::string_view);
using W4A8Fn = at::Tensor(const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                          const at::Tensor&, const std::optional<at::Tensor>&, c10::SymInt, c10::string_view,
                          c10::string_view, const std::optional<at::Tensor>&);
using NormFn = std::tuple<at::Tensor, at::Tensor>(const at::Tensor&, const at::Tensor&, double,
                                                  const std::optional<at::Tensor>&);
using NormDqFn = std::tuple<at::Tensor, at::Tensor, at::Tensor>(const at::Tensor&, const at::Tensor&, double,
                                                                const std::optional<at::Tensor>&);
using NormLinearFn = at::Tensor(const at::Tensor&, const at::Tensor&, double, const at::Tensor&, const at::Tensor&,
                                const at::Tensor&, const std::optional<at::Tensor>&, c10::SymInt, c10::string_view,
                                c10::string_view);

// ----------------------------------------------------------------------------- W4A16 linear

// Returns an undefined tensor when the call is not for the fast path.
at::Tensor linear_fast(int64_t epi, const at::Tensor& x, const at::Tensor& qw, const at::Tensor& sc,
                       const at::Tensor& qz, const std::optional<at::Tensor>& bias,
                       const std::optional<at::Tensor>& residual, int64_t g, c10::string_view backend) {
  if (!backend_ok(backend) || x.dim() < 1 || qw.dim() != 2 || !x.is_cuda()) return {};
  const c10::Device dev = x.device();
  const int64_t k = x.size(-1), n = qw.size(0);
  at::Tensor x2 = x.reshape({-1, k});
  if (x2.stride(1) != 1) return {};
  const int64_t m = x2.size(0);
  if (m == 0 || n == 0 || x.scalar_type() != at::kHalf || !weights_ok(qw, sc, qz, k, g, dev) || !bias_ok(bias, n, dev))
    return {};
  if (epi == TF_EPILOGUE_SILU_MUL && n % 16 != 0) return {};
  at::Tensor r2;
  if (epi == TF_EPILOGUE_RESIDUAL) {
    const at::Tensor& r = *residual;
    if (r.scalar_type() != at::kHalf || !on(r, dev) || r.sizes() != at::IntArrayRef(with_last(x.sizes().slice(0, x.dim() - 1), n)))
      return {};
    r2 = r.reshape({-1, n});
    if (r2.stride(1) != 1) return {};
  }
  const Launch l = resolve(Key{kLinear, epi, m, n, k, g, dev.index()});
  count(l);
  c10::OptionalDeviceGuard guard(dev);
  x2 = aligned_rows(x2);
  const int64_t n_out = epi == TF_EPILOGUE_SILU_MUL ? n / 2 : n;
  at::Tensor out = at::empty({m, n_out}, x2.options());
  at::Tensor ws;
  if (l.need > 0) ws = at::empty({(std::max<int64_t>(l.need, 4) + 3) / 4}, x2.options().dtype(at::kFloat));
  const int64_t ldx = m > 1 ? x2.stride(0) : k;
  const int64_t ldr = r2.defined() ? (m > 1 ? r2.stride(0) : n) : 0;
  const int rc = api().linear(data<const uint16_t>(x2), ldx, data<const int32_t>(qw), data<const uint16_t>(sc),
                              data<const int32_t>(qz), static_cast<const uint16_t*>(ptr_or_null(bias)),
                              data<uint16_t>(out), n_out, m, n, k, static_cast<int32_t>(g), &l.cfg,
                              static_cast<int32_t>(epi), r2.defined() ? data<const uint16_t>(r2) : nullptr, ldr,
                              ws.defined() ? data<float>(ws) : nullptr, l.need,
                              c10::hip::getCurrentHIPStream(dev.index()).stream());
  check(rc, "tf_w4a16_linear_ex");
  return out.reshape(with_last(x.sizes().slice(0, x.dim() - 1), n_out));
}

at::Tensor w4a16_linear(const at::Tensor& x, const at::Tensor& qw, const at::Tensor& sc, const at::Tensor& qz,
                        const std::optional<at::Tensor>& bias, c10::SymInt group_size, c10::string_view backend) {
  const int64_t g = group_size.guard_int(__FILE__, __LINE__);
  at::Tensor y = linear_fast(TF_EPILOGUE_NONE, x, qw, sc, qz, bias, std::nullopt, g, backend);
  if (y.defined()) return y;
  return python_body<LinearFn>("tokenforge::_py_w4a16_linear", x, qw, sc, qz, bias, group_size, backend);
}

at::Tensor w4a16_linear_residual(const at::Tensor& x, const at::Tensor& qw, const at::Tensor& sc,
                                 const at::Tensor& qz, const std::optional<at::Tensor>& bias,
                                 const at::Tensor& residual, c10::SymInt group_size, c10::string_view backend) {
  const int64_t g = group_size.guard_int(__FILE__, __LINE__);
  at::Tensor y = linear_fast(TF_EPILOGUE_RESIDUAL, x, qw, sc, qz, bias, residual, g, backend);
  if (y.defined()) return y;
  return python_body<ResidualFn>("tokenforge::_py_w4a16_linear_residual", x, qw, sc, qz, bias, residual,
                                 group_size, backend);
}

at::Tensor w4a16_linear_silu_mul(const at::Tensor& x, const at::Tensor& qw, const at::Tensor& sc,
                                 const at::Tensor& qz, const std::optional<at::Tensor>& bias,
                                 c10::SymInt group_size, c10::string_view backend) {
  const int64_t g = group_size.guard_int(__FILE__, __LINE__);
  at::Tensor y = linear_fast(TF_EPILOGUE_SILU_MUL, x, qw, sc, qz, bias, std::nullopt, g, backend);
  if (y.defined()) return y;
  return python_body<LinearFn>("tokenforge::_py_w4a16_linear_silu_mul", x, qw, sc, qz, bias, group_size,
                                 backend);
}

// ----------------------------------------------------------------------------- W4A8 linear

at::Tensor w4a8_fast(const at::Tensor& x8, const at::Tensor& x_scale, const at::Tensor& qw, const at::Tensor& sc,
                     const at::Tensor& qz, const std::optional<at::Tensor>& bias, int64_t g,
                     c10::string_view backend, c10::string_view epilogue,
                     const std::optional<at::Tensor>& residual) {
  const int64_t epi = epilogue_code(epilogue);
  if (epi < 0 || !backend_ok(backend) || x8.dim() < 1 || qw.dim() != 2 || !x8.is_cuda()) return {};
  const c10::Device dev = x8.device();
  const int64_t k = x8.size(-1), n = qw.size(0);
  at::Tensor x2 = x8.reshape({-1, k});
  const int64_t m = x2.size(0);
  if (m == 0 || n == 0 || x8.scalar_type() != at::kFloat8_e4m3fn || !weights_ok(qw, sc, qz, k, g, dev) ||
      !bias_ok(bias, n, dev))
    return {};
  if (x_scale.scalar_type() != at::kFloat || !on(x_scale, dev) || (x_scale.numel() != 1 && x_scale.numel() != m))
    return {};
  if (epi == TF_EPILOGUE_SILU_MUL && n % 16 != 0) return {};
  if ((epi == TF_EPILOGUE_RESIDUAL) != residual.has_value()) return {};
  at::Tensor r2;
  if (residual.has_value()) {
    const at::Tensor& r = *residual;
    if (r.scalar_type() != at::kHalf || !on(r, dev) || r.numel() != m * n) return {};
    r2 = r.reshape({-1, n});
    if (r2.size(0) != m || r2.stride(1) != 1) return {};
  }
  const Launch l = resolve(Key{kW4A8, epi, m, n, k, g, dev.index()});
  count(l);
  c10::OptionalDeviceGuard guard(dev);
  const at::Tensor s2 = x_scale.reshape({-1}).contiguous();
  const int64_t xs_stride = s2.numel() == 1 ? 0 : 1;
  int64_t ldx8 = m > 1 ? x2.stride(0) : k;
  if (x2.stride(1) != 1 || ldx8 % 8 != 0 || reinterpret_cast<uintptr_t>(x2.data_ptr()) % 16 != 0) {
    x2 = x2.clone(at::MemoryFormat::Contiguous);
    ldx8 = k;
  }
  const int64_t n_out = epi == TF_EPILOGUE_SILU_MUL ? n / 2 : n;
  at::Tensor out = at::empty({m, n_out}, x2.options().dtype(at::kHalf));
  at::Tensor ws;
  if (l.need > 0) ws = at::empty({(std::max<int64_t>(l.need, 4) + 3) / 4}, x2.options().dtype(at::kFloat));
  const int64_t ldr = r2.defined() ? (m > 1 ? r2.stride(0) : n) : 0;
  const int rc = api().w4a8(data<const uint8_t>(x2), ldx8, data<const float>(s2), xs_stride, data<const int32_t>(qw),
                            data<const uint16_t>(sc), data<const int32_t>(qz),
                            static_cast<const uint16_t*>(ptr_or_null(bias)), data<uint16_t>(out), n_out, m, n, k,
                            static_cast<int32_t>(g), &l.cfg, static_cast<int32_t>(epi),
                            r2.defined() ? data<const uint16_t>(r2) : nullptr, ldr,
                            ws.defined() ? data<float>(ws) : nullptr, l.need,
                            c10::hip::getCurrentHIPStream(dev.index()).stream());
  check(rc, "tf_w4a8_linear_ex");
  return out.reshape(with_last(x8.sizes().slice(0, x8.dim() - 1), n_out));
}

at::Tensor w4a8_linear(const at::Tensor& x8, const at::Tensor& x_scale, const at::Tensor& qw, const at::Tensor& sc,
                       const at::Tensor& qz, const std::optional<at::Tensor>& bias, c10::SymInt group_size,
                       c10::string_view backend, c10::string_view epilogue,
                       const std::optional<at::Tensor>& residual) {
  const int64_t g = group_size.guard_int(__FILE__, __LINE__);
  at::Tensor y = w4a8_fast(x8, x_scale, qw, sc, qz, bias, g, backend, epilogue, residual);
  if (y.defined()) return y;
  return python_body<W4A8Fn>("tokenforge::_py_w4a8_linear", x8, x_scale, qw, sc, qz, bias, group_size, backend,
                             epilogue, residual);
}

// ----------------------------------------------------------------------------- RMSNorm + FP8

// (q, scale, dq) of the norm on a fast-path call; q undefined when the call is not one.
std::tuple<at::Tensor, at::Tensor, at::Tensor> norm_fast(const at::Tensor& x, const at::Tensor& w, double eps,
                                                         const std::optional<at::Tensor>& scale, bool dequant) {
  if (x.dim() < 1 || !x.is_cuda()) return {};
  const c10::Device dev = x.device();
  const int64_t h = x.size(-1);
  at::Tensor x2 = x.reshape({-1, h});
  if (x2.stride(1) != 1) return {};
  const int64_t t = x2.size(0);
  if (t == 0 || h == 0 || x.scalar_type() != at::kHalf || w.scalar_type() != at::kHalf || w.dim() != 1 ||
      w.size(0) != h || !w.is_contiguous() || !on(w, dev))
    return {};
  if (scale.has_value() && (scale->numel() != 1 || scale->scalar_type() != at::kFloat || !on(*scale, dev))) return {};
  c10::OptionalDeviceGuard guard(dev);
  at::Tensor q = at::empty({t, h}, x2.options().dtype(at::kFloat8_e4m3fn));
  at::Tensor s = scale.has_value() ? *scale : at::empty({t, 1}, x2.options().dtype(at::kFloat));
  at::Tensor dq = dequant ? at::empty({t, h}, x2.options()) : at::Tensor();
  const int64_t ldx = t > 1 ? x2.stride(0) : h;
  const int rc = api().norm(data<const uint16_t>(x2), ldx, data<const uint16_t>(w), data<uint8_t>(q), h,
                            data<float>(s), scale.has_value() ? 1 : 0, dequant ? data<uint16_t>(dq) : nullptr, h, t,
                            h, static_cast<float>(eps), TF_NORM_AUTO,
                            c10::hip::getCurrentHIPStream(dev.index()).stream());
  check(rc, "tf_rmsnorm_fp8_quant_ex");
  const auto lead = x.sizes().slice(0, x.dim() - 1);
  at::Tensor s_out = scale.has_value() ? s.clone() : s.reshape(with_last(lead, 1));
  return {q.reshape(x.sizes()), s_out, dequant ? dq.reshape(x.sizes()) : at::Tensor()};
}

std::tuple<at::Tensor, at::Tensor> rmsnorm_fp8_quant(const at::Tensor& x, const at::Tensor& w, double eps,
                                                     const std::optional<at::Tensor>& scale) {
  auto r = norm_fast(x, w, eps, scale, false);
  if (std::get<0>(r).defined()) return {std::get<0>(r), std::get<1>(r)};
  return python_body<NormFn>("tokenforge::_py_rmsnorm_fp8_quant", x, w, eps, scale);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> rmsnorm_fp8_quant_dequant(const at::Tensor& x, const at::Tensor& w,
                                                                         double eps,
                                                                         const std::optional<at::Tensor>& scale) {
  auto r = norm_fast(x, w, eps, scale, true);
  if (std::get<0>(r).defined()) return r;
  return python_body<NormDqFn>("tokenforge::_py_rmsnorm_fp8_quant_dequant", x, w, eps, scale);
}

// ----------------------------------------------------------------------------- norm + linear

at::Tensor norm_linear_fast(const at::Tensor& x, const at::Tensor& nw, double eps, const at::Tensor& qw,
                            const at::Tensor& sc, const at::Tensor& qz, const std::optional<at::Tensor>& bias,
                            int64_t g, c10::string_view backend, c10::string_view epilogue) {
  const int64_t epi = epilogue_code(epilogue);
  if ((epi != TF_EPILOGUE_NONE && epi != TF_EPILOGUE_SILU_MUL) || !backend_ok(backend) || x.dim() < 1 ||
      qw.dim() != 2 || !x.is_cuda())
    return {};
  const c10::Device dev = x.device();
  const int64_t k = x.size(-1), n = qw.size(0);
  at::Tensor x2 = x.reshape({-1, k});
  if (x2.stride(1) != 1) return {};
  const int64_t m = x2.size(0);
  if (m == 0 || n == 0 || x.scalar_type() != at::kHalf || !weights_ok(qw, sc, qz, k, g, dev) || !bias_ok(bias, n, dev))
    return {};
  if (nw.scalar_type() != at::kHalf || nw.dim() != 1 || nw.size(0) != k || !nw.is_contiguous() || !on(nw, dev))
    return {};
  if (epi == TF_EPILOGUE_SILU_MUL && n % 16 != 0) return {};
  const Launch l = resolve(Key{kNormLinear, epi, m, n, k, g, dev.index()});
  count(l);
  c10::OptionalDeviceGuard guard(dev);
  const int64_t n_out = epi == TF_EPILOGUE_SILU_MUL ? n / 2 : n;
  const auto out_shape = with_last(x.sizes().slice(0, x.dim() - 1), n_out);
  const hipStream_t stream = c10::hip::getCurrentHIPStream(dev.index()).stream();
  at::Tensor out = at::empty({m, n_out}, x2.options());
  if (l.fused) {
    x2 = aligned_rows(x2);
    const at::Tensor w = reinterpret_cast<uintptr_t>(nw.data_ptr()) % 16 == 0 ? nw : nw.clone();
    const int64_t ldx = m > 1 ? x2.stride(0) : k;
    const int rc = api().norm_linear(data<const uint16_t>(x2), ldx, data<const uint16_t>(w), static_cast<float>(eps),
                                     data<const int32_t>(qw), data<const uint16_t>(sc), data<const int32_t>(qz),
                                     static_cast<const uint16_t*>(ptr_or_null(bias)), data<uint16_t>(out), n_out, m,
                                     n, k, static_cast<int32_t>(g), &l.cfg, static_cast<int32_t>(epi), stream);
    check(rc, "tf_rmsnorm_fp8_w4a16_linear");
    return out.reshape(out_shape);
  }
  // The norm kernel writes fp16(q * scale), then the linear reads it.
  at::Tensor q = at::empty({m, k}, x2.options().dtype(at::kFloat8_e4m3fn));
  at::Tensor s = at::empty({m, 1}, x2.options().dtype(at::kFloat));
  at::Tensor a = at::empty({m, k}, x2.options());
  const int64_t ldx = m > 1 ? x2.stride(0) : k;
  int rc = api().norm(data<const uint16_t>(x2), ldx, data<const uint16_t>(nw), data<uint8_t>(q), k, data<float>(s), 0,
                      data<uint16_t>(a), k, m, k, static_cast<float>(eps), TF_NORM_AUTO, stream);
  check(rc, "tf_rmsnorm_fp8_quant_ex");
  at::Tensor ws;
  if (l.need > 0) ws = at::empty({(std::max<int64_t>(l.need, 4) + 3) / 4}, x2.options().dtype(at::kFloat));
  rc = api().linear(data<const uint16_t>(a), k, data<const int32_t>(qw), data<const uint16_t>(sc),
                    data<const int32_t>(qz), static_cast<const uint16_t*>(ptr_or_null(bias)), data<uint16_t>(out),
                    n_out, m, n, k, static_cast<int32_t>(g), &l.cfg, static_cast<int32_t>(epi), nullptr, 0,
                    ws.defined() ? data<float>(ws) : nullptr, l.need, stream);
  check(rc, "tf_w4a16_linear_ex");
  return out.reshape(out_shape);
}

at::Tensor rmsnorm_fp8_w4a16_linear(const at::Tensor& x, const at::Tensor& nw, double eps, const at::Tensor& qw,
                                    const at::Tensor& sc, const at::Tensor& qz,
                                    const std::optional<at::Tensor>& bias, c10::SymInt group_size,
                                    c10::string_view backend, c10::string_view epilogue) {
  const int64_t g = group_size.guard_int(__FILE__, __LINE__);
  at::Tensor y = norm_linear_fast(x, nw, eps, qw, sc, qz, bias, g, backend, epilogue);
  if (y.defined()) return y;
  return python_body<NormLinearFn>("tokenforge::_py_rmsnorm_fp8_w4a16_linear", x, nw, eps, qw, sc, qz, bias,
                                   group_size, backend, epilogue);
}

}  // namespace

// Schemas: the reference's three ops (ops.py:48-156) and this build's fused forms, with the
// private operators the fast paths use.
TORCH_LIBRARY(tokenforge, m) {
  m.set_python_module("tokenforge.kernels.ops");
  m.def("w4a16_linear(Tensor x, Tensor qweight_t, Tensor scales, Tensor qzeros, Tensor? bias, SymInt group_size, "
        "str backend) -> Tensor");
  m.def("w4a16_linear_residual(Tensor x, Tensor qweight_t, Tensor scales, Tensor qzeros, Tensor? bias, "
        "Tensor residual, SymInt group_size, str backend) -> Tensor");
  m.def("w4a16_linear_silu_mul(Tensor x, Tensor qweight_t, Tensor scales, Tensor qzeros, Tensor? bias, "
        "SymInt group_size, str backend) -> Tensor");
  m.def("w4a8_linear(Tensor x8, Tensor x_scale, Tensor qweight_t, Tensor scales, Tensor qzeros, Tensor? bias, "
        "SymInt group_size, str backend, str epilogue=\"none\", Tensor? residual=None) -> Tensor");
  m.def("w4a16_dequant(Tensor qweight_t, Tensor scales, Tensor qzeros, SymInt group_size) -> Tensor");
  m.def("rmsnorm_fp8_quant(Tensor x, Tensor weight, float eps, Tensor? scale) -> (Tensor, Tensor)");
  m.def("rmsnorm_fp8_quant_dequant(Tensor x, Tensor weight, float eps, Tensor? scale) -> (Tensor, Tensor, Tensor)");
  m.def("rmsnorm_fp8_w4a16_linear(Tensor x, Tensor norm_weight, float eps, Tensor qweight_t, Tensor scales, "
        "Tensor qzeros, Tensor? bias, SymInt group_size, str backend, str epilogue) -> Tensor");
  m.def("_bind_library(str path) -> ()");
  m.def("_native_calls() -> int[]");
  m.def("_clear_launch_cache() -> ()");
  m.def("_resolve_launch(int kind, int epilogue, int m, int n, int k, int group_size, int device) -> int[]");
}

TORCH_LIBRARY_IMPL(tokenforge, CUDA, m) {
  m.impl("w4a16_linear", &w4a16_linear);
  m.impl("w4a16_linear_residual", &w4a16_linear_residual);
  m.impl("w4a16_linear_silu_mul", &w4a16_linear_silu_mul);
  m.impl("w4a8_linear", &w4a8_linear);
  m.impl("rmsnorm_fp8_quant", &rmsnorm_fp8_quant);
  m.impl("rmsnorm_fp8_quant_dequant", &rmsnorm_fp8_quant_dequant);
  m.impl("rmsnorm_fp8_w4a16_linear", &rmsnorm_fp8_w4a16_linear);
}

TORCH_LIBRARY_IMPL(tokenforge, CompositeExplicitAutograd, m) {
  m.impl("_bind_library", &bind_library);
  m.impl("_native_calls", &native_calls);
  m.impl("_clear_launch_cache", &clear_launch_cache);
}
