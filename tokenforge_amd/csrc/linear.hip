// tf_w4a16_linear: argument checks (w4a16.py:149-175 semantics) and variant dispatch.
#include "linear.h"

namespace tf {
namespace {

struct Table {
  const Variant* gemv;
  int n_gemv;
  const Variant* stream;
  int n_stream;
  const Variant* gemm;
  int n_gemm;
  const Variant* gemm2;
  int n_gemm2;
  const Variant* gemm3;
  int n_gemm3;
  const Variant* gemm4;
  int n_gemm4;
  const Variant* gemm8;
  int n_gemm8;
  Table() {
    gemv = gemv_variants(&n_gemv);
    stream = gemv_stream_variants(&n_stream);
    gemm = gemm_variants(&n_gemm);
    gemm2 = gemm2_variants(&n_gemm2);
    gemm3 = gemm3_variants(&n_gemm3);
    gemm4 = gemm4_variants(&n_gemm4);
    gemm8 = gemm8_variants(&n_gemm8);
  }
  int size() const { return n_gemv + n_stream + n_gemm + n_gemm2 + n_gemm3 + n_gemm4 + n_gemm8; }
  const Variant& at(int i) const {
    if (i < n_gemv) return gemv[i];
    i -= n_gemv;
    if (i < n_stream) return stream[i];
    i -= n_stream;
    if (i < n_gemm) return gemm[i];
    i -= n_gemm;
    if (i < n_gemm2) return gemm2[i];
    i -= n_gemm2;
    if (i < n_gemm3) return gemm3[i];
    i -= n_gemm3;
    return i < n_gemm4 ? gemm4[i] : gemm8[i - n_gemm4];
  }
};

const Table& table() {
  static const Table t;
  return t;
}

bool same_variant(const tf_gemm_config& a, const tf_gemm_config& b) {
  return a.kernel == b.kernel && a.block_m == b.block_m && a.block_n == b.block_n &&
         a.block_k == b.block_k && a.num_warps == b.num_warps && a.num_stages == b.num_stages;
}

const Variant* find_variant(const tf_gemm_config& cfg) {
  const Table& t = table();
  for (int i = 0; i < t.size(); ++i)
    if (same_variant(t.at(i).cfg, cfg)) return &t.at(i);
  return nullptr;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_config(const tf_gemm_config& cfg, int32_t group_size) {
  if (cfg.split_k < 1 || cfg.split_k > kMaxSplitK)
    return fail(TF_EINVAL, "tf_w4a16_linear: split_k must be in [1, 16]");
  // The GEMV stream form (gemv_mfma, block_k 512) may split K across workgroups (fp32 partials
  // and the split-K reduce); the other gemv kernels split K across their waves only.
  const bool stream_form = cfg.kernel == TF_KERNEL_GEMV_MFMA && cfg.block_k == 512;
  if (cfg.kernel != TF_KERNEL_GEMM_MFMA && cfg.kernel != TF_KERNEL_GEMM_FP8 && !stream_form && cfg.split_k != 1)
    return fail(TF_EINVAL, "tf_w4a16_linear: gemv kernels split K across waves (num_warps); split_k must be 1");
  // block_k 128 marks the skinny kernel (gemm3.hip), which reads each lane's group itself;
  // the LDS-tile kernels need one scale per column and block.
  if (cfg.kernel == TF_KERNEL_GEMM_MFMA && cfg.block_k != 128 &&
      (cfg.block_k > group_size || group_size % cfg.block_k))
    return fail(TF_EINVAL, "tf_w4a16_linear: block_k must divide group_size");
  return TF_OK;
}

// Configs whose kernels read e4m3 x themselves: every GEMV config (they decode while staging x
// in LDS) and the fp8 GEMM (which multiplies the codes). The fp16 GEMM configs get x converted
// to fp16 first.
bool fuses_x8(const tf_gemm_config& cfg) {
  return cfg.kernel == TF_KERNEL_GEMV_MFMA || cfg.kernel == TF_KERNEL_GEMV_DOT || cfg.kernel == TF_KERNEL_GEMM_FP8;
}

constexpr int64_t kWsAlign = 256;
int64_t align_ws(int64_t b) { return (b + kWsAlign - 1) / kWsAlign * kWsAlign; }

// e4m3 [m, k] (row stride ldx8 bytes) -> fp16 [m, k] (row stride k); 8 values per thread.
__global__ void e4m3_rows_to_f16_kernel(const uint8_t* __restrict__ x8, int64_t ldx8, uint16_t* __restrict__ out,
                                        int m, int k) {
  const int64_t chunks = (int64_t)m * (k / 8);
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= chunks) return;
  const int64_t row = i / (k / 8);
  const int64_t c = i % (k / 8);
  const u2 codes = *reinterpret_cast<const u2*>(x8 + row * ldx8 + c * 8);
  *reinterpret_cast<u4*>(out + row * k + c * 8) = e4m3x8_to_f16(codes);
}

}  // namespace
}  // namespace tf

using namespace tf;

extern "C" int tf_num_variants(void) { return table().size(); }

extern "C" int tf_get_variant(int index, tf_gemm_config* out) {
  if (out == nullptr || index < 0 || index >= table().size())
    return fail(TF_EINVAL, "tf_get_variant: index out of range");
  *out = table().at(index).cfg;
  return TF_OK;
}

static int make_args(const uint16_t* x, int64_t ldx, const int32_t* qweight_t, const uint16_t* scales,
                     const int32_t* qzeros, const uint16_t* bias, uint16_t* out, int64_t ldo, int64_t m,
                     int64_t n, int64_t k, int32_t group_size, int32_t epilogue, const uint16_t* residual,
                     int64_t ldr, LinearArgs* a) {
  if (m < 0 || n < 0 || k < 0) return fail(TF_EINVAL, "tf_w4a16_linear: negative size");
  if (m > 0x7FFFFFFF || n > 0x7FFFFFFF || k > 0x7FFFFFFF)
    return fail(TF_EINVAL, "tf_w4a16_linear: size above 2^31");
  if (n % 8) return fail(TF_EINVAL, "tf_w4a16_linear: N must be a multiple of 8");
  if (int rc = check_group_size(group_size, k, "tf_w4a16_linear")) return rc;
  if (epilogue != TF_EPILOGUE_NONE && epilogue != TF_EPILOGUE_RESIDUAL && epilogue != TF_EPILOGUE_SILU_MUL)
    return fail(TF_EINVAL, "tf_w4a16_linear_ex: unknown epilogue");
  if (epilogue == TF_EPILOGUE_SILU_MUL && n % 16)
    return fail(TF_EINVAL, "tf_w4a16_linear_ex: the SiLU*mul epilogue needs N to be a multiple of 16");
  const int64_t n_out = epilogue == TF_EPILOGUE_SILU_MUL ? n / 2 : n;
  if (ldx < k || ldo < n_out) return fail(TF_EINVAL, "tf_w4a16_linear: row stride smaller than the row");
  if (epilogue == TF_EPILOGUE_RESIDUAL) {
    if (ldr < n) return fail(TF_EINVAL, "tf_w4a16_linear_ex: residual row stride smaller than the row");
    if (residual == out && ldr != ldo)
      return fail(TF_EINVAL, "tf_w4a16_linear_ex: a residual that is the output needs the output's row stride");
  }
  a->epilogue = epilogue;
  a->residual = epilogue == TF_EPILOGUE_RESIDUAL ? residual : nullptr;
  a->ldr = ldr;
  if (ldx % 8) return fail(TF_EINVAL, "tf_w4a16_linear: x row stride must be a multiple of 8 elements");
  a->x = x;
  a->ldx = ldx;
  a->qw = reinterpret_cast<const uint32_t*>(qweight_t);
  a->scales = scales;
  a->qz = reinterpret_cast<const uint32_t*>(qzeros);
  a->bias = bias;
  a->out = out;
  a->ldo = ldo;
  a->m = (int)m;
  a->n = (int)n;
  a->k = (int)k;
  a->log2g = log2_group(group_size);
  if (m == 0 || n == 0) return TF_OK;
  if (!x || !qweight_t || !scales || !qzeros || !out) return fail(TF_EINVAL, "tf_w4a16_linear: null pointer");
  if (epilogue == TF_EPILOGUE_RESIDUAL && !residual)
    return fail(TF_EINVAL, "tf_w4a16_linear_ex: the residual epilogue needs a residual tensor");
  if (!aligned16(x) || !aligned16(qweight_t))
    return fail(TF_EINVAL, "tf_w4a16_linear: x and qweight_t must be 16-byte aligned");
  return TF_OK;
}

extern "C" int64_t tf_w4a16_workspace_bytes_ex(int64_t m, int64_t n, int64_t k, int32_t group_size,
                                               const tf_gemm_config* cfg, int32_t epilogue) {
  if (cfg == nullptr) return 0;
  const Variant* v = find_variant(*cfg);
  if (v == nullptr || m <= 0 || n <= 0 || k <= 0 || cfg->block_k <= 0) return 0;
  LinearArgs a{};
  a.m = (int)m;
  a.n = (int)n;
  a.k = (int)k;
  a.log2g = log2_group(group_size);
  a.epilogue = epilogue;
  return v->workspace(a, *cfg);
}

extern "C" int64_t tf_w4a16_workspace_bytes(int64_t m, int64_t n, int64_t k, int32_t group_size,
                                            const tf_gemm_config* cfg) {
  return tf_w4a16_workspace_bytes_ex(m, n, k, group_size, cfg, TF_EPILOGUE_NONE);
}

extern "C" int tf_w4a16_linear_ex(const uint16_t* x, int64_t ldx, const int32_t* qweight_t,
                                  const uint16_t* scales, const int32_t* qzeros, const uint16_t* bias,
                                  uint16_t* out, int64_t ldo, int64_t m, int64_t n, int64_t k,
                                  int32_t group_size, const tf_gemm_config* cfg, int32_t epilogue,
                                  const uint16_t* residual, int64_t ldr, float* workspace,
                                  int64_t workspace_bytes, void* stream) {
  if (cfg == nullptr) return fail(TF_EINVAL, "tf_w4a16_linear: null config");
  LinearArgs a;
  if (int rc = make_args(x, ldx, qweight_t, scales, qzeros, bias, out, ldo, m, n, k, group_size, epilogue,
                         residual, ldr, &a))
    return rc;
  if (int rc = check_config(*cfg, group_size)) return rc;
  const Variant* v = find_variant(*cfg);
  if (v == nullptr) return fail(TF_EINVAL, "tf_w4a16_linear: config does not name a compiled variant");
  if (cfg->kernel == TF_KERNEL_GEMM_FP8)
    return fail(TF_EINVAL, "tf_w4a16_linear: the gemm_fp8 kernels take e4m3 activations (tf_w4a8_linear_ex)");
  if (m == 0 || n == 0) return TF_OK;
  const int64_t need = v->workspace(a, *cfg);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(TF_EINVAL, "tf_w4a16_linear: workspace too small for this split_k");
  return v->launch(a, *cfg, workspace, (hipStream_t)stream);
}

extern "C" int tf_w4a16_linear(const uint16_t* x, int64_t ldx, const int32_t* qweight_t,
                               const uint16_t* scales, const int32_t* qzeros, const uint16_t* bias,
                               uint16_t* out, int64_t ldo, int64_t m, int64_t n, int64_t k,
                               int32_t group_size, const tf_gemm_config* cfg, float* workspace,
                               int64_t workspace_bytes, void* stream) {
  return tf_w4a16_linear_ex(x, ldx, qweight_t, scales, qzeros, bias, out, ldo, m, n, k, group_size, cfg,
                            TF_EPILOGUE_NONE, nullptr, 0, workspace, workspace_bytes, stream);
}

extern "C" int64_t tf_w4a8_workspace_bytes_ex(int64_t m, int64_t n, int64_t k, int32_t group_size,
                                              const tf_gemm_config* cfg, int32_t epilogue) {
  if (cfg == nullptr || m <= 0 || n <= 0 || k <= 0) return 0;
  const int64_t own = tf_w4a16_workspace_bytes_ex(m, n, k, group_size, cfg, epilogue);
  return fuses_x8(*cfg) ? own : align_ws(m * k * 2) + own;
}

extern "C" int tf_w4a8_linear_ex(const uint8_t* x8, int64_t ldx8, const float* xscale, int64_t xscale_stride,
                                 const int32_t* qweight_t, const uint16_t* scales, const int32_t* qzeros,
                                 const uint16_t* bias, uint16_t* out, int64_t ldo, int64_t m, int64_t n, int64_t k,
                                 int32_t group_size, const tf_gemm_config* cfg, int32_t epilogue,
                                 const uint16_t* residual, int64_t ldr, float* workspace, int64_t workspace_bytes,
                                 void* stream) {
  if (cfg == nullptr) return fail(TF_EINVAL, "tf_w4a8_linear_ex: null config");
  if (ldx8 < k || ldx8 % 8) return fail(TF_EINVAL, "tf_w4a8_linear_ex: x row stride must be >= K and a multiple of 8");
  if (xscale_stride < 0) return fail(TF_EINVAL, "tf_w4a8_linear_ex: negative scale stride");
  if (m > 0 && n > 0) {
    if (x8 == nullptr || xscale == nullptr) return fail(TF_EINVAL, "tf_w4a8_linear_ex: null pointer");
    if ((reinterpret_cast<uintptr_t>(x8) & 15u) != 0)
      return fail(TF_EINVAL, "tf_w4a8_linear_ex: x must be 16-byte aligned");
  }
  const int64_t need = tf_w4a8_workspace_bytes_ex(m, n, k, group_size, cfg, epilogue);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(TF_EINVAL, "tf_w4a8_linear_ex: workspace too small");
  const bool fused = fuses_x8(*cfg);
  const bool convert = !fused && m > 0 && n > 0 && k > 0;
  // The kernels that stage x read the codes; for the others x is converted to fp16 into the
  // front of the workspace and the rest of the workspace is theirs. Every check runs before
  // anything is launched, so a rejected call leaves nothing queued on the stream.
  const uint16_t* x16 = reinterpret_cast<const uint16_t*>(x8);
  float* ws = workspace;
  int64_t ws_bytes = workspace_bytes;
  if (convert) {
    x16 = reinterpret_cast<const uint16_t*>(workspace);
    const int64_t front = align_ws(m * k * 2);
    ws = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) + front);
    ws_bytes = workspace_bytes - front;
  }
  LinearArgs a;
  if (int rc = make_args(x16, k, qweight_t, scales, qzeros, bias, out, ldo, m, n, k, group_size, epilogue,
                         residual, ldr, &a))
    return rc;
  if (fused) {
    a.x = nullptr;
    a.x8 = x8;
    a.ldx8 = ldx8;
  }
  a.xscale = xscale;
  a.xscale_stride = xscale_stride;
  if (int rc = check_config(*cfg, group_size)) return rc;
  const Variant* v = find_variant(*cfg);
  if (v == nullptr) return fail(TF_EINVAL, "tf_w4a8_linear_ex: config does not name a compiled variant");
  if (m == 0 || n == 0) return TF_OK;
  const int64_t own = v->workspace(a, *cfg);
  if (own > 0 && (ws == nullptr || ws_bytes < own)) return fail(TF_EINVAL, "tf_w4a8_linear_ex: workspace too small");
  if (v->check != nullptr)
    if (int rc = v->check(a, *cfg)) return rc;
  if (convert) {
    uint16_t* conv = reinterpret_cast<uint16_t*>(workspace);
    const int64_t chunks = m * (k / 8);
    e4m3_rows_to_f16_kernel<<<(unsigned)cdiv(chunks, 256), 256, 0, (hipStream_t)stream>>>(x8, ldx8, conv, (int)m,
                                                                                         (int)k);
    if (int rc = check_launch("tf_w4a8_linear_ex(e4m3 to fp16)")) return rc;
  }
  return v->launch(a, *cfg, ws, (hipStream_t)stream);
}

extern "C" int tf_rmsnorm_fp8_w4a16_linear(const uint16_t* x, int64_t ldx, const uint16_t* norm_weight, float eps,
                                           const int32_t* qweight_t, const uint16_t* scales, const int32_t* qzeros,
                                           const uint16_t* bias, uint16_t* out, int64_t ldo, int64_t m, int64_t n,
                                           int64_t k, int32_t group_size, const tf_gemm_config* cfg,
                                           int32_t epilogue, void* stream) {
  if (cfg == nullptr) return fail(TF_EINVAL, "tf_rmsnorm_fp8_w4a16_linear: null config");
  if (cfg->kernel != TF_KERNEL_GEMV_MFMA || cfg->block_k != 512)
    return fail(TF_EINVAL, "tf_rmsnorm_fp8_w4a16_linear: the RMSNorm prologue runs in the gemv stream form "
                           "(gemv_mfma, block_k 512, M <= 4)");
  if (epilogue == TF_EPILOGUE_RESIDUAL)
    return fail(TF_EINVAL, "tf_rmsnorm_fp8_w4a16_linear: epilogue none or silu_mul");
  LinearArgs a;
  if (int rc = make_args(x, ldx, qweight_t, scales, qzeros, bias, out, ldo, m, n, k, group_size, epilogue, nullptr,
                         0, &a))
    return rc;
  if (m > 0 && n > 0) {
    if (norm_weight == nullptr) return fail(TF_EINVAL, "tf_rmsnorm_fp8_w4a16_linear: null norm weight");
    if (!aligned16(norm_weight)) return fail(TF_EINVAL, "tf_rmsnorm_fp8_w4a16_linear: norm weight must be 16-byte aligned");
  }
  a.norm_w = norm_weight;
  a.norm_eps = eps;
  a.norm_inv_k = k > 0 ? 1.0 / (double)k : 0.0;
  if (int rc = check_config(*cfg, group_size)) return rc;
  const Variant* v = find_variant(*cfg);
  if (v == nullptr) return fail(TF_EINVAL, "tf_rmsnorm_fp8_w4a16_linear: config does not name a compiled variant");
  if (m == 0 || n == 0) return TF_OK;
  return v->launch(a, *cfg, nullptr, (hipStream_t)stream);
}
