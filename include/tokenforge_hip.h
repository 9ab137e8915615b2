/*
 * tokenforge_hip.h — C ABI of the MI355X (gfx950) quantized-linear hot path.
 *
 * Every entry point takes plain device pointers, element counts and a HIP stream
 * (passed as `void*`, i.e. a `hipStream_t`; NULL = the null stream). Nothing here
 * allocates or frees device memory, synchronizes with the host, or reads tensor
 * values on the host, with one documented exception (tf_pack_int4 writes a range
 * flag that the caller may read). All kernels are launched asynchronously on the
 * given stream. Outputs and workspaces are owned by the caller.
 *
 * Return value: 0 on success, otherwise a TF_E* code; tf_last_error() then returns a
 * message (thread-local) naming the argument that was rejected, or the HIP error.
 *
 * Dtypes: fp16 buffers are `uint16_t` bit patterns (IEEE binary16); fp8 buffers are
 * `uint8_t` OCP float8_e4m3fn codes; packed int4 buffers are `int32_t` words holding
 * eight 4-bit values in the AWQ nibble order (nibble i holds offset AWQ_ORDER[i],
 * AWQ_ORDER = {0,2,4,6,1,3,5,7}).
 *
 * The Python host side (tokenforge.kernels) binds these with ctypes; the citations
 * name the reference function (saransh-debugs/TokenForge) each entry point replaces.
 */
#ifndef TOKENFORGE_HIP_H
#define TOKENFORGE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TF_OK 0
#define TF_EINVAL 1   /* bad argument: shape, alignment, group size, config */
#define TF_ELAUNCH 2  /* HIP reported an error at launch */
#define TF_ERANGE 3   /* value out of range (tf_pack_int4) */

/* ABI version of this library. The autotune cache is keyed on it. */
int tf_abi_version(void);

/* Message for the last failing call on this host thread ("" if none). */
const char* tf_last_error(void);

/* --------------------------------------------------------------- packing / layout */

/* pack.py:42-54 pack_int4. values int32 [rows, n] in [0,15] -> packed int32
 * [rows, n/8], AWQ interleave. n % 8 == 0. If any value lies outside [0, 15],
 * *range_flag (device int32, caller-zeroed) is set to 1; the packed output is then
 * unspecified. range_flag may be NULL. */
int tf_pack_int4(const int32_t* values, int32_t* packed, int64_t rows, int64_t n,
                 int32_t* range_flag, void* stream);

/* pack.py:57-67 unpack_int4. packed int32 [rows, words] -> int32 [rows, 8*words]. */
int tf_unpack_int4(const int32_t* packed, int32_t* values, int64_t rows, int64_t words,
                   void* stream);

/* pack.py:141-143 repack_awq_to_tf. AWQ qweight int32 [k, n/8] (packed along N)
 * -> qweight_t int32 [n, k/8] (packed along K, same nibble interleave). Bit-exact.
 * k % 8 == 0, n % 8 == 0. */
int tf_awq_to_tf(const int32_t* qweight, int32_t* qweight_t, int64_t k, int64_t n,
                 void* stream);

/* pack.py:146-148 repack_tf_to_awq. Exact inverse of tf_awq_to_tf. */
int tf_tf_to_awq(const int32_t* qweight_t, int32_t* qweight, int64_t n, int64_t k,
                 void* stream);

/* The gfx950 tile layout: what pack_awq produces and every kernel below reads. Same
 * shapes and dtypes as the reference's TokenForge layout (qweight_t int32 [n, k/8], scales
 * fp16 [k/g, n], qzeros int32 [k/g, n/8]); positions differ. Rows come in tiles of 16
 * (t = row / 16, c = row % 16, r_t = min(16, n - 16 t)); with Q = k/32 and P = k/g:
 *   16-byte weight chunk (row, q) [its words 4q..4q+3 of the TokenForge layout]
 *                          -> chunk 16 t Q + 4 r_t (q / 4) + (q % 4) r_t + c
 *   scale (p, row)         -> element 16 t P + p r_t + c
 *   zero word (p, w)       -> word 2 t P + p (r_t / 8) + (w - 2 t), t = w / 2
 * so each 16-row x 128-K step of qweight_t is one contiguous 1 KB block in which lane
 * 16 g + c of a wave finds the MFMA B operand of column c, K block g. */

/* pack.py:171-181 pack_awq (the layout step; the AWQ -> TokenForge transposition is
 * tf_awq_to_tf): TokenForge-layout qweight_t, scales, qzeros -> the same three tensors in the
 * tile layout. No counterpart kernel in the reference, whose pack_awq keeps the TokenForge
 * layout. n % 8 == 0, k % group_size == 0; qweight buffers 16-byte aligned; out-of-place. */
int tf_tile_pack(const int32_t* qweight_t, const uint16_t* scales, const int32_t* qzeros,
                 int32_t* qweight_tile, uint16_t* scales_tile, int32_t* qzeros_tile, int64_t n,
                 int64_t k, int32_t group_size, void* stream);

/* pack.py:184-186 unpack_to_awq (the layout step): exact inverse of tf_tile_pack. */
int tf_tile_unpack(const int32_t* qweight_tile, const uint16_t* scales_tile,
                   const int32_t* qzeros_tile, int32_t* qweight_t, uint16_t* scales,
                   int32_t* qzeros, int64_t n, int64_t k, int32_t group_size, void* stream);

/* pack.py:83-107 awq_quantize: min-max asymmetric int4 of an fp32 weight [n, k] (finite
 * values) into AWQ format: qweight int32 [k, n/8], qzeros int32 [k/g, n/8], scales fp16
 * [k/g, n]; scale = fp16(max(max - min, 1e-5) / 15), zero = clamp(-rint(min / scale), 0,
 * 15), q = clamp(rint(w / scale) + zero, 0, 15), IEEE fp32 division, round half to even. */
int tf_awq_quantize(const float* weight, int64_t n, int64_t k, int32_t group_size,
                    int32_t* qweight, int32_t* qzeros, uint16_t* scales, void* stream);

/* --------------------------------------------------------------- dequant */

/* w4a16.py:235-264 w4a16_dequant (== pack.py:189-194 dequantize_tf).
 * qweight_t, scales, qzeros in the tile layout (above)
 * -> out fp16 [n, k] with out[n][k] = fp16(q - z) * s (one fp16 rounding). */
int tf_w4a16_dequant(const int32_t* qweight_t, const uint16_t* scales,
                     const int32_t* qzeros, uint16_t* out, int64_t n, int64_t k,
                     int32_t group_size, void* stream);

/* --------------------------------------------------------------- W4A16 linear */

/* Kernel families (the `kernel` field of tf_gemm_config). */
#define TF_KERNEL_GEMV_DOT 0   /* decode: in-register dequant + VALU dot2, M <= 4     */
#define TF_KERNEL_GEMV_MFMA 1  /* decode: in-register dequant + fp16 MFMA (M <= 32)   */
#define TF_KERNEL_GEMM_MFMA 2  /* prefill: LDS-staged dequant + fp16 MFMA, split-K    */
#define TF_KERNEL_GEMM_FP8 3   /* W4A8 prefill (tf_w4a8_linear_ex only): e4m3 x and exact
                                  e4m3 (q - z) on the fp8 MFMA, group scale in fp32 after each
                                  128-K group; group_size 128, N % 16 == 0, split-K           */

/* Launch configuration; the counterpart of config.py:23-68 GemmConfig. The tuple
 * (kernel, block_m, block_n, block_k, num_warps, num_stages) must name a compiled
 * variant (see tf_num_variants / tf_get_variant); split_k is a runtime value (1 for the gemv
 * kernels except the stream form, gemv_mfma with block_k 512, which splits K across workgroup
 * sets and adds the slices with the split-K reduce). */
typedef struct tf_gemm_config {
  int32_t kernel;
  int32_t block_m;
  int32_t block_n;
  int32_t block_k;
  int32_t split_k;
  int32_t num_warps;
  int32_t num_stages;
} tf_gemm_config;

/* Number of compiled variants, and variant i (split_k set to 1). */
int tf_num_variants(void);
int tf_get_variant(int index, tf_gemm_config* out);

/* Bytes of fp32 workspace tf_w4a16_linear needs for this problem and config
 * (0 when split_k == 1 or the kernel reduces on chip). */
int64_t tf_w4a16_workspace_bytes(int64_t m, int64_t n, int64_t k, int32_t group_size,
                                 const tf_gemm_config* cfg);

/* w4a16.py:178-232 w4a16_gemm and ops.py:86-88 _C.w4a16_gemv:
 *   out[m][n] = fp16( sum_k fp32(x[m][k]) * fp32(fp16(q[n][k] - z) * s) + fp32(bias[n]) )
 * x fp16 [m, k] with row stride ldx elements (16-byte aligned rows), qweight_t, scales and
 * qzeros in the tile layout (above), bias fp16 [n] or NULL,
 * out fp16 [m, n] with row stride ldo. Split-K partials are reduced in a fixed order
 * (bit-identical run to run). workspace: fp32, >= tf_w4a16_workspace_bytes. */
int tf_w4a16_linear(const uint16_t* x, int64_t ldx, const int32_t* qweight_t,
                    const uint16_t* scales, const int32_t* qzeros, const uint16_t* bias,
                    uint16_t* out, int64_t ldo, int64_t m, int64_t n, int64_t k,
                    int32_t group_size, const tf_gemm_config* cfg, float* workspace,
                    int64_t workspace_bytes, void* stream);

/* Fused epilogues of the linear. No counterpart in the reference, which runs these as
 * separate torch ops after the linear; for callers that would otherwise round-trip [m, n]
 * through memory between the linear and the next elementwise op.
 *   TF_EPILOGUE_NONE      out[m][n] = y[m][n]                           (tf_w4a16_linear)
 *   TF_EPILOGUE_RESIDUAL  out[m][n] = fp16(residual[m][n] + fp16(y[m][n]))
 *                         residual fp16 [m, n] with row stride ldr; out may be residual
 *                         itself (same pointer and stride), nothing else may overlap.
 *   TF_EPILOGUE_SILU_MUL  out[m][j] = fp16(fp16(silu(fp16(y[m][j]))) * fp16(y[m][n/2 + j]))
 *                         for j < n/2 (gate columns first, then up); n a multiple of 16;
 *                         silu(v) = v / (1 + exp(-v)) in fp32.
 * Each equals the unfused torch composition on fp16 tensors (the same roundings). */
#define TF_EPILOGUE_NONE 0
#define TF_EPILOGUE_RESIDUAL 1
#define TF_EPILOGUE_SILU_MUL 2

/* Workspace bytes of tf_w4a16_linear_ex (the LDS-tile GEMMs reduce a SiLU*mul epilogue
 * through fp32 partials even without split-K). */
int64_t tf_w4a16_workspace_bytes_ex(int64_t m, int64_t n, int64_t k, int32_t group_size,
                                    const tf_gemm_config* cfg, int32_t epilogue);

/* tf_w4a16_linear with an epilogue (see above); residual and ldr only for
 * TF_EPILOGUE_RESIDUAL. */
int tf_w4a16_linear_ex(const uint16_t* x, int64_t ldx, const int32_t* qweight_t,
                       const uint16_t* scales, const int32_t* qzeros, const uint16_t* bias,
                       uint16_t* out, int64_t ldo, int64_t m, int64_t n, int64_t k,
                       int32_t group_size, const tf_gemm_config* cfg, int32_t epilogue,
                       const uint16_t* residual, int64_t ldr, float* workspace,
                       int64_t workspace_bytes, void* stream);

/* tf_w4a16_linear_ex that allocates nothing. No counterpart in the reference: for callers that
 * cannot allocate device memory (code under HIP-graph capture that must not call hipMalloc,
 * tight serving loops, harnesses that forbid allocation). The workspace the kernels need
 * (split-K partials, the SiLU*mul rows of the LDS-tile GEMMs) comes from a fixed device array
 * of tf_noalloc_scratch_bytes() bytes (32 MiB) that each GPU holds until the process ends; a
 * call needing more is rejected (TF_EINVAL). Nothing needs clearing between calls. All calls
 * on one GPU share that array: calls that overlap in time on one GPU (other streams, other
 * host threads) race, and the caller must serialize them. Arguments as tf_w4a16_linear_ex
 * without the workspace. */
int64_t tf_noalloc_scratch_bytes(void);
int tf_w4a16_linear_ex_noalloc(const uint16_t* x, int64_t ldx, const int32_t* qweight_t,
                               const uint16_t* scales, const int32_t* qzeros, const uint16_t* bias,
                               uint16_t* out, int64_t ldo, int64_t m, int64_t n, int64_t k,
                               int32_t group_size, const tf_gemm_config* cfg, int32_t epilogue,
                               const uint16_t* residual, int64_t ldr, void* stream);

/* W4A8: the linear on FP8 activations, e.g. tf_rmsnorm_fp8_quant's codes and scales. No
 * counterpart in the reference, which never feeds its FP8 output to a linear.
 *   out[m][n] = fp16( xscale[m] * sum_k e4m3(x8[m][k]) * fp16((q[n][k] - z) * s) + bias[n] )
 * x8 e4m3fn codes [m, k], row stride ldx8 bytes (a multiple of 8; 16-byte aligned base);
 * xscale fp32, row m at xscale[m * xscale_stride] (stride 0: one scale for every row).
 * e4m3 values are exact in fp16, so with xscale = 1 this equals tf_w4a16_linear on the
 * decoded x bit for bit. Epilogues as tf_w4a16_linear_ex (applied after the row scale).
 * The GEMV configs decode the codes while staging x in LDS; the GEMM configs decode x to fp16
 * into the workspace first. Every check runs before anything is launched. */
int64_t tf_w4a8_workspace_bytes_ex(int64_t m, int64_t n, int64_t k, int32_t group_size,
                                   const tf_gemm_config* cfg, int32_t epilogue);
int tf_w4a8_linear_ex(const uint8_t* x8, int64_t ldx8, const float* xscale, int64_t xscale_stride,
                      const int32_t* qweight_t, const uint16_t* scales, const int32_t* qzeros,
                      const uint16_t* bias, uint16_t* out, int64_t ldo, int64_t m, int64_t n,
                      int64_t k, int32_t group_size, const tf_gemm_config* cfg, int32_t epilogue,
                      const uint16_t* residual, int64_t ldr, float* workspace,
                      int64_t workspace_bytes, void* stream);

/* --------------------------------------------------------------- RMSNorm + FP8 */

/* rmsnorm_fp8.py:76-117 rmsnorm_fp8_quant (semantics of reference.py:35-56):
 *   y = fp16(fp16(x * rstd) * w),  rstd = 1 / sqrt(sum(x^2) / h + eps)
 *   dynamic: scale[t] = max(amax|y| / 448, 1/(448*512)) is written;
 *   static (static_scale != 0): scale[0] is read, not written.
 *   q = e4m3fn(RNE(clamp(y / scale, -448, 448)))
 * x fp16 [t, h] (row stride ldx), w fp16 [h], q uint8 [t, h] (row stride ldq),
 * scale fp32 [t] (dynamic) or [1] (static). */
int tf_rmsnorm_fp8_quant(const uint16_t* x, int64_t ldx, const uint16_t* weight,
                         uint8_t* q, int64_t ldq, float* scale, int32_t static_scale,
                         int64_t t, int64_t h, float eps, void* stream);

/* tf_rmsnorm_fp8_quant that also writes dq fp16 [t, h] (row stride lddq) =
 * fp16(fp32(q) * scale): the fp16 activation a W4A16 linear reads when it is fed from the
 * codes, which the reference computes as a separate torch expression
 * `(q.to(torch.float32) * scale).to(torch.float16)` (no kernel counterpart in the reference;
 * for callers that feed a W4A16 linear from the norm's FP8 output in one launch).
 * dq == NULL is tf_rmsnorm_fp8_quant. */
int tf_rmsnorm_fp8_quant_dq(const uint16_t* x, int64_t ldx, const uint16_t* weight,
                            uint8_t* q, int64_t ldq, float* scale, int32_t static_scale,
                            uint16_t* dq, int64_t lddq, int64_t t, int64_t h, float eps,
                            void* stream);

/* Kernel forms of the norm (same bits either way): */
#define TF_NORM_AUTO 0           /* the library's choice (currently row per workgroup)               */
#define TF_NORM_ROW_PER_BLOCK 1  /* up to 4 waves share a row, LDS reductions (any h, any alignment)  */
#define TF_NORM_ROW_PER_WAVE 2   /* 4 independent rows per workgroup, one per wave, wave reductions;
                                    needs h % 8 == 0, 16-byte aligned rows (and 8-byte q) and h <= 8192 */

/* tf_rmsnorm_fp8_quant_dq with the kernel form chosen by the caller (for tuning and tests;
 * the reference has a single Triton kernel, rmsnorm_fp8.py:44-73). TF_EINVAL when the form
 * does not apply to the arguments. */
int tf_rmsnorm_fp8_quant_ex(const uint16_t* x, int64_t ldx, const uint16_t* weight, uint8_t* q,
                            int64_t ldq, float* scale, int32_t static_scale, uint16_t* dq,
                            int64_t lddq, int64_t t, int64_t h, float eps, int32_t form,
                            void* stream);

/* tf_rmsnorm_fp8_quant_dq (dynamic scale) followed by tf_w4a16_linear_ex on its dq output, in
 * one decode launch: out = linear(dq(rmsnorm_fp8_quant(x, norm_weight, eps))), bit for bit the
 * two calls. No counterpart in the reference, which runs rmsnorm_fp8_quant (rmsnorm_fp8.py:76)
 * and the linear (ops.py:48) as separate kernels; for decode callers (M <= 4) that would
 * otherwise launch the norm on its own. Only the gemv stream form runs it (cfg gemv_mfma with
 * block_k 512 and block_m 4, split_k 1; M <= 4); epilogue NONE or SILU_MUL; the codes and
 * scales are not written.
 * x fp16 [m, k] (row stride ldx), norm_weight fp16 [k] (16-byte aligned); the linear's other
 * arguments as tf_w4a16_linear_ex (no workspace). */
int tf_rmsnorm_fp8_w4a16_linear(const uint16_t* x, int64_t ldx, const uint16_t* norm_weight, float eps,
                                const int32_t* qweight_t, const uint16_t* scales, const int32_t* qzeros,
                                const uint16_t* bias, uint16_t* out, int64_t ldo, int64_t m, int64_t n,
                                int64_t k, int32_t group_size, const tf_gemm_config* cfg,
                                int32_t epilogue, void* stream);

/* Test hook for the e4m3fn encoding used by tf_rmsnorm_fp8_quant
 * (rmsnorm_fp8.py:29-41 _round_to_e4m3_grid + cast): fp32 [count] -> uint8 [count], through
 * the same hardware conversion (v_cvt_pk_fp8_f32) and NaN handling as that kernel.
 * Inputs must lie in [-448, 448] or be NaN. */
int tf_e4m3_encode(const float* in, uint8_t* out, int64_t count, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TOKENFORGE_HIP_H */
