/*
 * joyomni_hip -- C ABI of the MI355X (gfx950) quantized-DiT hot path.
 *
 * libjoyomni_hip.so exports exactly the functions below. Signatures carry only
 * plain pointers, sizes and enums: device pointers to caller-owned memory, and
 * the HIP stream (hipStream_t) to launch on as `void *stream` (NULL = the null
 * stream). No function allocates, synchronises or retains a pointer after it
 * returns. Every argument rule is checked before anything is launched; a
 * failed check returns JOY_ERR_INVALID_ARGUMENT (or JOY_ERR_UNSUPPORTED) and
 * joy_last_error() describes it, using the reference's TORCH_CHECK wording
 * where one exists.
 *
 * Each entry point cites the reference interface it replaces (paths relative
 * to the reference repository root).
 */
#ifndef JOYOMNI_HIP_H_
#define JOYOMNI_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define JOY_ABI_VERSION 1

#if defined(__GNUC__) || defined(__clang__)
#define JOY_API __attribute__((visibility("default")))
#else
#define JOY_API
#endif

typedef enum {
  JOY_OK = 0,
  JOY_ERR_INVALID_ARGUMENT = 1, /* a reference TORCH_CHECK would have failed; nothing launched */
  JOY_ERR_UNSUPPORTED = 2,      /* legal for the reference, not supported by this build */
  JOY_ERR_HIP = 3               /* the HIP runtime rejected the launch */
} joy_status;

typedef enum { JOY_DTYPE_BF16 = 0, JOY_DTYPE_FP16 = 1 } joy_dtype;

/* Rounding of the activation quantiser's element step. */
typedef enum {
  JOY_QUANT_DIVIDE = 0,    /* q = e4m3fn(clamp(x / s)): deploy/xvideo/models/dit/fp8_linear.py:38-43 */
  JOY_QUANT_RECIPROCAL = 1 /* q = e4m3fn(clamp(x * (1/s))): joyomni_ops/csrc/per_token_quant_fp8_rocm.hip:72-77 */
} joy_quant_rounding;

typedef enum {
  JOY_EPILOGUE_NONE = 0,
  JOY_EPILOGUE_GELU_TANH = 1 /* gelu(round(out), approximate="tanh"): deploy/xvideo/models/dit/dit.py:87-89 */
} joy_epilogue;

/* Interface version (JOY_ABI_VERSION of the built library). */
JOY_API int joy_abi_version(void);

/* Message for the last non-OK status returned on the calling thread ("" if none). */
JOY_API const char *joy_last_error(void);

/*
 * Dynamic per-token FP8 quantisation.
 * Replaces: sgl_per_token_quant_fp8(Tensor input, Tensor! output_q, Tensor! output_s)
 *   schema joyomni_ops/csrc/pybind.cpp:68-69, impl joyomni_ops/csrc/per_token_quant_fp8_rocm.hip:96-123
 *   (rounding JOY_QUANT_RECIPROCAL), and the model's formula
 *   deploy/xvideo/models/dit/fp8_linear.py:38-43 (rounding JOY_QUANT_DIVIDE).
 * input: [M, K] bf16 or fp16 (input_dtype), contiguous; output_q: [M, K] e4m3fn;
 * output_s: [M] fp32, s[m] = max(absmax_k |x|, 1e-8) / 448.
 */
JOY_API joy_status joy_per_token_quant_fp8(const void *input, int input_dtype, void *output_q,
                                   float *output_s, int64_t M, int64_t K, int rounding,
                                   void *stream);

/*
 * Row/column-scaled FP8 GEMM with fused epilogue.
 * Replaces: fp8_scaled_mm(Tensor mat_a, Tensor mat_b, Tensor scales_a, Tensor scales_b,
 *           ScalarType out_dtype, Tensor? bias) -> Tensor
 *   schema joyomni_ops/csrc/pybind.cpp:71-73, impl joyomni_ops/csrc/fp8_gemm.cu:1450-1546,
 *   and the ROCm call torch._scaled_mm(..., use_fast_accum=True) at
 *   deploy/xvideo/models/dit/fp8_linear.py:124-132.
 * mat_a: e4m3fn [M, K] row-major. mat_b: e4m3fn (K, N) column-major, i.e. W[N, K]
 * row-major. scales_a [M], scales_b [N] fp32. bias: [N] of out_dtype or NULL.
 * out: caller-allocated [M, N] row-major of out_dtype (the reference allocates it).
 *   out[m,n] = round(fma(acc[m,n] * scales_b[n], scales_a[m], bias[n])) (fp8_gemm.cu:99-136)
 * Reference rules kept: K % 16 == 0, N % 8 == 0 (16-byte rows), out_dtype bf16/fp16.
 * This build also needs mat_a, mat_b 16-byte aligned and out, scales_b
 * 16-byte aligned (JOY_ERR_UNSUPPORTED otherwise).
 */
JOY_API joy_status joy_fp8_scaled_mm(const void *mat_a, const void *mat_b, const float *scales_a,
                             const float *scales_b, const void *bias, void *out, int out_dtype,
                             int64_t M, int64_t N, int64_t K, int epilogue, void *stream);

/*
 * In-place per-head q/k RMSNorm + interleaved RoPE.
 * Replaces: fused_qk_norm_rope_3d_paired(Tensor! q, Tensor! k, int seq_len, int num_heads,
 *           float eps, Tensor q_weight, Tensor k_weight, Tensor cos, Tensor sin, Tensor? k_pre_rope)
 *   schema joyomni_ops/csrc/pybind.cpp:53-55, impl
 *   joyomni_ops/csrc/fused_qknorm_rope_3d_kernel.cu:280-319 (kernel :44-106).
 * q, k: bf16 [batch, seq_len*num_heads, head_dim] contiguous, overwritten.
 * q_weight, k_weight: bf16 [head_dim]. cos, sin: bf16 [seq_len, head_dim/2].
 * k_pre_rope: bf16 like k, or NULL: receives the normalised K before rotation.
 * head_dim in {64, 128, 256}.
 */
JOY_API joy_status joy_fused_qk_norm_rope_3d_paired(void *q, void *k, int64_t batch, int64_t seq_len,
                                            int64_t num_heads, int64_t head_dim, float eps,
                                            const void *q_weight, const void *k_weight,
                                            const void *cos, const void *sin, void *k_pre_rope,
                                            void *stream);

/*
 * Fused QKV split + q/k RMSNorm + 3-D RoPE + KV-ring write (new op, no single
 * reference counterpart). It performs, in one pass over the QKV GEMM output:
 *   the split       rearrange(qkv, "B L (K H D) -> K B L H D")   deploy/xvideo/models/dit/dit.py:409-411
 *   the contiguous copies and norm+RoPE of                        deploy/xvideo/models/dit/sgl_fused_ops.py:122-168
 *                                                                 joyomni_ops/csrc/fused_qknorm_rope_3d_kernel.cu:44-106
 *   the cache write of pre-RoPE K and compact V                   deploy/xvideo/models/dit/dit.py:446-451,867-882
 * qkv: bf16 [seq_len, 3*num_heads*head_dim] with row stride qkv_row_stride (elements).
 * q_out, k_out: bf16 [seq_len, num_heads, head_dim] with token strides (elements);
 *   k_out may be NULL.
 * cache_k, cache_v: bf16 rings [num_slots, slot_capacity, num_heads, head_dim]
 *   (either both NULL or both set); tokens go to rows slot_offset .. slot_offset+seq_len-1
 *   of slot `slot`: cache_k gets the normalised pre-RoPE K, cache_v a copy of V.
 */
JOY_API joy_status joy_fused_qkv_norm_rope_cache(const void *qkv, int64_t qkv_row_stride, int64_t seq_len,
                                         int64_t num_heads, int64_t head_dim, float eps,
                                         const void *q_weight, const void *k_weight,
                                         const void *cos, const void *sin, void *q_out,
                                         int64_t q_out_stride, void *k_out, int64_t k_out_stride,
                                         void *cache_k, void *cache_v, int64_t num_slots,
                                         int64_t slot_capacity, int64_t slot, int64_t slot_offset,
                                         void *stream);

#ifdef __cplusplus
}
#endif

#endif /* JOYOMNI_HIP_H_ */
