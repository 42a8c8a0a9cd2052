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

#define JOY_ABI_VERSION 10

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

typedef enum { JOY_DTYPE_BF16 = 0, JOY_DTYPE_FP16 = 1, JOY_DTYPE_FP32 = 2 } joy_dtype;

typedef enum { JOY_NORM_LAYER = 0, JOY_NORM_RMS = 1 } joy_norm_type;

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
 * Optional set-up (no reference counterpart): resolves, for every visible device, the
 * per-device library state that an entry point otherwise sets up on its first call on
 * that device -- today the address of joy_fp8_scaled_mm_noalloc's scratch array
 * (hipGetSymbolAddress, which may load the code object). Call it once per process before
 * capturing into a HIP graph a joy_fp8_scaled_mm_noalloc call that may be the first on its
 * device, so that the captured call makes no runtime query. Allocates nothing; leaves the
 * caller's current device unchanged; returns JOY_OK with no visible device.
 */
JOY_API joy_status joy_init(void);

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
 * workspace: caller-owned device memory for split-K partial sums (16-byte aligned), or
 *   NULL. With workspace_bytes >= joy_fp8_scaled_mm_workspace_size(M, N, K) the small-M
 *   plans split K over more blocks (fp32 partials, summed in a fixed order, so results do
 *   not depend on timing); with less, the same tiles run without the split. Like the
 *   reference op's output allocation, the torch layer allocates it (fp8_gemm.cu:1486).
 */
JOY_API joy_status joy_fp8_scaled_mm(const void *mat_a, const void *mat_b, const float *scales_a,
                             const float *scales_b, const void *bias, void *out, int out_dtype,
                             int64_t M, int64_t N, int64_t K, int epilogue, void *workspace,
                             int64_t workspace_bytes, void *stream);

/*
 * Bytes of workspace that joy_fp8_scaled_mm / joy_fp8_scaled_mm_gated_residual can use
 * for an (M, N, K) problem on the current device; 0 when no plan splits K (then the
 * workspace argument may be NULL). Negative sizes return 0. No reference counterpart:
 * the reference's CUTLASS/hipBLASLt GEMMs allocate their own workspaces internally.
 */
JOY_API int64_t joy_fp8_scaled_mm_workspace_size(int64_t M, int64_t N, int64_t K);

/*
 * Bytes of the library-owned split-K scratch that joy_fp8_scaled_mm_noalloc uses
 * (one file-scope device array, held by every GPU the library runs on until the
 * process ends).
 */
#define JOY_FP8_NOALLOC_SCRATCH_BYTES (32LL * 1024 * 1024)

/*
 * joy_fp8_scaled_mm without a workspace argument: allocates nothing (no hipMalloc, no
 * hipFree, no allocating library call), for callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid it). No counterpart in
 * the reference. Same arguments, rules and results as joy_fp8_scaled_mm with a
 * workspace of joy_fp8_scaled_mm_workspace_size(M, N, K) bytes; the split-K partial
 * sums go to the library's scratch array of JOY_FP8_NOALLOC_SCRATCH_BYTES instead.
 * Problems whose split-K plan needs more scratch than that return
 * JOY_ERR_UNSUPPORTED before anything is launched. Every call on one GPU shares that
 * GPU's scratch: calls that overlap on one GPU (different streams or threads) race.
 * The scratch address is resolved by joy_init() or, failing that, on the first call on
 * each device (call joy_init() before capturing such a first call into a HIP graph).
 */
JOY_API joy_status joy_fp8_scaled_mm_noalloc(const void *mat_a, const void *mat_b, const float *scales_a,
                                             const float *scales_b, const void *bias, void *out, int out_dtype,
                                             int64_t M, int64_t N, int64_t K, int epilogue, void *stream);

/*
 * FP8 GEMM with the gated residual of the DiT block fused into its epilogue (new
 * op, no single reference counterpart): the out-projection / FFN-down Fp8Linear
 * (fp8_linear.py:114-141) followed by fused_add_gate = torch.addcmul(residual, y,
 * gate) (deploy/xvideo/models/dit/sgl_fused_ops.py:302-305, dit.py:525-528,535-538):
 *   y        = round(fma(acc[m,n] * scales_b[n], scales_a[m], bias[n]))   as joy_fp8_scaled_mm
 *   out[m,n] = round(residual[m,n] + y * gate[n])                        (fp32, one rounding)
 * residual: [M, N] of out_dtype with row stride residual_stride (elements); gate: [N]
 * of out_dtype. out may be residual itself (in place; then residual_stride == N).
 * Argument rules and workspace otherwise as joy_fp8_scaled_mm.
 */
JOY_API joy_status joy_fp8_scaled_mm_gated_residual(const void *mat_a, const void *mat_b,
                                            const float *scales_a, const float *scales_b,
                                            const void *bias, const void *residual,
                                            int64_t residual_stride, const void *gate, void *out,
                                            int out_dtype, int64_t M, int64_t N, int64_t K,
                                            void *workspace, int64_t workspace_bytes, void *stream);

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
 * q_out, k_out, v_out: bf16 [seq_len, num_heads, head_dim] with token strides (elements);
 *   each may be NULL (q_out NULL: Q is not read, as in the reference's cache-only
 *   forward, dit.py:446-459). v_out receives V itself (e.g. the video rows of the
 *   joint attention V, dit.py:489-496), so the joint pack need not copy them.
 * cache_k, cache_v: bf16 rings [num_slots, slot_capacity, num_heads, head_dim]
 *   (either both NULL or both set). The first cache_tokens tokens (0 <= cache_tokens
 *   <= seq_len; kv_cache_write_seq_len of dit.py:449-451, e.g. the current chunk
 *   without its ref-video tokens) go to rows slot_offset .. slot_offset+cache_tokens-1
 *   of slot `slot`: cache_v gets a copy of V; cache_k gets the normalised K before
 *   rotation (cache_post_rope == 0, kv_cache_pre_rope=True) or the rotated K
 *   (cache_post_rope != 0, the reference's default post-RoPE cache, dit.py:432-433).
 */
JOY_API joy_status joy_fused_qkv_norm_rope_cache(const void *qkv, int64_t qkv_row_stride, int64_t seq_len,
                                         int64_t num_heads, int64_t head_dim, float eps,
                                         const void *q_weight, const void *k_weight,
                                         const void *cos, const void *sin, void *q_out,
                                         int64_t q_out_stride, void *k_out, int64_t k_out_stride,
                                         void *v_out, int64_t v_out_stride,
                                         void *cache_k, void *cache_v, int64_t num_slots,
                                         int64_t slot_capacity, int64_t slot, int64_t slot_offset,
                                         int64_t cache_tokens, int cache_post_rope, void *stream);

/*
 * The QKV projection and joy_fused_qkv_norm_rope_cache in one call (new op, no single
 * reference counterpart): the image stream's QKV Fp8Linear (deploy/xvideo/models/dit/dit.py:409,
 * fp8_linear.py:114-141 on quantised activations) followed by the split, q/k RMSNorm, RoPE and
 * ring write of dit.py:409-451 -- joy_fp8_scaled_mm (bf16 out, [M, 3*num_heads*head_dim]) then
 * joy_fused_qkv_norm_rope_cache with seq_len = M and qkv its output, with the same results bit
 * for bit. Where the shape allows (head_dim 128, an even num_heads, K % 256 == 0, 32-bit
 * offsets) the GEMM's epilogue does the norm, rotation and writes itself, so the QKV rows never
 * reach HBM; the tiles of a last, partial round (and other shapes entirely) go through
 * `scratch` (bf16 [M, 3*num_heads*head_dim]) and the standalone kernel.
 * GEMM arguments as joy_fp8_scaled_mm (mat_b: [3*num_heads*head_dim, K] e4m3fn, bias bf16 or
 * NULL); norm/RoPE/ring arguments as joy_fused_qkv_norm_rope_cache (cos/sin [M, head_dim/2]).
 * scratch: 16-byte aligned device memory of at least joy_fp8_qkv_norm_rope_cache_scratch_size
 * bytes (may be NULL when that is 0) when cos / sin are 16-byte aligned and every output's
 * ((rows - 1) * stride + num_heads * head_dim) * 2 is below 2^31; otherwise M * 3 * num_heads *
 * head_dim * 2 bytes (the call then runs the GEMM and the standalone kernel). Too little
 * scratch for the call is JOY_ERR_INVALID_ARGUMENT, before any launch.
 */
JOY_API joy_status joy_fp8_qkv_norm_rope_cache(const void *mat_a, const void *mat_b, const float *scales_a,
                                               const float *scales_b, const void *bias, int64_t M, int64_t K,
                                               int64_t num_heads, int64_t head_dim, float eps,
                                               const void *q_weight, const void *k_weight, const void *cos,
                                               const void *sin, void *q_out, int64_t q_out_stride, void *k_out,
                                               int64_t k_out_stride, void *v_out, int64_t v_out_stride,
                                               void *cache_k, void *cache_v, int64_t num_slots,
                                               int64_t slot_capacity, int64_t slot, int64_t slot_offset,
                                               int64_t cache_tokens, int cache_post_rope, void *scratch,
                                               int64_t scratch_bytes, void *stream);

/* Bytes of scratch joy_fp8_qkv_norm_rope_cache needs with 16-byte aligned cos / sin and outputs of
 * token stride num_heads * head_dim (0 when every tile takes the fused epilogue). */
JOY_API int64_t joy_fp8_qkv_norm_rope_cache_scratch_size(int64_t M, int64_t K, int64_t num_heads,
                                                         int64_t head_dim);

/*
 * A bf16 [len, num_heads, head_dim] view with a dense last dimension: element
 * (t, h, d) is at ((const uint16_t *)ptr)[t * stride_token + h * stride_head + d]
 * (strides in elements). This is what a reference [1, L, H, D] tensor with
 * stride(3) == 1 passes (fused_joint_qkv_pack.cu:222-229), e.g. the q/k/v
 * slices of the QKV projection output.
 */
typedef struct {
  const void *ptr;
  int64_t len;
  int64_t stride_token;
  int64_t stride_head;
} joy_bf16_view;

/*
 * Joint-attention Q/K/V pack with text Q/K RMSNorm.
 * Replaces: fused_joint_qkv_pack(Tensor img_q, Tensor img_k, Tensor img_v, Tensor txt_q,
 *           Tensor txt_k, Tensor txt_v, Tensor? cached_k, Tensor? cached_v,
 *           Tensor txt_q_weight, Tensor txt_k_weight, float eps) -> (Tensor, Tensor, Tensor)
 *   schema joyomni_ops/csrc/pybind.cpp:56-59, impl joyomni_ops/csrc/fused_joint_qkv_pack.cu:237-342
 *   (kernel :81-164).
 *   out_q = [img_q | rms(txt_q)]            dense [img_len + txt_len, H, D]
 *   out_k = [cached_k | img_k | rms(txt_k)]  dense [cache_len + img_len + txt_len, H, D]
 *   out_v = [cached_v | img_v | txt_v]       same shape as out_k
 *   rms(x) = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)  (two roundings, :58-79)
 * cached_k, cached_v: NULL (or ptr NULL) for no cache; both or neither.
 * Outputs are caller-allocated (the reference allocates them, :290-293).
 * head_dim must be 128 (reference rule); img_len, txt_len, num_heads > 0.
 */
JOY_API joy_status joy_fused_joint_qkv_pack(const joy_bf16_view *img_q, const joy_bf16_view *img_k,
                                    const joy_bf16_view *img_v, const joy_bf16_view *txt_q,
                                    const joy_bf16_view *txt_k, const joy_bf16_view *txt_v,
                                    const joy_bf16_view *cached_k, const joy_bf16_view *cached_v,
                                    const void *txt_q_weight, const void *txt_k_weight, float eps,
                                    int64_t num_heads, int64_t head_dim, void *out_q, void *out_k,
                                    void *out_v, void *stream);

/*
 * The condition (text) segment of the joint pack, written where the caller says
 * (new op): with the video rows of the joint Q/K/V written by
 * joy_fused_qkv_norm_rope_cache and the cached rows by joy_fused_cached_kv_pack,
 * this completes the joint attention operands of fused_joint_qkv_pack
 * (joyomni_ops/csrc/fused_joint_qkv_pack.cu:81-164,237-342; dit.py:489-496) without
 * copying the cached and video rows a second time.
 *   out_q = rms(txt_q), out_k = rms(txt_k), out_v = txt_v     dense [txt_len, H, D] each
 *   rms(x) = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)        (two roundings, :58-79)
 * Argument rules as joy_fused_joint_qkv_pack (head_dim 128, txt_len, num_heads > 0).
 */
JOY_API joy_status joy_fused_text_qkv_pack(const joy_bf16_view *txt_q, const joy_bf16_view *txt_k,
                                   const joy_bf16_view *txt_v, const void *txt_q_weight,
                                   const void *txt_k_weight, float eps, int64_t num_heads,
                                   int64_t head_dim, void *out_q, void *out_k, void *out_v,
                                   void *stream);

/*
 * Rotate and pack one or two pre-RoPE cached K segments with their V.
 * Replaces: fused_cached_kv_pack(Tensor key0, Tensor value0, Tensor? key1, Tensor? value1,
 *           Tensor cos, Tensor sin) -> (Tensor, Tensor)
 *   schema joyomni_ops/csrc/pybind.cpp:60-62, impl joyomni_ops/csrc/fused_joint_qkv_pack.cu:344-415
 *   (kernel :166-220).
 *   out_k[t] = rotate(key[t]) with pair (2i, 2i+1):
 *     o_2i = k_2i * c - k_2i+1 * s ; o_2i+1 = k_2i * s + k_2i+1 * c, c, s = cos/sin[t * D + 2i]
 *   out_v[t] = value[t]; t runs over key0's tokens, then key1's.
 * cos, sin: fp32 [len0 + len1, head_dim] (full width, repeat_interleave layout).
 * key1/value1: NULL (or ptr NULL) for one segment; both or neither.
 * Outputs: caller-allocated dense [len0 + len1, H, D], e.g. the cached rows at the
 * head of the joint attention K / V. A ring slot (rows of cache_k[slot]) is a valid
 * key view, so this reads the KV ring directly.
 * head_dim must be 128; len0, num_heads > 0; len1 > 0 when present.
 */
JOY_API joy_status joy_fused_cached_kv_pack(const joy_bf16_view *key0, const joy_bf16_view *value0,
                                    const joy_bf16_view *key1, const joy_bf16_view *value1,
                                    const float *cos, const float *sin, int64_t num_heads,
                                    int64_t head_dim, void *out_k, void *out_v, void *stream);

/*
 * Joint-attention forward (new op): per head, out = softmax(q k^T * scale) v,
 * non-causal, no mask, bf16 inputs and output, fp32 softmax and accumulation.
 * Replaces: _sdpa_attention(query, key, value) at deploy/xvideo/models/dit/dit.py:154-167,
 *   i.e. F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2),
 *   v.transpose(1, 2), is_causal=False) on bf16 [1, S, H, D] tensors (default scale
 *   1/sqrt(D)), as called on the joint Q / K / V at dit.py:489-498.
 * q: view of q->len query tokens; k, v: views of the same number of key tokens
 *   (k->len > 0), all [len, num_heads, head_dim] with 16-byte aligned rows.
 * out: caller-allocated bf16 [q->len, num_heads, head_dim], heads dense, token stride
 *   out_stride_token (elements, >= num_heads * head_dim), 16-byte aligned rows.
 * head_dim must be 128 (JOY_ERR_UNSUPPORTED otherwise). scale > 0 (1/sqrt(head_dim)
 * reproduces the reference default).
 */
JOY_API joy_status joy_attention_fwd(const joy_bf16_view *q, const joy_bf16_view *k, const joy_bf16_view *v,
                                     void *out, int64_t out_stride_token, int64_t num_heads, int64_t head_dim,
                                     float scale, void *stream);

/*
 * (Layer|RMS)Norm + adaLN scale/shift.
 * Replaces: fused_norm_scale_shift(Tensor x, Tensor? gamma_opt, Tensor? beta_opt, Tensor scale,
 *           Tensor shift, int norm_type, float eps) -> Tensor
 *   schema joyomni_ops/csrc/pybind.cpp:63-65, impl joyomni_ops/csrc/fused_norm_scale_shift.cu:236-275
 *   (kernel :97-182), called by fused_layernorm_modulate (deploy/xvideo/models/dit/sgl_fused_ops.py:46-91).
 *   LayerNorm: out = ((x - mean) * rsqrt(var + eps) * gamma + beta) * (1 + scale) + shift
 *   RMSNorm:   out = (x * rsqrt(mean(x^2) + eps) * gamma) * (1 + scale) + shift
 * x: [M, N] of dtype (bf16, fp16 or fp32), rows x_row_stride elements apart.
 * gamma, beta: [N] of dtype or NULL; as in the reference, beta is applied only
 *   together with gamma (LayerNorm), and gamma without beta means beta = 0.
 * scale, shift: dense [mod_rows, N] of dtype, mod_rows 1 (broadcast) or M.
 * out: caller-allocated dense [M, N] of dtype (the reference allocates it).
 * Reference rules kept: N % 4 == 0, norm_type 0 or 1.
 */
JOY_API joy_status joy_fused_norm_scale_shift(const void *x, int64_t x_row_stride, int dtype,
                                      const void *gamma, const void *beta, const void *scale,
                                      const void *shift, int64_t mod_rows, void *out, int64_t M,
                                      int64_t N, int norm_type, float eps, void *stream);

/*
 * (Layer|RMS)Norm + adaLN scale/shift emitting the per-token FP8 quantisation of
 * its output (new op, no reference counterpart: it fuses
 * fused_layernorm_modulate (sgl_fused_ops.py:46-91) with the activation
 * quantiser of the Fp8Linear that consumes it, fp8_linear.py:38-43 / :57-74).
 * y = the bf16/fp16 output of joy_fused_norm_scale_shift (same arguments);
 * output_s[m] = max(absmax_n |y[m, n]|, 1e-8) / 448,
 * output_q[m, n] = e4m3fn(clamp(y / s)) (JOY_QUANT_DIVIDE) or clamp(y * (1/s)) (JOY_QUANT_RECIPROCAL),
 * bit-identical to joy_per_token_quant_fp8 applied to y. out (y itself) may be NULL.
 * dtype must be bf16 or fp16.
 */
JOY_API joy_status joy_fused_norm_scale_shift_fp8(const void *x, int64_t x_row_stride, int dtype,
                                          const void *gamma, const void *beta, const void *scale,
                                          const void *shift, int64_t mod_rows, void *out,
                                          void *output_q, float *output_s, int rounding, int64_t M,
                                          int64_t N, int norm_type, float eps, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* JOYOMNI_HIP_H_ */
