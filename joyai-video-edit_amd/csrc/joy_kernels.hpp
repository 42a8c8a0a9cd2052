// Internal launch interface between the C ABI (capi.hip) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace joy {

// Token-strided [tokens, H, D] bf16 views (strides in elements per token).
struct NormRopeArgs {
  const uint16_t* q_in;  // null: Q is neither read nor written
  const uint16_t* k_in;
  const uint16_t* v_in;  // may be null
  int64_t in_stride;
  uint16_t* q_out;
  int64_t q_out_stride;
  uint16_t* k_out;  // may be null
  int64_t k_out_stride;
  uint16_t* kpre_out;  // may be null
  int64_t kpre_stride;
  uint16_t* v_out;  // may be null (requires v_in)
  int64_t v_out_stride;
  uint16_t* v_out2 = nullptr;  // second V destination (joint attention V rows); may be null
  int64_t v_out2_stride = 0;
  const uint16_t* q_weight;
  const uint16_t* k_weight;
  const uint16_t* cos;  // [table_len, D/2]
  const uint16_t* sin;
  int64_t n_tokens;   // tokens processed (B * L)
  int64_t table_len;  // cos/sin row = token % table_len
  int64_t cache_tokens;  // kpre_out / v_out are written for tokens < cache_tokens
  bool cache_post_rope;  // kpre_out receives the rotated K instead of the normalised K
  int num_heads;
  float eps;
};

struct GemmArgs {
  const void* A;  // e4m3fn [M, K] row-major
  const void* W;  // e4m3fn [N, K] row-major (== (K, N) column-major)
  const float* scales_a;
  const float* scales_b;
  const void* bias;  // out dtype [N] or null
  void* C;           // [M, N] with row stride ldc
  int M, N, K;
  int64_t ldc;
  bool out_bf16;
  bool gelu;
  bool force_generic;
  // gated residual epilogue: C = round(residual + round(gemm) * gate[n]) when residual != null
  const void* residual;  // [M, N] of out dtype, row stride ldr (may equal C with ldr == ldc)
  int64_t ldr;
  const void* gate;  // [N] of out dtype
  // split-K workspace (16-byte aligned) or null; used when workspace_bytes covers
  // fp8_gemm_workspace_bytes(M, N, K)
  void* workspace;
  int64_t workspace_bytes;
};

// bf16 [len, H, D] view: element (t, h, d) at ptr[t * stride_token + h * stride_head + d].
struct RowView {
  const uint16_t* ptr;  // null = absent segment
  int64_t stride_token;
  int64_t stride_head;
};

// fused_joint_qkv_pack: outputs are dense [rows, 128].
struct JointPackArgs {
  RowView img_q, img_k, img_v, txt_q, txt_k, txt_v, cache_k, cache_v;
  const uint16_t* txt_q_weight;
  const uint16_t* txt_k_weight;
  uint16_t* out_q;
  uint16_t* out_k;
  uint16_t* out_v;
  int64_t img_len, txt_len, cache_len;
  int heads;
  float eps;
};

// fused_cached_kv_pack: cos/sin fp32 [len0 + len1, 128]; outputs dense [rows, 128].
struct CachedPackArgs {
  RowView key0, value0, key1, value1;
  const float* cos;
  const float* sin;
  uint16_t* out_k;
  uint16_t* out_v;
  int64_t len0, len1;
  int heads;
};

// Attention forward: bf16 [len, H, 128] views; out [q_len, H, 128] with token stride.
struct AttnArgs {
  RowView q, k, v;
  uint16_t* out;
  int64_t out_stride_token;
  int64_t q_len, k_len;
  int heads;
  float scale_log2e;  // softmax scale * log2(e)
};

// (Layer|RMS)Norm + adaLN scale/shift, optionally + per-token FP8 of the output.
struct NormModArgs {
  const void* x;        // [M, N] rows with stride x_stride (elements)
  int64_t x_stride;
  const void* gamma;    // [N] or null
  const void* beta;     // [N] or null (LayerNorm only; used only with gamma)
  const void* scale;    // [mod_rows, N] dense
  const void* shift;
  int64_t mod_rows;     // 1 (broadcast) or M
  void* out;            // [M, N] dense of the input dtype, or null (FP8 variant only)
  void* out_q;          // e4m3fn [M, N] or null (plain variant)
  float* out_s;         // [M]
  int64_t M, N;
  int dtype;            // 0 bf16, 1 fp16, 2 fp32
  int norm_type;        // 0 LayerNorm, 1 RMSNorm
  float eps;
  bool divide;          // FP8 rounding: x / s (true) or x * (1/s)
};

hipError_t launch_per_token_quant(const void* in, bool in_fp16, void* q, float* s, int64_t M,
                                  int64_t K, bool divide, hipStream_t st);
hipError_t launch_qk_norm_rope(const NormRopeArgs& a, int head_dim, hipStream_t st);
hipError_t launch_fp8_gemm(const GemmArgs& g, hipStream_t st);
// The QKV projection (bf16 [M, 3 * heads * head_dim] = g) with the norm/RoPE/ring outputs of a
// (its inputs ignored) written by the GEMM's epilogue where the shape allows it; g.C is the
// scratch for the tiles (or the whole GEMM) that go through the standalone kernel.
hipError_t launch_fp8_gemm_qkv(const GemmArgs& g, const NormRopeArgs& a, int head_dim, hipStream_t st);
int64_t fp8_gemm_qkv_scratch_bytes(int M, int N, int K, int num_heads, int head_dim);
// The scratch a given call needs: also counts what only the call's pointers and strides decide
// (16-byte aligned cos / sin, 31-bit output offsets), which send it to the unfused path.
int64_t fp8_gemm_qkv_call_scratch_bytes(const GemmArgs& g, const NormRopeArgs& a, int head_dim);
// Workspace bytes the GEMM of this shape can use on the current device (0: none).
int64_t fp8_gemm_workspace_bytes(int M, int N, int K);
hipError_t launch_norm_modulate(const NormModArgs& a, hipStream_t st);
hipError_t launch_joint_qkv_pack(const JointPackArgs& a, hipStream_t st);
hipError_t launch_cached_kv_pack(const CachedPackArgs& a, hipStream_t st);
hipError_t launch_attention_fwd(const AttnArgs& a, hipStream_t st);

// Compute units of the current device, and workgroups of `threads` threads of `kern` that
// stay resident per CU (HIP occupancy API, at least 1); both cached (device_info.hip).
int device_cus();
int resident_blocks(const void* kern, int threads);

}  // namespace joy
