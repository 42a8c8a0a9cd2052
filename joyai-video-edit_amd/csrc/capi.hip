// C ABI of libjoyomni_hip: argument validation (mirroring the reference's
// TORCH_CHECKs), then one kernel launch on the caller's stream.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "../../include/joyomni_hip.h"
#include "joy_kernels.hpp"

namespace {

thread_local char g_err[512] = "";

joy_status fail(joy_status st, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return st;
}

joy_status ok() {
  g_err[0] = '\0';
  return JOY_OK;
}

joy_status hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail(JOY_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

// The norm/RoPE kernel indexes (token, head) units with 32-bit integers.
constexpr int64_t kMaxUnits = 0x7ff00000LL;

// Argument rules of the GEMM entry points; fills g. *empty: nothing to launch (M or N is 0).
// out_optional: out may be null (the fused QKV projection's scratch when no tile needs it).
joy_status gemm_args(const void* mat_a, const void* mat_b, const float* scales_a, const float* scales_b,
                     const void* bias, void* out, int out_dtype, int64_t M, int64_t N, int64_t K, int epilogue,
                     const void* residual, int64_t residual_stride, const void* gate, void* workspace,
                     int64_t workspace_bytes, bool out_optional, joy::GemmArgs& g, bool* empty) {
  *empty = false;
  if (M < 0 || N < 0 || K < 0) return fail(JOY_ERR_INVALID_ARGUMENT, "mat_a and mat_b shapes cannot be multiplied");
  if (K % 16 != 0)
    return fail(JOY_ERR_INVALID_ARGUMENT, "mat_a must be multiple of 16 bytes for memory alignment");
  if (out_dtype != JOY_DTYPE_BF16 && out_dtype != JOY_DTYPE_FP16)
    return fail(JOY_ERR_INVALID_ARGUMENT, "out_dtype must be Half or BFloat16");
  if (N % 8 != 0)
    return fail(JOY_ERR_INVALID_ARGUMENT, "out must be multiple of 16 bytes for memory alignment");
  if (epilogue != JOY_EPILOGUE_NONE && epilogue != JOY_EPILOGUE_GELU_TANH)
    return fail(JOY_ERR_INVALID_ARGUMENT, "unknown epilogue %d", epilogue);
  if (M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL)
    return fail(JOY_ERR_UNSUPPORTED, "dimensions above 2^31-1 are not supported");
  if (residual && residual_stride < N) return fail(JOY_ERR_INVALID_ARGUMENT, "residual row stride must be >= N");
  if (residual && !gate) return fail(JOY_ERR_INVALID_ARGUMENT, "gate must be non-null");
  if (residual && residual == out && residual_stride != N)
    return fail(JOY_ERR_INVALID_ARGUMENT, "an in-place residual must have row stride N");
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace))
    return fail(JOY_ERR_INVALID_ARGUMENT, "workspace_bytes must be >= 0, with a workspace when > 0");
  if (workspace && !aligned(workspace, 16))
    return fail(JOY_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  if (M == 0 || N == 0) {
    *empty = true;
    return ok();
  }
  if ((!out && !out_optional) || !scales_a || !scales_b || (K > 0 && (!mat_a || !mat_b)))
    return fail(JOY_ERR_INVALID_ARGUMENT, "mat_a, mat_b, scales and out must be non-null");
  if (!aligned(mat_a, 16) || !aligned(mat_b, 16) || !aligned(out, 16) || !aligned(scales_b, 16))
    return fail(JOY_ERR_UNSUPPORTED, "mat_a, mat_b, out and scales_b must be 16-byte aligned");
  if (!aligned(scales_a, 4) || (bias && !aligned(bias, 2)) || (residual && (!aligned(residual, 2) || !aligned(gate, 2))))
    return fail(JOY_ERR_INVALID_ARGUMENT, "scales_a, bias, residual and gate must be naturally aligned");
  g = joy::GemmArgs{};
  g.A = mat_a;
  g.W = mat_b;
  g.scales_a = scales_a;
  g.scales_b = scales_b;
  g.bias = bias;
  g.C = out;
  g.M = (int)M;
  g.N = (int)N;
  g.K = (int)K;
  g.ldc = N;
  g.out_bf16 = out_dtype == JOY_DTYPE_BF16;
  g.gelu = epilogue == JOY_EPILOGUE_GELU_TANH;
  g.force_generic = (K == 0);
  g.residual = residual;
  g.ldr = residual_stride;
  g.gate = gate;
  g.workspace = workspace;
  g.workspace_bytes = workspace ? workspace_bytes : 0;
  return ok();
}

joy_status scaled_mm_common(const void* mat_a, const void* mat_b, const float* scales_a, const float* scales_b,
                            const void* bias, void* out, int out_dtype, int64_t M, int64_t N, int64_t K,
                            int epilogue, const void* residual, int64_t residual_stride, const void* gate,
                            void* workspace, int64_t workspace_bytes, void* stream) {
  joy::GemmArgs g;
  bool empty;
  const joy_status st = gemm_args(mat_a, mat_b, scales_a, scales_b, bias, out, out_dtype, M, N, K, epilogue, residual,
                                  residual_stride, gate, workspace, workspace_bytes, false, g, &empty);
  if (st != JOY_OK || empty) return st;
  return hip_status(joy::launch_fp8_gemm(g, (hipStream_t)stream),
                    residual ? "fp8_scaled_mm_gated_residual launch" : "fp8_scaled_mm launch");
}


// Split-K scratch of joy_fp8_scaled_mm_noalloc: one device array per GPU, part of the
// library's code object. Host code never passes the array's name to a kernel (on the
// host it is a stand-in, not a device address); it uses the per-device address that
// hipGetSymbolAddress returns, fetched once per device on that device's first call.
static __device__ __align__(256) unsigned char scratch[JOY_FP8_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Address of the scratch array on device `dev`, which must be the current device.
joy_status resolve_scratch(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return fail(JOY_ERR_UNSUPPORTED, "device %d: at most %d devices", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e, "hipGetSymbolAddress(scratch)");
    g_scratch_ptr[dev] = p;
  }
  return JOY_OK;
}

joy_status scratch_for_current_device(void** out) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "hipGetDevice");
  const joy_status st = resolve_scratch(dev);
  if (st != JOY_OK) return st;
  *out = g_scratch_ptr[dev];
  return JOY_OK;
}

// Argument rules of the fused norm/RoPE/ring ops; fills a. With qkv == nullptr (the fused QKV
// projection, whose GEMM makes the input) the input checks are skipped and a's inputs stay
// null. *empty: nothing to launch.
joy_status norm_rope_args(const void* qkv, int64_t qkv_row_stride, int64_t seq_len, int64_t num_heads,
                          int64_t head_dim, float eps, const void* q_weight, const void* k_weight, const void* cos,
                          const void* sin, void* q_out, int64_t q_out_stride, void* k_out, int64_t k_out_stride,
                          void* v_out, int64_t v_out_stride, void* cache_k, void* cache_v, int64_t num_slots,
                          int64_t slot_capacity, int64_t slot, int64_t slot_offset, int64_t cache_tokens,
                          int cache_post_rope, joy::NormRopeArgs& a, bool* empty) {
  *empty = false;
  if (seq_len < 0 || num_heads < 0) return fail(JOY_ERR_INVALID_ARGUMENT, "seq_len and num_heads must be >= 0");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(JOY_ERR_INVALID_ARGUMENT, "Unsupported head_dim: %lld", (long long)head_dim);
  if (num_heads > 0x7fffffffLL) return fail(JOY_ERR_UNSUPPORTED, "num_heads too large");
  const int64_t E = num_heads * head_dim;
  if (qkv && qkv_row_stride < 3 * E) return fail(JOY_ERR_INVALID_ARGUMENT, "qkv row stride must be >= 3*num_heads*head_dim");
  if ((q_out && q_out_stride < E) || (k_out && k_out_stride < E) || (v_out && v_out_stride < E))
    return fail(JOY_ERR_INVALID_ARGUMENT, "q_out/k_out/v_out token stride must be >= num_heads*head_dim");
  if ((cache_k == nullptr) != (cache_v == nullptr))
    return fail(JOY_ERR_INVALID_ARGUMENT, "cache_k and cache_v must be provided together");
  if (cache_k) {
    if (num_slots <= 0 || slot_capacity < 0)
      return fail(JOY_ERR_INVALID_ARGUMENT, "cache must have num_slots > 0 and slot_capacity >= 0");
    if (slot < 0 || slot >= num_slots)
      return fail(JOY_ERR_INVALID_ARGUMENT, "slot %lld out of range [0, %lld)", (long long)slot,
                  (long long)num_slots);
    if (cache_tokens < 0 || cache_tokens > seq_len)
      return fail(JOY_ERR_INVALID_ARGUMENT, "cache_tokens %lld out of range [0, seq_len = %lld]",
                  (long long)cache_tokens, (long long)seq_len);
    if (slot_offset < 0 || slot_offset + cache_tokens > slot_capacity)
      return fail(JOY_ERR_INVALID_ARGUMENT, "tokens [%lld, %lld) do not fit a slot of %lld tokens",
                  (long long)slot_offset, (long long)(slot_offset + cache_tokens), (long long)slot_capacity);
  }
  if ((!q_out && !k_out && !v_out && !cache_k) || seq_len == 0 || num_heads == 0) {  // nothing to write
    *empty = true;
    return ok();
  }
  if (seq_len * num_heads > kMaxUnits)
    return fail(JOY_ERR_UNSUPPORTED, "seq_len*num_heads above 2^31 - 2^20");
  if (!q_weight || !k_weight || !cos || !sin)
    return fail(JOY_ERR_INVALID_ARGUMENT, "qkv, weights and cos/sin must be non-null");
  if ((qkv && (qkv_row_stride % 8)) || (q_out && (q_out_stride % 8)) || (k_out && (k_out_stride % 8)) ||
      (v_out && (v_out_stride % 8)))
    return fail(JOY_ERR_UNSUPPORTED, "token strides must be multiples of 8 elements");
  if ((qkv && !aligned(qkv, 16)) || (q_out && !aligned(q_out, 16)) || (k_out && !aligned(k_out, 16)) ||
      (v_out && !aligned(v_out, 16)) ||
      (cache_k && (!aligned(cache_k, 16) || !aligned(cache_v, 16))) || !aligned(q_weight, 16) ||
      !aligned(k_weight, 16) || !aligned(cos, 8) || !aligned(sin, 8))
    return fail(JOY_ERR_UNSUPPORTED, "tensors must be 16-byte aligned (cos/sin 8-byte)");
  const uint16_t* base = (const uint16_t*)qkv;
  a = joy::NormRopeArgs{};
  a.q_in = q_out && qkv ? base : nullptr;
  a.k_in = qkv ? base + E : nullptr;
  a.v_in = (cache_v || v_out) && qkv ? base + 2 * E : nullptr;
  a.in_stride = qkv_row_stride;
  a.q_out = (uint16_t*)q_out;
  a.q_out_stride = q_out_stride;
  a.k_out = (uint16_t*)k_out;
  a.k_out_stride = k_out_stride;
  const int64_t slot_base = cache_k ? (slot * slot_capacity + slot_offset) * E : 0;
  a.kpre_out = cache_k ? (uint16_t*)cache_k + slot_base : nullptr;
  a.kpre_stride = E;
  a.v_out = cache_v ? (uint16_t*)cache_v + slot_base : nullptr;
  a.v_out_stride = E;
  a.v_out2 = (uint16_t*)v_out;
  a.v_out2_stride = v_out_stride;
  a.q_weight = (const uint16_t*)q_weight;
  a.k_weight = (const uint16_t*)k_weight;
  a.cos = (const uint16_t*)cos;
  a.sin = (const uint16_t*)sin;
  a.n_tokens = seq_len;
  a.table_len = seq_len;
  a.cache_tokens = cache_k ? cache_tokens : 0;
  a.cache_post_rope = cache_post_rope != 0;
  a.num_heads = (int)num_heads;
  a.eps = eps;
  return ok();
}



}  // namespace

extern "C" {

int joy_abi_version(void) { return JOY_ABI_VERSION; }

const char* joy_last_error(void) { return g_err; }

joy_status joy_init(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
    (void)hipGetLastError();  // no visible device: nothing to resolve
    return ok();
  }
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return hip_status(e, "hipGetDevice");
  for (int d = 0; d < n && d < kMaxDevices; ++d) {
    e = hipSetDevice(d);
    if (e != hipSuccess) return hip_status(e, "hipSetDevice");
    const joy_status st = resolve_scratch(d);
    if (st != JOY_OK) {
      (void)hipSetDevice(cur);
      return st;
    }
  }
  return hip_status(hipSetDevice(cur), "hipSetDevice");
}

joy_status joy_per_token_quant_fp8(const void* input, int input_dtype, void* output_q,
                                   float* output_s, int64_t M, int64_t K, int rounding,
                                   void* stream) {
  if (M < 0 || K < 0) return fail(JOY_ERR_INVALID_ARGUMENT, "input must be [M, K]");
  if (input_dtype != JOY_DTYPE_BF16 && input_dtype != JOY_DTYPE_FP16)
    return fail(JOY_ERR_INVALID_ARGUMENT, "input must be bfloat16 or float16");
  if (rounding != JOY_QUANT_DIVIDE && rounding != JOY_QUANT_RECIPROCAL)
    return fail(JOY_ERR_INVALID_ARGUMENT, "rounding must be JOY_QUANT_DIVIDE or JOY_QUANT_RECIPROCAL");
  if (M > 0 && !output_s) return fail(JOY_ERR_INVALID_ARGUMENT, "output_s must contain one scale per row");
  if (M > 0 && K > 0 && (!input || !output_q))
    return fail(JOY_ERR_INVALID_ARGUMENT, "input and output_q must be non-null");
  if (M > 0x7fffffffLL * 4) return fail(JOY_ERR_UNSUPPORTED, "M too large");
  if (M == 0) return ok();
  return hip_status(joy::launch_per_token_quant(input, input_dtype == JOY_DTYPE_FP16, output_q,
                                                output_s, M, K, rounding == JOY_QUANT_DIVIDE,
                                                (hipStream_t)stream),
                    "per_token_quant_fp8 launch");
}


joy_status joy_fp8_scaled_mm(const void* mat_a, const void* mat_b, const float* scales_a,
                             const float* scales_b, const void* bias, void* out, int out_dtype,
                             int64_t M, int64_t N, int64_t K, int epilogue, void* workspace,
                             int64_t workspace_bytes, void* stream) {
  return scaled_mm_common(mat_a, mat_b, scales_a, scales_b, bias, out, out_dtype, M, N, K, epilogue, nullptr, 0,
                          nullptr, workspace, workspace_bytes, stream);
}

joy_status joy_fp8_scaled_mm_noalloc(const void* mat_a, const void* mat_b, const float* scales_a,
                                     const float* scales_b, const void* bias, void* out, int out_dtype, int64_t M,
                                     int64_t N, int64_t K, int epilogue, void* stream) {
  const int64_t need = joy_fp8_scaled_mm_workspace_size(M, N, K);
  if (need > JOY_FP8_NOALLOC_SCRATCH_BYTES)
    return fail(JOY_ERR_UNSUPPORTED,
                "fp8_scaled_mm_noalloc: the split-K plan of %lldx%lldx%lld needs %lld bytes of scratch, "
                "the library holds %lld",
                (long long)M, (long long)N, (long long)K, (long long)need, (long long)JOY_FP8_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need > 0) {
    const joy_status st = scratch_for_current_device(&ws);
    if (st != JOY_OK) return st;
  }
  return scaled_mm_common(mat_a, mat_b, scales_a, scales_b, bias, out, out_dtype, M, N, K, epilogue, nullptr, 0,
                          nullptr, ws, need, stream);
}

int64_t joy_fp8_scaled_mm_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL) return 0;
  return joy::fp8_gemm_workspace_bytes((int)M, (int)N, (int)K);
}

joy_status joy_fp8_scaled_mm_gated_residual(const void* mat_a, const void* mat_b, const float* scales_a,
                                            const float* scales_b, const void* bias, const void* residual,
                                            int64_t residual_stride, const void* gate, void* out, int out_dtype,
                                            int64_t M, int64_t N, int64_t K, void* workspace,
                                            int64_t workspace_bytes, void* stream) {
  if (!residual) return fail(JOY_ERR_INVALID_ARGUMENT, "residual must be non-null");
  return scaled_mm_common(mat_a, mat_b, scales_a, scales_b, bias, out, out_dtype, M, N, K, JOY_EPILOGUE_NONE,
                          residual, residual_stride, gate, workspace, workspace_bytes, stream);
}

joy_status joy_fused_qk_norm_rope_3d_paired(void* q, void* k, int64_t batch, int64_t seq_len,
                                            int64_t num_heads, int64_t head_dim, float eps,
                                            const void* q_weight, const void* k_weight,
                                            const void* cos, const void* sin, void* k_pre_rope,
                                            void* stream) {
  if (batch < 0 || seq_len < 0 || num_heads < 0)
    return fail(JOY_ERR_INVALID_ARGUMENT, "q must be 3D [batch, seq_len*num_heads, head_dim]");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(JOY_ERR_INVALID_ARGUMENT, "Unsupported head_dim for fused_qk_norm_rope_3d_paired: %lld",
                (long long)head_dim);
  if (num_heads > 0x7fffffffLL) return fail(JOY_ERR_UNSUPPORTED, "num_heads too large");
  const int64_t units = batch * seq_len * num_heads;
  if (units == 0) return ok();
  if (units > kMaxUnits) return fail(JOY_ERR_UNSUPPORTED, "batch*seq_len*num_heads above 2^31 - 2^20");
  if (!q || !k || !q_weight || !k_weight || !cos || !sin)
    return fail(JOY_ERR_INVALID_ARGUMENT, "q, k, weights and cos/sin must be non-null");
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(q_weight, 16) || !aligned(k_weight, 16) ||
      !aligned(cos, 8) || !aligned(sin, 8) || (k_pre_rope && !aligned(k_pre_rope, 16)))
    return fail(JOY_ERR_UNSUPPORTED, "q, k, k_pre_rope and weights must be 16-byte aligned, cos/sin 8-byte aligned");
  joy::NormRopeArgs a;
  a.q_in = (const uint16_t*)q;
  a.k_in = (const uint16_t*)k;
  a.v_in = nullptr;
  a.in_stride = num_heads * head_dim;
  a.q_out = (uint16_t*)q;
  a.q_out_stride = a.in_stride;
  a.k_out = (uint16_t*)k;
  a.k_out_stride = a.in_stride;
  a.kpre_out = (uint16_t*)k_pre_rope;
  a.kpre_stride = a.in_stride;
  a.v_out = nullptr;
  a.v_out_stride = 0;
  a.q_weight = (const uint16_t*)q_weight;
  a.k_weight = (const uint16_t*)k_weight;
  a.cos = (const uint16_t*)cos;
  a.sin = (const uint16_t*)sin;
  a.n_tokens = batch * seq_len;
  a.table_len = seq_len;
  a.cache_tokens = batch * seq_len;  // k_pre_rope (if given) for every token
  a.cache_post_rope = false;
  a.num_heads = (int)num_heads;
  a.eps = eps;
  return hip_status(joy::launch_qk_norm_rope(a, (int)head_dim, (hipStream_t)stream),
                    "fused_qk_norm_rope_3d_paired launch");
}

joy_status joy_fused_qkv_norm_rope_cache(const void* qkv, int64_t qkv_row_stride, int64_t seq_len,
                                         int64_t num_heads, int64_t head_dim, float eps,
                                         const void* q_weight, const void* k_weight,
                                         const void* cos, const void* sin, void* q_out,
                                         int64_t q_out_stride, void* k_out, int64_t k_out_stride,
                                         void* v_out, int64_t v_out_stride,
                                         void* cache_k, void* cache_v, int64_t num_slots,
                                         int64_t slot_capacity, int64_t slot, int64_t slot_offset,
                                         int64_t cache_tokens, int cache_post_rope, void* stream) {
  joy::NormRopeArgs a;
  bool empty;
  // a null qkv is checked as the fused QKV projection's (no input) and refused below
  const joy_status st = norm_rope_args(qkv, qkv_row_stride, seq_len, num_heads, head_dim, eps, q_weight, k_weight, cos,
                                       sin, q_out, q_out_stride, k_out, k_out_stride, v_out, v_out_stride, cache_k,
                                       cache_v, num_slots, slot_capacity, slot, slot_offset, cache_tokens,
                                       cache_post_rope, a, &empty);
  if (st != JOY_OK || empty) return st;
  if (!qkv) return fail(JOY_ERR_INVALID_ARGUMENT, "qkv, weights and cos/sin must be non-null");
  return hip_status(joy::launch_qk_norm_rope(a, (int)head_dim, (hipStream_t)stream),
                    "fused_qkv_norm_rope_cache launch");
}

int64_t joy_fp8_qkv_norm_rope_cache_scratch_size(int64_t M, int64_t K, int64_t num_heads, int64_t head_dim) {
  if (M <= 0 || K <= 0 || num_heads <= 0 || head_dim <= 0 || M > 0x7fffffffLL || K > 0x7fffffffLL ||
      3 * num_heads * head_dim > 0x7fffffffLL)
    return 0;
  return joy::fp8_gemm_qkv_scratch_bytes((int)M, (int)(3 * num_heads * head_dim), (int)K, (int)num_heads,
                                         (int)head_dim);
}

joy_status joy_fp8_qkv_norm_rope_cache(const void* mat_a, const void* mat_b, const float* scales_a,
                                       const float* scales_b, const void* bias, int64_t M, int64_t K,
                                       int64_t num_heads, int64_t head_dim, float eps, const void* q_weight,
                                       const void* k_weight, const void* cos, const void* sin, void* q_out,
                                       int64_t q_out_stride, void* k_out, int64_t k_out_stride, void* v_out,
                                       int64_t v_out_stride, void* cache_k, void* cache_v, int64_t num_slots,
                                       int64_t slot_capacity, int64_t slot, int64_t slot_offset,
                                       int64_t cache_tokens, int cache_post_rope, void* scratch,
                                       int64_t scratch_bytes, void* stream) {
  joy::NormRopeArgs a;
  bool empty_n;
  joy_status st = norm_rope_args(nullptr, 0, M, num_heads, head_dim, eps, q_weight, k_weight, cos, sin, q_out,
                                 q_out_stride, k_out, k_out_stride, v_out, v_out_stride, cache_k, cache_v, num_slots,
                                 slot_capacity, slot, slot_offset, cache_tokens, cache_post_rope, a, &empty_n);
  if (st != JOY_OK) return st;
  const int64_t N = 3 * num_heads * head_dim;
  if (scratch_bytes < 0 || (scratch_bytes > 0 && !scratch))
    return fail(JOY_ERR_INVALID_ARGUMENT, "scratch_bytes must be >= 0, with a scratch buffer when > 0");
  joy::GemmArgs g;
  bool empty_g;
  st = gemm_args(mat_a, mat_b, scales_a, scales_b, bias, scratch, JOY_DTYPE_BF16, M, N, K, JOY_EPILOGUE_NONE, nullptr,
                 0, nullptr, nullptr, 0, true, g, &empty_g);
  if (st != JOY_OK || empty_n || empty_g) return st;
  // the size query's figure, or M x N bf16 where this call's pointers or strides rule the fused
  // epilogue out (cos / sin not 16-byte aligned, output offsets past 2^31 bytes)
  const int64_t need = joy::fp8_gemm_qkv_call_scratch_bytes(g, a, (int)head_dim);
  if (scratch_bytes < need)
    return fail(JOY_ERR_INVALID_ARGUMENT,
                "fp8_qkv_norm_rope_cache: %lld bytes of scratch needed for this call, %lld given (cos/sin not "
                "16-byte aligned or output offsets past 2^31 bytes need the M x 3*num_heads*head_dim bf16 buffer)",
                (long long)need, (long long)scratch_bytes);
  return hip_status(joy::launch_fp8_gemm_qkv(g, a, (int)head_dim, (hipStream_t)stream),
                    "fp8_qkv_norm_rope_cache launch");
}

}  // extern "C"

namespace {

bool present(const joy_bf16_view* v) { return v != nullptr && v->ptr != nullptr; }

joy::RowView row_view(const joy_bf16_view* v) {
  joy::RowView r;
  r.ptr = present(v) ? (const uint16_t*)v->ptr : nullptr;
  r.stride_token = present(v) ? v->stride_token : 0;
  r.stride_head = present(v) ? v->stride_head : 0;
  return r;
}

// Largest row count of the pack kernels' grid (16 rows per workgroup).
constexpr int64_t kMaxPackRows = 0xffffffffLL * 16;

joy_status norm_common(const void* x, int64_t x_row_stride, int dtype, const void* gamma, const void* beta,
                       const void* scale, const void* shift, int64_t mod_rows, void* out, void* output_q,
                       float* output_s, int rounding, int64_t M, int64_t N, int norm_type, float eps,
                       bool fp8, void* stream) {
  // checks of fused_norm_scale_shift.cu:243-257
  if (M < 0 || N < 0) return fail(JOY_ERR_INVALID_ARGUMENT, "x must be 2D [M, N]");
  if (N % 4 != 0) return fail(JOY_ERR_INVALID_ARGUMENT, "N must be divisible by 4");
  if (mod_rows != 1 && mod_rows != M)
    return fail(JOY_ERR_INVALID_ARGUMENT, "scale/shift rows must be 1 (broadcast) or M (per-row modulation)");
  if (norm_type != JOY_NORM_LAYER && norm_type != JOY_NORM_RMS)
    return fail(JOY_ERR_INVALID_ARGUMENT, "norm_type must be 0 (layer) or 1 (rms)");
  if (dtype != JOY_DTYPE_BF16 && dtype != JOY_DTYPE_FP16 && dtype != JOY_DTYPE_FP32)
    return fail(JOY_ERR_INVALID_ARGUMENT, "Unsupported dtype; use float32/float16/bfloat16");
  if (fp8 && dtype == JOY_DTYPE_FP32)
    return fail(JOY_ERR_INVALID_ARGUMENT, "the FP8 variant needs bfloat16 or float16 input");
  if (fp8 && rounding != JOY_QUANT_DIVIDE && rounding != JOY_QUANT_RECIPROCAL)
    return fail(JOY_ERR_INVALID_ARGUMENT, "rounding must be JOY_QUANT_DIVIDE or JOY_QUANT_RECIPROCAL");
  if (x_row_stride < N) return fail(JOY_ERR_INVALID_ARGUMENT, "x row stride must be >= N");
  if (M == 0 || N == 0) return ok();
  if (!x || !scale || !shift) return fail(JOY_ERR_INVALID_ARGUMENT, "x, scale and shift must be non-null");
  if (fp8 ? (!output_q || !output_s) : !out)
    return fail(JOY_ERR_INVALID_ARGUMENT, fp8 ? "output_q and output_s must be non-null" : "out must be non-null");
  const uintptr_t esz = dtype == JOY_DTYPE_FP32 ? 4 : 2;
  if (!aligned(x, esz) || !aligned(scale, esz) || !aligned(shift, esz) || (gamma && !aligned(gamma, esz)) ||
      (beta && !aligned(beta, esz)) || (out && !aligned(out, esz)) || (output_s && !aligned(output_s, 4)))
    return fail(JOY_ERR_INVALID_ARGUMENT, "tensors must be naturally aligned");
  joy::NormModArgs a;
  a.x = x;
  a.x_stride = x_row_stride;
  a.gamma = gamma;
  a.beta = gamma ? beta : nullptr;  // the reference applies beta only with gamma (:125-166)
  a.scale = scale;
  a.shift = shift;
  a.mod_rows = mod_rows;
  a.out = out;
  a.out_q = fp8 ? output_q : nullptr;
  a.out_s = fp8 ? output_s : nullptr;
  a.M = M;
  a.N = N;
  a.dtype = dtype;
  a.norm_type = norm_type;
  a.eps = eps;
  a.divide = rounding == JOY_QUANT_DIVIDE;
  return hip_status(joy::launch_norm_modulate(a, (hipStream_t)stream),
                    fp8 ? "fused_norm_scale_shift_fp8 launch" : "fused_norm_scale_shift launch");
}


}  // namespace

extern "C" {


joy_status joy_fused_norm_scale_shift(const void* x, int64_t x_row_stride, int dtype, const void* gamma,
                                      const void* beta, const void* scale, const void* shift,
                                      int64_t mod_rows, void* out, int64_t M, int64_t N, int norm_type,
                                      float eps, void* stream) {
  return norm_common(x, x_row_stride, dtype, gamma, beta, scale, shift, mod_rows, out, nullptr, nullptr,
                     JOY_QUANT_DIVIDE, M, N, norm_type, eps, false, stream);
}

joy_status joy_fused_norm_scale_shift_fp8(const void* x, int64_t x_row_stride, int dtype, const void* gamma,
                                          const void* beta, const void* scale, const void* shift,
                                          int64_t mod_rows, void* out, void* output_q, float* output_s,
                                          int rounding, int64_t M, int64_t N, int norm_type, float eps,
                                          void* stream) {
  return norm_common(x, x_row_stride, dtype, gamma, beta, scale, shift, mod_rows, out, output_q, output_s,
                     rounding, M, N, norm_type, eps, true, stream);
}

joy_status joy_fused_joint_qkv_pack(const joy_bf16_view* img_q, const joy_bf16_view* img_k,
                                    const joy_bf16_view* img_v, const joy_bf16_view* txt_q,
                                    const joy_bf16_view* txt_k, const joy_bf16_view* txt_v,
                                    const joy_bf16_view* cached_k, const joy_bf16_view* cached_v,
                                    const void* txt_q_weight, const void* txt_k_weight, float eps,
                                    int64_t num_heads, int64_t head_dim, void* out_q, void* out_k,
                                    void* out_v, void* stream) {
  // checks of fused_joint_qkv_pack.cu:246-284
  if (!present(img_q) || !present(img_k) || !present(img_v) || !present(txt_q) || !present(txt_k) ||
      !present(txt_v))
    return fail(JOY_ERR_INVALID_ARGUMENT, "img/txt q, k, v must be non-null");
  if (head_dim != 128) return fail(JOY_ERR_INVALID_ARGUMENT, "fused_joint_qkv_pack requires head_dim=128");
  const int64_t img_len = img_q->len;
  if (img_len <= 0 || num_heads <= 0)
    return fail(JOY_ERR_INVALID_ARGUMENT, "image length and heads must be positive");
  if (img_k->len != img_len || img_v->len != img_len)
    return fail(JOY_ERR_INVALID_ARGUMENT, "image Q/K/V lengths must match");
  const int64_t txt_len = txt_q->len;
  if (txt_len <= 0 || txt_k->len != txt_len || txt_v->len != txt_len)
    return fail(JOY_ERR_INVALID_ARGUMENT, "text Q/K/V lengths must match and be positive");
  if (!txt_q_weight || !txt_k_weight)
    return fail(JOY_ERR_INVALID_ARGUMENT, "txt_q_weight and txt_k_weight must be non-null");
  if (present(cached_k) != present(cached_v))
    return fail(JOY_ERR_INVALID_ARGUMENT,
                "cached_k and cached_v must either both be present or both be absent");
  const int64_t cache_len = present(cached_k) ? cached_k->len : 0;
  if (cache_len < 0 || (present(cached_v) && cached_v->len != cache_len))
    return fail(JOY_ERR_INVALID_ARGUMENT, "cached K/V lengths must match");
  if (!out_q || !out_k || !out_v) return fail(JOY_ERR_INVALID_ARGUMENT, "out_q, out_k and out_v must be non-null");
  if (num_heads > 0x7fffffffLL) return fail(JOY_ERR_UNSUPPORTED, "num_heads too large");
  if ((img_len + txt_len) * num_heads + 2 * (cache_len + img_len + txt_len) * num_heads > kMaxPackRows)
    return fail(JOY_ERR_UNSUPPORTED, "too many rows for one launch");
  joy::JointPackArgs a;
  a.img_q = row_view(img_q);
  a.img_k = row_view(img_k);
  a.img_v = row_view(img_v);
  a.txt_q = row_view(txt_q);
  a.txt_k = row_view(txt_k);
  a.txt_v = row_view(txt_v);
  a.cache_k = row_view(cached_k);
  a.cache_v = row_view(cached_v);
  a.txt_q_weight = (const uint16_t*)txt_q_weight;
  a.txt_k_weight = (const uint16_t*)txt_k_weight;
  a.out_q = (uint16_t*)out_q;
  a.out_k = (uint16_t*)out_k;
  a.out_v = (uint16_t*)out_v;
  a.img_len = img_len;
  a.txt_len = txt_len;
  a.cache_len = cache_len;
  a.heads = (int)num_heads;
  a.eps = eps;
  return hip_status(joy::launch_joint_qkv_pack(a, (hipStream_t)stream), "fused_joint_qkv_pack launch");
}

joy_status joy_fused_text_qkv_pack(const joy_bf16_view* txt_q, const joy_bf16_view* txt_k,
                                   const joy_bf16_view* txt_v, const void* txt_q_weight,
                                   const void* txt_k_weight, float eps, int64_t num_heads,
                                   int64_t head_dim, void* out_q, void* out_k, void* out_v, void* stream) {
  // the condition segment of fused_joint_qkv_pack, with its checks (fused_joint_qkv_pack.cu:246-284)
  if (!present(txt_q) || !present(txt_k) || !present(txt_v))
    return fail(JOY_ERR_INVALID_ARGUMENT, "txt q, k, v must be non-null");
  if (head_dim != 128) return fail(JOY_ERR_INVALID_ARGUMENT, "fused_text_qkv_pack requires head_dim=128");
  const int64_t txt_len = txt_q->len;
  if (txt_len <= 0 || num_heads <= 0 || txt_k->len != txt_len || txt_v->len != txt_len)
    return fail(JOY_ERR_INVALID_ARGUMENT, "text Q/K/V lengths must match and be positive");
  if (!txt_q_weight || !txt_k_weight)
    return fail(JOY_ERR_INVALID_ARGUMENT, "txt_q_weight and txt_k_weight must be non-null");
  if (!out_q || !out_k || !out_v) return fail(JOY_ERR_INVALID_ARGUMENT, "out_q, out_k and out_v must be non-null");
  if (num_heads > 0x7fffffffLL) return fail(JOY_ERR_UNSUPPORTED, "num_heads too large");
  if (3 * txt_len * num_heads > kMaxPackRows) return fail(JOY_ERR_UNSUPPORTED, "too many rows for one launch");
  joy::JointPackArgs a;
  a.img_q = a.img_k = a.img_v = row_view(nullptr);
  a.cache_k = a.cache_v = row_view(nullptr);
  a.txt_q = row_view(txt_q);
  a.txt_k = row_view(txt_k);
  a.txt_v = row_view(txt_v);
  a.txt_q_weight = (const uint16_t*)txt_q_weight;
  a.txt_k_weight = (const uint16_t*)txt_k_weight;
  a.out_q = (uint16_t*)out_q;
  a.out_k = (uint16_t*)out_k;
  a.out_v = (uint16_t*)out_v;
  a.img_len = 0;
  a.txt_len = txt_len;
  a.cache_len = 0;
  a.heads = (int)num_heads;
  a.eps = eps;
  return hip_status(joy::launch_joint_qkv_pack(a, (hipStream_t)stream), "fused_text_qkv_pack launch");
}

joy_status joy_fused_cached_kv_pack(const joy_bf16_view* key0, const joy_bf16_view* value0,
                                    const joy_bf16_view* key1, const joy_bf16_view* value1,
                                    const float* cos, const float* sin, int64_t num_heads,
                                    int64_t head_dim, void* out_k, void* out_v, void* stream) {
  // checks of fused_joint_qkv_pack.cu:351-381
  if (!present(key0) || !present(value0))
    return fail(JOY_ERR_INVALID_ARGUMENT, "key0 and value0 must be non-null");
  if (head_dim != 128) return fail(JOY_ERR_INVALID_ARGUMENT, "fused_cached_kv_pack requires head_dim=128");
  const int64_t len0 = key0->len;
  if (len0 <= 0 || num_heads <= 0) return fail(JOY_ERR_INVALID_ARGUMENT, "cache length and heads must be positive");
  if (value0->len != len0) return fail(JOY_ERR_INVALID_ARGUMENT, "key0/value0 lengths must match");
  if (present(key1) != present(value1))
    return fail(JOY_ERR_INVALID_ARGUMENT, "key1 and value1 must either both be present or both be absent");
  const int64_t len1 = present(key1) ? key1->len : 0;
  if (present(key1) && (len1 <= 0 || value1->len != len1))
    return fail(JOY_ERR_INVALID_ARGUMENT, "key1/value1 lengths must match and be positive");
  if (!cos || !sin) return fail(JOY_ERR_INVALID_ARGUMENT, "cos and sin must be non-null");
  if (!out_k || !out_v) return fail(JOY_ERR_INVALID_ARGUMENT, "out_k and out_v must be non-null");
  if (num_heads > 0x7fffffffLL) return fail(JOY_ERR_UNSUPPORTED, "num_heads too large");
  if (2 * (len0 + len1) * num_heads > kMaxPackRows)
    return fail(JOY_ERR_UNSUPPORTED, "too many rows for one launch");
  joy::CachedPackArgs a;
  a.key0 = row_view(key0);
  a.value0 = row_view(value0);
  a.key1 = row_view(key1);
  a.value1 = row_view(value1);
  a.cos = cos;
  a.sin = sin;
  a.out_k = (uint16_t*)out_k;
  a.out_v = (uint16_t*)out_v;
  a.len0 = len0;
  a.len1 = len1;
  a.heads = (int)num_heads;
  return hip_status(joy::launch_cached_kv_pack(a, (hipStream_t)stream), "fused_cached_kv_pack launch");
}


joy_status joy_attention_fwd(const joy_bf16_view* q, const joy_bf16_view* k, const joy_bf16_view* v, void* out,
                             int64_t out_stride_token, int64_t num_heads, int64_t head_dim, float scale,
                             void* stream) {
  if (head_dim != 128) return fail(JOY_ERR_UNSUPPORTED, "attention_fwd supports head_dim=128 only");
  if (!q || !k || !v) return fail(JOY_ERR_INVALID_ARGUMENT, "q, k and v views must be non-null");
  if (q->len < 0 || k->len < 0 || v->len != k->len)
    return fail(JOY_ERR_INVALID_ARGUMENT, "key and value must have the same sequence length");
  if (num_heads <= 0 || num_heads > 65535) return fail(JOY_ERR_INVALID_ARGUMENT, "num_heads must be in [1, 65535]");
  if (!(scale > 0.0f) || !(scale < INFINITY)) return fail(JOY_ERR_INVALID_ARGUMENT, "scale must be positive and finite");
  if (out_stride_token < num_heads * head_dim)
    return fail(JOY_ERR_INVALID_ARGUMENT, "out token stride must be >= num_heads * head_dim");
  if (q->len == 0) return ok();
  if (k->len == 0) return fail(JOY_ERR_INVALID_ARGUMENT, "attention over an empty key sequence is undefined");
  if (!present(q) || !present(k) || !present(v) || !out)
    return fail(JOY_ERR_INVALID_ARGUMENT, "q, k, v and out must be non-null");
  const joy_bf16_view* views[3] = {q, k, v};
  for (const joy_bf16_view* w : views) {
    if (!aligned(w->ptr, 16) || w->stride_token % 8 != 0 || w->stride_head % 8 != 0)
      return fail(JOY_ERR_UNSUPPORTED, "q, k, v need 16-byte aligned rows (pointer and strides multiples of 8)");
  }
  if (!aligned(out, 16) || out_stride_token % 8 != 0)
    return fail(JOY_ERR_UNSUPPORTED, "out needs 16-byte aligned rows");
  if (num_heads * ((q->len + 31) / 32 + 8) > 0x7fffffffLL)
    return fail(JOY_ERR_UNSUPPORTED, "num_heads * query blocks of 32 above 2^31");
  joy::AttnArgs a;
  a.q = row_view(q);
  a.k = row_view(k);
  a.v = row_view(v);
  a.out = (uint16_t*)out;
  a.out_stride_token = out_stride_token;
  a.q_len = q->len;
  a.k_len = k->len;
  a.heads = (int)num_heads;
  a.scale_log2e = scale * 1.4426950408889634f;
  return hip_status(joy::launch_attention_fwd(a, (hipStream_t)stream), "attention_fwd launch");
}

}  // extern "C"
