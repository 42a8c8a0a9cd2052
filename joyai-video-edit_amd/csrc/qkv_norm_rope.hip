// Fused QKV split + per-head q/k RMSNorm + interleaved 3-D RoPE + KV-ring write (bf16).
//
// Per (token, head), following joyomni_ops/csrc/fused_qknorm_rope_3d_kernel.cu:68-105:
//   r     = rsqrt(sum_d x_d^2 / D + eps)                     fp32
//   xh_d  = x_d * r * w_d                                    fp32
//   pair i = (2i, 2i+1) with c, s = bf16 cos/sin[token, i]
//   out_2i = xh_2i*c - xh_2i+1*s ; out_2i+1 = xh_2i*s + xh_2i+1*c   -> bf16 (RNE)
//   k_pre  = bf16(xh of K)   (pre-RoPE K kept by the KV cache)
//
// One kernel serves two callers:
//  * the reference's in-place op fused_qk_norm_rope_3d_paired (q, k separate
//    contiguous [B, L*H, D] tensors, outputs over the inputs);
//  * the fused op: q, k, v read straight from the QKV GEMM output row
//    [q(H*D) | k(H*D) | v(H*D)], roped q/k written to the attention operands and
//    the pre-RoPE k and v written into a slot of the KV ring.
// Every pointer is a token-strided [tokens, H, D] view, so outputs can land in
// any caller-owned buffer (ring slot, joint attention buffer) with no copy.
//
// Mapping: D/8 lanes own one head (8 bf16 = one 16-byte access per lane per
// tensor), so a wave64 covers 512/D heads of consecutive (token, head) units and
// every load and store is a fully coalesced 128-bit access. The RMS reduction
// runs over the D/8 lanes of a head with xor shuffles; RoPE pairs are adjacent
// inside a lane, so rotation needs no cross-lane traffic.
#include "joy_common.hpp"
#include "joy_kernels.hpp"

namespace joy {
namespace {

__device__ __forceinline__ void unpack_bf16x8(const uint4& v, float f[8]) {
  f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x);
  f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
  f[4] = bf16_lo(v.z); f[5] = bf16_hi(v.z);
  f[6] = bf16_lo(v.w); f[7] = bf16_hi(v.w);
}

__device__ __forceinline__ uint4 pack_bf16x8(const float f[8]) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                    pack_bf16x2(f[6], f[7]));
}

template <int LPH>
__device__ __forceinline__ float head_sum(float v) {
#pragma unroll
  for (int off = LPH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

template <int D>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(NormRopeArgs a) {
  constexpr int LPH = D / 8;           // lanes per head
  constexpr int HPW = kWave / LPH;     // heads per wave
  const int lane = threadIdx.x & 63;
  const int li = lane % LPH;
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t unit = wave * HPW + lane / LPH;  // (token, head) index
  const int64_t units = a.n_tokens * a.num_heads;
  const bool valid = unit < units;
  const int64_t u = valid ? unit : units - 1;
  const int64_t token = u / a.num_heads;
  const int head = (int)(u - token * a.num_heads);
  const int64_t trow = token % a.table_len;
  const int64_t hoff = (int64_t)head * D + li * 8;

  const uint16_t* qi = a.q_in + token * a.in_stride + hoff;
  const uint16_t* ki = a.k_in + token * a.in_stride + hoff;
  uint4 qv = *(const uint4*)qi;
  uint4 kv = *(const uint4*)ki;
  uint4 vv = make_uint4(0, 0, 0, 0);
  if (a.v_in) vv = *(const uint4*)(a.v_in + token * a.in_stride + hoff);
  const uint4 qwv = *(const uint4*)(a.q_weight + li * 8);
  const uint4 kwv = *(const uint4*)(a.k_weight + li * 8);
  const uint2 cv = *(const uint2*)(a.cos + trow * (D / 2) + li * 4);
  const uint2 sv = *(const uint2*)(a.sin + trow * (D / 2) + li * 4);

  float q[8], k[8], qw[8], kw[8];
  unpack_bf16x8(qv, q);
  unpack_bf16x8(kv, k);
  unpack_bf16x8(qwv, qw);
  unpack_bf16x8(kwv, kw);
  const float c[4] = {bf16_lo(cv.x), bf16_hi(cv.x), bf16_lo(cv.y), bf16_hi(cv.y)};
  const float s[4] = {bf16_lo(sv.x), bf16_hi(sv.x), bf16_lo(sv.y), bf16_hi(sv.y)};

  float ssq = 0.f, ssk = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    ssq = __builtin_fmaf(q[j], q[j], ssq);
    ssk = __builtin_fmaf(k[j], k[j], ssk);
  }
  ssq = head_sum<LPH>(ssq);
  ssk = head_sum<LPH>(ssk);
  const float inv_d = 1.0f / (float)D;
  const float rq = __builtin_amdgcn_rsqf(ssq * inv_d + a.eps);
  const float rk = __builtin_amdgcn_rsqf(ssk * inv_d + a.eps);

  float qo[8], ko[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    q[j] = q[j] * rq * qw[j];
    k[j] = k[j] * rk * kw[j];
  }
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    qo[2 * p] = q[2 * p] * c[p] - q[2 * p + 1] * s[p];
    qo[2 * p + 1] = q[2 * p] * s[p] + q[2 * p + 1] * c[p];
    ko[2 * p] = k[2 * p] * c[p] - k[2 * p + 1] * s[p];
    ko[2 * p + 1] = k[2 * p] * s[p] + k[2 * p + 1] * c[p];
  }
  if (!valid) return;
  *(uint4*)(a.q_out + token * a.q_out_stride + hoff) = pack_bf16x8(qo);
  if (a.k_out) *(uint4*)(a.k_out + token * a.k_out_stride + hoff) = pack_bf16x8(ko);
  if (a.kpre_out) *(uint4*)(a.kpre_out + token * a.kpre_stride + hoff) = pack_bf16x8(k);
  if (a.v_out) *(uint4*)(a.v_out + token * a.v_out_stride + hoff) = vv;
}

}  // namespace

hipError_t launch_qk_norm_rope(const NormRopeArgs& a, int head_dim, hipStream_t st) {
  const int64_t units = a.n_tokens * a.num_heads;
  if (units == 0) return hipSuccess;
  const int hpw = kWave / (head_dim / 8);
  const int64_t waves = (units + hpw - 1) / hpw;
  const int wpb = 4;
  const dim3 grid((unsigned)((waves + wpb - 1) / wpb));
  const dim3 block(wpb * kWave);
  switch (head_dim) {
    case 64:
      hipLaunchKernelGGL(qk_norm_rope_kernel<64>, grid, block, 0, st, a);
      break;
    case 128:
      hipLaunchKernelGGL(qk_norm_rope_kernel<128>, grid, block, 0, st, a);
      break;
    case 256:
      hipLaunchKernelGGL(qk_norm_rope_kernel<256>, grid, block, 0, st, a);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace joy
