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
//    [q(H*D) | k(H*D) | v(H*D)], roped q/k written to the attention operands,
//    the pre-RoPE (or rotated) k and v of the first cache_tokens tokens written
//    into a slot of the KV ring and, optionally, v also into the attention V
//    operand. Without a q output, q is not read (cache-only forward).
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

// 16-byte global access; NT marks streaming (non-temporal) traffic.
template <bool NT>
__device__ __forceinline__ uint4 ld16(const uint16_t* p) {
  if constexpr (NT) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
    return make_uint4(v[0], v[1], v[2], v[3]);
  }
  return *(const uint4*)p;
}
template <bool NT>
__device__ __forceinline__ void st16(uint16_t* p, const uint4& v) {
  if constexpr (NT) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store((u32x4){v.x, v.y, v.z, v.w}, (u32x4*)p);
  } else {
    *(uint4*)p = v;
  }
}

// the tree over the head's lanes of head_rsqrt's comment: offsets LPH / 2, ..., 1
template <int LPH>
__device__ __forceinline__ float head_sum(float v) {
#pragma unroll
  for (int off = LPH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// UPT groups of (64 / (D/8)) consecutive (token, head) units per wave; every
// lane issues all of its 16-byte loads before any arithmetic.
template <int D, int UPT, bool NT>
__global__ __launch_bounds__(512) void qk_norm_rope_kernel(NormRopeArgs a) {
  constexpr int LPH = D / 8;           // lanes per head
  constexpr int HPW = kWave / LPH;     // heads per wave per group
  const int lane = threadIdx.x & 63;
  const int li = lane % LPH;
  const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int units = (int)(a.n_tokens * a.num_heads);

  int token[UPT], hoff[UPT];
  bool valid[UPT];
  uint4 qv[UPT], kv[UPT], vv[UPT];
  uint2 cv[UPT], sv[UPT];
#pragma unroll
  for (int r = 0; r < UPT; ++r) {
    const int unit = (wave * UPT + r) * HPW + lane / LPH;
    valid[r] = unit < units;
    const int u = valid[r] ? unit : units - 1;
    token[r] = u / a.num_heads;
    hoff[r] = (u - token[r] * a.num_heads) * D + li * 8;
    const int64_t in = (int64_t)token[r] * a.in_stride + hoff[r];
    qv[r] = a.q_in ? ld16<NT>(a.q_in + in) : make_uint4(0, 0, 0, 0);
    kv[r] = ld16<NT>(a.k_in + in);
    if (a.v_in) vv[r] = ld16<NT>(a.v_in + in);
    const int64_t trow = (int64_t)(token[r] % a.table_len) * (D / 2) + li * 4;
    cv[r] = *(const uint2*)(a.cos + trow);
    sv[r] = *(const uint2*)(a.sin + trow);
  }
  const uint4 qwv = *(const uint4*)(a.q_weight + li * 8);
  const uint4 kwv = *(const uint4*)(a.k_weight + li * 8);
  float qw[8], kw[8];
  unpack_bf16x8(qwv, qw);
  unpack_bf16x8(kwv, kw);
  const float inv_d = 1.0f / (float)D;

#pragma unroll
  for (int r = 0; r < UPT; ++r) {
    float q[8], k[8];
    unpack_bf16x8(qv[r], q);
    unpack_bf16x8(kv[r], k);
    const float c[4] = {bf16_lo(cv[r].x), bf16_hi(cv[r].x), bf16_lo(cv[r].y), bf16_hi(cv[r].y)};
    const float s[4] = {bf16_lo(sv[r].x), bf16_hi(sv[r].x), bf16_lo(sv[r].y), bf16_hi(sv[r].y)};
    float ssq = 0.f, ssk = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ssq = __builtin_fmaf(q[j], q[j], ssq);
      ssk = __builtin_fmaf(k[j], k[j], ssk);
    }
    ssq = head_sum<LPH>(ssq);
    ssk = head_sum<LPH>(ssk);
    const float rq = head_rsqrt(ssq, inv_d, a.eps);
    const float rk = head_rsqrt(ssk, inv_d, a.eps);
    float qo[8], ko[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      q[j] = q[j] * rq * qw[j];
      k[j] = k[j] * rk * kw[j];
    }
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      rope_pair(q[2 * p], q[2 * p + 1], c[p], s[p], qo[2 * p], qo[2 * p + 1]);
      rope_pair(k[2 * p], k[2 * p + 1], c[p], s[p], ko[2 * p], ko[2 * p + 1]);
    }
    if (!valid[r]) continue;
    const int64_t t = token[r];
    if (a.q_in) st16<NT>(a.q_out + t * a.q_out_stride + hoff[r], pack_bf16x8(qo));
    if (a.k_out) st16<NT>(a.k_out + t * a.k_out_stride + hoff[r], pack_bf16x8(ko));
    if (t < a.cache_tokens) {
      if (a.kpre_out)
        st16<NT>(a.kpre_out + t * a.kpre_stride + hoff[r], pack_bf16x8(a.cache_post_rope ? ko : k));
      if (a.v_out) st16<NT>(a.v_out + t * a.v_out_stride + hoff[r], vv[r]);
    }
    if (a.v_out2) st16<NT>(a.v_out2 + t * a.v_out2_stride + hoff[r], vv[r]);
  }
}

// Launch: two (token, head) groups per wave (UPT = 2), non-temporal traffic, 4 waves per
// workgroup. Measured on four MI355X boxes at L = 10800, H = 40 against one group per wave and
// 8 waves per workgroup (graph-replayed, same-process A/B, bit-identical): 127.9 / 134.1 / 126.9 /
// 127.0 us against 132.4 / 133.9 / 131.2 / 131.8; four or more groups per wave were faster on one
// box only (UPT 4: 128.5-129.6 / 129.4-130.4 / 129.6-129.8 us), eight slower everywhere.
template <int D>
hipError_t launch_norm_rope_d(const NormRopeArgs& a, hipStream_t st) {
  constexpr int UPT = 2, WPB = 4;
  constexpr int HPW = kWave / (D / 8);
  const int64_t units = a.n_tokens * a.num_heads;
  const int64_t waves = (units + HPW * UPT - 1) / (HPW * UPT);
  hipLaunchKernelGGL((qk_norm_rope_kernel<D, UPT, true>), dim3((unsigned)((waves + WPB - 1) / WPB)),
                     dim3(WPB * kWave), 0, st, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_qk_norm_rope(const NormRopeArgs& a, int head_dim, hipStream_t st) {
  if (a.n_tokens * a.num_heads == 0) return hipSuccess;
  switch (head_dim) {
    case 64:
      return launch_norm_rope_d<64>(a, st);
    case 128:
      return launch_norm_rope_d<128>(a, st);
    case 256:
      return launch_norm_rope_d<256>(a, st);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace joy
