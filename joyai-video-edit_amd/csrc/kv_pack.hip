// Joint-attention operand packing on gfx950 (bf16, head_dim 128).
//
// Two ops of the reference's cache read side:
//  * fused_joint_qkv_pack (joyomni_ops/csrc/fused_joint_qkv_pack.cu:81-164):
//      Q = [img_q | rms(txt_q)]
//      K = [cached_k | img_k | rms(txt_k)]
//      V = [cached_v | img_v | txt_v]
//    where rms(x) = bf16(bf16(x * r) * w), r = rsqrt(sum x^2 / D + eps): the
//    model's two-rounding RMSNorm (fused_joint_qkv_pack.cu:58-79, dit.py:292-296).
//  * fused_cached_kv_pack (fused_joint_qkv_pack.cu:166-220): rotate one or two
//    pre-RoPE cached K segments with fp32 full-width tables, pair (2i, 2i+1)
//    using cos/sin[token * D + 2i], and pack them with their V.
//
// Mapping: one (token, head) row of 128 bf16 = 256 bytes belongs to 16 lanes
// (16 bytes each), so a wave moves 4 rows with fully coalesced 128-bit
// accesses and the RMS reduction is a 4-step xor shuffle inside the 16 lanes.
// The cached pack gives each 16-lane group one token and 8 of its heads, so
// the token's fp32 table entries are read once per 8 heads.
// Output rows are dense [rows, 128]; source rows are strided views
// (token stride, head stride) like the reference's [1, L, H, D] inputs, which
// is how the V slices of the QKV projection are passed without a copy.
// VEC = every source pointer and stride allows 16-byte accesses; otherwise the
// same kernel loads and stores 2-byte elements.
#include "joy_common.hpp"
#include "joy_kernels.hpp"

namespace joy {
namespace {

constexpr int kD = 128;          // head_dim of both reference ops
constexpr int kLPR = kD / 8;     // lanes per row
constexpr int kRPW = kWave / kLPR;  // rows per wave
constexpr int kWPB = 4;          // waves per workgroup

// 16-byte accesses are non-temporal: every K / V row is read and written once per launch
// (measured 12 % faster on the cached pack, 4 % on the joint pack, than default-policy accesses).
template <bool VEC>
__device__ __forceinline__ uint4 load8(const uint16_t* p) {
  if constexpr (VEC) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
    return make_uint4(v[0], v[1], v[2], v[3]);
  } else {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = (uint32_t)p[2 * j] | ((uint32_t)p[2 * j + 1] << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
}

template <bool VEC>
__device__ __forceinline__ void store8(uint16_t* p, const uint4& v) {
  if constexpr (VEC) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store((u32x4){v.x, v.y, v.z, v.w}, (u32x4*)p);
  } else {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      p[2 * j] = (uint16_t)(w[j] & 0xffffu);
      p[2 * j + 1] = (uint16_t)(w[j] >> 16);
    }
  }
}

__device__ __forceinline__ void unpack8(const uint4& v, float f[8]) {
  f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x);
  f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
  f[4] = bf16_lo(v.z); f[5] = bf16_hi(v.z);
  f[6] = bf16_lo(v.w); f[7] = bf16_hi(v.w);
}

__device__ __forceinline__ uint4 pack8(const float f[8]) {
  return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                    pack_bf16x2(f[6], f[7]));
}

__device__ __forceinline__ float bf16_round(float x) { return __uint_as_float(f32_to_bf16_bits(x) << 16); }

__device__ __forceinline__ float row_sum(float v) {
#pragma unroll
  for (int off = kLPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ const uint16_t* row_ptr(const RowView& v, int64_t row, int heads) {
  const int64_t t = row / heads;
  const int64_t h = row - t * heads;
  return v.ptr + t * v.stride_token + h * v.stride_head;
}

// U groups of kRPW consecutive rows per wave: every lane issues its U loads before any
// arithmetic (one row per 16-lane group left each lane a single 16-byte load in flight).
template <bool VEC, int U>
__global__ __launch_bounds__(kWPB * kWave) void joint_qkv_pack_kernel(JointPackArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int li = lane % kLPR;
  const int64_t row0 = ((int64_t)blockIdx.x * kWPB + (threadIdx.x >> 6)) * U * kRPW + lane / kLPR;
  const int64_t img_rows = a.img_len * a.heads;
  const int64_t txt_rows = a.txt_len * a.heads;
  const int64_t cache_rows = a.cache_len * a.heads;
  const int64_t q_rows = img_rows + txt_rows;
  const int64_t kv_rows = cache_rows + q_rows;

  uint4 x[U];
  uint16_t* dst[U];
  const uint16_t* w[U];
  bool valid[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t row = row0 + u * kRPW;
    valid[u] = row < q_rows + 2 * kv_rows;
    // source row, destination row and (for text Q/K) the norm weight of this row
    RowView src;
    int64_t srow;
    w[u] = nullptr;
    if (row < q_rows) {
      dst[u] = a.out_q + row * kD;
      if (row < img_rows) {
        src = a.img_q;
        srow = row;
      } else {
        src = a.txt_q;
        srow = row - img_rows;
        w[u] = a.txt_q_weight;
      }
    } else {
      const bool is_v = row >= q_rows + kv_rows;
      const int64_t kv = is_v ? row - q_rows - kv_rows : row - q_rows;
      dst[u] = (is_v ? a.out_v : a.out_k) + kv * kD;
      if (kv < cache_rows) {
        src = is_v ? a.cache_v : a.cache_k;
        srow = kv;
      } else if (kv < cache_rows + img_rows) {
        src = is_v ? a.img_v : a.img_k;
        srow = kv - cache_rows;
      } else {
        src = is_v ? a.txt_v : a.txt_k;
        srow = kv - cache_rows - img_rows;
        if (!is_v) w[u] = a.txt_k_weight;
      }
    }
    x[u] = make_uint4(0, 0, 0, 0);
    if (valid[u]) x[u] = load8<VEC>(row_ptr(src, srow, a.heads) + li * 8);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float f[8];
    unpack8(x[u], f);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(f[j], f[j], ss);
    ss = row_sum(ss);  // every lane takes part, whatever its row needs
    if (!valid[u]) continue;
    uint4 y = x[u];
    if (w[u]) {
      const float r = __builtin_amdgcn_rsqf(ss * (1.0f / kD) + a.eps);
      float wf[8];
      unpack8(load8<VEC>(w[u] + li * 8), wf);
#pragma unroll
      for (int j = 0; j < 8; ++j) f[j] = bf16_round(f[j] * r) * wf[j];
      y = pack8(f);
    }
    store8<VEC>(dst[u] + li * 8, y);
  }
}

// One 16-lane group per (token, group of kHPG heads): the token's cos/sin entries
// are loaded once into registers and reused for every head of the group, and
// the group's K and V rows are all in flight before any arithmetic.
constexpr int kHPG = 8;

template <bool VEC>
__global__ __launch_bounds__(kWPB * kWave) void cached_kv_pack_kernel(CachedPackArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int li = lane % kLPR;
  const int64_t unit =
      ((int64_t)blockIdx.x * kWPB + (threadIdx.x >> 6)) * kRPW + lane / kLPR;
  const int groups = (a.heads + kHPG - 1) / kHPG;
  const int64_t tokens = a.len0 + a.len1;
  if (unit >= tokens * groups) return;
  const int64_t t = unit / groups;
  const int h0 = (int)(unit - t * groups) * kHPG;
  const bool second = t >= a.len0;
  const int64_t st = second ? t - a.len0 : t;
  const RowView kv_k = second ? a.key1 : a.key0;
  const RowView kv_v = second ? a.value1 : a.value0;
  const uint16_t* kp = kv_k.ptr + st * kv_k.stride_token + li * 8;
  const uint16_t* vp = kv_v.ptr + st * kv_v.stride_token + li * 8;

  uint4 kx[kHPG], vx[kHPG];
#pragma unroll
  for (int j = 0; j < kHPG; ++j) {
    const int h = min(h0 + j, a.heads - 1);
    kx[j] = load8<VEC>(kp + h * kv_k.stride_head);
    vx[j] = load8<VEC>(vp + h * kv_v.stride_head);
  }
  // Pair p of this lane is (li*8 + 2p, li*8 + 2p + 1); its angle entry is the
  // even column t*D + li*8 + 2p of the full-width tables.
  const int64_t tab = t * kD + li * 8;
  float c[4], s[4];
  if constexpr (VEC) {
    const float4 c0 = *(const float4*)(a.cos + tab), c1 = *(const float4*)(a.cos + tab + 4);
    const float4 s0 = *(const float4*)(a.sin + tab), s1 = *(const float4*)(a.sin + tab + 4);
    c[0] = c0.x; c[1] = c0.z; c[2] = c1.x; c[3] = c1.z;
    s[0] = s0.x; s[1] = s0.z; s[2] = s1.x; s[3] = s1.z;
  } else {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      c[p] = a.cos[tab + 2 * p];
      s[p] = a.sin[tab + 2 * p];
    }
  }
  uint16_t* ok = a.out_k + t * a.heads * kD + li * 8;
  uint16_t* ov = a.out_v + t * a.heads * kD + li * 8;
#pragma unroll
  for (int j = 0; j < kHPG; ++j) {
    const int h = h0 + j;
    if (h >= a.heads) break;
    float f[8], o[8];
    unpack8(kx[j], f);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      o[2 * p] = f[2 * p] * c[p] - f[2 * p + 1] * s[p];
      o[2 * p + 1] = f[2 * p] * s[p] + f[2 * p + 1] * c[p];
    }
    store8<VEC>(ok + h * kD, pack8(o));
    store8<VEC>(ov + h * kD, vx[j]);
  }
}

__host__ bool view_vec_ok(const RowView& v) {
  return v.ptr == nullptr ||
         ((uintptr_t)v.ptr % 16 == 0 && v.stride_token % 8 == 0 && v.stride_head % 8 == 0);
}

dim3 grid_for_rows(int64_t rows) {
  const int64_t per_block = (int64_t)kWPB * kRPW;
  return dim3((unsigned)((rows + per_block - 1) / per_block));
}

}  // namespace

hipError_t launch_joint_qkv_pack(const JointPackArgs& a, hipStream_t st) {
  const int64_t rows = (a.img_len + a.txt_len) * a.heads +
                       2 * (a.cache_len + a.img_len + a.txt_len) * a.heads;
  if (rows == 0) return hipSuccess;
  const bool vec = view_vec_ok(a.img_q) && view_vec_ok(a.img_k) && view_vec_ok(a.img_v) &&
                   view_vec_ok(a.txt_q) && view_vec_ok(a.txt_k) && view_vec_ok(a.txt_v) &&
                   view_vec_ok(a.cache_k) && view_vec_ok(a.cache_v) &&
                   (uintptr_t)a.txt_q_weight % 16 == 0 && (uintptr_t)a.txt_k_weight % 16 == 0 &&
                   (uintptr_t)a.out_q % 16 == 0 && (uintptr_t)a.out_k % 16 == 0 &&
                   (uintptr_t)a.out_v % 16 == 0;
  // two row groups per wave: 347 -> 330 us at 32400 cached + 10800 + 512 tokens (four: no further gain)
  constexpr int U = 2;
  const dim3 grid((unsigned)((rows + (int64_t)kWPB * kRPW * U - 1) / ((int64_t)kWPB * kRPW * U)));
  if (vec)
    hipLaunchKernelGGL((joint_qkv_pack_kernel<true, U>), grid, dim3(kWPB * kWave), 0, st, a);
  else
    hipLaunchKernelGGL((joint_qkv_pack_kernel<false, U>), grid, dim3(kWPB * kWave), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_cached_kv_pack(const CachedPackArgs& a, hipStream_t st) {
  const int64_t rows = (a.len0 + a.len1) * ((a.heads + kHPG - 1) / kHPG);  // 16-lane units
  if (rows == 0) return hipSuccess;
  const bool vec = view_vec_ok(a.key0) && view_vec_ok(a.value0) && view_vec_ok(a.key1) &&
                   view_vec_ok(a.value1) && (uintptr_t)a.cos % 16 == 0 && (uintptr_t)a.sin % 16 == 0 &&
                   (uintptr_t)a.out_k % 16 == 0 && (uintptr_t)a.out_v % 16 == 0;
  if (vec)
    hipLaunchKernelGGL(cached_kv_pack_kernel<true>, grid_for_rows(rows), dim3(kWPB * kWave), 0, st, a);
  else
    hipLaunchKernelGGL(cached_kv_pack_kernel<false>, grid_for_rows(rows), dim3(kWPB * kWave), 0, st, a);
  return hipGetLastError();
}

}  // namespace joy
