// (Layer|RMS)Norm + adaLN modulation, optionally emitting the per-token FP8
// quantisation of its output directly (gfx950).
//
//   mean = sum x / N                                  (LayerNorm only)
//   r    = rsqrt(sum (x - mean)^2 / N + eps)          (LayerNorm)
//        = rsqrt(sum x^2 / N + eps)                   (RMSNorm)
//   y    = T(((x - mean) * r * g + b) * (1 + scale) + shift)      LayerNorm
//        = T((x * r * g) * (1 + scale) + shift)                   RMSNorm
// following joyomni_ops/csrc/fused_norm_scale_shift.cu:97-182 (g = 1, b = 0 when
// absent; scale/shift per row or one row broadcast over all rows).
//
// FP8 variant (no reference counterpart; it fuses the norm with the activation
// quantiser that every Fp8Linear runs on this output, fp8_linear.py:38-43):
// the row of rounded y values is quantised in the same pass,
//   s = max(absmax |y|, 1e-8) / 448,  q = e4m3fn(clamp(y / s))   (or y * (1/s)),
// so q and s are bit-identical to per_token_quant_fp8 applied to y, while y
// itself never has to reach HBM (optional output).
//
// Vector path (bf16/fp16, N % 8 == 0, 16-byte aligned rows, N <= 8192): the row
// is held in registers as 16-byte vectors, so x is read once -- by one wave64
// (N <= 2048, and the FP8 variant at N = 4096 / 5120 with a broadcast modulation
// row: xor-shuffle reductions) or by the waves of a workgroup (longer rows; wave
// partial sums meet in LDS). Other shapes and fp32 take a scalar kernel that
// re-reads the row per pass.
#include "joy_common.hpp"
#include "joy_kernels.hpp"

namespace joy {
namespace {

template <int DT>  // 0 bf16, 1 fp16, 2 fp32
__device__ __forceinline__ float load_elem(const void* p, int64_t i) {
  if constexpr (DT == 0) return __uint_as_float((uint32_t)((const uint16_t*)p)[i] << 16);
  if constexpr (DT == 1) return fp16_bits_to_f32(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}

template <int DT>
__device__ __forceinline__ float round_elem(float v) {
  if constexpr (DT == 0) return __uint_as_float(f32_to_bf16_bits(v) << 16);
  if constexpr (DT == 1) return round_fp16(v);
  return v;
}

template <int DT>
__device__ __forceinline__ void store_elem(void* p, int64_t i, float v) {
  if constexpr (DT == 0) ((uint16_t*)p)[i] = (uint16_t)f32_to_bf16_bits(v);
  if constexpr (DT == 1) ((uint16_t*)p)[i] = (uint16_t)f32_to_fp16_bits(v);
  if constexpr (DT == 2) ((float*)p)[i] = v;
}

template <bool kFp16>
__device__ __forceinline__ void unpack8(const uint4& v, float f[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (kFp16) {
      f[2 * i] = fp16_bits_to_f32(w[i] & 0xffffu);
      f[2 * i + 1] = fp16_bits_to_f32(w[i] >> 16);
    } else {
      f[2 * i] = bf16_lo(w[i]);
      f[2 * i + 1] = bf16_hi(w[i]);
    }
  }
}

template <bool kFp16>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (kFp16) return pack_fp16x2(lo, hi);
  return pack_bf16x2(lo, hi);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t o = __shfl_xor(v, off, kWave);
    v = o > v ? o : v;
  }
  return v;
}

// Software fp32 -> e4m3fn (RNE, no saturation) for rows whose absmax is not
// finite, where torch's NaN/sign behaviour is wanted.
__device__ uint32_t e4m3fn_soft(float x) {
  const uint32_t b = __float_as_uint(x);
  const uint32_t sign = (b >> 24) & 0x80u;
  if ((b & 0x7f800000u) == 0x7f800000u) return 0x7fu | sign;
  const float a = fabsf(x);
  if (a < 0.015625f) return (uint32_t)__builtin_rintf(a * 512.0f) | sign;
  const uint32_t ab = __float_as_uint(a);
  const uint32_t r = (ab + 0x7ffffu + ((ab >> 20) & 1u)) >> 20;
  const int e8 = (int)(r >> 3) - 127 + 7;
  const uint32_t m3 = r & 7u;
  if (e8 > 15 || (e8 == 15 && m3 == 7u)) return 0x7fu | sign;
  return (((uint32_t)e8 << 3) | m3) | sign;
}

// Quantiser scale from the 16-bit absmax pattern; false when it is inf/NaN.
template <bool kFp16>
__device__ __forceinline__ bool fp8_row_scale(uint32_t amax_bits, float& s) {
  const uint32_t inf_bits = kFp16 ? 0x7c00u : 0x7f80u;
  const float amax = kFp16 ? fp16_bits_to_f32(amax_bits) : __uint_as_float(amax_bits << 16);
  if (amax_bits >= inf_bits) {
    s = amax / kFp8Max;
    return false;
  }
  s = fmaxf(amax, 1.0e-8f) / kFp8Max;
  return true;
}

// WPR waves own one row (WPR = 1: one row per wave, shuffle reductions only;
// WPR = 4: the workgroup owns one row, so a long row's arithmetic is spread over
// the four SIMDs, registers stay low and the wave results meet in LDS in a fixed
// order). VPT 16-byte vectors (8 elements) per lane: nvec = N / 8 <= 64 * WPR * VPT.
template <bool kFp16, int NORM, bool kFp8, bool kDivide, int VPT, int WPR>
__global__ __launch_bounds__(256) void norm_mod_vec(NormModArgs a) {
  static_assert(WPR == 1 || WPR == 4, "one row per wave or per workgroup");
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row = WPR == 4 ? (int64_t)blockIdx.x : (int64_t)blockIdx.x * 4 + wave;
  if (WPR == 1 && row >= a.M) return;  // (WPR == 4: the grid is exactly M workgroups)
  const int t = WPR == 4 ? (int)threadIdx.x : lane;  // thread index within the row
  constexpr int STRIDE = 64 * WPR;
  const int nvec = (int)(a.N / 8);
  const uint4* src = (const uint4*)((const uint16_t*)a.x + row * a.x_stride);
  const int64_t mrow = a.mod_rows == 1 ? 0 : row;
  const uint4* scv = (const uint4*)((const uint16_t*)a.scale + mrow * a.N);
  const uint4* shv = (const uint4*)((const uint16_t*)a.shift + mrow * a.N);
  __shared__ float red[4];
  __shared__ uint32_t red_u[4];
  auto row_sum = [&](float v) -> float {
    v = wave_sum(v);
    if constexpr (WPR == 1) return v;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    const float r = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return r;
  };

  uint4 v[VPT];
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int idx = t + i * STRIDE;
    v[i] = idx < nvec ? src[idx] : make_uint4(0, 0, 0, 0);
    float f[8];
    unpack8<kFp16>(v[i], f);
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += NORM == 0 ? f[j] : f[j] * f[j];
  }
  float mean = 0.f, r;
  if constexpr (NORM == 0) {
    mean = row_sum(sum) / (float)a.N;
    float var = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int idx = t + i * STRIDE;
      if (idx < nvec) {
        float f[8];
        unpack8<kFp16>(v[i], f);
#pragma unroll
        for (int j = 0; j < 8; ++j) var += (f[j] - mean) * (f[j] - mean);
      }
    }
    r = __builtin_amdgcn_rsqf(row_sum(var) / (float)a.N + a.eps);
  } else {
    r = __builtin_amdgcn_rsqf(row_sum(sum) / (float)a.N + a.eps);
  }

  // y, rounded to the activation type, overwrites v
  uint32_t amax = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int idx = t + i * STRIDE;
    if (idx >= nvec) continue;
    float f[8], sc[8], sh[8], g[8], b[8];
    unpack8<kFp16>(v[i], f);
    unpack8<kFp16>(scv[idx], sc);
    unpack8<kFp16>(shv[idx], sh);
    if (a.gamma) {
      unpack8<kFp16>(((const uint4*)a.gamma)[idx], g);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) g[j] = 1.f;
    }
    if (a.beta && NORM == 0) {
      unpack8<kFp16>(((const uint4*)a.beta)[idx], b);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) b[j] = 0.f;
    }
    float y[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (NORM == 0)
        y[j] = ((f[j] - mean) * r * g[j] + b[j]) * (1.f + sc[j]) + sh[j];
      else
        y[j] = (f[j] * r * g[j]) * (1.f + sc[j]) + sh[j];
    }
    v[i] = make_uint4(pack2<kFp16>(y[0], y[1]), pack2<kFp16>(y[2], y[3]), pack2<kFp16>(y[4], y[5]),
                      pack2<kFp16>(y[6], y[7]));
    if (a.out) ((uint4*)((uint16_t*)a.out + row * a.N))[idx] = v[i];
    if constexpr (kFp8) {
      const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = w[j] & 0x7fffu, hi = (w[j] >> 16) & 0x7fffu;
        amax = lo > amax ? lo : amax;
        amax = hi > amax ? hi : amax;
      }
    }
  }
  if constexpr (kFp8) {
    amax = wave_max_u32(amax);
    if constexpr (WPR == 4) {
      if (lane == 0) red_u[wave] = amax;
      __syncthreads();
      const uint32_t m01 = red_u[0] > red_u[1] ? red_u[0] : red_u[1];
      const uint32_t m23 = red_u[2] > red_u[3] ? red_u[2] : red_u[3];
      amax = m01 > m23 ? m01 : m23;
    }
    float s;
    const bool finite = fp8_row_scale<kFp16>(amax, s);
    if (t == 0) a.out_s[row] = s;
    const float rs = 1.0f / s;
    uint2* dst = (uint2*)((uint8_t*)a.out_q + row * a.N);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int idx = t + i * STRIDE;
      if (idx >= nvec) continue;
      float f[8];
      unpack8<kFp16>(v[i], f);
      uint2 o;
      if (finite) {  // no clamp needed (see norm_mod_rows)
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = kDivide ? div_by_scale(f[j], s, rs) : f[j] * rs;
        o.x = pack_fp8x4(f[0], f[1], f[2], f[3]);
        o.y = pack_fp8x4(f[4], f[5], f[6], f[7]);
      } else {
        uint32_t bq[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) bq[j] = e4m3fn_soft(clamp_fp8(kDivide ? f[j] / s : f[j] * rs));
        o.x = bq[0] | (bq[1] << 8) | (bq[2] << 16) | (bq[3] << 24);
        o.y = bq[4] | (bq[5] << 8) | (bq[6] << 16) | (bq[7] << 24);
      }
      dst[idx] = o;
    }
  }
}

// Non-temporal 16- / 8-byte accesses for the row walk: every byte is touched once (measured
// 8 % faster than plain accesses on the bf16 output, M = 10800, N = 5120).
__device__ __forceinline__ uint4 nt_load16(const uint4* p) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void nt_store16(uint4* p, const uint4& v) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store((u32x4){v.x, v.y, v.z, v.w}, (u32x4*)p);
}
__device__ __forceinline__ void nt_store8(uint2* p, const uint2& v) {
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  __builtin_nontemporal_store((u32x2){v.x, v.y}, (u32x2*)p);
}

typedef unsigned short us2 __attribute__((ext_vector_type(2)));

// max over the |x| 16-bit patterns of 8 packed values (bf16 and fp16 order like their magnitude)
__device__ __forceinline__ uint32_t absmax8(uint32_t acc, const uint4& v) {
  us2 m = __builtin_bit_cast(us2, acc);
  m = __builtin_elementwise_max(m, __builtin_bit_cast(us2, v.x & 0x7fff7fffu));
  m = __builtin_elementwise_max(m, __builtin_bit_cast(us2, v.y & 0x7fff7fffu));
  m = __builtin_elementwise_max(m, __builtin_bit_cast(us2, v.z & 0x7fff7fffu));
  m = __builtin_elementwise_max(m, __builtin_bit_cast(us2, v.w & 0x7fff7fffu));
  return __builtin_bit_cast(uint32_t, m);
}

// Long rows with one broadcast modulation row and no affine weights (the adaLN
// case of the model): each workgroup walks rows blockIdx.x, +gridDim.x, ...
// with blockDim = nvec / VPT threads rounded up to whole waves (N = 5120: 320
// threads, exactly VPT = 2 vectors each, so no wave idles at the barriers);
// 1 + scale and shift live in fp32 registers for all its rows, the next row's
// 16-byte vectors are loaded while the current row is computed, x is unpacked
// once, and the wave partial sums meet in LDS in wave order with one barrier
// per reduction (consecutive reductions alternate between two LDS slots, so a
// slot is only rewritten after a barrier that every reader of its previous use
// has passed).
constexpr int kMaxRowWaves = 8;

template <bool kFp16, int NORM, bool kFp8, bool kDivide, int VPT>
__global__ __launch_bounds__(64 * kMaxRowWaves) void norm_mod_rows(NormModArgs a) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int nwaves = blockDim.x >> 6;
  const int stride = blockDim.x;
  const int nvec = (int)(a.N / 8);
  __shared__ float red[2][kMaxRowWaves];
  __shared__ uint32_t red_u[kMaxRowWaves];
  int slot = 0;
  auto row_sum = [&](float v) -> float {
    v = wave_sum(v);
    if (lane == 0) red[slot][wave] = v;
    __syncthreads();
    float r = red[slot][0];
    for (int w = 1; w < nwaves; ++w) r += red[slot][w];
    slot ^= 1;
    return r;
  };

  float sc1[VPT][8], shf[VPT][8];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int idx = t + i * stride;
    float sc[8];
    const bool in = idx < nvec;
    unpack8<kFp16>(in ? ((const uint4*)a.scale)[idx] : make_uint4(0, 0, 0, 0), sc);
    unpack8<kFp16>(in ? ((const uint4*)a.shift)[idx] : make_uint4(0, 0, 0, 0), shf[i]);
#pragma unroll
    for (int j = 0; j < 8; ++j) sc1[i][j] = 1.f + sc[j];
  }

  auto load_row = [&](int64_t row, uint4 (&v)[VPT]) {
    const uint4* src = (const uint4*)((const uint16_t*)a.x + row * a.x_stride);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int idx = t + i * stride;
      v[i] = idx < nvec ? nt_load16(src + idx) : make_uint4(0, 0, 0, 0);
    }
  };
  uint4 nxt[VPT];
  int64_t row = blockIdx.x;
  if (row < a.M) load_row(row, nxt);
  for (; row < a.M; row += gridDim.x) {
    float x[VPT][8];
#pragma unroll
    for (int i = 0; i < VPT; ++i) unpack8<kFp16>(nxt[i], x[i]);
    if (row + gridDim.x < a.M) load_row(row + gridDim.x, nxt);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) sum += NORM == 0 ? x[i][j] : x[i][j] * x[i][j];
    float mean = 0.f, r;
    if constexpr (NORM == 0) {
      mean = row_sum(sum) / (float)a.N;
      float var = 0.f;
#pragma unroll
      for (int i = 0; i < VPT; ++i) {
#pragma unroll
        for (int j = 0; j < 8; ++j) x[i][j] -= mean;  // x - mean, reused below
        if (t + i * stride < nvec) {
#pragma unroll
          for (int j = 0; j < 8; ++j) var += x[i][j] * x[i][j];
        }
      }
      r = __builtin_amdgcn_rsqf(row_sum(var) / (float)a.N + a.eps);
    } else {
      r = __builtin_amdgcn_rsqf(row_sum(sum) / (float)a.N + a.eps);
    }
    uint4 y[VPT];
    uint32_t amax = 0;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      float o[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float n = x[i][j] * r;
        o[j] = n * sc1[i][j] + shf[i][j];
      }
      y[i] = make_uint4(pack2<kFp16>(o[0], o[1]), pack2<kFp16>(o[2], o[3]), pack2<kFp16>(o[4], o[5]),
                        pack2<kFp16>(o[6], o[7]));
      const int idx = t + i * stride;
      if (idx < nvec) {
        if (a.out) nt_store16((uint4*)((uint16_t*)a.out + row * a.N) + idx, y[i]);
        if constexpr (kFp8) amax = absmax8(amax, y[i]);
      }
    }
    if constexpr (kFp8) {
      amax = (amax & 0xffffu) > (amax >> 16) ? (amax & 0xffffu) : (amax >> 16);
      amax = wave_max_u32(amax);
      if (lane == 0) red_u[wave] = amax;
      __syncthreads();
      amax = red_u[0];
      for (int w = 1; w < nwaves; ++w) amax = red_u[w] > amax ? red_u[w] : amax;
      float s;
      const bool finite = fp8_row_scale<kFp16>(amax, s);
      if (t == 0) a.out_s[row] = s;
      const float rs = 1.0f / s;
      uint2* dst = (uint2*)((uint8_t*)a.out_q + row * a.N);
#pragma unroll
      for (int i = 0; i < VPT; ++i) {
        const int idx = t + i * stride;
        if (idx >= nvec) continue;
        float f[8];
        unpack8<kFp16>(y[i], f);
        uint2 o;
        if (finite) {
          // no clamp: with a finite scale |y| * (1 / s) (and y / s) stays below 464, the midpoint
          // between 448 and the next e4m3 step, so the conversion rounds it to 448 as clamp-then-cast
          // does (checked over every bf16 and fp16 absmax, both roundings)
#pragma unroll
          for (int j = 0; j < 8; ++j) f[j] = kDivide ? div_by_scale(f[j], s, rs) : f[j] * rs;
          o.x = pack_fp8x4(f[0], f[1], f[2], f[3]);
          o.y = pack_fp8x4(f[4], f[5], f[6], f[7]);
        } else {
          uint32_t bq[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) bq[j] = e4m3fn_soft(clamp_fp8(kDivide ? f[j] / s : f[j] * rs));
          o.x = bq[0] | (bq[1] << 8) | (bq[2] << 16) | (bq[3] << 24);
          o.y = bq[4] | (bq[5] << 8) | (bq[6] << 16) | (bq[7] << 24);
        }
        nt_store8(dst + idx, o);
      }
    }
  }
}

// One wave per row for the model's rows (N = 512 NV: 4096, 5120), broadcast modulation, no affine
// weights: the row is held in the wave's registers, unpacked to fp32 once (8 NV values per lane),
// every reduction is a wave shuffle (no LDS round trip, no barrier per row), and 1 + scale and shift
// live in LDS as fp32, read by every wave of the workgroup. Waves walk rows wave_id, + total waves;
// the next row's vectors are loaded while the current row is computed. The FP8 pass quantises the
// row as rounded to the output dtype, kept as fp32 in the same registers. Same arithmetic per element as
// norm_mod_rows (x - mean, * r, * (1 + scale) + shift, one rounding; the quantiser of the rounded
// row), the row sums accumulated per lane in element order and then over the lanes.
template <bool kFp16, int NORM, bool kFp8, bool kDivide, int NV>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void norm_mod_wave_rows(NormModArgs a) {
  constexpr int N = 512 * NV;
  __shared__ __attribute__((aligned(16))) float sc1_l[N];
  __shared__ __attribute__((aligned(16))) float shf_l[N];
  const int t = threadIdx.x, lane = t & 63;
  for (int i = t; i < N / 8; i += blockDim.x) {
    float sc[8], sh[8];
    unpack8<kFp16>(((const uint4*)a.scale)[i], sc);
    unpack8<kFp16>(((const uint4*)a.shift)[i], sh);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      sc1_l[i * 8 + j] = 1.f + sc[j];
      shf_l[i * 8 + j] = sh[j];
    }
  }
  __syncthreads();
  const int waves = gridDim.x * (blockDim.x >> 6);
  int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (t >> 6);
  auto load_row = [&](int64_t r, uint4 (&v)[NV]) {
    const uint4* src = (const uint4*)((const uint16_t*)a.x + r * a.x_stride);
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = nt_load16(src + lane + 64 * i);
  };
  uint4 nxt[NV];
  if (row < a.M) load_row(row, nxt);
  for (; row < a.M; row += waves) {
    // the row unpacked to fp32 once, then the next row's loads issued into the freed vectors
    float f[NV][8];
#pragma unroll
    for (int i = 0; i < NV; ++i) unpack8<kFp16>(nxt[i], f[i]);
    if (row + waves < a.M) load_row(row + waves, nxt);
    // row sums: per lane over its NV vectors in element order, then over the lanes
    float mean = 0.f, r;
    if constexpr (NORM == 0) {
      float part = 0.f;
#pragma unroll
      for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) part += f[i][j];
      mean = wave_sum(part) / (float)N;
      part = 0.f;
#pragma unroll
      for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float d = f[i][j] - mean;
          part += d * d;
        }
      r = __builtin_amdgcn_rsqf(wave_sum(part) / (float)N + a.eps);
    } else {
      float part = 0.f;
#pragma unroll
      for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) part += f[i][j] * f[i][j];
      r = __builtin_amdgcn_rsqf(wave_sum(part) / (float)N + a.eps);
    }
    uint32_t amax = 0;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      // one vector's modulation operands at a time (hoisting every vector's LDS reads to the top
      // holds 16 NV more registers)
      asm volatile("" ::: "memory");
      const int e0 = (lane + 64 * i) * 8;
      const float4 c0 = *(const float4*)&sc1_l[e0], c1 = *(const float4*)&sc1_l[e0 + 4];
      const float4 h0 = *(const float4*)&shf_l[e0], h1 = *(const float4*)&shf_l[e0 + 4];
      const float cs[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
      const float hs[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
      float o[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float n = NORM == 0 ? (f[i][j] - mean) * r : f[i][j] * r;
        o[j] = n * cs[j] + hs[j];
      }
      const uint4 y = make_uint4(pack2<kFp16>(o[0], o[1]), pack2<kFp16>(o[2], o[3]), pack2<kFp16>(o[4], o[5]),
                                 pack2<kFp16>(o[6], o[7]));
      if (a.out) nt_store16((uint4*)((uint16_t*)a.out + row * N) + lane + 64 * i, y);
      if constexpr (kFp8) {
        amax = absmax8(amax, y);
        unpack8<kFp16>(y, f[i]);  // the rounded row, which the quantiser sees
      }
    }
    if constexpr (kFp8) {
      amax = (amax & 0xffffu) > (amax >> 16) ? (amax & 0xffffu) : (amax >> 16);
      // wave-uniform, so that the quantisation below takes one scalar branch per row rather than
      // an exec-mask branch per vector
      amax = __builtin_amdgcn_readfirstlane(wave_max_u32(amax));
      float s;
      const bool finite = fp8_row_scale<kFp16>(amax, s);
      if (lane == 0) a.out_s[row] = s;
      const float rs = 1.0f / s;
      uint2* dst = (uint2*)((uint8_t*)a.out_q + row * N);
      if (finite) {  // no clamp needed (see norm_mod_rows)
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          float q[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) q[j] = kDivide ? div_by_scale(f[i][j], s, rs) : f[i][j] * rs;
          nt_store8(dst + lane + 64 * i, make_uint2(pack_fp8x4_reuse(q[0], q[1], q[2], q[3]),
                                                    pack_fp8x4_reuse(q[4], q[5], q[6], q[7])));
        }
      } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          uint32_t bq[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) bq[j] = e4m3fn_soft(clamp_fp8(kDivide ? f[i][j] / s : f[i][j] * rs));
          nt_store8(dst + lane + 64 * i, make_uint2(bq[0] | (bq[1] << 8) | (bq[2] << 16) | (bq[3] << 24),
                                                    bq[4] | (bq[5] << 8) | (bq[6] << 16) | (bq[7] << 24)));
        }
      }
    }
  }
}

// Any N, any alignment, bf16/fp16/fp32: one wave per row, the row re-read per pass.
template <int DT, int NORM, bool kFp8, bool kDivide>
__global__ __launch_bounds__(256) void norm_mod_scalar(NormModArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= a.M) return;
  const int64_t xb = row * a.x_stride;
  const int64_t mb = (a.mod_rows == 1 ? 0 : row) * a.N;
  float sum = 0.f;
  for (int64_t k = lane; k < a.N; k += kWave) {
    const float f = load_elem<DT>(a.x, xb + k);
    sum += NORM == 0 ? f : f * f;
  }
  float mean = 0.f, r;
  if constexpr (NORM == 0) {
    mean = wave_sum(sum) / (float)a.N;
    float var = 0.f;
    for (int64_t k = lane; k < a.N; k += kWave) {
      const float d = load_elem<DT>(a.x, xb + k) - mean;
      var += d * d;
    }
    r = __builtin_amdgcn_rsqf(wave_sum(var) / (float)a.N + a.eps);
  } else {
    r = __builtin_amdgcn_rsqf(wave_sum(sum) / (float)a.N + a.eps);
  }
  auto y_at = [&](int64_t k) {
    const float f = load_elem<DT>(a.x, xb + k);
    const float g = a.gamma ? load_elem<DT>(a.gamma, k) : 1.f;
    const float b = (a.beta && NORM == 0) ? load_elem<DT>(a.beta, k) : 0.f;
    const float sc = load_elem<DT>(a.scale, mb + k), sh = load_elem<DT>(a.shift, mb + k);
    float y;
    if constexpr (NORM == 0)
      y = ((f - mean) * r * g + b) * (1.f + sc) + sh;
    else
      y = (f * r * g) * (1.f + sc) + sh;
    return round_elem<DT>(y);
  };
  uint32_t amax = 0;
  for (int64_t k = lane; k < a.N; k += kWave) {
    const float y = y_at(k);
    if (a.out) store_elem<DT>(a.out, row * a.N + k, y);
    if constexpr (kFp8) {
      const uint32_t bits = DT == 1 ? f32_to_fp16_bits(y)
                                    : (__float_as_uint(y) >> 16);
      const uint32_t m = bits & 0x7fffu;
      amax = m > amax ? m : amax;
    }
  }
  if constexpr (kFp8) {
    amax = wave_max_u32(amax);
    float s;
    const bool finite = fp8_row_scale<DT == 1>(amax, s);
    if (lane == 0) a.out_s[row] = s;
    const float rs = 1.0f / s;
    uint8_t* dst = (uint8_t*)a.out_q + row * a.N;
    for (int64_t k = lane; k < a.N; k += kWave) {
      const float y = y_at(k);
      const float t = finite ? (kDivide ? div_by_scale(y, s, rs) : y * rs) : (kDivide ? y / s : y * rs);
      dst[k] = (uint8_t)e4m3fn_soft(clamp_fp8(t));
    }
  }
}

template <int DT, int NORM, bool kFp8, bool kDivide>
hipError_t launch_dt(const NormModArgs& a, hipStream_t st) {
  const dim3 block(256);
  const bool vec = DT != 2 && a.N % 8 == 0 && a.x_stride % 8 == 0 && a.N <= 64 * 8 * 16 &&
                   (uintptr_t)a.x % 16 == 0 && (uintptr_t)a.scale % 16 == 0 &&
                   (uintptr_t)a.shift % 16 == 0 && (uintptr_t)a.gamma % 16 == 0 &&
                   (uintptr_t)a.beta % 16 == 0 && (uintptr_t)a.out % 16 == 0 && (uintptr_t)a.out_q % 8 == 0;
  if constexpr (DT != 2) {
    if (vec) {
      const int nvec = (int)(a.N / 8);
      // the model's row lengths with a broadcast modulation row: one wave per row (M 10800, N 5120,
      // FP8 output: 40.2 -> 34.2 us with reciprocal rounding, 43.8 -> 38.4 us with division, against
      // the workgroup row walk below; bf16 output 41.4 vs 40.1 us). The plain op takes the same
      // kernel so that its output and the FP8 op's bf16 output are the same bits.
      if (a.mod_rows == 1 && !a.gamma && a.M > 1 && (a.N == 4096 || a.N == 5120)) {
        auto kern = a.N == 5120 ? norm_mod_wave_rows<DT == 1, NORM, kFp8, kDivide, 10>
                                : norm_mod_wave_rows<DT == 1, NORM, kFp8, kDivide, 8>;
        const int64_t slots = (int64_t)device_cus() * resident_blocks((const void*)kern, 256) * 4;
        const int64_t wgs = ((a.M < slots ? a.M : slots) + 3) / 4;
        hipLaunchKernelGGL(kern, dim3((unsigned)wgs), dim3(256), 0, st, a);
        return hipGetLastError();
      }
      if (nvec > 256 && a.mod_rows == 1 && !a.gamma && a.M > 1) {
        // long rows, broadcast modulation, no affine weights: persistent row walk
        // with VPT = 2 vectors per thread and nvec / 2 threads (rounded to waves)
        auto kern = norm_mod_rows<DT == 1, NORM, kFp8, kDivide, 2>;
        const int threads = ((nvec + 1) / 2 + 63) / 64 * 64;
        if (threads <= 64 * kMaxRowWaves) {
          const int64_t slots = (int64_t)device_cus() * resident_blocks((const void*)kern, threads);
          const dim3 grid((unsigned)(a.M < slots ? a.M : slots));
          hipLaunchKernelGGL(kern, grid, dim3(threads), 0, st, a);
          return hipGetLastError();
        }
      }
      if (nvec > 256) {  // long rows: one workgroup per row
        const dim3 grid((unsigned)a.M);
        const int need = (nvec + 255) / 256;
#define JOY_NORM_ROW(V)                                                                              \
  if (need <= V) {                                                                                   \
    hipLaunchKernelGGL((norm_mod_vec<DT == 1, NORM, kFp8, kDivide, V, 4>), grid, block, 0, st, a);  \
    return hipGetLastError();                                                                        \
  }
        JOY_NORM_ROW(2)
        JOY_NORM_ROW(3)
        JOY_NORM_ROW(4)
#undef JOY_NORM_ROW
      } else {  // short rows: one wave per row
        const dim3 grid((unsigned)((a.M + 3) / 4));
        const int need = (nvec + 63) / 64;
#define JOY_NORM_WAVE(V)                                                                             \
  if (need <= V) {                                                                                   \
    hipLaunchKernelGGL((norm_mod_vec<DT == 1, NORM, kFp8, kDivide, V, 1>), grid, block, 0, st, a);  \
    return hipGetLastError();                                                                        \
  }
        JOY_NORM_WAVE(1)
        JOY_NORM_WAVE(2)
        JOY_NORM_WAVE(4)
#undef JOY_NORM_WAVE
      }
    }
  }
  const dim3 grid((unsigned)((a.M + 3) / 4));
  hipLaunchKernelGGL((norm_mod_scalar<DT, NORM, kFp8, kDivide>), grid, block, 0, st, a);
  return hipGetLastError();
}

template <int DT, bool kFp8, bool kDivide>
hipError_t launch_norm(const NormModArgs& a, hipStream_t st) {
  return a.norm_type == 0 ? launch_dt<DT, 0, kFp8, kDivide>(a, st) : launch_dt<DT, 1, kFp8, kDivide>(a, st);
}

}  // namespace

hipError_t launch_norm_modulate(const NormModArgs& a, hipStream_t st) {
  if (a.M == 0 || a.N == 0) return hipSuccess;
  if (!a.out_q) {
    if (a.dtype == 0) return launch_norm<0, false, true>(a, st);
    if (a.dtype == 1) return launch_norm<1, false, true>(a, st);
    return launch_norm<2, false, true>(a, st);
  }
  if (a.dtype == 0) return a.divide ? launch_norm<0, true, true>(a, st) : launch_norm<0, true, false>(a, st);
  return a.divide ? launch_norm<1, true, true>(a, st) : launch_norm<1, true, false>(a, st);
}

}  // namespace joy
