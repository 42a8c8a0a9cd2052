// Dynamic per-token (row-wise) activation quantisation to OCP e4m3fn on gfx950.
//
//   s[m] = max(absmax_k |x[m,k]|, 1e-8) / 448
//   q[m,k] = e4m3fn(clamp(x[m,k] / s[m], -448, 448))            (DIVIDE)
//   q[m,k] = e4m3fn(clamp(x[m,k] * (1 / s[m]), -448, 448))      (RECIPROCAL)
//
// DIVIDE is the reference model formula (deploy/xvideo/models/dit/fp8_linear.py:38-43);
// RECIPROCAL is the reference's gfx950 kernel (joyomni_ops/csrc/per_token_quant_fp8_rocm.hip:66-78).
//
// Design: one wave64 owns one row. Each lane keeps its share of the row in
// registers as 16-byte vectors, so the row is read from HBM exactly once. The
// absmax runs on the 16-bit patterns (|x| = bits & 0x7fff orders like the
// value for bf16 and fp16, NaN above inf) with packed u16 max, then one
// cross-lane reduction. Quantised bytes leave as 8-byte stores per lane, which
// a wave turns into fully coalesced 512-byte segments.
#include "joy_common.hpp"
#include "joy_kernels.hpp"

namespace joy {
namespace {

typedef unsigned short us2 __attribute__((ext_vector_type(2)));

template <bool kFp16>
__device__ __forceinline__ float half_to_f32(uint32_t bits16) {
  if constexpr (kFp16) return fp16_bits_to_f32(bits16);
  return __uint_as_float(bits16 << 16);
}

// fp16 values are converted arithmetically (exact, denormals kept; kFinite: every
// value of the row is finite, so inf / NaN need no select): plain fp32 arithmetic
// on the converted values, with no register barrier that would make the widest rows
// spill.
template <bool kFp16, bool kFinite>
__device__ __forceinline__ void unpack8(const uint4& v, float f[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (kFp16 && kFinite) {
      f[2 * i] = fp16_finite_bits_to_f32(w[i] & 0xffffu);
      f[2 * i + 1] = fp16_finite_bits_to_f32(w[i] >> 16);
    } else if constexpr (kFp16) {
      f[2 * i] = fp16_bits_to_f32_arith(w[i] & 0xffffu);
      f[2 * i + 1] = fp16_bits_to_f32_arith(w[i] >> 16);
    } else {
      f[2 * i] = bf16_lo(w[i]);
      f[2 * i + 1] = bf16_hi(w[i]);
    }
  }
}

__device__ __forceinline__ uint32_t absmax_bits(uint32_t acc, const uint4& v) {
  us2 a = __builtin_bit_cast(us2, acc);
  a = __builtin_elementwise_max(a, __builtin_bit_cast(us2, v.x & 0x7fff7fffu));
  a = __builtin_elementwise_max(a, __builtin_bit_cast(us2, v.y & 0x7fff7fffu));
  a = __builtin_elementwise_max(a, __builtin_bit_cast(us2, v.z & 0x7fff7fffu));
  a = __builtin_elementwise_max(a, __builtin_bit_cast(us2, v.w & 0x7fff7fffu));
  return __builtin_bit_cast(uint32_t, a);
}

// Software fp32 -> e4m3fn (RNE, no saturation), for rows holding inf/NaN where
// torch's exact NaN/sign behaviour is wanted.
__device__ uint32_t f32_to_e4m3fn_soft(float x) {
  uint32_t b = __float_as_uint(x);
  uint32_t sign = (b >> 24) & 0x80u;
  if ((b & 0x7f800000u) == 0x7f800000u) return 0x7fu | sign;
  float a = fabsf(x);
  if (a < 0.015625f) return (uint32_t)__builtin_rintf(a * 512.0f) | sign;
  uint32_t ab = __float_as_uint(a);
  uint32_t r = (ab + 0x7ffffu + ((ab >> 20) & 1u)) >> 20;
  int e8 = (int)(r >> 3) - 127 + 7;
  uint32_t m3 = r & 7u;
  if (e8 > 15 || (e8 == 15 && m3 == 7u)) return 0x7fu | sign;
  return (((uint32_t)e8 << 3) | m3) | sign;
}

// Row-scale from the reduced 16-bit absmax pattern. Returns false for a
// non-finite absmax (inf or NaN in the row).
template <bool kFp16>
__device__ __forceinline__ bool row_scale(uint32_t amax_bits, float& s) {
  const uint32_t inf_bits = kFp16 ? 0x7c00u : 0x7f80u;
  float amax = half_to_f32<kFp16>(amax_bits);
  if (amax_bits >= inf_bits) {
    s = amax / kFp8Max;  // inf or NaN, like torch: clamp_min keeps both
    return false;
  }
  s = fmaxf(amax, 1.0e-8f) / kFp8Max;
  return true;
}

template <bool kDivide>
__device__ __forceinline__ float scale_value(float x, float s, float r) {
  if constexpr (kDivide) return div_by_scale(x, s, r);
  return x * r;
}

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// Streaming (non-temporal) 16-byte load / 8-byte store: rows are read and
// written exactly once.
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
  const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void st_stream(uint2* p, const uint2& v) {
  __builtin_nontemporal_store((u32x2){v.x, v.y}, (u32x2*)p);
}

// VPT = 16-byte vectors per lane (row length K = 8 * nvec, nvec <= 64 * VPT).
template <bool kFp16, bool kDivide, int VPT>
__global__ __launch_bounds__(256) void quant_rows_vec(const uint4* __restrict__ in,
                                                      uint2* __restrict__ out_q,
                                                      float* __restrict__ out_s, int64_t rows,
                                                      int nvec) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint4* src = in + row * nvec;
  uint4 v[VPT];
  uint32_t amax = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int idx = lane + i * kWave;
    if (idx < nvec) {
      v[i] = ld_stream(&src[idx]);
    } else {
      v[i] = make_uint4(0, 0, 0, 0);
    }
    amax = absmax_bits(amax, v[i]);
  }
  amax = (amax & 0xffffu) > (amax >> 16) ? (amax & 0xffffu) : (amax >> 16);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    uint32_t o = __shfl_xor(amax, off, kWave);
    amax = o > amax ? o : amax;
  }
  float s;
  const bool finite = row_scale<kFp16>(amax, s);
  if (lane == 0) out_s[row] = s;
  const float r = 1.0f / s;
  uint2* dst = out_q + row * nvec;
  if (finite) {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int idx = lane + i * kWave;
      if (idx < nvec) {
        // No clamp needed on rows with a finite scale: |x| <= absmax, so the scaled value is at
        // most 448 * (1 + 2^-23) (448.00003 for 15 % of the bf16 absmax values, both roundings),
        // below 464, the midpoint to the next e4m3 step, so the conversion rounds it to 448.
        float f[8];
        unpack8<kFp16, true>(v[i], f);
#pragma unroll
        for (int j = 0; j < 8; ++j)
          f[j] = scale_value<kDivide>(f[j], s, r);
        uint2 o;
        o.x = pack_fp8x4(f[0], f[1], f[2], f[3]);
        o.y = pack_fp8x4(f[4], f[5], f[6], f[7]);
        st_stream(&dst[idx], o);
      }
    }
  } else {
    // rows holding inf / NaN (cold): read the row again rather than index v[] from a
    // rolled loop, so that v[] stays in registers
#pragma unroll 1
    for (int idx = lane; idx < nvec; idx += kWave) {
      float f[8];
      unpack8<kFp16, false>(src[idx], f);
      uint32_t b[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float t = kDivide ? f[j] / s : f[j] * r;
        b[j] = f32_to_e4m3fn_soft(clamp_fp8(t));
      }
      uint2 o;
      o.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
      o.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
      dst[idx] = o;
    }
  }
}

// Any K (including K % 8 != 0 or unaligned rows): one wave per row, two passes.
template <bool kFp16, bool kDivide>
__global__ __launch_bounds__(256) void quant_rows_scalar(const uint16_t* __restrict__ in,
                                                         uint8_t* __restrict__ out_q,
                                                         float* __restrict__ out_s, int64_t rows,
                                                         int64_t K) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint16_t* src = in + row * K;
  uint32_t amax = 0;
  for (int64_t k = lane; k < K; k += kWave) {
    uint32_t a = src[k] & 0x7fffu;
    amax = a > amax ? a : amax;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    uint32_t o = __shfl_xor(amax, off, kWave);
    amax = o > amax ? o : amax;
  }
  float s;
  const bool finite = row_scale<kFp16>(amax, s);
  if (lane == 0) out_s[row] = s;
  const float r = 1.0f / s;
  uint8_t* dst = out_q + row * K;
  for (int64_t k = lane; k < K; k += kWave) {
    float x = half_to_f32<kFp16>(src[k]);
    float t = finite ? scale_value<kDivide>(x, s, r) : (kDivide ? x / s : x * r);
    dst[k] = (uint8_t)f32_to_e4m3fn_soft(clamp_fp8(t));
  }
}

template <bool kFp16, bool kDivide>
hipError_t launch_quant(const void* in, void* q, float* s, int64_t M, int64_t K, hipStream_t st) {
  constexpr int kRowsPerBlock = 4;
  const dim3 grid((unsigned)((M + kRowsPerBlock - 1) / kRowsPerBlock));
  const dim3 block(kRowsPerBlock * kWave);
  const bool aligned = ((uintptr_t)in % 16 == 0) && ((uintptr_t)q % 8 == 0) && (K % 8 == 0);
  const int64_t nvec = K / 8;
  if (aligned && nvec <= 64 * 32) {
    const int need = (int)((nvec + 63) / 64);
#define JOY_QUANT_CASE(V)                                                                       \
  if (need <= V) {                                                                              \
    hipLaunchKernelGGL((quant_rows_vec<kFp16, kDivide, V>), grid, block, 0, st,                 \
                       (const uint4*)in, (uint2*)q, s, M, (int)nvec);                           \
    return hipGetLastError();                                                                   \
  }
    JOY_QUANT_CASE(1)
    JOY_QUANT_CASE(2)
    JOY_QUANT_CASE(4)
    JOY_QUANT_CASE(8)
    JOY_QUANT_CASE(12)
    JOY_QUANT_CASE(16)
    JOY_QUANT_CASE(24)
    JOY_QUANT_CASE(32)
#undef JOY_QUANT_CASE
  }
  hipLaunchKernelGGL((quant_rows_scalar<kFp16, kDivide>), grid, block, 0, st, (const uint16_t*)in,
                     (uint8_t*)q, s, M, K);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_per_token_quant(const void* in, bool in_fp16, void* q, float* s, int64_t M,
                                  int64_t K, bool divide, hipStream_t st) {
  if (M == 0) return hipSuccess;
  if (in_fp16) {
    return divide ? launch_quant<true, true>(in, q, s, M, K, st)
                  : launch_quant<true, false>(in, q, s, M, K, st);
  }
  return divide ? launch_quant<false, true>(in, q, s, M, K, st)
                : launch_quant<false, false>(in, q, s, M, K, st);
}

}  // namespace joy
