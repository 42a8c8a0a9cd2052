// Shared device helpers for the gfx950 kernels of libjoyomni_hip.
//
// Number formats are handled at the bit level so that every rounding is
// explicit: bf16 <-> fp32 (RNE), fp16 -> fp32, and fp32 -> OCP e4m3fn through
// the CDNA4 v_cvt_pk_fp8_f32 instruction (RNE, OCP encoding on gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace joy {

constexpr int kWave = 64;          // CDNA wavefront width
constexpr float kFp8Max = 448.0f;  // torch.finfo(torch.float8_e4m3fn).max

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 bits, round to nearest even, NaN kept quiet.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t b = __float_as_uint(f);
  if ((b & 0x7fffffffu) > 0x7f800000u) return (b >> 16) | 0x40u;
  return (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
}

typedef __bf16 bf16x2_vt __attribute__((ext_vector_type(2)));
typedef float f32x2_vt __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16 pair, round to nearest even: one v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_vt v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_vt));
}

// fp16 bits -> fp32 (exact).
__device__ __forceinline__ float fp16_bits_to_f32(uint32_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)v;
}

__device__ __forceinline__ uint32_t pack_fp16x2(float lo, float hi) {
  uint16_t a = __builtin_bit_cast(uint16_t, (_Float16)lo);
  uint16_t b = __builtin_bit_cast(uint16_t, (_Float16)hi);
  return (uint32_t)a | ((uint32_t)b << 16);
}

// Four fp32 values -> four e4m3fn bytes packed little-endian (RNE).
__device__ __forceinline__ uint32_t pack_fp8x4(float a, float b, float c, float d) {
  uint32_t w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return w;
}

// Clamp to the finite e4m3fn range; NaN passes through like torch.clamp.
__device__ __forceinline__ float clamp_fp8(float v) {
  v = v > kFp8Max ? kFp8Max : v;
  v = v < -kFp8Max ? -kFp8Max : v;
  return v;
}

// Correctly rounded x / s given r = RN(1/s): one multiply, two fma, sign fix.
// Equality with IEEE division after the e4m3fn cast is proven exhaustively over
// every (16-bit x, quantiser scale s) pair by oracle_check_device_division.
__device__ __forceinline__ float div_by_scale(float x, float s, float r) {
  float q0 = x * r;
  float e = __builtin_fmaf(-q0, s, x);
  float q1 = __builtin_fmaf(e, r, q0);
  return __builtin_copysignf(q1, x);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

}  // namespace joy
