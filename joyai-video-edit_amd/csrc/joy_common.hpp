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

// Value barrier around fp16 conversions (an empty asm: no instruction). Without it
// the compiler folds fma + fp32 -> fp16 rounding into one v_fma_mixlo_f16, a single
// rounding of the exact result where the reference's fp32 arithmetic rounds twice
// (to fp32, then to fp16), and folds fp16 -> fp32 conversions into mixed-precision
// FMA sources. Pinning the fp32 value keeps v_cvt_f32_f16 / v_cvt_pk_f16_f32 and
// plain fp32 arithmetic, so fp16 results follow the fp32 formula bit for bit.
__device__ __forceinline__ float pin_f32(float v) {
  __asm__("" : "+v"(v));
  return v;
}

// fp16 bits -> fp32 (exact, denormals kept).
__device__ __forceinline__ float fp16_bits_to_f32(uint32_t h) {
  const _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
  return pin_f32((float)v);
}

// fp16 bits of a finite value -> fp32 (exact, denormals kept), without a conversion
// instruction: the 15 magnitude bits placed at the fp32 exponent/mantissa position
// read as x * 2^-112 (an fp32 denormal for fp16 denormals), and one exact multiply
// by 2^112 restores x. For rows known to be finite; inf / NaN bits give large finite
// values.
__device__ __forceinline__ float fp16_finite_bits_to_f32(uint32_t h) {
  const float scaled = __uint_as_float(((h & 0x7fffu) << 13) | ((h & 0x8000u) << 16));
  return scaled * 0x1p112f;
}

// fp16 bits -> fp32, exact for every value (inf / NaN bits rebuilt with the fp32
// exponent), without a conversion instruction.
__device__ __forceinline__ float fp16_bits_to_f32_arith(uint32_t h) {
  const uint32_t special = ((h & 0x7fffu) << 13) | 0x7f800000u | ((h & 0x8000u) << 16);
  return (h & 0x7c00u) == 0x7c00u ? __uint_as_float(special) : fp16_finite_bits_to_f32(h);
}

// fp32 -> fp16 bits, round to nearest even, from the fp32 value.
__device__ __forceinline__ uint32_t f32_to_fp16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)pin_f32(f));
}

// fp32 -> fp16 -> fp32 (the value an fp16 store keeps).
__device__ __forceinline__ float round_fp16(float f) {
  return fp16_bits_to_f32(f32_to_fp16_bits(f));
}

typedef _Float16 f16x2_vt __attribute__((ext_vector_type(2)));

// Two fp32 -> packed fp16 pair, round to nearest even (v_cvt_pk_f16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_fp16x2(float lo, float hi) {
  const f32x2_vt v = {pin_f32(lo), pin_f32(hi)};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_vt));
}

// Four fp32 values -> four e4m3fn bytes packed little-endian (RNE).
__device__ __forceinline__ uint32_t pack_fp8x4(float a, float b, float c, float d) {
  uint32_t w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return w;
}

// The same bytes as pack_fp8x4 without a zeroed register: the first conversion keeps the upper
// half of its destination, which the second overwrites, so a's bits may stand there.
__device__ __forceinline__ uint32_t pack_fp8x4_reuse(float a, float b, float c, float d) {
  const uint32_t w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int)__float_as_uint(a), false);
  return __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
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

// Per-head q/k RMSNorm and rotation (fused_qknorm_rope_3d_kernel.cu:68-105), written with
// explicit fma so that the standalone norm/RoPE kernel and the QKV GEMM epilogue, which
// hold a head's elements in different lane layouts, give the same bits. The sum of squares
// is fma(x_j, x_j, s) over 8 consecutive elements (from 0), then a tree over the head's G =
// D / 8 groups of 8 (group index = element / 8): g with g ^ (G / 2), then G / 4, ..., 1.
__device__ __forceinline__ float head_rsqrt(float ss, float inv_d, float eps) {
  return __builtin_amdgcn_rsqf(__builtin_fmaf(ss, inv_d, eps));
}
// pair (x0, x1) rotated by (c, s): (x0 c - x1 s, x0 s + x1 c)
__device__ __forceinline__ void rope_pair(float x0, float x1, float c, float s, float& o0, float& o1) {
  o0 = __builtin_fmaf(x0, c, -(x1 * s));
  o1 = __builtin_fmaf(x0, s, x1 * c);
}

}  // namespace joy
