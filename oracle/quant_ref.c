/*
 * Independent C restatement of the per-token FP8 quantiser -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg load
 * this library (oracle/liboracle.so), and only as a checker.
 *
 * oracle_quant_rows follows:
 *   variant 0 (division):   deploy/xvideo/models/dit/fp8_linear.py:38-43
 *   variant 1 (reciprocal): joyomni_ops/csrc/per_token_quant_fp8_rocm.hip:60-78
 * s = max(absmax, 1e-8f) / 448 (IEEE single division), q = e4m3fn_rne(clamp(x/s or x*(1/s))).
 *
 * oracle_check_device_division proves, by exhaustion over the quantiser's whole
 * input domain, that the device's division formula
 *     r = 1/s (correctly rounded, once per row)
 *     q0 = x*r ; e = fma(-q0, s, x) ; q1 = copysign(fma(e, r, q0), x)
 * produces the same e4m3fn byte as correctly rounded x/s, for every 16-bit
 * input x (bf16 or fp16 bit patterns) and every scale s that the quantiser can
 * produce (s = max(a, 1e-8)/448 for every finite 16-bit absmax a), restricted
 * to |x| <= a as in any real row.
 *
 * Pins: tests/test_oracle_quant.py compares oracle_quant_rows with the numpy
 * oracle and with torch's own CPU ops on the same inputs.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define FP8_MAX 448.0f

static inline float bits_f32(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

static inline float bf16_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

static inline float fp16_f32(uint16_t h) {
  uint32_t s = (uint32_t)(h >> 15) << 31;
  uint32_t e = (h >> 10) & 0x1f;
  uint32_t m = h & 0x3ff;
  if (e == 0) {
    float v = ldexpf((float)m, -24);
    return s ? -v : v;
  }
  if (e == 31) return bits_f32(s | 0x7f800000u | (m << 13));
  return bits_f32(s | ((e - 15 + 127) << 23) | (m << 13));
}

/* float -> OCP e4m3fn, round to nearest even, no saturation (torch semantics). */
uint8_t oracle_f32_to_e4m3fn(float x) {
  uint32_t b = f32_bits(x);
  uint8_t sign = (uint8_t)((b >> 24) & 0x80);
  if (!isfinite(x)) return (uint8_t)(0x7f | sign);
  float a = fabsf(x);
  if (a < 0.015625f) { /* 2^-6: subnormal step 2^-9 */
    float k = nearbyintf(a * 512.0f); /* exact scaling, default mode = RNE */
    return (uint8_t)((uint8_t)k | sign);
  }
  uint32_t ab = f32_bits(a);
  uint32_t lsb = (ab >> 20) & 1u;
  uint32_t r = (ab + 0x7ffffu + lsb) >> 20;
  int e8 = (int)(r >> 3) - 127 + 7;
  uint32_t m3 = r & 7u;
  if (e8 > 15 || (e8 == 15 && m3 == 7)) return (uint8_t)(0x7f | sign);
  return (uint8_t)(((uint32_t)e8 << 3 | m3) | sign);
}

static inline float clamp_keep_nan(float v) {
  if (v > FP8_MAX) return FP8_MAX;
  if (v < -FP8_MAX) return -FP8_MAX;
  return v;
}

void oracle_quant_rows(const uint16_t* x, int is_fp16, int64_t M, int64_t K, int variant,
                       uint8_t* q, float* s) {
  for (int64_t m = 0; m < M; ++m) {
    const uint16_t* row = x + m * K;
    float amax = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      float v = is_fp16 ? fp16_f32(row[k]) : bf16_f32(row[k]);
      float av = fabsf(v);
      if (av > amax || isnan(av)) amax = av;
    }
    float sc = fmaxf(amax, 1e-8f) / FP8_MAX;
    if (isnan(amax)) sc = amax;
    s[m] = sc;
    float inv = 1.0f / sc;
    for (int64_t k = 0; k < K; ++k) {
      float v = is_fp16 ? fp16_f32(row[k]) : bf16_f32(row[k]);
      float t = variant == 0 ? v / sc : v * inv;
      q[m * K + k] = oracle_f32_to_e4m3fn(clamp_keep_nan(t));
    }
  }
}

/* Device division formula (see header). */
static inline float device_div(float x, float s, float r) {
  float q0 = x * r;
  float e = fmaf(-q0, s, x);
  float q1 = fmaf(e, r, q0);
  return copysignf(q1, x);
}

/*
 * Exhaustive check. Scales are enumerated from absmax values a_idx in
 * [a_begin, a_end) over the positive finite 16-bit patterns; every x with
 * |x| <= a is tested. Returns the number of (x, s) pairs whose fp8 bytes
 * differ; *n_pairs receives the number of pairs tested; the first mismatch is
 * stored in first_x / first_a (bit patterns) when non-null.
 */
int64_t oracle_check_device_division(int is_fp16, uint32_t a_begin, uint32_t a_end,
                                     int64_t* n_pairs, uint32_t* first_x, uint32_t* first_a) {
  int64_t bad = 0, pairs = 0;
  for (uint32_t ab = a_begin; ab < a_end; ++ab) {
    float a = is_fp16 ? fp16_f32((uint16_t)ab) : bf16_f32((uint16_t)ab);
    if (!isfinite(a) || a < 0.0f) continue;
    float s = fmaxf(a, 1e-8f) / FP8_MAX;
    float r = 1.0f / s;
    for (uint32_t xb = 0; xb < 65536u; ++xb) {
      float x = is_fp16 ? fp16_f32((uint16_t)xb) : bf16_f32((uint16_t)xb);
      if (!(fabsf(x) <= a)) continue;
      ++pairs;
      float qd = x / s;
      float qm = device_div(x, s, r);
      if (f32_bits(qd) == f32_bits(qm)) continue;
      if (oracle_f32_to_e4m3fn(clamp_keep_nan(qd)) != oracle_f32_to_e4m3fn(clamp_keep_nan(qm))) {
        if (bad == 0 && first_x) { *first_x = xb; *first_a = ab; }
        ++bad;
      }
    }
  }
  if (n_pairs) *n_pairs = pairs;
  return bad;
}
