// FP8 (e4m3fn) x FP8 -> bf16/fp16 GEMM with row/column scales and fused epilogue, gfx950.
//
//   out[m, n] = round( fma( acc[m, n] * scales_b[n], scales_a[m], bias[n] ) )
//   acc[m, n] = sum_k A[m, k] * W[n, k]          (fp32 accumulation in MFMA)
//
// Contract: joyomni_ops/csrc/fp8_gemm.cu:1450-1487 (A row-major [M,K], B the
// (K,N) column-major matrix == W[N,K] row-major, scales fp32, bias of out
// dtype); epilogue order of fp8_gemm.cu:99-136. Optional GELU-tanh epilogue
// applies F.gelu(approximate="tanh") to the rounded output, as the reference
// model does after its up-projection (deploy/xvideo/models/dit/dit.py:87-89).
//
// Large-M kernel (MFMA-bound):
//  * macro tile 256x256, K step 128 bytes, 256 threads = 4 waves in 2x2, each
//    wave owns a 128x128 sub-tile as 4x4 v_mfma_f32_32x32x64_f8f6f4 tiles
//    (256 fp32 accumulators per lane, held in AGPR/VGPR);
//  * both operands are K-contiguous, so a lane's MFMA fragment (32 K-bytes of
//    one row) is two 16-byte LDS reads. The MFMA takes W as its "A" operand and
//    the activation as "B", so each lane ends with 4 consecutive output columns
//    of one output row -> 8-byte stores;
//  * global -> LDS with gfx950 16-byte direct-to-LDS loads
//    (global_load_lds_dwordx4), double-buffered in two static LDS halves
//    (128 KiB of the 160 KiB), one barrier per K step;
//  * LDS rows are 128 bytes = 8 chunks of 16 bytes; chunk c of row r is stored at
//    c ^ swz(r), swz(r) = (r & 7) ^ ((r >> 3) & 1), which makes both the
//    direct-to-LDS writes and the fragment reads bank-conflict free for 8- and
//    16-lane service groups;
//  * blockIdx -> tile mapping is XCD-aware (consecutive workgroups land on
//    different XCDs, so each XCD gets a contiguous tile range) and grouped
//    (GROUP_M tile-rows share B columns in one XCD's L2).
#include <stdlib.h>

#include "joy_common.hpp"
#include "joy_kernels.hpp"

namespace joy {
namespace {

constexpr int BK = 128;
#ifndef JOY_BM
#define JOY_BM 256
#define JOY_BN 256
#define JOY_WM 2
#define JOY_WN 4
#endif

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

__device__ __forceinline__ v16f mfma_32x32x64_fp8(const v8i& a, const v8i& b, const v16f& c) {
  // Scale operands of zero select the plain (unscaled) f8f6f4 MFMA; format 0 = e4m3.
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ void wait_vmem_all() {
  // s_waitcnt vmcnt(0): gfx9 encoding, expcnt and lgkmcnt left at their maxima.
  __builtin_amdgcn_s_waitcnt(0x0f70);
}

// GELU, tanh form: 0.5 x (1 + tanh(u)) == x * sigmoid(2u), u = sqrt(2/pi) (x + 0.044715 x^3).
// exp2 / rcp hardware approximations (~1 ulp fp32) are far below bf16 resolution.
__device__ __forceinline__ float gelu_tanh(float x) {
  const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
  const float k1 = 0.044715f;
  const float u2 = 2.0f * k0 * __builtin_fmaf(k1 * x, x * x, x);
  const float e = __builtin_amdgcn_exp2f(-u2 * 1.4426950408889634f);  // exp(-2u)
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two fp32 -> packed 16-bit pair, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
template <bool kBf16>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  if constexpr (kBf16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
}

// Value of a packed 16-bit pair element (exact).
template <bool kBf16>
__device__ __forceinline__ float unpack_lo(uint32_t w) {
  if constexpr (kBf16) return __uint_as_float(w << 16);
  return fp16_bits_to_f32(w & 0xffffu);
}
template <bool kBf16>
__device__ __forceinline__ float unpack_hi(uint32_t w) {
  if constexpr (kBf16) return __uint_as_float(w & 0xffff0000u);
  return fp16_bits_to_f32(w >> 16);
}

// Epilogue of one wave's FN x FM grid of 32x32 MFMA tiles. acc[i][j][r] holds
// output row m_base + 32j + (lane % 32) and column n_base + 32i + 8(r/4) + 4g + r%4.
// Column operands (scale, bias) are loaded once per lane up front, then every
// output quad is rounded, optionally passed through GELU, and stored as 8 bytes.
template <bool kBf16, bool kGelu, int FN, int FM>
__device__ __forceinline__ void store_tile(const v16f (&acc)[FN][FM], int m_base, int n_base,
                                           int frow, int g, const float* __restrict__ sa,
                                           const float* __restrict__ sb,
                                           const uint16_t* __restrict__ bias,
                                           uint16_t* __restrict__ C, int M, int N, int64_t ldc) {
  float4 sbv[FN][4];
  uint2 bv[FN][4];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n_base + i * 32 + q * 8 + g * 4;
      const bool ok = n < N;
      sbv[i][q] = ok ? *(const float4*)(sb + n) : make_float4(0.f, 0.f, 0.f, 0.f);
      bv[i][q] = (ok && bias) ? *(const uint2*)(bias + n) : make_uint2(0u, 0u);
    }
  float sav[FM];
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int m = m_base + j * 32 + frow;
    sav[j] = m < M ? sa[m] : 0.0f;
  }
  // interior wave tiles (all but the last tile row/column) store without guards
  const bool interior = (m_base + 32 * FM <= M) && (n_base + 32 * FN <= N);
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int m = m_base + j * 32 + frow;
    if (!interior && m >= M) continue;
    uint16_t* crow = C + (int64_t)m * ldc;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n_base + i * 32 + q * 8 + g * 4;
        if (!interior && n >= N) continue;
        const float sbe[4] = {sbv[i][q].x, sbv[i][q].y, sbv[i][q].z, sbv[i][q].w};
        const float be[4] = {unpack_lo<kBf16>(bv[i][q].x), unpack_hi<kBf16>(bv[i][q].x),
                             unpack_lo<kBf16>(bv[i][q].y), unpack_hi<kBf16>(bv[i][q].y)};
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = __builtin_fmaf(acc[i][j][q * 4 + e] * sbe[e], sav[j], be[e]);
        uint2 pk = make_uint2(pack2<kBf16>(o[0], o[1]), pack2<kBf16>(o[2], o[3]));
        if constexpr (kGelu) {
          // the reference applies GELU to the rounded GEMM output and rounds again
          pk = make_uint2(pack2<kBf16>(gelu_tanh(unpack_lo<kBf16>(pk.x)), gelu_tanh(unpack_hi<kBf16>(pk.x))),
                          pack2<kBf16>(gelu_tanh(unpack_lo<kBf16>(pk.y)), gelu_tanh(unpack_hi<kBf16>(pk.y))));
        }
        *(uint2*)(crow + n) = pk;
      }
    }
  }
}

template <bool kBf16>
__device__ __forceinline__ float round_out(float v) {
  if constexpr (kBf16) return __uint_as_float(f32_to_bf16_bits(v) << 16);
  return (float)(_Float16)v;
}

template <bool kBf16>
__device__ __forceinline__ float bias_value(const uint16_t* bias, int64_t n) {
  if (!bias) return 0.0f;
  if constexpr (kBf16) return __uint_as_float((uint32_t)bias[n] << 16);
  return fp16_bits_to_f32(bias[n]);
}

struct TileCoord {
  int tm, tn;
};

__device__ __forceinline__ TileCoord map_tile(int b, int tiles_m, int tiles_n, int group_m) {
  const int T = tiles_m * tiles_n;
  // XCD-aware: hardware deals workgroups round-robin to the 8 XCDs.
  const int xcd = b & 7, local = b >> 3, q = T >> 3, rem = T & 7;
  const int t = xcd < rem ? xcd * (q + 1) + local : rem * (q + 1) + (xcd - rem) * q + local;
  const int per_group = group_m * tiles_n;
  const int g = t / per_group;
  const int first_m = g * group_m;
  const int gsz = min(tiles_m - first_m, group_m);
  const int r = t - g * per_group;
  return {first_m + r % gsz, r / gsz};
}

template <bool kBf16, bool kGelu, int BM, int BN, int WAVES_M, int WAVES_N>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64, 1) void fp8_gemm_tiled(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ sa,
    const float* __restrict__ sb, const uint16_t* __restrict__ bias, uint16_t* __restrict__ C,
    int M, int N, int K, int64_t ldc, int tiles_m, int tiles_n, int group_m) {
  constexpr int NW = WAVES_M * WAVES_N;      // waves per workgroup
  constexpr int WTM = BM / WAVES_M;          // wave tile rows (activation rows)
  constexpr int WTN = BN / WAVES_N;          // wave tile cols (weight rows)
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int IA = BM / 8 / NW, IW = BN / 8 / NW;  // 8-row load instructions per wave
  static_assert(IA * 8 * NW == BM && IW * 8 * NW == BN, "tile rows must split over waves");
  __shared__ __attribute__((aligned(1024))) uint8_t lds_a0[BM * BK];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_w0[BN * BK];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_a1[BM * BK];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_w1[BN * BK];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const TileCoord tc = map_tile(blockIdx.x, tiles_m, tiles_n, group_m);
  const int m0 = tc.tm * BM, n0 = tc.tn * BN;

  // ---- global -> LDS addressing: wave w fills rows [w*IA*8, (w+1)*IA*8) of
  // the activation tile (and likewise for W) with 8-row x 128-byte instructions.
  const int lrow = lane >> 3;   // row within an 8-row instruction
  const int lchunk = lane & 7;  // physical 16-byte chunk this lane writes
  int64_t ga[IA], gw[IW];
#pragma unroll
  for (int i = 0; i < IA; ++i) {
    const int row = (wave * IA + i) * 8 + lrow;
    const int c = lchunk ^ swz(row);  // logical chunk whose bytes land here
    ga[i] = (int64_t)min(m0 + row, M - 1) * K + c * 16;
  }
#pragma unroll
  for (int i = 0; i < IW; ++i) {
    const int row = (wave * IW + i) * 8 + lrow;
    const int c = lchunk ^ swz(row);
    gw[i] = (int64_t)min(n0 + row, N - 1) * K + c * 16;
  }
  auto issue = [&](uint8_t* la, uint8_t* lw, int kt) {
    const int64_t koff = (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < IA; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(A + ga[i] + koff),
                                       (lds_void*)(la + (wave * IA + i) * 8 * BK), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < IW; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(W + gw[i] + koff),
                                       (lds_void*)(lw + (wave * IW + i) * 8 * BK), 16, 0, 0);
  };

  // ---- fragment addressing: wave (wm, wn) owns activation rows [WTM*wm, +WTM)
  // and weight rows [WTN*wn, +WTN). A lane reads row (l % 32) of a 32-row
  // fragment, K bytes [32g, 32g+32) of the 64-byte MFMA step, g = l / 32.
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int frow = lane & 31, g = lane >> 5;
  // All fragment rows are frow + 32*f (+ multiples of 32), so swz(row) == swz(frow).
  const int sw = swz(frow);
  const int off00 = ((0 + g * 2) ^ sw) * 16, off01 = ((1 + g * 2) ^ sw) * 16;
  const int off10 = ((4 + g * 2) ^ sw) * 16, off11 = ((5 + g * 2) ^ sw) * 16;
  v16f acc[FN][FM];  // [weight-fragment][activation-fragment]
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = (v16f){};

  auto compute = [&](const uint8_t* la, const uint8_t* lw) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int o0 = kk ? off10 : off00, o1 = kk ? off11 : off01;
      v8i fw[FN], fa[FM];
#pragma unroll
      for (int f = 0; f < FN; ++f) {
        const uint8_t* rw = lw + (wn * WTN + f * 32 + frow) * BK;
        const v4i lo = *(const v4i*)(rw + o0);
        const v4i hi = *(const v4i*)(rw + o1);
        fw[f] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int f = 0; f < FM; ++f) {
        const uint8_t* ra = la + (wm * WTM + f * 32 + frow) * BK;
        const v4i lo = *(const v4i*)(ra + o0);
        const v4i hi = *(const v4i*)(ra + o1);
        fa[f] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = mfma_32x32x64_fp8(fw[i], fa[j], acc[i][j]);
    }
  };

  // Single-exit loop over pairs of K steps (buffer 0 then buffer 1), so the
  // accumulators stay in place across iterations; an odd last step follows.
  const int nk = K / BK;
  issue(lds_a0, lds_w0, 0);
  wait_vmem_all();
  __syncthreads();
  for (int kt = 0; kt + 1 < nk; kt += 2) {
    issue(lds_a1, lds_w1, kt + 1);
    compute(lds_a0, lds_w0);
    wait_vmem_all();
    __syncthreads();
    if (kt + 2 < nk) issue(lds_a0, lds_w0, kt + 2);
    compute(lds_a1, lds_w1);
    wait_vmem_all();
    __syncthreads();
  }
  if (nk & 1) compute(lds_a0, lds_w0);

  store_tile<kBf16, kGelu, FN, FM>(acc, m0 + wm * WTM, n0 + wn * WTN, frow, g, sa, sb, bias, C, M, N, ldc);
}

// ---------------------------------------------------------------------------
// Pipelined large-M kernel: K step KS bytes (64 or 128), STAGES-deep ring of LDS
// slots fed by direct-to-LDS loads issued STAGES-1 steps ahead, one barrier per
// step.
//
// LDS rows are KS bytes = KS/16 chunks of 16 bytes; logical chunk c of row r is
// stored at c ^ swz(r). Both swizzles were chosen by measuring
// SQ_LDS_BANK_CONFLICT on gfx950 (zero for the fragment reads below):
//   KS = 64:  swz(r) = (r >> 2) & 3
//   KS = 128: swz(r) = (r & 7) ^ ((r >> 3) & 1)
// Both are invariant under r -> r + 32, so a lane's fragment rows share its swizzle.
// With KS = 128 every DMA instruction moves whole 128-byte lines (8 rows x 128 B).
// ---------------------------------------------------------------------------
template <int KS>
__device__ __forceinline__ int swz_rows(int r) {
  if constexpr (KS == 64) return (r >> 2) & 3;
  return (r & 7) ^ ((r >> 3) & 1);
}

// s_waitcnt with vmcnt(n), expcnt/lgkmcnt at their maxima (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
}

__device__ __forceinline__ void block_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <bool kBf16, bool kGelu, int BM, int BN, int WAVES_M, int WAVES_N, int STAGES, int KS,
          int TOUCH>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64, 1) void fp8_gemm_pipe(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ sa,
    const float* __restrict__ sb, const uint16_t* __restrict__ bias, uint16_t* __restrict__ C,
    int M, int N, int K, int64_t ldc, int tiles_m, int tiles_n, int group_m) {
  constexpr int NW = WAVES_M * WAVES_N;
  constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int CPR = KS / 16;                        // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;                       // rows per DMA instruction
  constexpr int IA = BM / RPI / NW, IW = BN / RPI / NW;  // DMA instructions per wave
  constexpr int LOADS = IA + IW;                      // per wave per stage
  constexpr int A_BYTES = BM * KS, SLOT = (BM + BN) * KS;
  static_assert(KS == 64 || KS == 128, "K step");
  static_assert(IA * RPI * NW == BM && IW * RPI * NW == BN, "tile rows must split over waves");
  // TOUCH > 0: every lane also pulls one 128-byte line of the stage TOUCH steps
  // beyond the newest DMA stage into L2 (4-byte load into a scratch LDS area), so
  // the DMA for that stage later hits L2. One extra load per wave per step.
  constexpr int TPL = (BM + BN + NW * 64 - 1) / (NW * 64);  // touched rows per lane
  constexpr int TLOADS = TOUCH ? TPL : 0;
  constexpr int PER_STEP = LOADS + TLOADS;
  static_assert((STAGES - 2) * PER_STEP + TLOADS < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[STAGES * SLOT + (TOUCH ? 256 * NW : 0)];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const TileCoord tc = map_tile(blockIdx.x, tiles_m, tiles_n, group_m);
  const int m0 = tc.tm * BM, n0 = tc.tn * BN;

  // DMA addressing: lane l of an instruction writes row l / CPR, physical chunk l % CPR.
  const int lrow = lane / CPR, lchunk = lane % CPR;
  int64_t ga[IA], gw[IW];
#pragma unroll
  for (int i = 0; i < IA; ++i) {
    const int row = (wave * IA + i) * RPI + lrow;
    ga[i] = (int64_t)min(m0 + row, M - 1) * K + (lchunk ^ swz_rows<KS>(row)) * 16;
  }
#pragma unroll
  for (int i = 0; i < IW; ++i) {
    const int row = (wave * IW + i) * RPI + lrow;
    gw[i] = (int64_t)min(n0 + row, N - 1) * K + (lchunk ^ swz_rows<KS>(row)) * 16;
  }
  // touch addressing: thread t covers tile rows t, t + NW*64, ... (A rows first, then W)
  const uint8_t* tbase[TPL];
#pragma unroll
  for (int u = 0; u < TPL; ++u) {
    const int trow = min((int)threadIdx.x + u * NW * 64, BM + BN - 1);
    tbase[u] = trow < BM ? A + (int64_t)min(m0 + trow, M - 1) * K
                         : W + (int64_t)min(n0 + trow - BM, N - 1) * K;
  }
  const int nk = K / KS;
  auto touch = [&](int kt) {
    if constexpr (TOUCH > 0) {
      if (kt < nk) {
#pragma unroll
        for (int u = 0; u < TPL; ++u)
          __builtin_amdgcn_global_load_lds((const void*)(tbase[u] + (int64_t)kt * KS),
                                           (lds_void*)(lds + STAGES * SLOT + wave * 256), 4, 0, 0);
      }
    }
  };
  auto issue = [&](int slot, int kt) {
    const int64_t koff = (int64_t)kt * KS;
    uint8_t* base = lds + slot * SLOT;
#pragma unroll
    for (int i = 0; i < IA; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(A + ga[i] + koff),
                                       (lds_void*)(base + (wave * IA + i) * 1024), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < IW; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(W + gw[i] + koff),
                                       (lds_void*)(base + A_BYTES + (wave * IW + i) * 1024), 16, 0,
                                       0);
  };

  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int frow = lane & 31, g = lane >> 5;
  const int fsw = swz_rows<KS>(frow);  // fragment rows differ from frow by multiples of 32
  const int a_row0 = (wm * WTM + frow) * KS, w_row0 = A_BYTES + (wn * WTN + frow) * KS;

  v16f acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = (v16f){};

  auto compute = [&](int slot) {
    const uint8_t* base = lds + slot * SLOT;
#pragma unroll
    for (int kk = 0; kk < KS / 64; ++kk) {
      const int off0 = ((kk * 4 + 2 * g) ^ fsw) * 16, off1 = ((kk * 4 + 2 * g + 1) ^ fsw) * 16;
      v8i fw[FN], fa[FM];
#pragma unroll
      for (int f = 0; f < FN; ++f) {
        const uint8_t* r = base + w_row0 + f * 32 * KS;
        const v4i lo = *(const v4i*)(r + off0);
        const v4i hi = *(const v4i*)(r + off1);
        fw[f] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int f = 0; f < FM; ++f) {
        const uint8_t* r = base + a_row0 + f * 32 * KS;
        const v4i lo = *(const v4i*)(r + off0);
        const v4i hi = *(const v4i*)(r + off1);
        fa[f] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = mfma_32x32x64_fp8(fw[i], fa[j], acc[i][j]);
    }
  };

#pragma unroll
  for (int t = STAGES - 1; t < STAGES - 1 + TOUCH; ++t) touch(t);
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < nk) {
      issue(s, s);
      touch(s + STAGES - 1 + TOUCH);
    }
  int slot = 0;
  for (int kt = 0; kt < nk; ++kt) {
    // stage kt has landed once at most the loads issued after it are in flight:
    // its own step's touch plus (STAGES-2) full steps
    if (kt + STAGES - 2 < nk) {
      wait_vmcnt<(STAGES - 2) * PER_STEP + TLOADS>();
    } else {
      wait_vmcnt<0>();
    }
    block_barrier();  // stage kt visible to all waves; slot of stage kt-1 is free
    if (kt + STAGES - 1 < nk) {
      issue(slot == 0 ? STAGES - 1 : slot - 1, kt + STAGES - 1);
      touch(kt + STAGES - 1 + TOUCH);
    }
    compute(slot);
    slot = slot + 1 == STAGES ? 0 : slot + 1;
  }

  store_tile<kBf16, kGelu, FN, FM>(acc, m0 + wm * WTM, n0 + wn * WTN, frow, g, sa, sb, bias, C, M, N, ldc);
}

// Generic fallback for any M, N, K with K % 16 == 0: one wave computes a 32x32
// output tile straight from global memory (no LDS), zero-padding K to 64.
template <bool kBf16, bool kGelu>
__global__ __launch_bounds__(256) void fp8_gemm_generic(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ sa,
    const float* __restrict__ sb, const uint16_t* __restrict__ bias, uint16_t* __restrict__ C,
    int M, int N, int K, int64_t ldc, int tiles_n) {
  const int lane = threadIdx.x & 63;
  const int tile = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int tm = tile / tiles_n, tn = tile % tiles_n;
  const int m0 = tm * 32, n0 = tn * 32;
  if (m0 >= M) return;
  const int frow = lane & 31, g = lane >> 5;
  const int am = min(m0 + frow, M - 1);
  const int wn = min(n0 + frow, N - 1);
  const uint8_t* ar = A + (int64_t)am * K;
  const uint8_t* wr = W + (int64_t)wn * K;
  v16f acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
  for (int k0 = 0; k0 < K; k0 += 64) {
    int fa[8], fw[8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int kb = k0 + g * 32 + h * 16;  // 16-byte granule; K % 16 == 0
      v4i va = {0, 0, 0, 0}, vw = {0, 0, 0, 0};
      if (kb < K) {
        va = *(const v4i*)(ar + kb);
        vw = *(const v4i*)(wr + kb);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        fa[h * 4 + e] = va[e];
        fw[h * 4 + e] = vw[e];
      }
    }
    const v8i a8 = {fa[0], fa[1], fa[2], fa[3], fa[4], fa[5], fa[6], fa[7]};
    const v8i w8 = {fw[0], fw[1], fw[2], fw[3], fw[4], fw[5], fw[6], fw[7]};
    acc = mfma_32x32x64_fp8(w8, a8, acc);
  }
  const int m = m0 + frow;
  if (m >= M) return;
  const float s_a = sa[m];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int n = n0 + (r >> 2) * 8 + g * 4 + (r & 3);
    if (n >= N) continue;
    float v = round_out<kBf16>(__builtin_fmaf(acc[r] * sb[n], s_a, bias_value<kBf16>(bias, n)));
    if constexpr (kGelu) v = round_out<kBf16>(gelu_tanh(v));
    uint16_t bits;
    if constexpr (kBf16) {
      bits = (uint16_t)f32_to_bf16_bits(v);
    } else {
      bits = __builtin_bit_cast(uint16_t, (_Float16)v);
    }
    C[(int64_t)m * ldc + n] = bits;
  }
}

// Large-M kernel variant and L2 tile grouping (tuning switches while the
// pipelined kernel is evaluated): JOY_GEMM_VARIANT, JOY_GEMM_GROUP_M.
int gemm_variant() {
  static const int v = [] {
    const char* e = getenv("JOY_GEMM_VARIANT");
    return e ? atoi(e) : 3;
  }();
  return v;
}

int gemm_group_m() {
  static const int v = [] {
    const char* e = getenv("JOY_GEMM_GROUP_M");
    return e ? atoi(e) : 4;
  }();
  return v;
}

template <bool kBf16, bool kGelu, int BM, int BN, int WM_, int WN_, int ST, int KS, int TOUCH = 0>
hipError_t launch_pipe(const GemmArgs& g, hipStream_t st) {
  const int tiles_m = (g.M + BM - 1) / BM, tiles_n = (g.N + BN - 1) / BN;
  hipLaunchKernelGGL((fp8_gemm_pipe<kBf16, kGelu, BM, BN, WM_, WN_, ST, KS, TOUCH>), dim3(tiles_m * tiles_n),
                     dim3(WM_ * WN_ * 64), 0, st, (const uint8_t*)g.A, (const uint8_t*)g.W,
                     g.scales_a, g.scales_b, (const uint16_t*)g.bias, (uint16_t*)g.C, g.M, g.N, g.K,
                     g.ldc, tiles_m, tiles_n, gemm_group_m());
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Ring kernel: 256x256 tile, K step 128 bytes (whole 128-byte lines per DMA
// instruction), LDS used as a ring of five 32 KiB half-stages (the A half and the
// W half of a K step), i.e. all 160 KiB. While step kt is computed, A(kt+1),
// W(kt+1) and A(kt+2) are in flight: 1.5 steps of loads instead of 1 for a
// two-slot double buffer. Half h of the sequence A0 W0 A1 W1 ... lives in slot h % 5.
// ---------------------------------------------------------------------------
template <bool kBf16, bool kGelu, int WAVES_M, int WAVES_N>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64, 1) void fp8_gemm_ring(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ sa,
    const float* __restrict__ sb, const uint16_t* __restrict__ bias, uint16_t* __restrict__ C,
    int M, int N, int K, int64_t ldc, int tiles_m, int tiles_n, int group_m) {
  constexpr int BM = 256, BN = 256, KS = 128, HALF = 256 * KS;  // 32 KiB
  constexpr int NW = WAVES_M * WAVES_N;
  constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int RPI = 8;                 // rows per DMA instruction (8 x 128 B)
  constexpr int IH = 256 / RPI / NW;     // DMA instructions per wave per half
  __shared__ __attribute__((aligned(1024))) uint8_t lds[5 * HALF];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const TileCoord tc = map_tile(blockIdx.x, tiles_m, tiles_n, group_m);
  const int m0 = tc.tm * BM, n0 = tc.tn * BN;

  const int lrow = lane >> 3, lchunk = lane & 7;
  int64_t ga[IH], gw[IH];
#pragma unroll
  for (int i = 0; i < IH; ++i) {
    const int row = (wave * IH + i) * RPI + lrow;
    const int c = (lchunk ^ swz_rows<KS>(row)) * 16;
    ga[i] = (int64_t)min(m0 + row, M - 1) * K + c;
    gw[i] = (int64_t)min(n0 + row, N - 1) * K + c;
  }
  auto issue_half = [&](const uint8_t* src, const int64_t (&off)[IH], int slot, int kt) {
    const int64_t koff = (int64_t)kt * KS;
    uint8_t* base = lds + slot * HALF;
#pragma unroll
    for (int i = 0; i < IH; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(src + off[i] + koff),
                                       (lds_void*)(base + (wave * IH + i) * 1024), 16, 0, 0);
  };

  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int frow = lane & 31, g = lane >> 5;
  const int fsw = swz_rows<KS>(frow);
  const int a_row0 = (wm * WTM + frow) * KS, w_row0 = (wn * WTN + frow) * KS;

  v16f acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = (v16f){};

  auto compute = [&](int slot_a, int slot_w) {
    const uint8_t* ba = lds + slot_a * HALF + a_row0;
    const uint8_t* bw = lds + slot_w * HALF + w_row0;
#pragma unroll
    for (int kk = 0; kk < KS / 64; ++kk) {
      const int off0 = ((kk * 4 + 2 * g) ^ fsw) * 16, off1 = ((kk * 4 + 2 * g + 1) ^ fsw) * 16;
      v8i fw[FN], fa[FM];
#pragma unroll
      for (int f = 0; f < FN; ++f) {
        const v4i lo = *(const v4i*)(bw + f * 32 * KS + off0);
        const v4i hi = *(const v4i*)(bw + f * 32 * KS + off1);
        fw[f] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int f = 0; f < FM; ++f) {
        const v4i lo = *(const v4i*)(ba + f * 32 * KS + off0);
        const v4i hi = *(const v4i*)(ba + f * 32 * KS + off1);
        fa[f] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = mfma_32x32x64_fp8(fw[i], fa[j], acc[i][j]);
    }
  };

  const int nk = K / KS;
  // prologue: A0 W0 A1 -> slots 0 1 2
  issue_half(A, ga, 0, 0);
  issue_half(W, gw, 1, 0);
  if (nk > 1) issue_half(A, ga, 2, 1);
  int sa_slot = 0;  // slot of A(kt) = (2 kt) % 5; W(kt) is the next slot
  for (int kt = 0; kt < nk; ++kt) {
    // A(kt), W(kt) have landed once only A(kt+1) (issued after W(kt)) may be in flight
    if (kt + 1 < nk) {
      wait_vmcnt<IH>();
    } else {
      wait_vmcnt<0>();
    }
    block_barrier();  // step kt visible; the slots of step kt-1 are free
    const int sw_slot = sa_slot == 4 ? 0 : sa_slot + 1;
    // W(kt+1) goes to slot (2kt+3) % 5, A(kt+2) to (2kt+4) % 5: the slots of step kt-1
    const int s3 = sa_slot + 3 >= 5 ? sa_slot - 2 : sa_slot + 3;
    const int s4 = sa_slot + 4 >= 5 ? sa_slot - 1 : sa_slot + 4;
    if (kt + 1 < nk) issue_half(W, gw, s3, kt + 1);
    if (kt + 2 < nk) issue_half(A, ga, s4, kt + 2);
    compute(sa_slot, sw_slot);
    sa_slot = sa_slot + 2 >= 5 ? sa_slot - 3 : sa_slot + 2;
  }
  store_tile<kBf16, kGelu, FN, FM>(acc, m0 + wm * WTM, n0 + wn * WTN, frow, g, sa, sb, bias, C, M, N, ldc);
}

template <bool kBf16, bool kGelu, int WM_, int WN_>
hipError_t launch_ring(const GemmArgs& g, hipStream_t st) {
  const int tiles_m = (g.M + 255) / 256, tiles_n = (g.N + 255) / 256;
  hipLaunchKernelGGL((fp8_gemm_ring<kBf16, kGelu, WM_, WN_>), dim3(tiles_m * tiles_n),
                     dim3(WM_ * WN_ * 64), 0, st, (const uint8_t*)g.A, (const uint8_t*)g.W,
                     g.scales_a, g.scales_b, (const uint16_t*)g.bias, (uint16_t*)g.C, g.M, g.N, g.K,
                     g.ldc, tiles_m, tiles_n, gemm_group_m());
  return hipGetLastError();
}

template <bool kBf16, bool kGelu>
hipError_t launch_gemm_t(const GemmArgs& g, hipStream_t st) {
  const bool fast = (g.K % BK == 0) && (g.N % 8 == 0) && (g.ldc % 4 == 0) &&
                    ((uintptr_t)g.C % 8 == 0) && ((uintptr_t)g.scales_b % 16 == 0) &&
                    ((uintptr_t)g.A % 16 == 0) && ((uintptr_t)g.W % 16 == 0) &&
                    ((uintptr_t)g.bias % 8 == 0) && !g.force_generic;
  if (fast) {
    switch (gemm_variant()) {
      case 1:
        return launch_pipe<kBf16, kGelu, 256, 256, 2, 2, 4, 64>(g, st);
      case 2:
        return launch_pipe<kBf16, kGelu, 256, 256, 2, 4, 4, 64>(g, st);
      case 3:
        return launch_pipe<kBf16, kGelu, 256, 256, 2, 4, 2, 128>(g, st);
      case 4:
        return launch_pipe<kBf16, kGelu, 256, 256, 2, 2, 2, 128>(g, st);
      case 5:
        return launch_pipe<kBf16, kGelu, 256, 128, 2, 2, 3, 128>(g, st);
      case 6:
        return launch_pipe<kBf16, kGelu, 128, 256, 2, 2, 3, 128>(g, st);
      case 7:
        return launch_pipe<kBf16, kGelu, 256, 256, 2, 4, 2, 128, 2>(g, st);
      case 8:
        return launch_pipe<kBf16, kGelu, 256, 256, 2, 4, 2, 128, 3>(g, st);
      case 9:
        return launch_pipe<kBf16, kGelu, 256, 256, 2, 2, 2, 128, 2>(g, st);
      case 10:
        return launch_ring<kBf16, kGelu, 2, 4>(g, st);
      case 11:
        return launch_ring<kBf16, kGelu, 2, 2>(g, st);
      default:
        break;
    }
    constexpr int BM = JOY_BM, BN = JOY_BN, WM_ = JOY_WM, WN_ = JOY_WN;
    const int tiles_m = (g.M + BM - 1) / BM, tiles_n = (g.N + BN - 1) / BN;
    hipLaunchKernelGGL((fp8_gemm_tiled<kBf16, kGelu, BM, BN, WM_, WN_>), dim3(tiles_m * tiles_n),
                       dim3(WM_ * WN_ * 64), 0, st, (const uint8_t*)g.A, (const uint8_t*)g.W,
                       g.scales_a, g.scales_b, (const uint16_t*)g.bias, (uint16_t*)g.C, g.M, g.N,
                       g.K, g.ldc, tiles_m, tiles_n, 4);
    return hipGetLastError();
  }
  const int tiles_m = (g.M + 31) / 32, tiles_n = (g.N + 31) / 32;
  const int tiles = tiles_m * tiles_n;
  hipLaunchKernelGGL((fp8_gemm_generic<kBf16, kGelu>), dim3((tiles + 3) / 4), dim3(256), 0, st,
                     (const uint8_t*)g.A, (const uint8_t*)g.W, g.scales_a, g.scales_b,
                     (const uint16_t*)g.bias, (uint16_t*)g.C, g.M, g.N, g.K, g.ldc, tiles_n);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_fp8_gemm(const GemmArgs& g, hipStream_t st) {
  if (g.M == 0 || g.N == 0) return hipSuccess;
  if (g.out_bf16) {
    return g.gelu ? launch_gemm_t<true, true>(g, st) : launch_gemm_t<true, false>(g, st);
  }
  return g.gelu ? launch_gemm_t<false, true>(g, st) : launch_gemm_t<false, false>(g, st);
}

}  // namespace joy
