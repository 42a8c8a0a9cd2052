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

__device__ __forceinline__ float gelu_tanh(float x) {
  const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
  const float k1 = 0.044715f;
  return 0.5f * x * (1.0f + tanhf(k0 * (x + k1 * x * x * x)));
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

  // ---- epilogue. acc[i][j][r]: output row m = activation fragment j, lane % 32;
  // output col n = weight fragment i, 8*(r/4) + 4*g + r%4.
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int m = m0 + wm * WTM + j * 32 + frow;
    if (m >= M) continue;
    const float s_a = sa[m];
    uint16_t* crow = C + (int64_t)m * ldc;
#pragma unroll
    for (int i = 0; i < FN; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * WTN + i * 32 + q * 8 + g * 4;
        if (n >= N) continue;
        const float4 s_b = *(const float4*)(sb + n);
        const float sbv[4] = {s_b.x, s_b.y, s_b.z, s_b.w};
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float t = acc[i][j][q * 4 + e] * sbv[e];
          float v = round_out<kBf16>(__builtin_fmaf(t, s_a, bias_value<kBf16>(bias, n + e)));
          if constexpr (kGelu) v = round_out<kBf16>(gelu_tanh(v));
          o[e] = v;
        }
        uint2 pk;
        if constexpr (kBf16) {
          pk.x = pack_bf16x2(o[0], o[1]);
          pk.y = pack_bf16x2(o[2], o[3]);
        } else {
          pk.x = pack_fp16x2(o[0], o[1]);
          pk.y = pack_fp16x2(o[2], o[3]);
        }
        *(uint2*)(crow + n) = pk;
      }
    }
  }
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

template <bool kBf16, bool kGelu>
hipError_t launch_gemm_t(const GemmArgs& g, hipStream_t st) {
  const bool fast = (g.K % BK == 0) && (g.N % 8 == 0) && (g.ldc % 4 == 0) &&
                    ((uintptr_t)g.C % 8 == 0) && ((uintptr_t)g.scales_b % 16 == 0) &&
                    ((uintptr_t)g.A % 16 == 0) && ((uintptr_t)g.W % 16 == 0) && !g.force_generic;
  if (fast) {
    constexpr int BM = JOY_BM, BN = JOY_BN, WM_ = JOY_WM, WN_ = JOY_WN;
    const int tiles_m = (g.M + BM - 1) / BM, tiles_n = (g.N + BN - 1) / BN;
    hipLaunchKernelGGL((fp8_gemm_tiled<kBf16, kGelu, BM, BN, WM_, WN_>), dim3(tiles_m * tiles_n),
                       dim3(WM_ * WN_ * 64), 0, st, (const uint8_t*)g.A, (const uint8_t*)g.W, g.scales_a, g.scales_b,
                       (const uint16_t*)g.bias, (uint16_t*)g.C, g.M, g.N, g.K, g.ldc, tiles_m,
                       tiles_n, 4);
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
