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
// Optional gated-residual epilogue: out = round(residual[m, n] + round(gemm) * gate[n]),
// the reference block's projection + fused_add_gate pair (dit.py:525-528, 535-538;
// sgl_fused_ops.py:302-305); residual and output may be the same buffer.
//
// Kernels by problem shape:
//  * fp8_gemm_4q (K % 256 == 0, M % 4 == 0, M > 512): persistent 256x256 tiles, one
//    workgroup per CU walking the whole rounds, 128-byte K steps through a 2-slot ring,
//    16x16x128 MFMAs;
//  * fp8_gemm_4k (M <= 512, and long-K GEMMs of less than one round): deep-K tiles
//    with register-staged operands and optional split-K;
//  * fp8_gemm_4n (129-512 rows with N % 80 == 0, e.g. N 5120): one round of narrow
//    BM x 80 tiles, no K split;
//  * fp8_gemm_4h (K % 128 == 0): one 256x128 or 128x128 tile per workgroup with the
//    persistent kernel's 128-byte K steps; the sub-tiles of the last, partial round and
//    single-round GEMMs of <= 2048 rows that 256x128 tiles fill best;
//  * fp8_gemm_4w (any M, N with K % 64 == 0): one tile per workgroup; the sub-tiles of
//    the last, partial round when K % 128 != 0 and the remaining shapes. Its layout:
//  * 256 threads = 4 waves in 2x2, one wave per SIMD; macro tile 256x256 (one workgroup
//    per CU), 256x128 or 128x128 sub-tiles for the tiles of a last, partial round, so
//    more CUs share it;
//  * each wave accumulates its sub-tile as 32x32 tiles of
//    v_mfma_f32_32x32x64_f8f6f4 (up to 256 fp32 accumulators per lane, AGPRs);
//    the MFMA takes W as its "A" operand and the activation as "B";
//  * both operands are K-contiguous; they reach LDS with gfx950 16-byte
//    direct-to-LDS loads (global_load_lds_dwordx4) into a 5-deep ring of 64-byte
//    K steps, one barrier per step, with fragments of the next step read into a
//    second register set while the current step's MFMAs run;
//  * the epilogue rounds the tile into LDS and writes whole row segments with
//    16-byte stores;
//  * blockIdx -> tile mapping is XCD-aware (each XCD gets a contiguous range of
//    tile positions) and grouped (4 tile rows walk the tile columns together,
//    so one XCD's L2 serves both operands).
// A one-wave-per-32x32-tile kernel straight from global memory covers every
// other shape with K % 16 == 0.
#include <stdlib.h>

#include <type_traits>

#include "joy_common.hpp"
#include "joy_kernels.hpp"

namespace joy {
namespace {

constexpr int kGroupM = 4;  // tile rows per group of the tile order

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ v16f mfma_32x32x64_fp8(const v8i& a, const v8i& b, const v16f& c) {
  // Scale operands of zero select the plain (unscaled) f8f6f4 MFMA; format 0 = e4m3.
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// GELU, tanh form: 0.5 x (1 + tanh(u)) == x * sigmoid(2u), u = sqrt(2/pi) (x + 0.044715 x^3),
// with exp(-2u) = exp2(x (c0 + c1 x^2)), c0 = -2 sqrt(2/pi) log2(e), c1 = 0.044715 c0: seven
// VALU operations per value. exp2 / rcp hardware approximations (~1 ulp fp32) are far below
// bf16 resolution.
__device__ __forceinline__ float gelu_tanh(float x) {
  constexpr float c0 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;
  constexpr float c1 = 0.044715f * c0;
  const float e = __builtin_amdgcn_exp2f(x * __builtin_fmaf(x * x, c1, c0));  // exp(-2u)
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// Two fp32 -> packed 16-bit pair, round to nearest even (v_cvt_pk_bf16_f32 /
// v_cvt_pk_f16_f32 on gfx950).
template <bool kBf16>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (kBf16) return pack_bf16x2(lo, hi);
  return pack_fp16x2(lo, hi);
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

// Column operands of one wave's 128-column slice, loaded once per tile (ahead of
// the main loop, so their latency is hidden): scales_b and bias for the four
// consecutive output columns n_base + 32i + 8q + 4g of every accumulator quad.
template <int FN>
struct ColOperands {
  float4 sb[FN][4];
  uint2 bias[FN][4];
};

template <int FN>
__device__ __forceinline__ void load_col_operands(ColOperands<FN>& c, int n_base, int g, int N,
                                                  const float* __restrict__ sb,
                                                  const uint16_t* __restrict__ bias) {
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = n_base + i * 32 + q * 8 + g * 4;
      const bool ok = n < N;
      c.sb[i][q] = ok ? *(const float4*)(sb + n) : make_float4(0.f, 0.f, 0.f, 0.f);
      c.bias[i][q] = (ok && bias) ? *(const uint2*)(bias + n) : make_uint2(0u, 0u);
    }
}

// Optional gated residual of the epilogue (fused_add_gate, sgl_fused_ops.py:302-305):
// out = round(residual + round(gemm) * gate[n]) -- the GEMM output is rounded first,
// as the reference rounds the projection before torch.addcmul.
struct ResidualArgs {
  const uint16_t* ptr;
  int64_t ld;
  const uint16_t* gate;
};

// Epilogue kinds, a template parameter so that the plain and GELU kernels carry no
// residual registers. kEpiPartial writes the raw fp32 accumulators of a K range
// (split-K) to a workspace; the reduce kernel applies one of the other kinds. kEpiQkv
// (persistent kernel only): the QKV projection's q/k RMSNorm, RoPE and KV-ring write on
// the rounded tile instead of storing it (QkvEpi).
enum Epi : int { kEpiPlain = 0, kEpiGelu = 1, kEpiResidual = 2, kEpiPartial = 3, kEpiQkv = 4 };

// Outputs of the fused QKV epilogue, each a bf16 [rows, heads, 128] view with a token stride
// (elements): 0 rotated q, 1 rotated k, 2 ring K (normalised, or rotated when kpre_rotated),
// 3 ring V, 4 a second V (the joint attention V). dst null or rows 0: not written; bytes is
// the buffer range ((rows - 1) * stride + heads * 128) * 2, so rows past `rows` fall outside.
struct QkvEpi {
  uint16_t* dst[5];
  int64_t stride[5];
  int bytes[5];
  int rows[5];
  const uint16_t* q_weight;  // [128]
  const uint16_t* k_weight;
  const uint16_t* cos;  // [M, 64]: token m uses row m
  const uint16_t* sin;
  int heads;
  float eps;
  bool kpre_rotated;
};

template <bool kBf16>
__device__ __forceinline__ uint32_t gated_pair(uint32_t y, uint32_t x, uint32_t g) {
  return pack2<kBf16>(__builtin_fmaf(unpack_lo<kBf16>(y), unpack_lo<kBf16>(g), unpack_lo<kBf16>(x)),
                      __builtin_fmaf(unpack_hi<kBf16>(y), unpack_hi<kBf16>(g), unpack_hi<kBf16>(x)));
}

// Epilogue through LDS: the wave's (32*FN) x (32*FM) tile is rounded to 16-bit, written
// to a private LDS staging area [32*FM rows][32*FN columns] with a row pitch of
// 32*FN*2 + 16 bytes (16 lanes x 16 bytes cover all banks once for the 8-byte writes
// and for the 16-byte reads), then read back row-wise so that each global store
// instruction writes 64 x 16 contiguous bytes (whole row segments).
template <bool kBf16, int kEpi, int FN, int FM>
__device__ __forceinline__ void store_tile_lds(const v16f (&acc)[FN][FM], const ColOperands<FN>& col,
                                               const float (&sav)[FM], uint8_t* stage, int m_base,
                                               int n_base, int lane, uint16_t* __restrict__ C,
                                               int M, int N, int64_t ldc, const ResidualArgs& res) {
  constexpr int ROW_BYTES = 32 * FN * 2;
  constexpr int PITCH = ROW_BYTES + 16;
  const int frow = lane & 31, g = lane >> 5;
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    uint8_t* srow = stage + (j * 32 + frow) * PITCH;
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 s = col.sb[i][q];
        const uint2 bb = col.bias[i][q];
        const float sbe[4] = {s.x, s.y, s.z, s.w};
        const float be[4] = {unpack_lo<kBf16>(bb.x), unpack_hi<kBf16>(bb.x), unpack_lo<kBf16>(bb.y),
                             unpack_hi<kBf16>(bb.y)};
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = __builtin_fmaf(acc[i][j][q * 4 + e] * sbe[e], sav[j], be[e]);
        uint2 pk = make_uint2(pack2<kBf16>(o[0], o[1]), pack2<kBf16>(o[2], o[3]));
        if constexpr (kEpi == kEpiGelu) {
          // the reference applies GELU to the rounded GEMM output and rounds again
          pk = make_uint2(pack2<kBf16>(gelu_tanh(unpack_lo<kBf16>(pk.x)), gelu_tanh(unpack_hi<kBf16>(pk.x))),
                          pack2<kBf16>(gelu_tanh(unpack_lo<kBf16>(pk.y)), gelu_tanh(unpack_hi<kBf16>(pk.y))));
        }
        *(uint2*)(srow + (i * 32 + q * 8 + g * 4) * 2) = pk;
      }
  }
  // read back: CPL lanes per row, 64/CPL rows per instruction (FN = 3: 12 lanes per row,
  // 5 rows per instruction, lanes 60..63 idle and the last instruction's rows past the
  // tile skipped)
  constexpr int CPL = ROW_BYTES / 16;
  constexpr int RPI = 64 / CPL;
  constexpr int ROWS = 32 * FM;
  const int rr = lane / CPL, cc = lane % CPL;
  const int n = n_base + cc * 8;
  uint4 gv = make_uint4(0, 0, 0, 0);
  if constexpr (kEpi == kEpiResidual)
    if (n < N) gv = *(const uint4*)(res.gate + n);
#pragma unroll
  for (int r0 = 0; r0 < ROWS; r0 += RPI) {
    const int r = r0 + rr;
    if constexpr (RPI * CPL != 64 || ROWS % RPI != 0)
      if (rr >= RPI || r >= ROWS) continue;
    uint4 v = *(const uint4*)(stage + r * PITCH + cc * 16);
    const int m = m_base + r;
    if (m < M && n < N) {
      if constexpr (kEpi == kEpiResidual) {
        const uint4 x = *(const uint4*)(res.ptr + (int64_t)m * res.ld + n);
        v = make_uint4(gated_pair<kBf16>(v.x, x.x, gv.x), gated_pair<kBf16>(v.y, x.y, gv.y),
                       gated_pair<kBf16>(v.z, x.z, gv.z), gated_pair<kBf16>(v.w, x.w, gv.w));
      }
      typedef unsigned u32x4 __attribute__((ext_vector_type(4)));  // written once: non-temporal
      __builtin_nontemporal_store((u32x4){v.x, v.y, v.z, v.w}, (u32x4*)(C + (int64_t)m * ldc + n));
    }
  }
}

template <bool kBf16>
__device__ __forceinline__ float round_out(float v) {
  if constexpr (kBf16) return __uint_as_float(f32_to_bf16_bits(v) << 16);
  return round_fp16(v);
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

// XCD-aware position of block b of nblocks: hardware deals workgroups round-robin
// to the 8 XCDs; give each XCD a contiguous range of positions so its L2 sees
// neighbouring tiles.
__device__ __forceinline__ int xcd_position(int b, int nblocks) {
  const int xcd = b & 7, local = b >> 3, q = nblocks >> 3, rem = nblocks & 7;
  return xcd < rem ? xcd * (q + 1) + local : rem * (q + 1) + (xcd - rem) * q + local;
}

__device__ __forceinline__ TileCoord map_tile(int b, int nblocks, int tiles_m, int tiles_n,
                                              int group_m, int base) {
  int t = b;
  if (nblocks > 0) t = xcd_position(b, nblocks);
  t += base;
  // grouped order: group_m tile rows walk the tile columns together
  const int per_group = group_m * tiles_n;
  const int grp = t / per_group;
  const int first_m = grp * group_m;
  const int gsz = min(tiles_m - first_m, group_m);
  const int r = t - grp * per_group;
  return {first_m + r % gsz, r / gsz};
}

// LDS rows of the operand ring are KS bytes = KS/16 chunks of 16 bytes; logical
// chunk c of row r is stored at c ^ swz(r). The KS = 64 and 128 swizzles were chosen
// by measuring SQ_LDS_BANK_CONFLICT on gfx950 (zero for the fragment reads):
//   KS = 64:  swz(r) = (r >> 2) & 3
//   KS = 128: swz(r) = (r & 7) ^ ((r >> 3) & 1)
//   KS >= 256: swz(r) = r & 15 (16 consecutive rows reading one logical chunk hit 16
//              distinct 16-byte bank groups of a row pitch that is a multiple of 256 B)
// All are invariant under r -> r + 32, so a lane's fragment rows share its swizzle.
template <int KS>
__device__ __forceinline__ int swz_rows(int r) {
  if constexpr (KS == 64) {
    return (r >> 2) & 3;
  } else if constexpr (KS == 128) {
    return (r & 7) ^ ((r >> 3) & 1);
  } else {
    return r & 15;
  }
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

// Generic fallback for any M, N, K with K % 16 == 0: one wave computes a 32x32
// output tile straight from global memory (no LDS), zero-padding K to 64.
template <bool kBf16, int kEpi>
__global__ __launch_bounds__(256) void fp8_gemm_generic(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ sa,
    const float* __restrict__ sb, const uint16_t* __restrict__ bias, uint16_t* __restrict__ C,
    int M, int N, int K, int64_t ldc, int tiles_n, ResidualArgs res) {
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
    if constexpr (kEpi == kEpiGelu) v = round_out<kBf16>(gelu_tanh(v));
    if constexpr (kEpi == kEpiResidual)
      v = round_out<kBf16>(__builtin_fmaf(v, bias_value<kBf16>(res.gate, n),
                                          bias_value<kBf16>(res.ptr, (int64_t)m * res.ld + n)));
    uint16_t bits;
    if constexpr (kBf16) {
      bits = (uint16_t)f32_to_bf16_bits(v);
    } else {
      bits = (uint16_t)f32_to_fp16_bits(v);
    }
    C[(int64_t)m * ldc + n] = bits;
  }
}

// Instruction interleave of one main-loop iteration (N MFMAs, R fragment reads, L
// DMAs) as sched_group_barrier groups emitted after MFMA number I: ceil(R/N) reads
// and one DMA after each MFMA until both run out. (Spreading the DMAs over the whole
// iteration, or reads first and DMAs last, measured the same on MI355X.)
template <int I, int N, int R, int L>
__device__ __forceinline__ void sched_pattern() {
  if constexpr (I < N) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    constexpr int RD = (R + N - 1) / N;
    if constexpr (I * RD < R) __builtin_amdgcn_sched_group_barrier(0x100, RD, 0);  // LDS reads
    constexpr int LD = (L + N - 1) / N;
    if constexpr (I * LD < L) __builtin_amdgcn_sched_group_barrier(0x020, LD, 0);  // DMAs
    sched_pattern<I + 1, N, R, L>();
  }
}

// ---------------------------------------------------------------------------
// Four-wave software-pipelined kernel: BM x BN tile (256x256 for the bulk of a
// large GEMM; 128-row/column tiles for the last, partial round), one wave per
// SIMD, each wave a (BM/2) x (BN/2) sub-tile of 32x32 MFMA tiles (up to 256 fp32
// accumulators per lane, in AGPRs).
//
// LDS is a ring of S stages of one 64-byte K step ((BM + BN) rows x 64 B).
// Iteration kt computes on fragments of step kt already in registers while it
//   * reads the fragments of step kt+1 from LDS into the other register set, and
//   * DMAs step kt+S into the slot of step kt (free: its fragments were read in
//     iteration kt-1 and every wave passed this iteration's barrier),
// with the three instruction streams interleaved one MFMA at a time. The loop body
// is one basic block: past the last step the DMA re-fetches the last step (a slot
// nobody reads again) and the extra fragment read is discarded, so every iteration
// waits on the same constant vmcnt.
//
// Tile source. Bulk launch (sub_log2 == -1): block b takes position
// xcd_position(b) of the grouped 256x256 tile order, positions [0, gridDim.x).
// Tail launch (sub_log2 >= 0): block b takes sub-tile (b mod 2^sub_log2) of the
// 256x256 tile at position tile_base + (b >> sub_log2).
// Small-M launch (sub_log2 == -2): BM x BN tiles of a tiles_m x tiles_n grid,
// M fastest within each XCD's contiguous range (the M tiles of one weight tile
// run together, so W is fetched once per XCD).
// Split-K launch (sub_log2 == -3, kEpi == kEpiPartial): BM x BN tiles times
// `splits` K ranges; position -> (M tile fastest, N tile, split), and split s
// covers K steps [s*nk/splits, (s+1)*nk/splits). The tile's fp32 sums go to
// ws[s][m][n] (row-major [M, N] per split) for the reduce kernel.
// ---------------------------------------------------------------------------
// Origin and K range of one block's tile.
struct TileJob {
  int m0, n0;
  int k_step0, nk;  // K steps [k_step0, k_step0 + nk) of the kernel's step size
  int split;
};

template <int BM, int BN, int KS = 64>
__device__ __forceinline__ TileJob decode_job(int K, int tiles_m, int tiles_n, int group_m, int tile_base,
                                              int sub_log2, int splits) {
  TileJob j;
  j.k_step0 = 0;
  j.nk = K / KS;
  j.split = 0;
  if (sub_log2 == -3) {
    int p = xcd_position(blockIdx.x, gridDim.x);
    const int tm = p % tiles_m;
    p /= tiles_m;
    const int tn = p % tiles_n;
    j.split = p / tiles_n;
    j.m0 = tm * BM;
    j.n0 = tn * BN;
    const int nk_all = j.nk;
    j.k_step0 = (int)((int64_t)j.split * nk_all / splits);
    j.nk = (int)((int64_t)(j.split + 1) * nk_all / splits) - j.k_step0;
  } else if (sub_log2 == -2) {
    const TileCoord tc = map_tile(blockIdx.x, gridDim.x, tiles_n, tiles_m, 1, 0);
    j.m0 = tc.tn * BM;
    j.n0 = tc.tm * BN;
  } else if (sub_log2 == -4) {
    // 128x128 sub-tiles of a last round over tiles_m whole 256-row tile rows (the 256x256
    // tiles from tile_base on, four each), then the top halves of the partial tile row below
    // them (at most 128 rows remain there), one 128-column block each
    const int na = (tiles_m * tiles_n - tile_base) << 2;
    const int w = (int)blockIdx.x;
    if (w < na) {
      const TileCoord tc = map_tile(w >> 2, -1, tiles_m, tiles_n, group_m, tile_base);
      j.m0 = tc.tm * 256 + (w & 1) * 128;
      j.n0 = tc.tn * 256 + ((w >> 1) & 1) * 128;
    } else {
      j.m0 = tiles_m * 256;
      j.n0 = (w - na) * 128;
    }
  } else if (sub_log2 < 0) {
    const TileCoord tc = map_tile(blockIdx.x, gridDim.x, tiles_m, tiles_n, group_m, 0);
    j.m0 = tc.tm * 256;
    j.n0 = tc.tn * 256;
  } else {
    const TileCoord tc = map_tile(blockIdx.x >> sub_log2, -1, tiles_m, tiles_n, group_m, tile_base);
    const int sub = blockIdx.x & ((1 << sub_log2) - 1);
    constexpr int SUB_M = 256 / BM;
    j.m0 = tc.tm * 256 + (sub % SUB_M) * BM;
    j.n0 = tc.tn * 256 + (sub / SUB_M) * BN;
  }
  return j;
}

// Per-wave global addresses of the operand rows for K steps of KS bytes: one load
// instruction covers RPI = 1024 / KS rows; lane l covers row l / (KS/16) and fetches
// logical 16-byte chunk (l % (KS/16)) ^ swz(row), which lands in physical chunk
// l % (KS/16) of that LDS row (so the LDS write is 1 KB contiguous).
template <int IA, int IW, int KS = 64>
__device__ __forceinline__ void operand_rows(const uint8_t* A, const uint8_t* W, int M, int N, int K,
                                             const TileJob& job, int wave, int lane, const uint8_t* (&pa)[IA],
                                             const uint8_t* (&pw)[IW]) {
  constexpr int CPR = KS / 16, RPI = 64 / CPR;
  const int lrow = lane / CPR, lchunk = lane % CPR;
  const int64_t k0 = (int64_t)job.k_step0 * KS;
#pragma unroll
  for (int i = 0; i < IA; ++i) {
    const int row = (wave * IA + i) * RPI + lrow;
    pa[i] = A + (int64_t)min(job.m0 + row, M - 1) * K + k0 + (lchunk ^ swz_rows<KS>(row)) * 16;
  }
#pragma unroll
  for (int i = 0; i < IW; ++i) {
    const int row = (wave * IW + i) * RPI + lrow;
    pw[i] = W + (int64_t)min(job.n0 + row, N - 1) * K + k0 + (lchunk ^ swz_rows<KS>(row)) * 16;
  }
}

// End of a tile: raw fp32 sums to the split-K workspace (kEpiPartial), or the
// scaled, rounded tile staged through LDS and stored as whole row segments.
template <bool kBf16, int kEpi, int BM, int BN>
__device__ __forceinline__ void finish_tile(const v16f (&acc)[BN / 64][BM / 64], const TileJob& job, uint8_t* lds,
                                            int wave, int lane, int M, int N, const float* __restrict__ sa,
                                            const float* __restrict__ sb, const uint16_t* __restrict__ bias,
                                            uint16_t* __restrict__ C, int64_t ldc, const ResidualArgs& res,
                                            float* __restrict__ ws) {
  constexpr int WTM = BM / 2, WTN = BN / 2, FM = WTM / 32, FN = WTN / 32;
  constexpr int STAGE_BYTES = WTM * (WTN * 2 + 16);
  const int wm = wave >> 1, wn = wave & 1;
  const int frow = lane & 31, g = lane >> 5;
  if constexpr (kEpi == kEpiPartial) {
    // lane (frow, g) holds rows m, columns n..n+3 of each 32x32 tile; 16-byte
    // stores, 32 contiguous bytes per row and (i, q)
    wait_vmcnt<0>();  // no load into LDS or registers outlives the block
    float* wsp = ws + (int64_t)job.split * M * N;
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int m = job.m0 + wm * WTM + j * 32 + frow;
      if (m >= M) continue;
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = job.n0 + wn * WTN + i * 32 + q * 8 + g * 4;
          if (n < N)
            *(float4*)(wsp + (int64_t)m * N + n) =
                make_float4(acc[i][j][q * 4], acc[i][j][q * 4 + 1], acc[i][j][q * 4 + 2], acc[i][j][q * 4 + 3]);
        }
    }
  } else {
    // epilogue operands; their latency overlaps the drain of the last loads and the barrier
    ColOperands<FN> col;
    load_col_operands<FN>(col, job.n0 + wn * WTN, g, N, sb, bias);
    float sav[FM];
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int m = job.m0 + wm * WTM + j * 32 + frow;
      sav[j] = m < M ? sa[m] : 0.0f;
    }
    // every wave's loads and fragment reads are done before LDS is reused for staging
    wait_vmcnt<0>();
    __builtin_amdgcn_s_waitcnt(0x0070);
    block_barrier();
    store_tile_lds<kBf16, kEpi, FN, FM>(acc, col, sav, lds + wave * STAGE_BYTES, job.m0 + wm * WTM,
                                         job.n0 + wn * WTN, lane, C, M, N, ldc, res);
  }
}

template <bool kBf16, int kEpi, int BM, int BN, int S>
__global__ __launch_bounds__(256, 1) void fp8_gemm_4w(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ sa,
    const float* __restrict__ sb, const uint16_t* __restrict__ bias, uint16_t* __restrict__ C,
    int M, int N, int K, int64_t ldc, int tiles_m, int tiles_n, int group_m, int tile_base,
    int sub_log2, ResidualArgs res, float* __restrict__ ws, int splits) {
  constexpr int KS = 64, NW = 4;
  constexpr int WTM = BM / 2, WTN = BN / 2;  // wave sub-tile
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int RPI = 16;                    // rows per DMA instruction (16 x 64 B)
  constexpr int IA = BM / RPI / NW, IW = BN / RPI / NW;
  constexpr int A_BYTES = BM * KS, SLOT = (BM + BN) * KS;
  constexpr int LOADS = IA + IW;
  constexpr int NMFMA = FM * FN, NREAD = 2 * (FM + FN);
  static_assert(IA * RPI * NW == BM && IW * RPI * NW == BN, "tile rows must split over waves");
  static_assert((S - 2) * LOADS < 64, "vmcnt range");
  constexpr int STAGE_BYTES = WTM * (WTN * 2 + 16);  // epilogue staging per wave
  constexpr int LDS_BYTES = S * SLOT > NW * STAGE_BYTES ? S * SLOT : NW * STAGE_BYTES;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const TileJob job = decode_job<BM, BN>(K, tiles_m, tiles_n, group_m, tile_base, sub_log2, splits);
  const int nk = job.nk;
  const uint8_t* pa[IA];
  const uint8_t* pw[IW];
  operand_rows<IA, IW>(A, W, M, N, K, job, wave, lane, pa, pw);
  auto issue = [&](int slot, int kt) {
    const int64_t koff = (int64_t)min(kt, nk - 1) * KS;
    uint8_t* base = lds + slot * SLOT;
#pragma unroll
    for (int i = 0; i < IA; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(pa[i] + koff),
                                       (lds_void*)(base + (wave * IA + i) * 1024), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < IW; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(pw[i] + koff),
                                       (lds_void*)(base + A_BYTES + (wave * IW + i) * 1024), 16, 0, 0);
  };

  const int wm = wave >> 1, wn = wave & 1;
  const int frow = lane & 31, g = lane >> 5;
  const int fsw = swz_rows<KS>(frow);
  const int off0 = ((2 * g) ^ fsw) * 16, off1 = ((2 * g + 1) ^ fsw) * 16;
  const int a_row0 = (wm * WTM + frow) * KS, w_row0 = A_BYTES + (wn * WTN + frow) * KS;

  v16f acc[FN][FM];  // [weight fragment][activation fragment]
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = (v16f){};

  v8i fw0[FN], fa0[FM], fw1[FN], fa1[FM];
  auto read_frags = [&](int slot, v8i (&fw)[FN], v8i (&fa)[FM]) {
    const uint8_t* base = lds + slot * SLOT;
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
  };
  auto mfmas = [&](const v8i (&fw)[FN], const v8i (&fa)[FM]) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) acc[i][j] = mfma_32x32x64_fp8(fw[i], fa[j], acc[i][j]);
  };
  // One iteration: wait for step kt+1 (own DMAs) and for this wave's fragment reads,
  // barrier, then DMA step kt+S into slot(kt), read step kt+1 from slot(kt+1), MFMA step kt.
  auto iteration = [&](int kt, int slot, int next_slot, const v8i (&fw)[FN], const v8i (&fa)[FM],
                       v8i (&nw)[FN], v8i (&na)[FM]) {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(((S - 2) * LOADS & 15) | ((((S - 2) * LOADS) >> 4) << 14) | 0x0070);
    block_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue(slot, kt + S);
    read_frags(next_slot, nw, na);
    mfmas(fw, fa);
    sched_pattern<0, NMFMA, NREAD, LOADS>();
    __builtin_amdgcn_sched_barrier(0);
  };

  // prologue: steps 0..S-1 into slots 0..S-1, fragments of step 0
#pragma unroll
  for (int s = 0; s < S; ++s) issue(s, s);
  wait_vmcnt<(S - 1) * LOADS>();
  block_barrier();
  read_frags(0, fw0, fa0);

  int slot = 0;
  int kt = 0;
  for (; kt + 2 <= nk; kt += 2) {
    const int s1 = slot + 1 == S ? 0 : slot + 1;
    const int s2 = s1 + 1 == S ? 0 : s1 + 1;
    iteration(kt, slot, s1, fw0, fa0, fw1, fa1);
    iteration(kt + 1, s1, s2, fw1, fa1, fw0, fa0);
    slot = s2;
  }
  if (kt < nk) {  // odd step count: last step's fragments are in set 0
    mfmas(fw0, fa0);
  }
  finish_tile<kBf16, kEpi, BM, BN>(acc, job, lds, wave, lane, M, N, sa, sb, bias, C, ldc, res, ws);
}

template <int J>
using IC = std::integral_constant<int, J>;

// Calls f(IC<I>{}), ..., f(IC<N-1>{}) (compile-time indices for register arrays).
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(IC<I>{});
    static_for<I + 1, N>(f);
  }
}

// ---------------------------------------------------------------------------
// Direct-to-LDS operand loads of the persistent and one-tile 128-byte-step kernels. They are
// inline asm: the compiler does not track them (through the builtins it cannot tell an
// epilogue LDS access from the ring slots the DMAs write and waits for every DMA in flight).
// m0 is written only by these asm statements. vmcnt is in order on gfx9 for loads and stores
// alike, so the kernels wait on constant counts.
// ---------------------------------------------------------------------------
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma_buf16(uint32_t lds_addr, uint32_t voff, __amdgpu_buffer_rsrc_t rsrc, int soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds_addr), "v"(voff), "s"(rsrc),
               "s"(soff)
               : "m0");
}
__device__ __forceinline__ void dma_glb16(uint32_t lds_addr, const void* p) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_addr), "v"(p) : "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t lds_u32(lds_void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}

template <int W>
__device__ __forceinline__ void wait_vmcnt_lgkm0() {
  static_assert(W >= 0 && W < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((W & 15) | ((W >> 4) << 14) | 0x0070);
}

// ---------------------------------------------------------------------------
// Persistent bulk kernel (plain, GELU and gated-residual epilogues): gridDim.x workgroups
// (a multiple of 8, one per CU) each walk the tiles b, b + gridDim.x, ... of the XCD-ordered
// grouped tile order. The operand ring runs on across tiles: during the last 2 K steps of a
// tile the ring fetches the next tile's first 2 steps, so a new tile starts on data already in
// LDS, and the epilogue's stores drain while the next tile's MFMAs run.
//
//   * K steps of 128 bytes in a ring of S = 2 slots: every operand row of a step is one
//     128-byte request (a 64-byte-step ring of the same kernel made twice the L2 requests and
//     ran 2-6 % slower on the cfg-2 GEMMs). Steps go through buffer loads straight into LDS
//     (row offsets are 32-bit: M*K, N*K < 2^31); a step's DMA is issued during step t - 2's
//     second phase and waited for in step t - 1, so it has one step to land.
//   * Per-tile column scales, bias and row scales arrive by one DMA per wave with the tile's
//     step 2 into side_lds.
//   * Each wait is a constant count: none of a step's own DMAs may be outstanding when the
//     next step is read, except in a tile's first step, whose wait (for step 1, fetched during
//     the previous tile) also counts the NST epilogue stores issued after it (2 NST with the
//     fused QKV epilogue, of which the wait leaves 63).
//   * MFMA: v_mfma_scale_f32_16x16x128_f8f6f4, 16 x 16 tiles that each consume a whole
//     128-byte K step. On random e4m3 operands this instruction sustains a higher shader clock
//     than 32x32x64 at the same MFMA density (MI355X, one wave per SIMD, operands in registers:
//     2.04 vs 1.87 GHz, both 100 % MFMA-busy; re-read from LDS every step: 1.98 vs 1.83 GHz),
//     i.e. it draws less power per FLOP, and the part runs these GEMMs power-limited. The
//     GEMM tests that compare it with the 32x32x64 kernels find the same bits; on random
//     M 10800 operands a few FFN-down outputs differ by <= 2 ulp (the MFMAs sum a 128-byte
//     K step in another order).
//
// Tile BM x BN (BM = 256, BN = 128, 192 or 256), 4 waves in 2 x 2, each a 128 x (BN/2)
// sub-tile = 8 x FN MFMA tiles of 16 x 16 (FN = BN/32; 4 fp32 accumulators each). Operand
// lanes: lane l holds row l % 16 of its fragment, K bytes [32 (l / 16), +32) of the step;
// accumulator lane l, element e = output (m = l % 16, n = 4 (l / 16) + e) of its tile (the
// MFMA's "A" operand is W, its "B" operand the activations).
//
// Step t (slot t & 1), two phases of FH x 8 MFMAs (FH = FN / 2):
//   A: W fragments [0, FH) x every A fragment, i-major, while W fragments [FH, FN) of step t
//      are read from the slot;
//   wait for step t + 1, one barrier;
//   B: W fragments [FH, FN) x every A fragment, j-major; after column j's MFMAs its A registers
//      take fragment j of step t + 1, W fragments [0, FH) of step t + 1 are read alongside (both
//      from the other slot), and an eighth of the DMAs of step t + 2 into this slot are issued.
// Registers: 8 x FN x 4 accumulators (AGPRs) + FN + 8 fragments of 8 VGPRs (128 at BN = 256).
// The epilogue stages each 16-row chunk of the wave's sub-tile through a padded LDS area
// (row pitch BN + 16 bytes: the 8-byte writes of 16 rows and the 16-byte row reads each
// cover distinct banks) and stores 16-byte row segments with buffer stores, NSTC per chunk
// for every wave whatever M and N (out-of-range lanes store past the buffer's range).
// ---------------------------------------------------------------------------
// The value of lane ^ 16 without the LDS crossbar: v_permlane16_swap with both operands x
// gives lane l {x[l & ~16], x[l | 16]}.
__device__ __forceinline__ float xor16_value(float v, int lane) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((lane & 16) ? r[0] : r[1]);
}
// v + (the value of lane ^ 32): v_permlane32_swap with both operands gives {x[l], x[l ^ 32]} in an
// order that depends on the half; the sum of the two is the same bits in both.
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ v4f mfma_16x16x128_fp8(const v8i& a, const v8i& b, const v4f& c) {
  // Scale operands of zero select the plain (unscaled) f8f6f4 MFMA; format 0 = e4m3.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

template <bool kBf16, int kEpi, int BN>
__global__ __launch_bounds__(256, 1) void fp8_gemm_4q(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ sa,
    const float* __restrict__ sb, const uint16_t* __restrict__ bias, uint16_t* __restrict__ C,
    int M, int N, int K, int64_t ldc, int tiles_m, int tiles_n, int group_m, int ntiles, ResidualArgs res,
    QkvEpi qe) {
  static_assert(kEpi == kEpiPlain || kEpi == kEpiGelu || kEpi == kEpiResidual || kEpi == kEpiQkv, "epilogues");
  static_assert(kEpi != kEpiQkv || (BN == 256 && kBf16), "fused QKV epilogue: 256-wide tiles (one head per wave), bf16");
  static_assert(BN == 128 || BN == 192 || BN == 256, "tile widths");
  constexpr int BM = 256, KS = 128, NW = 4, S = 2;
  constexpr int WTM = BM / 2, WTN = BN / 2, FM = WTM / 16, FN = WTN / 16, FH = FN / 2;
  constexpr int CPR = KS / 16, RPL = 64 / CPR;  // 8 chunks per row, 8 rows per DMA instruction
  constexpr int IA = BM / RPL / NW, IW = BN / RPL / NW, LOADS = IA + IW;
  constexpr int A_BYTES = BM * KS, SLOT = (BM + BN) * KS;
  constexpr int CPL = WTN / 8;             // 16-byte chunks of a staged row
  constexpr int PITCH = WTN * 2 + 16;      // staged row pitch
  constexpr int NSTC = 16 * CPL / 64;      // stores per 16-row chunk and wave
  constexpr int NST = FM * NSTC;           // stores per tile and wave
  constexpr int STAGE = 16 * PITCH;
  static_assert(FN % 2 == 0 && (16 * CPL) % 64 == 0, "phases and store shapes");
  static_assert(S * SLOT + 4096 + NW * STAGE <= 160 * 1024, "LDS");
  static_assert(LOADS + NST + 1 < 64, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[S * SLOT];
  __shared__ __attribute__((aligned(1024))) uint8_t side_lds[4096];
  __shared__ __attribute__((aligned(16))) uint8_t stage_lds[NW * STAGE];
  __shared__ __attribute__((aligned(16))) uint16_t w_lds[kEpi == kEpiQkv ? 256 : 8];  // q then k norm weights

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int frow = lane & 15, g = lane >> 4;
  if constexpr (kEpi == kEpiQkv) {
    // before the first DMA, so that the wait for these loads counts nothing else
    if (threadIdx.x < 32) {
      const uint16_t* src = threadIdx.x < 16 ? qe.q_weight + threadIdx.x * 8 : qe.k_weight + (threadIdx.x - 16) * 8;
      *(uint4*)(w_lds + threadIdx.x * 8) = *(const uint4*)src;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the prologue's barrier publishes them
  }
  const int fsw = swz_rows<KS>(frow);
  // fragment byte offsets of the lane's two 16-byte chunks (logical chunks 2g, 2g + 1; the
  // swizzle is invariant under row -> row + 16)
  const int fo0 = ((2 * g) ^ fsw) * 16, fo1 = ((2 * g + 1) ^ fsw) * 16;
  const int a_row0 = (wm * WTM + frow) * KS, w_row0 = A_BYTES + (wn * WTN + frow) * KS;
  const int nk = K / KS;  // even (K % 256 == 0)
  const int P = gridDim.x;
  const bool has_bias = bias != nullptr;
  const __amdgpu_buffer_rsrc_t crs =
      __builtin_amdgcn_make_buffer_rsrc(C, 0, (int)(((int64_t)(M - 1) * ldc + N) * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, (int)((int64_t)M * K), 0x00020000);
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void*)W, 0, (int)((int64_t)N * K), 0x00020000);
  const __amdgpu_buffer_rsrc_t rrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)res.ptr, 0, kEpi == kEpiResidual ? (int)(((int64_t)(M - 1) * res.ld + N) * 2) : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t grs =
      __builtin_amdgcn_make_buffer_rsrc((void*)res.gate, 0, kEpi == kEpiResidual ? N * 2 : 0, 0x00020000);

  int b = blockIdx.x;
  if (b >= ntiles) return;
  TileCoord tc = map_tile(b, ntiles, tiles_m, tiles_n, group_m, 0);
  int m0 = tc.tm * BM, n0 = tc.tn * BN;

  uint32_t oa[IA], ow[IW];
  auto set_rows = [&](int mm, int nn) {
    const int lrow = lane / CPR, lchunk = lane % CPR;
#pragma unroll
    for (int i = 0; i < IA; ++i) {
      const int row = (wave * IA + i) * RPL + lrow;
      // rows past M (N) fall outside the descriptor's range and load zeros (never stored)
      oa[i] = (uint32_t)(mm + row) * (uint32_t)K + (uint32_t)((lchunk ^ swz_rows<KS>(row)) * 16);
    }
#pragma unroll
    for (int i = 0; i < IW; ++i) {
      const int row = (wave * IW + i) * RPL + lrow;
      ow[i] = (uint32_t)(nn + row) * (uint32_t)K + (uint32_t)((lchunk ^ swz_rows<KS>(row)) * 16);
    }
  };
  set_rows(m0, n0);
  auto issue = [&](int slot, int koff) {
    const uint32_t base = lds_u32((lds_void*)(lds + slot * SLOT));
#pragma unroll
    for (int i = 0; i < IA; ++i) dma_buf16(base + (wave * IA + i) * 1024, oa[i], ars, koff);
#pragma unroll
    for (int i = 0; i < IW; ++i) dma_buf16(base + A_BYTES + (wave * IW + i) * 1024, ow[i], wrs, koff);
  };
  auto issue_side = [&](int mm, int nn) {
    const int lr = min(lane, (M - mm) / 4 - 1), lc = min(lane, (N - nn) / 4 - 1), lb = min(lane, (N - nn) / 8 - 1);
    const void* ps = sa + mm + 4 * lr;
    const void* pc = sb + nn + 4 * lc;
    const void* pb = has_bias ? (const void*)(bias + nn + 8 * lb) : pc;
    const void* src = wave == 0 ? ps : (wave == 2 ? pb : pc);
    dma_glb16(lds_u32((lds_void*)(side_lds + wave * 1024)), src);
  };

  v4f acc[FN][FM];
  v8i fw[FN], fa[FM];
  auto frag = [&](const uint8_t* r) {
    const v4i lo = *(const v4i*)(r + fo0);
    const v4i hi = *(const v4i*)(r + fo1);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  };
  auto mma = [&](int i, int j, auto zero) {
    if constexpr (decltype(zero)::value)
      acc[i][j] = mfma_16x16x128_fp8(fw[i], fa[j], (v4f){});
    else
      acc[i][j] = mfma_16x16x128_fp8(fw[i], fa[j], acc[i][j]);
  };
  using F = std::false_type;
  using T_ = std::true_type;
  auto step = [&](auto slotc, auto zero, auto wait, bool side, int koff, auto nextc) {
    constexpr int SL = decltype(slotc)::value;
    constexpr bool NEXT = decltype(nextc)::value;
    const uint8_t* wcur = lds + SL * SLOT + w_row0;
    const uint8_t* anext = lds + (SL ^ 1) * SLOT + a_row0;
    const uint8_t* wnext = lds + (SL ^ 1) * SLOT + w_row0;
    // phase A: W fragments [0, FH) x every A fragment, reading this step's W fragments [FH, FN)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int f = FH; f < FN; ++f) fw[f] = frag(wcur + f * 16 * KS);
#pragma unroll
    for (int i = 0; i < FH; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) mma(i, j, zero);
    sched_pattern<0, FH * FM, (FN - FH) * 2, 0>();
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt_lgkm0<decltype(wait)::value>();
    block_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (side) issue_side(m0, n0);
    __builtin_amdgcn_sched_barrier(0);
    // phase B: W fragments [FH, FN) x A fragment j, j-major; once column j is issued, its A
    // registers take the next step's fragment j, and the next step's W fragments [0, FH) (free
    // since phase A) are read alongside. The DMAs of step t + 2 into this slot are spread over
    // the columns, LOADS / FM after each: issued as one block after the barrier they left the
    // MFMAs idle while the four waves queued 4 x LOADS DMA instructions (11 % slower over the
    // QKV, out-projection and FFN-down GEMMs, bit-identical).
    const uint32_t dbase = lds_u32((lds_void*)(lds + SL * SLOT));
#pragma unroll
    for (int j = 0; j < FM; ++j) {
#pragma unroll
      for (int i = FH; i < FN; ++i) mma(i, j, zero);
      if constexpr (NEXT) {
        fa[j] = frag(anext + j * 16 * KS);
        if (j < FH) fw[j] = frag(wnext + j * 16 * KS);
      }
#pragma unroll
      for (int d = j * LOADS / FM; d < (j + 1) * LOADS / FM; ++d) {
        if (d < IA)
          dma_buf16(dbase + (wave * IA + d) * 1024, oa[d], ars, koff);
        else
          dma_buf16(dbase + A_BYTES + (wave * IW + d - IA) * 1024, ow[d - IA], wrs, koff);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // prologue: steps 0 and 1 of the first tile, both landed before the first step (whose wait then
  // counts the same outstanding operations as on every later tile)
  issue(0, 0);
  issue(1, KS);
  wait_vmcnt<0>();
  block_barrier();
  for (;;) {
    // the first step's A fragments and W fragments [0, FH) (slot 0: landed before the last barrier)
#pragma unroll
    for (int f = 0; f < FM; ++f) fa[f] = frag(lds + a_row0 + f * 16 * KS);
#pragma unroll
    for (int f = 0; f < FH; ++f) fw[f] = frag(lds + w_row0 + f * 16 * KS);
    // step 0: its wait is for step 1, issued before the previous tile's NST epilogue stores (the
    // fused QKV epilogue issues 2 NST stores, and on q / k tiles table loads that it has waited for,
    // after step 1's last DMA: up to 63 of them may still be in flight)
    step(IC<0>{}, T_{}, IC<kEpi == kEpiQkv ? 63 : NST>{}, true, 2 * KS, T_{});
    step(IC<1>{}, F{}, IC<0>{}, false, 3 * KS, T_{});
    for (int kt = 2; kt + 2 < nk; kt += 2) {
      step(IC<0>{}, F{}, IC<0>{}, false, (kt + 2) * KS, T_{});
      step(IC<1>{}, F{}, IC<0>{}, false, (kt + 3) * KS, T_{});
    }
    // last two steps: DMA the next tile's steps 0 and 1, or re-fetch this tile's last step into
    // slots nobody reads again
    const int bn = b + P;
    const bool more = bn < ntiles;
    const int tm0 = m0, tn0 = n0;
    int koffB = (nk - 1) * KS, dk = 0;
    if (more) {
      tc = map_tile(bn, ntiles, tiles_m, tiles_n, group_m, 0);
      m0 = tc.tm * BM;
      n0 = tc.tn * BN;
      set_rows(m0, n0);
      koffB = 0;
      dk = KS;
    }
    step(IC<0>{}, F{}, IC<0>{}, false, koffB, T_{});
    step(IC<1>{}, F{}, IC<0>{}, false, koffB + dk, F{});

    // epilogue of tile (tm0, tn0)
    {
      int lane_e;  // an opaque copy of the lane index keeps the epilogue's addresses out of the main loop
      asm volatile("v_mov_b32 %0, %1" : "=v"(lane_e) : "v"(lane));
      const int er = lane_e & 15, eg = lane_e >> 4;
      const float* sa_l = (const float*)(side_lds);
      const float* sb_l = (const float*)(side_lds + 1024);
      const uint16_t* bias_l = (const uint16_t*)(side_lds + 2048);
      uint8_t* stage = stage_lds + wave * STAGE;
      const int mw = tm0 + wm * WTM, nw0 = tn0 + wn * WTN;
      typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
      if constexpr (kEpi == kEpiQkv) {
        // this wave's 128 columns are one head of q, k or v (the three blocks are 256-aligned)
        const int eh = qe.heads * 128, region = tn0 / eh, head = (nw0 - region * eh) >> 7;
        // the two outputs of the tile: q (rotated q, -), k (rotated k, ring K), v (ring V, joint V)
        const int o1 = region == 0 ? 0 : (region == 1 ? 1 : 3), o2 = region == 1 ? 2 : 4;
        const __amdgpu_buffer_rsrc_t rs1 = __builtin_amdgcn_make_buffer_rsrc(qe.dst[o1], 0, qe.bytes[o1], 0x00020000);
        const __amdgpu_buffer_rsrc_t rs2 =
            __builtin_amdgcn_make_buffer_rsrc(qe.dst[o2], 0, region == 0 ? 0 : qe.bytes[o2], 0x00020000);
        const int64_t st1 = qe.stride[o1], st2 = qe.stride[o2];
        const uint16_t* w_l = w_lds + (region == 1 ? 128 : 0);
        // rows of the chunk staged through LDS, then stored as 16-byte row segments (NSTC per
        // lane, for every output and every wave: rows past the output's range fall outside it)
        auto stage_store = [&](const uint2 (&v)[FN], const __amdgpu_buffer_rsrc_t& rs, int64_t stride, int j) {
          uint8_t* srow = stage + er * PITCH + eg * 8;
#pragma unroll
          for (int i = 0; i < FN; ++i) *(uint2*)(srow + i * 32) = v[i];
          asm volatile("" ::: "memory");
#pragma unroll
          for (int k = 0; k < NSTC; ++k) {
            const int idx = k * 64 + lane_e, r = idx / CPL, c = idx % CPL;
            const uint4 x = *(const uint4*)(stage + r * PITCH + c * 16);
            const int m = mw + j * 16 + r;
            const uint32_t off =
                m < M ? (uint32_t)(((int64_t)m * stride + head * 128 + c * 8) * 2) : 0x80000000u;
            __builtin_amdgcn_raw_buffer_store_b128((u32x4){x.x, x.y, x.z, x.w}, rs, (int)off, 0, 2);
          }
          asm volatile("" ::: "memory");
        };
        // RoPE tables of chunk j: the cos and sin rows (128 bytes) of its 16 tokens, 16 bytes per
        // lane and load (lane l: piece l & 7 of row (l >> 3) + 8 (k & 1) of table k >> 1), loaded one
        // chunk ahead (vmcnt is in order: loads issued after the previous chunk's stores would wait
        // for them too), then passed through the staging area (rows of 136 bytes: the lanes' 4-byte
        // reads of one pair column hit distinct banks) to the lanes that rotate each pair
        // zeroed, so that the v tiles (which load no tables) carry no values across tiles: left
        // undefined, 32 registers of them were spilled around every tile's K loop
        u32x4 tb[4] = {}, tbn[4] = {};
        auto load_tables = [&](int j, u32x4 (&t)[4]) {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int tok = min(mw + j * 16 + (lane_e >> 3) + 8 * (k & 1), M - 1);
            t[k] = *(const u32x4*)(((k >> 1) ? qe.sin : qe.cos) + (int64_t)tok * 64 + (lane_e & 7) * 8);
          }
        };
        if (region < 2) load_tables(0, tb);
#pragma unroll
        for (int j = 0; j < FM; ++j) {
          int jz;  // re-read the column operands per chunk rather than holding them in registers
          asm volatile("v_mov_b32 %0, 0" : "=v"(jz));
          if (region < 2 && j + 1 < FM) load_tables(j + 1, tbn);
          // the GEMM's rounded output (as the plain epilogue stores it)
          const float s_a = sa_l[wm * WTM + j * 16 + er];
          uint2 yb[FN];
#pragma unroll
          for (int i = 0; i < FN; ++i) {
            const int c = wn * WTN + i * 16 + eg * 4;
            const float4 sv = *(const float4*)(sb_l + c + jz);
            const uint2 bb = *(const uint2*)(bias_l + c + jz);
            const float sbe[4] = {sv.x, sv.y, sv.z, sv.w};
            const float be[4] = {has_bias ? bf16_lo(bb.x) : 0.0f, has_bias ? bf16_hi(bb.x) : 0.0f,
                                 has_bias ? bf16_lo(bb.y) : 0.0f, has_bias ? bf16_hi(bb.y) : 0.0f};
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = __builtin_fmaf(acc[i][j][e] * sbe[e], s_a, be[e]);
            yb[i] = make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]));
          }
          if (region == 2) {
            stage_store(yb, rs1, st1, j);
            stage_store(yb, rs2, st2, j);
            continue;
          }
          // the lane's 16 pairs i * 8 + eg * 2 and + 1 (i < FN) of token er
          uint32_t cw[FN], sw[FN];
          {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              uint8_t* d = stage + ((k >> 1) * 16 + (lane_e >> 3) + 8 * (k & 1)) * 136 + (lane_e & 7) * 16;
              *(uint2*)d = make_uint2(tb[k][0], tb[k][1]);
              *(uint2*)(d + 8) = make_uint2(tb[k][2], tb[k][3]);
            }
            asm volatile("" ::: "memory");
#pragma unroll
            for (int i = 0; i < FN; ++i) {
              cw[i] = *(const uint32_t*)(stage + er * 136 + (i * 8 + eg * 2) * 2);
              sw[i] = *(const uint32_t*)(stage + (16 + er) * 136 + (i * 8 + eg * 2) * 2);
            }
            asm volatile("" ::: "memory");
          }
          // head RMSNorm: lane (er, eg) holds elements i * 16 + eg * 4 + e of token er's head, so
          // element group 2 i + (eg >> 1) (8 elements) is split over lanes eg and eg ^ 1: the even
          // lane's 4-term fma chain continues in the odd lane, whose 8 group sums then take the
          // tree g ^ 8 (i ^ 4), g ^ 4 (i ^ 2), g ^ 2 (i ^ 1) in the lane and g ^ 1 across lanes
          // eg and eg ^ 2 -- the order of the standalone kernel (head_rsqrt)
          float yv[FN][4], s8[FN];
#pragma unroll
          for (int i = 0; i < FN; ++i) {
            yv[i][0] = bf16_lo(yb[i].x);
            yv[i][1] = bf16_hi(yb[i].x);
            yv[i][2] = bf16_lo(yb[i].y);
            yv[i][3] = bf16_hi(yb[i].y);
            float c4 = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) c4 = __builtin_fmaf(yv[i][e], yv[i][e], c4);
            float t = xor16_value(c4, lane_e);
#pragma unroll
            for (int e = 0; e < 4; ++e) t = __builtin_fmaf(yv[i][e], yv[i][e], t);
            s8[i] = t;
          }
          const float l10 = s8[0] + s8[4], l11 = s8[1] + s8[5], l12 = s8[2] + s8[6], l13 = s8[3] + s8[7];
          const float l3 = (l10 + l12) + (l11 + l13);
          const float l4 = xor32_sum(l3);
          const float l4p = xor16_value(l4, lane_e);
          const float r = head_rsqrt((eg & 1) ? l4 : l4p, 1.0f / 128.0f, qe.eps);
          float xh[FN][4];
          uint2 kb[FN], ob[FN];
#pragma unroll
          for (int i = 0; i < FN; ++i) {
            const uint2 wv = *(const uint2*)(w_l + i * 16 + eg * 4 + jz);
            const float w[4] = {bf16_lo(wv.x), bf16_hi(wv.x), bf16_lo(wv.y), bf16_hi(wv.y)};
#pragma unroll
            for (int e = 0; e < 4; ++e) xh[i][e] = yv[i][e] * r * w[e];
            kb[i] = make_uint2(pack_bf16x2(xh[i][0], xh[i][1]), pack_bf16x2(xh[i][2], xh[i][3]));
            float ro[4];
            rope_pair(xh[i][0], xh[i][1], bf16_lo(cw[i]), bf16_lo(sw[i]), ro[0], ro[1]);
            rope_pair(xh[i][2], xh[i][3], bf16_hi(cw[i]), bf16_hi(sw[i]), ro[2], ro[3]);
            ob[i] = make_uint2(pack_bf16x2(ro[0], ro[1]), pack_bf16x2(ro[2], ro[3]));
          }
          stage_store(ob, rs1, st1, j);
          if (region == 1 && !qe.kpre_rotated)
            stage_store(kb, rs2, st2, j);
          else
            stage_store(ob, rs2, st2, j);  // q: a range of 0 bytes (nothing stored, same count)
#pragma unroll
          for (int k = 0; k < 4; ++k) tb[k] = tbn[k];
        }
      } else {
      // the gate of the 8 output columns each lane stores in read-back instruction k (fixed per tile)
      u32x4 gv[NSTC];
#pragma unroll
      for (int k = 0; k < NSTC; ++k) {
        gv[k] = (u32x4){0, 0, 0, 0};
        if constexpr (kEpi == kEpiResidual) {
          const int n = nw0 + ((k * 64 + lane_e) % CPL) * 8;
          gv[k] = __builtin_amdgcn_raw_buffer_load_b128(grs, n < N ? n * 2 : 0x40000000, 0, 0);
        }
      }
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        int jz;  // re-read the column operands per chunk rather than holding them in registers
        asm volatile("v_mov_b32 %0, 0" : "=v"(jz));
        // gated residual: the row segments this lane stores for chunk j, loaded before the chunk's
        // arithmetic so that their latency overlaps it
        u32x4 rx[NSTC];
        if constexpr (kEpi == kEpiResidual) {
#pragma unroll
          for (int k = 0; k < NSTC; ++k) {
            const int idx = k * 64 + lane_e, r = idx / CPL, c = idx % CPL;
            const int m = mw + j * 16 + r, n = nw0 + c * 8;
            const uint32_t roff = (m < M && n < N) ? (uint32_t)(((int64_t)m * res.ld + n) * 2) : 0x80000000u;
            rx[k] = __builtin_amdgcn_raw_buffer_load_b128(rrs, (int)roff, 0, 0);
          }
        }
        const float s_a = sa_l[wm * WTM + j * 16 + er];
        uint8_t* srow = stage + er * PITCH + eg * 8;
#pragma unroll
        for (int i = 0; i < FN; ++i) {
          const int c = wn * WTN + i * 16 + eg * 4;
          const float4 sv = *(const float4*)(sb_l + c + jz);
          const uint2 bb = *(const uint2*)(bias_l + c + jz);
          const float sbe[4] = {sv.x, sv.y, sv.z, sv.w};
          const float be[4] = {has_bias ? unpack_lo<kBf16>(bb.x) : 0.0f, has_bias ? unpack_hi<kBf16>(bb.x) : 0.0f,
                               has_bias ? unpack_lo<kBf16>(bb.y) : 0.0f, has_bias ? unpack_hi<kBf16>(bb.y) : 0.0f};
          float o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = __builtin_fmaf(acc[i][j][e] * sbe[e], s_a, be[e]);
          uint2 pk = make_uint2(pack2<kBf16>(o[0], o[1]), pack2<kBf16>(o[2], o[3]));
          if constexpr (kEpi == kEpiGelu) {
            pk = make_uint2(pack2<kBf16>(gelu_tanh(unpack_lo<kBf16>(pk.x)), gelu_tanh(unpack_hi<kBf16>(pk.x))),
                            pack2<kBf16>(gelu_tanh(unpack_lo<kBf16>(pk.y)), gelu_tanh(unpack_hi<kBf16>(pk.y))));
          }
          *(uint2*)(srow + i * 32) = pk;
        }
        // other lanes' rows are read next: the compiler must not reuse an earlier read of the same
        // address (LDS is in order within the wave, so no hardware wait is needed)
        asm volatile("" ::: "memory");
#pragma unroll
        for (int k = 0; k < NSTC; ++k) {
          const int idx = k * 64 + lane_e, r = idx / CPL, c = idx % CPL;
          uint4 v = *(const uint4*)(stage + r * PITCH + c * 16);
          const int m = mw + j * 16 + r, n = nw0 + c * 8;
          const uint32_t off = (m < M && n < N) ? (uint32_t)(((int64_t)m * ldc + n) * 2) : 0x80000000u;
          if constexpr (kEpi == kEpiResidual) {
            const u32x4 x = rx[k];
            v = make_uint4(gated_pair<kBf16>(v.x, x[0], gv[k][0]), gated_pair<kBf16>(v.y, x[1], gv[k][1]),
                           gated_pair<kBf16>(v.z, x[2], gv[k][2]), gated_pair<kBf16>(v.w, x[3], gv[k][3]));
          }
          // cache policy 2 = nt: the output is written once
          __builtin_amdgcn_raw_buffer_store_b128((u32x4){v.x, v.y, v.z, v.w}, crs, (int)off, 0, 2);
        }
        asm volatile("" ::: "memory");
      }
      }
    }
    if (!more) break;
    b = bn;
  }
  wait_vmcnt<0>();
}


// ---------------------------------------------------------------------------
// One tile per workgroup with 128-byte K steps through an S-slot ring (the sub-tiles of a
// persistent launch's last round, and single-round direct launches), 32x32x64 MFMAs: the
// MFMAs of a step's first 64-byte half while its second half is read, a wait for the next
// step and one barrier, then the second half's MFMAs with the reads of the next step's first
// half and the DMA of step t + S into the slot just finished spread among them.
// ---------------------------------------------------------------------------
template <bool kBf16, int kEpi, int BM, int BN, int S>
__global__ __launch_bounds__(256, 1) void fp8_gemm_4h(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ sa,
    const float* __restrict__ sb, const uint16_t* __restrict__ bias, uint16_t* __restrict__ C,
    int M, int N, int K, int64_t ldc, int tiles_m, int tiles_n, int group_m, int tile_base,
    int sub_log2, ResidualArgs res) {
  constexpr int KS = 128, NW = 4;
  constexpr int WTM = BM / 2, WTN = BN / 2, FM = WTM / 32, FN = WTN / 32;
  constexpr int CPR = KS / 16, RPL = 64 / CPR;  // 8 rows per DMA instruction
  constexpr int IA = BM / RPL / NW, IW = BN / RPL / NW, LOADS = IA + IW;
  constexpr int A_BYTES = BM * KS, SLOT = (BM + BN) * KS;
  constexpr int NMFMA = FM * FN, NREAD = 2 * (FM + FN);
  static_assert(IA * RPL * NW == BM && IW * RPL * NW == BN, "tile rows must split over waves");
  static_assert(S >= 2 && (S - 1) * LOADS < 64, "vmcnt range");
  constexpr int STAGE_BYTES = WTM * (WTN * 2 + 16);
  constexpr int LDS_BYTES = S * SLOT > NW * STAGE_BYTES ? S * SLOT : NW * STAGE_BYTES;
  static_assert(LDS_BYTES <= 160 * 1024, "LDS of one CU");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const TileJob job = decode_job<BM, BN, KS>(K, tiles_m, tiles_n, group_m, tile_base, sub_log2, 1);
  const int nk = job.nk;
  const uint8_t* pa[IA];
  const uint8_t* pw[IW];
  operand_rows<IA, IW, KS>(A, W, M, N, K, job, wave, lane, pa, pw);
  auto issue = [&](int slot, int kt) {
    const int64_t koff = (int64_t)min(kt, nk - 1) * KS;
    uint8_t* base = lds + slot * SLOT;
#pragma unroll
    for (int i = 0; i < IA; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(pa[i] + koff),
                                       (lds_void*)(base + (wave * IA + i) * 1024), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < IW; ++i)
      __builtin_amdgcn_global_load_lds((const void*)(pw[i] + koff),
                                       (lds_void*)(base + A_BYTES + (wave * IW + i) * 1024), 16, 0, 0);
  };

  const int wm = wave >> 1, wn = wave & 1;
  const int frow = lane & 31, g = lane >> 5;
  const int fsw = swz_rows<KS>(frow);
  const int a_row0 = (wm * WTM + frow) * KS, w_row0 = A_BYTES + (wn * WTN + frow) * KS;

  v16f acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = (v16f){};
  v8i fwx[FN], fax[FM], fwy[FN], fay[FM];
  // fragments of 64-byte half h of the step in `slot`
  auto read_frags = [&](int slot, int h, v8i (&fw)[FN], v8i (&fa)[FM]) {
    const uint8_t* base = lds + slot * SLOT;
    const int o0 = ((4 * h + 2 * g) ^ fsw) * 16, o1 = ((4 * h + 2 * g + 1) ^ fsw) * 16;
#pragma unroll
    for (int f = 0; f < FN; ++f) {
      const uint8_t* r = base + w_row0 + f * 32 * KS;
      const v4i lo = *(const v4i*)(r + o0);
      const v4i hi = *(const v4i*)(r + o1);
      fw[f] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
#pragma unroll
    for (int f = 0; f < FM; ++f) {
      const uint8_t* r = base + a_row0 + f * 32 * KS;
      const v4i lo = *(const v4i*)(r + o0);
      const v4i hi = *(const v4i*)(r + o1);
      fa[f] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
  };
  auto mfmas = [&](const v8i (&fw)[FN], const v8i (&fa)[FM]) {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) acc[i][j] = mfma_32x32x64_fp8(fw[i], fa[j], acc[i][j]);
  };

  // prologue: steps 0 .. S-1 into slots 0 .. S-1, the first half of step 0
#pragma unroll
  for (int s = 0; s < S; ++s) issue(s, s);
  wait_vmcnt<(S - 1) * LOADS>();
  block_barrier();
  read_frags(0, 0, fwx, fax);
  int slot = 0;
  for (int kt = 0; kt < nk; ++kt) {
    const int next = slot + 1 == S ? 0 : slot + 1;
    __builtin_amdgcn_sched_barrier(0);
    read_frags(slot, 1, fwy, fay);
    mfmas(fwx, fax);
    sched_pattern<0, NMFMA, NREAD, 0>();
    __builtin_amdgcn_sched_barrier(0);
    // step kt + 1 has landed (steps kt + 2 .. kt + S - 1 may still be in flight) and every wave
    // has read this slot: refill it with step kt + S (past the end, the last step again)
    wait_vmcnt_lgkm0<(S - 2) * LOADS>();
    block_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // second half: after each MFMA, its share of the next step's first-half fragments (past the
    // last step: a slot nobody uses) and of the refill DMAs of step kt + S into this slot --
    // issued as one block after the barrier, the DMAs left the MFMAs idle while the four waves
    // queued them
    {
      const int64_t koff = (int64_t)min(kt + S, nk - 1) * KS;
      uint8_t* dst = lds + slot * SLOT;
      const uint8_t* src = lds + next * SLOT;
      const int o0 = ((2 * g) ^ fsw) * 16, o1 = ((2 * g + 1) ^ fsw) * 16;
      static_for<0, NMFMA>([&](auto qc) {
        constexpr int Q = decltype(qc)::value, I = Q / FM, J = Q % FM;
        acc[I][J] = mfma_32x32x64_fp8(fwy[I], fay[J], acc[I][J]);
        if constexpr (Q < FN + FM) {
          const uint8_t* r = src + (Q < FN ? w_row0 + Q * 32 * KS : a_row0 + (Q - FN) * 32 * KS);
          const v4i lo = *(const v4i*)(r + o0);
          const v4i hi = *(const v4i*)(r + o1);
          const v8i f = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          if constexpr (Q < FN) fwx[Q] = f; else fax[Q - FN] = f;
        }
        constexpr int LD = (LOADS + NMFMA - 1) / NMFMA;
#pragma unroll
        for (int d = Q * LD; d < (Q + 1) * LD && d < LOADS; ++d) {
          if (d < IA)
            __builtin_amdgcn_global_load_lds((const void*)(pa[d] + koff), (lds_void*)(dst + (wave * IA + d) * 1024),
                                             16, 0, 0);
          else
            __builtin_amdgcn_global_load_lds((const void*)(pw[d - IA] + koff),
                                             (lds_void*)(dst + A_BYTES + (wave * IW + d - IA) * 1024), 16, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      });
      static_assert(NMFMA >= FN + FM, "one fragment read per MFMA");
    }
    slot = next;
  }
  finish_tile<kBf16, kEpi, BM, BN>(acc, job, lds, wave, lane, M, N, sa, sb, bias, C, ldc, res, nullptr);
}

// Instruction interleave of one deep-K iteration: N MFMAs with the R fragment reads
// spread over all of them, the L global loads after the first L MFMAs and the L
// LDS writes after the last L.
template <int I, int N, int R, int L>
__device__ __forceinline__ void sched_pattern_k() {
  if constexpr (I < N) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    constexpr int RD = (R + N - 1) / N;
    if constexpr (I * RD < R) __builtin_amdgcn_sched_group_barrier(0x100, RD, 0);  // LDS reads
    if constexpr (I < L) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);        // one global load
    if constexpr (I >= N - L) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);   // one LDS write
    sched_pattern_k<I + 1, N, R, L>();
  }
}

// ---------------------------------------------------------------------------
// Deep-K register-staged kernel for grids of at most a few rounds (small M): the
// tiles, waves, MFMA fragments, launch modes and epilogue of fp8_gemm_4w, with K
// steps of KS = 128..512 bytes so that each barrier covers KS/64 MFMA k-steps and
// each load instruction reads whole 256..512-byte row runs, and with operands
// going global -> VGPR -> LDS (16-byte loads, 1 KB-contiguous LDS writes). Small-M
// GEMMs are bound by the bytes each CU keeps in flight against ~2 us of loaded
// memory latency, which deep steps and register staging raise; the 64-byte-step
// DMA kernel streams W at under 3 TB/s on these shapes.
//
// U staging buffers of one K step live in VGPRs (step j in buffer j % U); LDS holds
// NS slots of one step (step j in slot j % NS), and steps are written AHEAD = NS - 1
// iterations before they are used. Iteration t (after one barrier):
//   * loads step t+AHEAD+U-1 into its staging buffer (that buffer's previous step,
//     t+AHEAD-1, was written to LDS in iteration t-1),
//   * runs the MFMAs of step t, reading the fragments of k-step s+1 while the MFMAs
//     of k-step s run,
//   * writes step t+AHEAD into slot (t+AHEAD) % NS = (t-1) % NS: step t-1's slot,
//     whose reads every wave completed before this iteration's barrier.
// With NS = 3 step t+1 (written in iteration t-1) is already visible, so the
// fragments of its first k-step are read during step t's last MFMAs.
// ---------------------------------------------------------------------------
template <bool kBf16, int kEpi, int BM, int BN, int KS, int U, int NS>
__global__ __launch_bounds__(256, 1) void fp8_gemm_4k(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ sa,
    const float* __restrict__ sb, const uint16_t* __restrict__ bias, uint16_t* __restrict__ C,
    int M, int N, int K, int64_t ldc, int tiles_m, int tiles_n, int group_m, int tile_base,
    int sub_log2, ResidualArgs res, float* __restrict__ ws, int splits) {
  constexpr int NW = 4;
  constexpr int WTM = BM / 2, WTN = BN / 2;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int CPR = KS / 16, RPI = 64 / CPR;
  constexpr int IA = BM / RPI / NW, IW = BN / RPI / NW;
  constexpr int A_BYTES = BM * KS, SLOT = (BM + BN) * KS;
  constexpr int LOADS = IA + IW;
  constexpr int SUBS = KS / 64;
  constexpr int NMFMA = FM * FN, NREAD = 2 * (FM + FN);
  constexpr int AHEAD = NS - 1;
  constexpr int UNR = U % NS == 0 ? U : U * NS;  // lcm(U, NS) for NS in {2, 3}
  static_assert(KS >= 128 && KS <= 512, "deep K steps only");
  static_assert(NS == 2 || NS == 3, "two or three LDS slots");
  static_assert(U >= 2, "at least two staging buffers");
  static_assert(UNR % U == 0 && UNR % NS == 0, "buffer and slot indices compile-time in the unrolled loop");
  static_assert(IA * RPI * NW == BM && IW * RPI * NW == BN, "tile rows must split over waves");
  constexpr int STAGE_BYTES = WTM * (WTN * 2 + 16);
  constexpr int LDS_BYTES = NS * SLOT > NW * STAGE_BYTES ? NS * SLOT : NW * STAGE_BYTES;
  static_assert(LDS_BYTES <= 160 * 1024, "LDS of one CU");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const TileJob job = decode_job<BM, BN, KS>(K, tiles_m, tiles_n, group_m, tile_base, sub_log2, splits);
  const int nk = job.nk;
  const uint8_t* pa[IA];
  const uint8_t* pw[IW];
  operand_rows<IA, IW, KS>(A, W, M, N, K, job, wave, lane, pa, pw);

  v4i stg[U][LOADS];
  // W with default-policy loads also where a single row of tiles reads every W byte once:
  // non-temporal loads there were 1.1 us faster with 256-byte steps (M 64 x N 15360), are level
  // with the 512-byte steps in back-to-back launches (20.0 us), and 3 us slower for a launch that
  // starts on an idle device (25.9 vs 22.9 us)
  auto gload = [&](auto bc, int kt) {
    constexpr int B = decltype(bc)::value;
    const int64_t koff = (int64_t)min(kt, nk - 1) * KS;
#pragma unroll
    for (int i = 0; i < IA; ++i) stg[B][i] = *(const v4i*)(pa[i] + koff);
#pragma unroll
    for (int i = 0; i < IW; ++i) stg[B][IA + i] = *(const v4i*)(pw[i] + koff);
  };
  auto lwrite = [&](auto bc, int slot) {
    constexpr int B = decltype(bc)::value;
    uint8_t* base = lds + slot * SLOT + lane * 16;
#pragma unroll
    for (int i = 0; i < IA; ++i) *(v4i*)(base + (wave * IA + i) * 1024) = stg[B][i];
#pragma unroll
    for (int i = 0; i < IW; ++i) *(v4i*)(base + A_BYTES + (wave * IW + i) * 1024) = stg[B][IA + i];
  };

  const int wm = wave >> 1, wn = wave & 1;
  const int frow = lane & 31, g = lane >> 5;
  const int fsw = swz_rows<KS>(frow);
  const int a_row0 = (wm * WTM + frow) * KS, w_row0 = A_BYTES + (wn * WTN + frow) * KS;

  v16f acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = (v16f){};

  v8i fw[2][FN], fa[2][FM];
  // fragments of k-step KK (64 bytes: logical chunks 4 KK + 2 g and + 1) of the step in `slot`
  auto read_frags = [&](auto sc, auto kc, int slot) {
    constexpr int SL = decltype(sc)::value, KK = decltype(kc)::value;
    const uint8_t* base = lds + slot * SLOT;
    const int o0 = ((4 * KK + 2 * g) ^ fsw) * 16, o1 = ((4 * KK + 2 * g + 1) ^ fsw) * 16;
#pragma unroll
    for (int f = 0; f < FN; ++f) {
      const uint8_t* r = base + w_row0 + f * 32 * KS;
      const v4i lo = *(const v4i*)(r + o0);
      const v4i hi = *(const v4i*)(r + o1);
      fw[SL][f] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
#pragma unroll
    for (int f = 0; f < FM; ++f) {
      const uint8_t* r = base + a_row0 + f * 32 * KS;
      const v4i lo = *(const v4i*)(r + o0);
      const v4i hi = *(const v4i*)(r + o1);
      fa[SL][f] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
  };
  auto mfmas = [&](auto sc) {
    constexpr int SL = decltype(sc)::value;
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) acc[i][j] = mfma_32x32x64_fp8(fw[SL][i], fa[SL][j], acc[i][j]);
  };
  // k-step KK of a step uses fragment set KK % 2 (SUBS is even, so a step starts in set 0)
  auto iteration = [&](auto jc, int t) {
    constexpr int J = decltype(jc)::value;
    constexpr int CUR = J % NS, NXT = (J + 1) % NS, WRT = (J + AHEAD) % NS;
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): own LDS writes and fragment reads done
    block_barrier();
    __builtin_amdgcn_sched_barrier(0);
    gload(IC<(J + AHEAD - 1) % U>{}, t + AHEAD + U - 1);
    if constexpr (NS == 2) read_frags(IC<0>{}, IC<0>{}, CUR);
    static_for<0, SUBS>([&](auto kc) {
      constexpr int KK = decltype(kc)::value;
      if constexpr (KK + 1 < SUBS) {
        read_frags(IC<(KK + 1) & 1>{}, IC<KK + 1>{}, CUR);
      } else if constexpr (NS == 3) {
        read_frags(IC<0>{}, IC<0>{}, NXT);  // first k-step of step t+1
      }
      mfmas(IC<KK & 1>{});
    });
    lwrite(IC<(J + AHEAD) % U>{}, WRT);
    sched_pattern_k<0, NMFMA * SUBS, NREAD * SUBS, LOADS>();
    __builtin_amdgcn_sched_barrier(0);
  };

  // prologue: steps 0..U-1 into the staging buffers, steps 0..AHEAD-1 into their slots,
  // steps U..U+AHEAD-2 into the freed buffers; with three slots, the first k-step of
  // step 0 into registers
  static_for<0, U>([&](auto bc) { gload(bc, decltype(bc)::value); });
  static_for<0, AHEAD>([&](auto bc) { lwrite(bc, decltype(bc)::value); });
  static_for<0, AHEAD - 1>([&](auto bc) { gload(bc, U + decltype(bc)::value); });
  if constexpr (NS == 3) {
    __builtin_amdgcn_s_waitcnt(0xc07f);
    block_barrier();
    read_frags(IC<0>{}, IC<0>{}, 0);
  }

  int kt = 0;
  for (; kt + UNR <= nk; kt += UNR) static_for<0, UNR>([&](auto jc) { iteration(jc, kt + decltype(jc)::value); });
  static_for<0, UNR - 1>([&](auto jc) {
    if (kt + decltype(jc)::value < nk) iteration(jc, kt + decltype(jc)::value);
  });
  finish_tile<kBf16, kEpi, BM, BN>(acc, job, lds, wave, lane, M, N, sa, sb, bias, C, ldc, res, ws);
}

ResidualArgs residual_args(const GemmArgs& g) {
  return ResidualArgs{(const uint16_t*)g.residual, g.ldr, (const uint16_t*)g.gate};
}


// Layout rules of the persistent kernel fp8_gemm_4q: K steps in pairs of 128 bytes, row scales
// read 4 at a time, 32-bit buffer offsets for the operands, the output and the residual.
bool persistent_ok(const GemmArgs& g) {
  constexpr int64_t kLim = 0x7fffffffLL;
  return g.K % 256 == 0 && g.K >= 512 && g.M % 4 == 0 && (int64_t)g.M * g.K <= kLim && (int64_t)g.N * g.K <= kLim &&
         ((int64_t)(g.M - 1) * g.ldc + g.N) * 2 <= kLim &&
         (!g.residual || ((int64_t)(g.M - 1) * g.ldr + g.N) * 2 <= kLim);
}

// One round of 256x128 tiles (tm x tn <= CUs), one tile per workgroup. The one-tile kernel's
// 3-slot ring beats the persistent 16x16x128 kernel here (1560 x 4096 -> 4096: 29.0 vs 30.0 us,
// 512 x 5120 -> 13824: 34.9 vs 38.9; same-process A/B, bit-identical).
template <bool kBf16, int kEpi>
hipError_t launch_one_round_256x128(const GemmArgs& g, int tm, int tn, hipStream_t st) {
  hipLaunchKernelGGL((fp8_gemm_4h<kBf16, kEpi, 256, 128, 3>), dim3(tm * tn), dim3(256), 0, st, (const uint8_t*)g.A,
                     (const uint8_t*)g.W, g.scales_a, g.scales_b, (const uint16_t*)g.bias, (uint16_t*)g.C, g.M, g.N,
                     g.K, g.ldc, tm, tn, 1, 0, -2, residual_args(g));
  return hipGetLastError();
}

// Full rounds of 256x256 tiles (one workgroup per CU), then the remaining tiles of
// the last, partial round split into 4 (128x128) or 2 (256x128) sub-tiles so that
// more CUs share that round. Both launches go to the same stream; the result does
// not depend on the split (every output element sums its K products in the same order).
template <bool kBf16, int kEpi>
hipError_t launch_4w(const GemmArgs& g, hipStream_t st) {
  int tiles_m = (g.M + 255) / 256;
  const int tiles_n = (g.N + 255) / 256;
  const int T = tiles_m * tiles_n, P = device_cus();
  int rem = T % P;
  int sub_log2 = 0;
  if (rem * 4 <= P) {
    sub_log2 = 2;
  } else if (rem * 2 <= P + P / 4) {
    sub_log2 = 1;
  } else {
    rem = 0;  // the last round is nearly full: no split
  }
  // With at most 128 rows in the last tile row, its 256x256 tiles are mostly padding: when the
  // whole tile rows' leftover tiles (as 128x128 quarters) and the last row's top halves (one
  // 128x128 tile per 128 columns) fit one round, that round takes a quarter tile's time instead
  // of a half (1560 x 4096 -> 12288: one round of 256 tiles, then 32 x 4 + 96 = 224 quarter tiles
  // instead of 80 x 2 half tiles)
  bool last_row_quarters = false;
  const int m_rows = g.M % 256;
  if (m_rows > 0 && m_rows <= 128 && g.M > 256 && g.K % 128 == 0) {
    const int tf = (g.M / 256) * tiles_n;
    const int lq = (tf % P) * 4 + (g.N + 127) / 128;
    const int cost_now = 4 * (T / P) + (rem == 0 ? 4 * ((T % P) != 0) : (sub_log2 == 2 ? 1 : 2));
    if (tf >= P && lq <= P && 4 * (tf / P) + 1 < cost_now) last_row_quarters = true;
  }
  if (last_row_quarters) {
    tiles_m = g.M / 256;
    rem = (tiles_m * tiles_n) % P;
    sub_log2 = -4;
  }
  constexpr int D = 5;  // DMA ring depth
  const int bulk = tiles_m * tiles_n - rem;
  // the persistent kernel takes the full rounds (or a single partial one) when its layout
  // rules hold (K steps in pairs of 128 bytes, row scales read 4 at a time, 32-bit buffer
  // offsets, a workgroup count that keeps the XCD mapping); with fewer tiles than CUs it
  // runs one tile per workgroup (1024 x 4096 -> 16384: 63 us vs 66 for the one-tile kernel,
  // 3120 x 4096 -> 4096: 53 vs 56, 1560 x 4096 -> 12288: 90 vs 95 with the sub-tile tail)
  bool persistent = false;
  if constexpr (kEpi == kEpiPlain || kEpi == kEpiGelu || kEpi == kEpiResidual) {
    persistent = persistent_ok(g) && P % 8 == 0 && bulk >= 1;
    if (persistent)
      hipLaunchKernelGGL((fp8_gemm_4q<kBf16, kEpi, 256>), dim3(bulk < P ? bulk : P), dim3(256), 0, st, (const uint8_t*)g.A,
                         (const uint8_t*)g.W, g.scales_a, g.scales_b, (const uint16_t*)g.bias, (uint16_t*)g.C, g.M, g.N,
                         g.K, g.ldc, tiles_m, tiles_n, kGroupM, bulk, residual_args(g), QkvEpi{});
  }
  if (bulk > 0 && !persistent) {
    auto kern = fp8_gemm_4w<kBf16, kEpi, 256, 256, D>;
    hipLaunchKernelGGL(kern, dim3(bulk), dim3(256), 0, st, (const uint8_t*)g.A, (const uint8_t*)g.W, g.scales_a,
                       g.scales_b, (const uint16_t*)g.bias, (uint16_t*)g.C, g.M, g.N, g.K, g.ldc, tiles_m, tiles_n,
                       kGroupM, 0, -1, residual_args(g), nullptr, 1);
  }
  if (last_row_quarters) {
    const int nq = rem * 4 + (g.N + 127) / 128;
    hipLaunchKernelGGL((fp8_gemm_4h<kBf16, kEpi, 128, 128, 4>), dim3(nq), dim3(256), 0, st, (const uint8_t*)g.A,
                       (const uint8_t*)g.W, g.scales_a, g.scales_b, (const uint16_t*)g.bias, (uint16_t*)g.C, g.M, g.N,
                       g.K, g.ldc, tiles_m, tiles_n, kGroupM, bulk, -4, residual_args(g));
  } else if (rem > 0) {
    if (sub_log2 == 2) {
      if (g.K % 128 == 0)
        hipLaunchKernelGGL((fp8_gemm_4h<kBf16, kEpi, 128, 128, 4>), dim3(rem << 2), dim3(256), 0, st,
                           (const uint8_t*)g.A, (const uint8_t*)g.W, g.scales_a, g.scales_b, (const uint16_t*)g.bias,
                           (uint16_t*)g.C, g.M, g.N, g.K, g.ldc, tiles_m, tiles_n, kGroupM, bulk, 2, residual_args(g));
      else
        hipLaunchKernelGGL((fp8_gemm_4w<kBf16, kEpi, 128, 128, D>), dim3(rem << 2), dim3(256), 0, st,
                           (const uint8_t*)g.A, (const uint8_t*)g.W, g.scales_a, g.scales_b, (const uint16_t*)g.bias,
                           (uint16_t*)g.C, g.M, g.N, g.K, g.ldc, tiles_m, tiles_n, kGroupM, bulk, 2,
                           residual_args(g), nullptr, 1);
    } else {
      if (g.K % 128 == 0)
        hipLaunchKernelGGL((fp8_gemm_4h<kBf16, kEpi, 256, 128, 3>), dim3(rem << 1), dim3(256), 0, st,
                           (const uint8_t*)g.A, (const uint8_t*)g.W, g.scales_a, g.scales_b, (const uint16_t*)g.bias,
                           (uint16_t*)g.C, g.M, g.N, g.K, g.ldc, tiles_m, tiles_n, kGroupM, bulk, 1, residual_args(g));
      else
        hipLaunchKernelGGL((fp8_gemm_4w<kBf16, kEpi, 256, 128, D>), dim3(rem << 1), dim3(256), 0, st,
                           (const uint8_t*)g.A, (const uint8_t*)g.W, g.scales_a, g.scales_b, (const uint16_t*)g.bias,
                           (uint16_t*)g.C, g.M, g.N, g.K, g.ldc, tiles_m, tiles_n, kGroupM, bulk, 1,
                           residual_args(g), nullptr, 1);
    }
  }
  return hipGetLastError();
}

// Fallback for small M when K is not a multiple of 128 (64-byte K steps, one launch):
// M <= 64: 64x64 tiles; otherwise 128x64 if its tiles fit one round of the CUs, else
// 128x128.
template <bool kBf16, int kEpi, int BM, int BN, int D>
hipError_t launch_direct(const GemmArgs& g, hipStream_t st) {
  const int tiles_m = (g.M + BM - 1) / BM, tiles_n = (g.N + BN - 1) / BN;
  auto kern = fp8_gemm_4w<kBf16, kEpi, BM, BN, D>;
  hipLaunchKernelGGL(kern, dim3(tiles_m * tiles_n), dim3(256), 0, st, (const uint8_t*)g.A, (const uint8_t*)g.W,
                     g.scales_a, g.scales_b, (const uint16_t*)g.bias, (uint16_t*)g.C, g.M, g.N, g.K, g.ldc, tiles_m,
                     tiles_n, 1, 0, -2, residual_args(g), nullptr, 1);
  return hipGetLastError();
}

// Split-K reduction and epilogue: thread t owns 8 consecutive columns of one row,
// sums the splits' fp32 partials in split order (so the result does not depend on
// which block finished first), then applies the epilogue of store_tile_lds.
template <bool kBf16, int kEpi>
__global__ __launch_bounds__(256) void fp8_gemm_splitk_reduce(
    const float* __restrict__ ws, int splits, const float* __restrict__ sa, const float* __restrict__ sb,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ C, int M, int N, int64_t ldc,
    ResidualArgs res) {
  const int groups = N >> 3;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)M * groups) return;
  const int m = (int)(t / groups), n = (int)(t - (int64_t)m * groups) * 8;
  const int64_t split_stride = (int64_t)M * N;
  const float* p = ws + (int64_t)m * N + n;
  float acc[8];
  {
    const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
    acc[0] = a.x; acc[1] = a.y; acc[2] = a.z; acc[3] = a.w;
    acc[4] = b.x; acc[5] = b.y; acc[6] = b.z; acc[7] = b.w;
  }
#pragma unroll 4
  for (int s = 1; s < splits; ++s) {
    const float* q = p + s * split_stride;
    const float4 a = *(const float4*)q, b = *(const float4*)(q + 4);
    acc[0] += a.x; acc[1] += a.y; acc[2] += a.z; acc[3] += a.w;
    acc[4] += b.x; acc[5] += b.y; acc[6] += b.z; acc[7] += b.w;
  }
  const float s_a = sa[m];
  const float4 sb0 = *(const float4*)(sb + n), sb1 = *(const float4*)(sb + n + 4);
  const float sbe[8] = {sb0.x, sb0.y, sb0.z, sb0.w, sb1.x, sb1.y, sb1.z, sb1.w};
  float be[8];
  if (bias) {
    const uint4 bb = *(const uint4*)(bias + n);
    const uint32_t w[4] = {bb.x, bb.y, bb.z, bb.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      be[2 * e] = unpack_lo<kBf16>(w[e]);
      be[2 * e + 1] = unpack_hi<kBf16>(w[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) be[e] = 0.0f;
  }
  uint32_t pk[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    pk[e] = pack2<kBf16>(__builtin_fmaf(acc[2 * e] * sbe[2 * e], s_a, be[2 * e]),
                         __builtin_fmaf(acc[2 * e + 1] * sbe[2 * e + 1], s_a, be[2 * e + 1]));
    if constexpr (kEpi == kEpiGelu)
      pk[e] = pack2<kBf16>(gelu_tanh(unpack_lo<kBf16>(pk[e])), gelu_tanh(unpack_hi<kBf16>(pk[e])));
  }
  uint4 v = make_uint4(pk[0], pk[1], pk[2], pk[3]);
  if constexpr (kEpi == kEpiResidual) {
    const uint4 gv = *(const uint4*)(res.gate + n);
    const uint4 x = *(const uint4*)(res.ptr + (int64_t)m * res.ld + n);
    v = make_uint4(gated_pair<kBf16>(v.x, x.x, gv.x), gated_pair<kBf16>(v.y, x.y, gv.y),
                   gated_pair<kBf16>(v.z, x.z, gv.z), gated_pair<kBf16>(v.w, x.w, gv.w));
  }
  *(uint4*)(C + (int64_t)m * ldc + n) = v;
}

// Deep-K launch of BM x BN tiles: one launch (splits == 1) or a split-K partial
// launch plus the reduce (splits > 1; ws holds splits * M * N floats).
template <bool kBf16, int kEpi, int BM, int BN, int KS, int U, int NS>
hipError_t launch_deepk(const GemmArgs& g, int splits, float* ws, hipStream_t st) {
  const int tiles_m = (g.M + BM - 1) / BM, tiles_n = (g.N + BN - 1) / BN;
  if (splits <= 1) {
    hipLaunchKernelGGL((fp8_gemm_4k<kBf16, kEpi, BM, BN, KS, U, NS>), dim3(tiles_m * tiles_n), dim3(256), 0, st,
                       (const uint8_t*)g.A, (const uint8_t*)g.W, g.scales_a, g.scales_b, (const uint16_t*)g.bias,
                       (uint16_t*)g.C, g.M, g.N, g.K, g.ldc, tiles_m, tiles_n, 1, 0, -2, residual_args(g), nullptr, 1);
    return hipGetLastError();
  }
  hipLaunchKernelGGL((fp8_gemm_4k<true, kEpiPartial, BM, BN, KS, U, NS>), dim3(tiles_m * tiles_n * splits), dim3(256), 0,
                     st, (const uint8_t*)g.A, (const uint8_t*)g.W, g.scales_a, g.scales_b, (const uint16_t*)g.bias,
                     (uint16_t*)g.C, g.M, g.N, g.K, g.ldc, tiles_m, tiles_n, 1, 0, -3, residual_args(g), ws, splits);
  const int64_t threads = (int64_t)g.M * (g.N / 8);
  hipLaunchKernelGGL((fp8_gemm_splitk_reduce<kBf16, kEpi>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     st, ws, splits, g.scales_a, g.scales_b, (const uint16_t*)g.bias, (uint16_t*)g.C, g.M, g.N,
                     g.ldc, residual_args(g));
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Narrow tiles for small M with N % 80 == 0 (the model's 5120-wide outputs at 129-512 tokens):
// BM x 80 tiles, BM = 64 or 128, so that one round of tiles fills the CUs without a K split
// (M 256 x N 5120: 4 x 64 tiles of 64 x 80; M 512: 4 x 64 of 128 x 80). These GEMMs are bound by
// the operand bytes each CU streams, (BM + BN) x K per tile, at 40-50 GB/s per CU when the
// operands come partly from HBM (a load-only probe of the same access pattern takes 18.8 us at
// M 512 x N 5120 with 128 x 80 tiles against 25.1 us with 128 x 128 tiles on 160 CUs, and
// 14.7 us at M 256 with 64 x 80 tiles); of the tile shapes that fill one round, the squarest
// moves the fewest bytes per CU.
//
// 4 x KH waves: wave w owns rows [(w % 4) BM/4, +BM/4) and all 80 columns, as FM x 5 tiles of
// v_mfma_scale_f32_16x16x128_f8f6f4 (operand lanes and accumulator layout as in fp8_gemm_4q:
// lane l holds row l % 16 of a fragment, K bytes [32 (l / 16), +32) of a 128-byte k-step;
// accumulator element e of lane l is output (row l % 16, column 4 (l / 16) + e)). K steps of
// 256 bytes staged global -> VGPR -> LDS as in fp8_gemm_4k: U staging buffers (2; 3 measured no
// faster) and two LDS slots; iteration t loads step t + U into the buffer that held step t, runs
// step t's MFMAs and writes step t + 1 into the slot of step t - 1 (read by every wave before the
// barrier). With KH = 2 the waves w and w + 4 share a row group, each taking one of the two MFMA
// k-steps of every K step (two waves per SIMD, so one wave's MFMAs run while the other waits);
// their sums are added at the end, (k-step 0) + (k-step 1), through LDS.
// Workgroup positions are XCD-ordered with the tile rows innermost, so the tiles that share
// a W panel run on one XCD and read it through one L2.
// ---------------------------------------------------------------------------
template <bool kBf16, int kEpi, int BM, int U, int KH>
__global__ __launch_bounds__(256 * KH, 1) void fp8_gemm_4n(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ W, const float* __restrict__ sa,
    const float* __restrict__ sb, const uint16_t* __restrict__ bias, uint16_t* __restrict__ C,
    int M, int N, int K, int64_t ldc, int tiles_m, ResidualArgs res) {
  static_assert(kEpi == kEpiPlain || kEpi == kEpiGelu || kEpi == kEpiResidual, "epilogues");
  static_assert(U == 2 || U == 3, "staging buffers");
  static_assert(KH == 1 || KH == 2, "waves per row group");
  constexpr int UNR = U == 2 ? 2 : 6;  // lcm(U, 2 slots)
  constexpr int BN = 80, KS = 256, NW = 4, NT = 256 * KH;
  constexpr int WTM = BM / NW, FM = WTM / 16, FN = BN / 16;
  constexpr int CPR = KS / 16;                                 // 16 chunks per row
  constexpr int ROWS = BM + BN, CHUNKS = ROWS * CPR;
  constexpr int L = (CHUNKS + NT - 1) / NT, LAST = CHUNKS - (L - 1) * NT;  // loads per thread; the last
  constexpr int SLOT = ROWS * KS, A_BYTES = BM * KS;                         // one by the first LAST threads
  static_assert(BM == 64 || BM == 128, "tile heights");
  static_assert(LAST % 64 == 0 && (NT / CPR) % 16 == 0 && BM % (NT / CPR) == 0, "whole waves per load, A or W rows");
  static_assert(2 * SLOT <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * SLOT];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = wave % NW, kh = wave / NW;  // row group; the MFMA k-step (of 2 per K step) with KH = 2
  const int pos = xcd_position(blockIdx.x, gridDim.x);
  const int m0 = (pos % tiles_m) * BM, n0 = (pos / tiles_m) * BN;
  const int nk = K / KS;

  // operand rows of this thread's loads: load i covers rows NT/16 i .. of the slot (A rows, then W
  // rows); the thread fetches logical chunk c ^ swz(row) into physical chunk c = tid % 16
  const uint8_t* src[L];
  const int lc = tid % CPR;
#pragma unroll
  for (int i = 0; i < L; ++i) {
    const int row = min(i * (NT / CPR) + tid / CPR, ROWS - 1);
    const int chunk = (lc ^ swz_rows<KS>(row)) * 16;
    src[i] = row < BM ? A + (int64_t)min(m0 + row, M - 1) * K + chunk : W + (int64_t)(n0 + row - BM) * K + chunk;
  }
  const bool last = LAST == NT || tid < LAST;  // wave-uniform
  v4i stg[U][L];
  auto gload = [&](auto bc, int kt) {
    constexpr int B = decltype(bc)::value;
    const int64_t koff = (int64_t)min(kt, nk - 1) * KS;
#pragma unroll
    for (int i = 0; i < L; ++i)
      if (i + 1 < L || last) stg[B][i] = *(const v4i*)(src[i] + koff);
  };
  auto lwrite = [&](auto bc, auto sc) {
    constexpr int B = decltype(bc)::value, SL = decltype(sc)::value;
    uint8_t* base = lds + SL * SLOT + tid * 16;
#pragma unroll
    for (int i = 0; i < L; ++i)
      if (i + 1 < L || last) *(v4i*)(base + i * NT * 16) = stg[B][i];
  };

  const int frow = lane & 15, g = lane >> 4;
  const int a_row0 = (rg * WTM + frow) * KS, w_row0 = A_BYTES + frow * KS;
  v4f acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = (v4f){};
  // fragment of k-step S (128 bytes: logical chunks 8 S + 2 g, + 1) of the row at r (the
  // swizzle of every fragment row is frow)
  auto frag = [&](const uint8_t* r, int s) {
    const v4i lo = *(const v4i*)(r + (((8 * s + 2 * g) ^ frow) << 4));
    const v4i hi = *(const v4i*)(r + (((8 * s + 2 * g + 1) ^ frow) << 4));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  };
  auto iteration = [&](auto jc, int t) {
    constexpr int J = decltype(jc)::value;  // t % UNR
    constexpr int SL = J % 2;
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): own LDS writes and fragment reads done
    block_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // into the buffer of step t (written to LDS in the last iteration); left to the compiler's
    // schedule among the MFMAs (issued as a block before them: M 512 x N 5120 25.3 -> 28.7 us)
    gload(IC<J % U>{}, t + U);
    const uint8_t* slot = lds + SL * SLOT;
#pragma unroll
    for (int s = 0; s < 2 / KH; ++s) {
      const int ks = KH == 2 ? kh : s;
      v8i fa[FM], fw[FN];
#pragma unroll
      for (int j = 0; j < FM; ++j) fa[j] = frag(slot + a_row0 + j * 16 * KS, ks);
#pragma unroll
      for (int i = 0; i < FN; ++i) fw[i] = frag(slot + w_row0 + i * 16 * KS, ks);
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = mfma_16x16x128_fp8(fw[i], fa[j], acc[i][j]);
    }
    lwrite(IC<(J + 1) % U>{}, IC<SL ^ 1>{});  // step t + 1 into the slot of step t - 1
    __builtin_amdgcn_sched_barrier(0);
  };

  static_for<0, U>([&](auto bc) { gload(bc, decltype(bc)::value); });
  lwrite(IC<0>{}, IC<0>{});
  int t = 0;
  for (; t + UNR <= nk; t += UNR) static_for<0, UNR>([&](auto jc) { iteration(jc, t + decltype(jc)::value); });
  static_for<0, UNR - 1>([&](auto jc) {
    if (t + decltype(jc)::value < nk) iteration(jc, t + decltype(jc)::value);
  });
  if constexpr (KH == 2) {
    // the second k-step's sums join the first's: acc = acc(k-step 0) + acc(k-step 1)
    wait_vmcnt_lgkm0<0>();  // also the last, unused prefetches
    block_barrier();
    v4f* xch = (v4f*)lds + (rg * FN * FM) * 64 + lane;
    if (kh == 1) {
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) xch[(i * FM + j) * 64] = acc[i][j];
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    block_barrier();
    if (kh == 1) return;
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) acc[i][j] += xch[(i * FM + j) * 64];
  }

  // epilogue: out = round(fma(acc * sb[n], sa[m], bias[n])), then GELU or the gated residual;
  // each lane stores 4 consecutive outputs (8 bytes) of one row per MFMA tile
#pragma unroll
  for (int j = 0; j < FM; ++j) {
    const int m = m0 + rg * WTM + j * 16 + frow;
    if (m >= M) continue;
    const float s_a = sa[m];
#pragma unroll
    for (int i = 0; i < FN; ++i) {
      const int n = n0 + i * 16 + 4 * g;
      const float4 sv = *(const float4*)(sb + n);
      const uint2 bb = bias ? *(const uint2*)(bias + n) : make_uint2(0u, 0u);
      const float sbe[4] = {sv.x, sv.y, sv.z, sv.w};
      const float be[4] = {unpack_lo<kBf16>(bb.x), unpack_hi<kBf16>(bb.x), unpack_lo<kBf16>(bb.y),
                           unpack_hi<kBf16>(bb.y)};
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = __builtin_fmaf(acc[i][j][e] * sbe[e], s_a, be[e]);
      uint2 pk = make_uint2(pack2<kBf16>(o[0], o[1]), pack2<kBf16>(o[2], o[3]));
      if constexpr (kEpi == kEpiGelu) {
        pk = make_uint2(pack2<kBf16>(gelu_tanh(unpack_lo<kBf16>(pk.x)), gelu_tanh(unpack_hi<kBf16>(pk.x))),
                        pack2<kBf16>(gelu_tanh(unpack_lo<kBf16>(pk.y)), gelu_tanh(unpack_hi<kBf16>(pk.y))));
      }
      if constexpr (kEpi == kEpiResidual) {
        const uint2 x = *(const uint2*)(res.ptr + (int64_t)m * res.ld + n);
        const uint2 gt = *(const uint2*)(res.gate + n);
        pk = make_uint2(gated_pair<kBf16>(pk.x, x.x, gt.x), gated_pair<kBf16>(pk.y, x.y, gt.y));
      }
      *(uint2*)(C + (int64_t)m * ldc + n) = pk;
    }
  }
}

// One round of BM x 80 tiles (fp8_gemm_4n).
template <bool kBf16, int kEpi, int BM, int U, int KH>
hipError_t launch_narrow(const GemmArgs& g, hipStream_t st) {
  const int tm = (g.M + BM - 1) / BM, tn = g.N / 80;
  hipLaunchKernelGGL((fp8_gemm_4n<kBf16, kEpi, BM, U, KH>), dim3(tm * tn), dim3(256 * KH), 0, st, (const uint8_t*)g.A,
                     (const uint8_t*)g.W, g.scales_a, g.scales_b, (const uint16_t*)g.bias, (uint16_t*)g.C, g.M, g.N,
                     g.K, g.ldc, tm, residual_args(g));
  return hipGetLastError();
}

// Small M (<= 512 rows): deep-K tiles (fp8_gemm_4k), split over K where the tiles
// alone would leave most CUs idle (splits = CUs / tiles, at most 8 and at least 4 K
// steps per split). Measured on MI355X with W read from HBM, K 5120 unless stated;
// the reference's hipBLASLt GEMM (torch._scaled_mm) on the same inputs in brackets,
// the 64-byte-step DMA kernel in braces:
//   M 64:  64x64 tiles, 256-byte K steps, 3 staging buffers, 2 LDS slots:
//          N 15360: 20.9 us (20.4) {28.4};  N 5120, 3 splits: 12.8 us (15.3) {23.9}
//   M 256: 128x128 tiles, 128-byte K steps, 3 staging buffers, 3 LDS slots:
//          N 15360: 35.0 us (41.1) {42.1};  N 5120, 3 splits: 21.6 us (30.4) {28.1}
//   M 512: N 5120: 128x128 as for M 256: 29.5 us (31.2) {35.7}
//          (N 15360 / 13824 take 256x128 one-tile-per-workgroup plans before these, in
//          launch_small_m)
//          128x256 tiles, 128-byte K steps, 2 staging buffers, 3 LDS slots, where they
//          fill 3/4 of the CUs or K is long enough to split:
//          N 15360: 56.7 us (54.6) {62.2};  N 13824: 53.4 us {58.6};
//          K 13824, N 5120, 3 splits: 57.2 us {80.9} (128x128 without split: 63.4 us)
constexpr int kSmallMaxM = 512;

struct SmallPlan {
  int kind;  // 0: no deep-K plan; 1: 64x64 / 256 B steps; 2: 128x128 / 128 B; 3: 128x256 / 128 B;
             // 4: 64x64 / 512 B steps (no K split)
  int splits;
};

SmallPlan small_plan(int M, int N, int K, bool allow_split) {
  if (M > kSmallMaxM || M <= 0 || N <= 0) return SmallPlan{0, 1};
  const int P = device_cus();
  auto tiles = [&](int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  auto splits_for = [&](int t, int ks) {
    if (!allow_split) return 1;
    int s = min(P / t, (K / ks) / 4);
    return max(1, min(s, 8));
  };
  if (M <= 64) {
    if (K % 256 != 0) return SmallPlan{0, 1};
    const int s = splits_for(tiles(64, 64), 256);
    // unsplit: 512-byte steps (M 64 x N 15360: 20.1 vs 20.5 us for 256-byte steps; with a K
    // split the 256-byte steps stay ahead: N 5120, 3 splits 13.8 vs 14.1 us)
    if (s == 1 && K % 512 == 0) return SmallPlan{4, 1};
    return SmallPlan{1, s};
  }
  if (K % 128 != 0) return SmallPlan{0, 1};
  if (M <= 256) return SmallPlan{2, splits_for(tiles(128, 128), 128)};
  const int t3 = tiles(128, 256);
  if (4 * t3 >= 3 * P) return SmallPlan{3, 1};
  if (K >= 8192 && allow_split) return SmallPlan{3, splits_for(t3, 128)};
  return SmallPlan{2, splits_for(tiles(128, 128), 128)};
}

// Tile height of the narrow-tile plan (fp8_gemm_4n), or 0: one round of BM x 80 tiles where it
// fills the CUs (N 5120: 64-row tiles at 129-256 rows, 128-row tiles at 449-512 rows with K below
// 8192). Measured against the deep-K plans (W from HBM, graph-replayed, K 5120): M 200 20.2 ->
// 15.8 us, M 256 21.9 -> 17.3 (no K split, no reduce launch), M 512 29.0 -> 24.6 (256 tiles
// against 160), with the gated residual 31.8 -> 25.4. Where the deep-K plan splits K over
// larger tiles it moves fewer bytes per CU and stays ahead: M 300 (3 x 64 tiles of 128 x 80)
// 24.8 vs 22.3 us, M 512 x K 13824 56.3 vs 50.7.
int narrow_bm(int M, int N, int K) {
  if (N % 80 != 0 || K % 256 != 0 || M <= 128 || M > kSmallMaxM) return 0;
  const int P = device_cus(), tn = N / 80;
  const int t128 = ((M + 127) / 128) * tn, t64 = ((M + 63) / 64) * tn;
  if (8 * t128 >= 7 * P && t128 <= P && K < 8192) return 128;
  if (4 * t64 >= 3 * P && t64 <= P) return 64;
  return 0;
}

template <bool kBf16, int kEpi>
hipError_t launch_small_m(const GemmArgs& g, hipStream_t st) {
  const int nbm = narrow_bm(g.M, g.N, g.K);
  // 128-row tiles with two waves per row group (each one of the two MFMA k-steps of a K step): 25.3 ->
  // 24.6 us at M 512 x N 5120; 64-row tiles with one (two: 17.4 -> 18.3 us at M 256)
  if (nbm == 128) return launch_narrow<kBf16, kEpi, 128, 2, 2>(g, st);
  if (nbm == 64) return launch_narrow<kBf16, kEpi, 64, 2, 1>(g, st);
  if (g.M > 256 && g.K % 128 == 0) {
    // 257-512 rows where 256x128 tiles fill 3/4 of the CUs: one tile per workgroup with
    // 128-byte K steps through the DMA ring (M 512 x N 15360: 43-45 us vs 47 for 128x256
    // deep-K tiles, hipBLASLt 48; x N 13824 with GELU 42 vs 46). With fewer tiles (N 5120)
    // the deep-K plans stay ahead (128x128 tiles: 30.3 vs 28.8 us).
    const int tm = (g.M + 255) / 256, tn = (g.N + 127) / 128, P = device_cus();
    if (4 * tm * tn >= 3 * P && tm * tn <= P) return launch_one_round_256x128<kBf16, kEpi>(g, tm, tn, st);
  }
  SmallPlan p = small_plan(g.M, g.N, g.K, true);
  if (p.splits > 1 && (g.workspace == nullptr || g.workspace_bytes < (int64_t)p.splits * g.M * g.N * 4))
    p = small_plan(g.M, g.N, g.K, false);  // no (or too small a) workspace: best plan without a split
  float* ws = (float*)g.workspace;
  switch (p.kind) {
    case 1:
      return launch_deepk<kBf16, kEpi, 64, 64, 256, 3, 2>(g, p.splits, ws, st);
    case 4:
      return launch_deepk<kBf16, kEpi, 64, 64, 512, 2, 2>(g, 1, nullptr, st);
    case 2:
      return launch_deepk<kBf16, kEpi, 128, 128, 128, 3, 3>(g, p.splits, ws, st);
    case 3:
      return launch_deepk<kBf16, kEpi, 128, 256, 128, 2, 3>(g, p.splits, ws, st);
    default:
      break;
  }
  if (g.M > 256) return launch_4w<kBf16, kEpi>(g, st);
  if (g.M <= 64) return launch_direct<kBf16, kEpi, 64, 64, 8>(g, st);
  const int64_t tiles_128x64 = (int64_t)((g.M + 127) / 128) * ((g.N + 63) / 64);
  if (tiles_128x64 <= device_cus()) return launch_direct<kBf16, kEpi, 128, 64, 6>(g, st);
  return launch_direct<kBf16, kEpi, 128, 128, 5>(g, st);
}

template <bool kBf16, int kEpi>
hipError_t launch_gemm_t(const GemmArgs& g, hipStream_t st) {
  // main kernel: 64-byte K steps, 16-byte operand rows and scale loads, 8-byte bias
  // loads, 16-byte output row segments
  const bool fast = !g.force_generic && g.K >= 64 && (g.K % 64 == 0) && (g.N % 8 == 0) &&
                    (g.ldc % 8 == 0) && ((uintptr_t)g.C % 16 == 0) &&
                    ((uintptr_t)g.scales_b % 16 == 0) && ((uintptr_t)g.A % 16 == 0) &&
                    ((uintptr_t)g.W % 16 == 0) && ((uintptr_t)g.bias % 8 == 0) &&
                    (!g.residual || ((uintptr_t)g.residual % 16 == 0 && g.ldr % 8 == 0 &&
                                     (uintptr_t)g.gate % 16 == 0));
  if (fast && g.M <= kSmallMaxM) return launch_small_m<kBf16, kEpi>(g, st);
  if (fast && g.M <= 2048 && g.K >= 4096 && g.K % 128 == 0) {
    // Less than one round of 256x256 tiles: deep-K 128-row tiles. Measured with W
    // from HBM, long K (the reference's 16384-wide FFN-down at 1024 / 1560 tokens):
    // 1024 x 16384 x 4096: 79.3 us vs 89.3 (256x256 + split tail); 1560 x 16384 x 4096:
    // 140.3 us vs 151.7. At K 4096 only where the 128-row tiles fit one round:
    // 1024 x 4096 x 4096 26.9 us vs 30.1, 1560 x 4096 x 4096 42.6 vs 44.2, while
    // 1024 x 4096 x 12288 (1.5 rounds of 128x256) takes 82.5 us vs 66.6.
    // Where neither 128-row tile fits one round but 256x192 tiles do (1024 x 4096 x 12288:
    // 256 tiles against 192 of 256x256), the 256x192 tiles fill every CU.
    const int P = device_cus();
    const int64_t t256 = (int64_t)((g.M + 255) / 256) * ((g.N + 255) / 256);
    const int64_t t128 = (int64_t)((g.M + 127) / 128) * ((g.N + 127) / 128);
    const int64_t t128x256 = (int64_t)((g.M + 127) / 128) * ((g.N + 255) / 256);
    const int64_t t256x192 = (int64_t)((g.M + 255) / 256) * ((g.N + 191) / 192);
    const int64_t t256x128 = (int64_t)((g.M + 255) / 256) * ((g.N + 127) / 128);
    if (t256 < P) {
      if (t128 <= P) return launch_deepk<kBf16, kEpi, 128, 128, 128, 3, 3>(g, 1, nullptr, st);
      // 256x128 tiles with 128-byte steps where they fill more CUs than 128x256 (1560 rows: 224
      // tiles against 208; 1560 x 4096 -> 4096 32.3 us vs 34.0, 1560 x 16384 -> 4096 109.7 vs 112.3)
      if (t256x128 <= P && t256x128 > t128x256)
        return launch_one_round_256x128<kBf16, kEpi>(g, (g.M + 255) / 256, (g.N + 127) / 128, st);
      if (t128x256 <= P) return launch_deepk<kBf16, kEpi, 128, 256, 128, 2, 3>(g, 1, nullptr, st);
      if (t256x192 <= P) {
        // 256x192 tiles filling the CUs (1024 x 4096 -> 12288: 256 tiles): the persistent kernel,
        // one tile per workgroup (38.9 vs 43.9 us for the one-tile 32x32x64 kernel, bit-identical)
        const int tm = (g.M + 255) / 256, tn = (g.N + 191) / 192;
        if (persistent_ok(g)) {
          hipLaunchKernelGGL((fp8_gemm_4q<kBf16, kEpi, 192>), dim3(tm * tn), dim3(256), 0, st, (const uint8_t*)g.A,
                             (const uint8_t*)g.W, g.scales_a, g.scales_b, (const uint16_t*)g.bias, (uint16_t*)g.C, g.M,
                             g.N, g.K, g.ldc, tm, tn, kGroupM, tm * tn, residual_args(g), QkvEpi{});
          return hipGetLastError();
        }
        hipLaunchKernelGGL((fp8_gemm_4h<kBf16, kEpi, 256, 192, 2>), dim3(tm * tn), dim3(256), 0, st,
                           (const uint8_t*)g.A, (const uint8_t*)g.W, g.scales_a, g.scales_b, (const uint16_t*)g.bias,
                           (uint16_t*)g.C, g.M, g.N, g.K, g.ldc, tm, tn, 1, 0, -2, residual_args(g));
        return hipGetLastError();
      }
      if (g.K >= 8192) return launch_deepk<kBf16, kEpi, 128, 256, 128, 2, 3>(g, 1, nullptr, st);
    }
  }
  if (fast) return launch_4w<kBf16, kEpi>(g, st);
  const int tiles_m = (g.M + 31) / 32, tiles_n = (g.N + 31) / 32;
  const int tiles = tiles_m * tiles_n;
  hipLaunchKernelGGL((fp8_gemm_generic<kBf16, kEpi>), dim3((tiles + 3) / 4), dim3(256), 0, st,
                     (const uint8_t*)g.A, (const uint8_t*)g.W, g.scales_a, g.scales_b,
                     (const uint16_t*)g.bias, (uint16_t*)g.C, g.M, g.N, g.K, g.ldc, tiles_n, residual_args(g));
  return hipGetLastError();
}

// q/k RMSNorm + RoPE and the KV-ring write of the tiles of a fused QKV projection that the
// persistent kernel leaves to the sub-tile launch (which stores them plainly in C): one
// workgroup per sub-tile of BMs rows x one head, 16 lanes per token as in the standalone
// kernel (same arithmetic order, head_rsqrt), the sub-tile order of fp8_gemm_4h.
template <int BMs>
__global__ __launch_bounds__(256) void qkv_tail_norm_rope(const uint16_t* __restrict__ C, int64_t ldc, int M,
                                                          int tiles_m, int tiles_n, int group_m, int tile_base,
                                                          int sub_log2, QkvEpi qe) {
  const TileJob job = decode_job<BMs, 128>(0, tiles_m, tiles_n, group_m, tile_base, sub_log2, 1);
  const int lane = threadIdx.x & 63, li = lane & 15;
  const int eh = qe.heads * 128, region = job.n0 / eh, head = (job.n0 - region * eh) >> 7;
  const int o1 = region == 0 ? 0 : (region == 1 ? 1 : 3), o2 = region == 1 ? 2 : 4;
  float w[8] = {};
  if (region < 2) {
    const uint4 wv = *(const uint4*)((region == 0 ? qe.q_weight : qe.k_weight) + li * 8);
    const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      w[2 * e] = bf16_lo(ww[e]);
      w[2 * e + 1] = bf16_hi(ww[e]);
    }
  }
  for (int u0 = 0; u0 < BMs; u0 += 16) {
    const int m = job.m0 + u0 + (int)(threadIdx.x >> 4);
    const int mr = min(m, M - 1);  // every lane takes part in the head's shuffles
    const uint4 x = *(const uint4*)(C + (int64_t)mr * ldc + job.n0 + li * 8);
    uint4 out1 = x, out2 = x;
    if (region < 2) {
      const uint32_t xw[4] = {x.x, x.y, x.z, x.w};
      float f[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f[2 * e] = bf16_lo(xw[e]);
        f[2 * e + 1] = bf16_hi(xw[e]);
      }
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(f[j], f[j], ss);
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) ss += __shfl_xor(ss, off, kWave);
      const float r = head_rsqrt(ss, 1.0f / 128.0f, qe.eps);
#pragma unroll
      for (int j = 0; j < 8; ++j) f[j] = f[j] * r * w[j];
      const uint2 cv = *(const uint2*)(qe.cos + (int64_t)mr * 64 + li * 4);
      const uint2 sv = *(const uint2*)(qe.sin + (int64_t)mr * 64 + li * 4);
      const float c[4] = {bf16_lo(cv.x), bf16_hi(cv.x), bf16_lo(cv.y), bf16_hi(cv.y)};
      const float sn[4] = {bf16_lo(sv.x), bf16_hi(sv.x), bf16_lo(sv.y), bf16_hi(sv.y)};
      float o[8];
#pragma unroll
      for (int p = 0; p < 4; ++p) rope_pair(f[2 * p], f[2 * p + 1], c[p], sn[p], o[2 * p], o[2 * p + 1]);
      out1 = make_uint4(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]), pack_bf16x2(o[4], o[5]),
                        pack_bf16x2(o[6], o[7]));
      out2 = (region == 1 && !qe.kpre_rotated)
                 ? make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                              pack_bf16x2(f[6], f[7]))
                 : out1;
    }
    if (m < M) {
      if (qe.dst[o1] && m < qe.rows[o1]) *(uint4*)(qe.dst[o1] + (int64_t)m * qe.stride[o1] + head * 128 + li * 8) = out1;
      if (region > 0 && qe.dst[o2] && m < qe.rows[o2])
        *(uint4*)(qe.dst[o2] + (int64_t)m * qe.stride[o2] + head * 128 + li * 8) = out2;
    }
  }
}

}  // namespace

int64_t fp8_gemm_workspace_bytes(int M, int N, int K) {
  if (K < 64 || K % 64 != 0 || N % 8 != 0 || narrow_bm(M, N, K) != 0) return 0;
  const SmallPlan p = small_plan(M, N, K, true);
  return p.splits > 1 ? (int64_t)p.splits * M * N * 4 : 0;
}

namespace {
// Tile plan of the fused QKV projection: the persistent kernel takes the whole rounds of 256x256
// tiles (or all tiles when the last round is nearly full), the rest run as 128x128 (sub 2) or
// 256x128 (sub 1) sub-tiles, as launch_4w splits them.
struct QkvPlan {
  int tiles_m, tiles_n, bulk, rem, sub_log2;
};
QkvPlan qkv_plan(int M, int N) {
  QkvPlan p;
  p.tiles_m = (M + 255) / 256;
  p.tiles_n = N / 256;
  const int T = p.tiles_m * p.tiles_n, P = device_cus();
  p.rem = T % P;
  p.sub_log2 = 0;
  if (p.rem * 4 <= P) {
    p.sub_log2 = 2;
  } else if (p.rem * 2 <= P + P / 4) {
    p.sub_log2 = 1;
  } else {
    p.rem = 0;
  }
  p.bulk = T - p.rem;
  return p;
}

bool qkv_fusable(const GemmArgs& g, const NormRopeArgs& a, int head_dim) {
  const int64_t eh = (int64_t)a.num_heads * 128;
  if (head_dim != 128 || !g.out_bf16 || g.gelu || g.residual || a.num_heads % 2 != 0 || g.N != 3 * eh) return false;
  if (a.n_tokens != g.M || a.table_len != g.M || !persistent_ok(g) || device_cus() % 8 != 0) return false;
  if ((uintptr_t)a.cos % 16 != 0 || (uintptr_t)a.sin % 16 != 0) return false;  // 16-byte table loads
  const int64_t strides[5] = {a.q_out_stride, a.k_out_stride, a.kpre_stride, a.v_out_stride, a.v_out2_stride};
  for (int i = 0; i < 5; ++i)
    if (((int64_t)g.M * strides[i] + eh) * 2 > 0x7fffffffLL) return false;  // 32-bit buffer offsets
  return true;
}
}  // namespace

int64_t fp8_gemm_qkv_scratch_bytes(int M, int N, int K, int num_heads, int head_dim) {
  if (M <= 0 || N <= 0) return 0;
  GemmArgs g{};
  g.M = M;
  g.N = N;
  g.K = K;
  g.ldc = N;
  g.out_bf16 = true;
  NormRopeArgs a{};
  a.num_heads = num_heads;
  a.n_tokens = a.table_len = M;
  a.q_out_stride = a.k_out_stride = a.kpre_stride = a.v_out_stride = a.v_out2_stride = (int64_t)num_heads * head_dim;
  if (qkv_fusable(g, a, head_dim) && qkv_plan(M, N).rem == 0) return 0;
  return (int64_t)M * N * 2;
}

int64_t fp8_gemm_qkv_call_scratch_bytes(const GemmArgs& g, const NormRopeArgs& a, int head_dim) {
  if (g.M <= 0 || g.N <= 0) return 0;
  if (qkv_fusable(g, a, head_dim) && qkv_plan(g.M, g.N).rem == 0) return 0;
  return (int64_t)g.M * g.N * 2;
}

hipError_t launch_fp8_gemm_qkv(const GemmArgs& g, const NormRopeArgs& a, int head_dim, hipStream_t st) {
  if (g.M == 0 || g.N == 0) return hipSuccess;
  if (!qkv_fusable(g, a, head_dim) || (qkv_plan(g.M, g.N).rem > 0 && g.C == nullptr)) {
    // the GEMM into C, then the standalone norm/RoPE kernel on it
    if (g.C == nullptr) return hipErrorInvalidValue;
    hipError_t e = launch_fp8_gemm(g, st);
    if (e != hipSuccess) return e;
    NormRopeArgs b = a;
    const uint16_t* c = (const uint16_t*)g.C;
    const int64_t eh = (int64_t)a.num_heads * head_dim;
    b.q_in = a.q_out ? c : nullptr;
    b.k_in = c + eh;
    b.v_in = (a.v_out || a.v_out2) ? c + 2 * eh : nullptr;
    b.in_stride = g.ldc;
    return launch_qk_norm_rope(b, head_dim, st);
  }
  QkvEpi qe{};
  uint16_t* dst[5] = {a.q_out, a.k_out, a.kpre_out, a.v_out, a.v_out2};
  const int64_t stride[5] = {a.q_out_stride, a.k_out_stride, a.kpre_stride, a.v_out_stride, a.v_out2_stride};
  const int64_t rows[5] = {g.M, g.M, a.cache_tokens, a.cache_tokens, g.M};
  for (int i = 0; i < 5; ++i) {
    const bool on = dst[i] != nullptr && rows[i] > 0;
    qe.dst[i] = on ? dst[i] : nullptr;
    qe.stride[i] = stride[i];
    qe.rows[i] = on ? (int)rows[i] : 0;
    qe.bytes[i] = on ? (int)(((rows[i] - 1) * stride[i] + (int64_t)a.num_heads * 128) * 2) : 0;
  }
  qe.q_weight = a.q_weight;
  qe.k_weight = a.k_weight;
  qe.cos = a.cos;
  qe.sin = a.sin;
  qe.heads = a.num_heads;
  qe.eps = a.eps;
  qe.kpre_rotated = a.cache_post_rope;
  const QkvPlan p = qkv_plan(g.M, g.N);
  const int P = device_cus();
  if (p.bulk > 0) {
    hipLaunchKernelGGL((fp8_gemm_4q<true, kEpiQkv, 256>), dim3(p.bulk < P ? p.bulk : P), dim3(256), 0, st,
                       (const uint8_t*)g.A, (const uint8_t*)g.W, g.scales_a, g.scales_b, (const uint16_t*)g.bias,
                       (uint16_t*)g.C, g.M, g.N, g.K, g.ldc, p.tiles_m, p.tiles_n, kGroupM, p.bulk, residual_args(g),
                       qe);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (p.rem == 0) return hipSuccess;
  const uint16_t* c = (const uint16_t*)g.C;
  if (p.sub_log2 == 2) {
    hipLaunchKernelGGL((fp8_gemm_4h<true, kEpiPlain, 128, 128, 4>), dim3(p.rem << 2), dim3(256), 0, st,
                       (const uint8_t*)g.A, (const uint8_t*)g.W, g.scales_a, g.scales_b, (const uint16_t*)g.bias,
                       (uint16_t*)g.C, g.M, g.N, g.K, g.ldc, p.tiles_m, p.tiles_n, kGroupM, p.bulk, 2, residual_args(g));
    hipLaunchKernelGGL((qkv_tail_norm_rope<128>), dim3(p.rem << 2), dim3(256), 0, st, c, g.ldc, g.M, p.tiles_m,
                       p.tiles_n, kGroupM, p.bulk, 2, qe);
  } else {
    hipLaunchKernelGGL((fp8_gemm_4h<true, kEpiPlain, 256, 128, 3>), dim3(p.rem << 1), dim3(256), 0, st,
                       (const uint8_t*)g.A, (const uint8_t*)g.W, g.scales_a, g.scales_b, (const uint16_t*)g.bias,
                       (uint16_t*)g.C, g.M, g.N, g.K, g.ldc, p.tiles_m, p.tiles_n, kGroupM, p.bulk, 1, residual_args(g));
    hipLaunchKernelGGL((qkv_tail_norm_rope<256>), dim3(p.rem << 1), dim3(256), 0, st, c, g.ldc, g.M, p.tiles_m,
                       p.tiles_n, kGroupM, p.bulk, 1, qe);
  }
  return hipGetLastError();
}

hipError_t launch_fp8_gemm(const GemmArgs& g, hipStream_t st) {
  if (g.M == 0 || g.N == 0) return hipSuccess;
  if (g.residual && g.gelu) return hipErrorInvalidValue;
  if (g.out_bf16) {
    if (g.residual) return launch_gemm_t<true, kEpiResidual>(g, st);
    return g.gelu ? launch_gemm_t<true, kEpiGelu>(g, st) : launch_gemm_t<true, kEpiPlain>(g, st);
  }
  if (g.residual) return launch_gemm_t<false, kEpiResidual>(g, st);
  return g.gelu ? launch_gemm_t<false, kEpiGelu>(g, st) : launch_gemm_t<false, kEpiPlain>(g, st);
}

}  // namespace joy
