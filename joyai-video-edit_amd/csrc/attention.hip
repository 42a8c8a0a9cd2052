// Joint-attention forward on gfx950: O = softmax(Q K^T * scale) V per head,
// non-causal, no mask, bf16 in / bf16 out, fp32 softmax and accumulation, head
// dim 128 -- the reference model's F.scaled_dot_product_attention(q, k, v,
// is_causal=False) (deploy/xvideo/models/dit/dit.py:154-167), which the block
// calls on the joint Q = [video | condition] and K, V = [cached | video |
// condition] (dit.py:489-498).
//
// Layout: Q, K, V and O are token-major [L, H, 128] views (token and head strides
// in elements), so the joint operands are read where the fused QKV / pack ops wrote
// them and O is written straight into the [L, H*128] rows the out-projection reads.
//
// One workgroup = 128 queries of one head (4 waves x 32 queries), one pass over the
// keys in tiles of 64 (flash attention with an online softmax). Per tile and wave:
//   * S^T = K Q^T: 16 v_mfma_f32_32x32x16_bf16 (K from LDS as the A operand, the
//     wave's 32 queries kept in registers as the B operand). In the 32x32 output a
//     lane holds 16 keys of ONE query, so the row max / row sum are in-lane plus one
//     exchange with lane ^ 32;
//   * online softmax in fp32 with exp2 (scale * log2 e folded into the scores);
//   * O^T += V^T P^T: 16 MFMAs; P^T is the B operand straight from the registers
//     that hold the scores (rounded to bf16), which fixes a permutation of the 16
//     keys of each MFMA; the A operand (V^T) comes from the key-major V tile with two
//     ds_read_b64_tr_b16 per MFMA, whose addresses apply the same permutation. The
//     O^T accumulator again gives each lane one query, so the rescale by
//     exp2(m_old - m_new) is per lane.
// K and V tiles reach LDS by direct-to-LDS DMA (double-buffered, the next tile in flight
// during the current one, one barrier per tile); LDS rows of 256 bytes store 16-byte
// chunk c at a row-dependent XOR of c (chunk_at, chunk_at_v).
//
// ds_read_b64_tr_b16 lane layout (measured on gfx950): within each group of 16
// lanes, lane a points at 4 consecutive 16-bit values M[a][0..3] and lane i receives
// M[4j + i/4][i % 4] for j = 0..3.
#include <type_traits>

#include "joy_common.hpp"
#include "joy_kernels.hpp"

namespace joy {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kD = 128;
constexpr int kBK = 64;                // keys per tile
constexpr int kRowB = kD * 2;          // bytes per K / V row
constexpr int kTileB = kBK * kRowB;    // 16 KB per K or V tile

template <int J>
using IC = std::integral_constant<int, J>;

// K tile: 16-byte chunk c of key row r at c ^ (r & 15) -- the fragment reads take 16 consecutive rows of one
// logical chunk. V tile: c ^ vsw(r) -- a transpose read takes rows 4n..4n+3 and logical chunks 4m..4m+3
// (32 lanes), which vsw spreads over 16 distinct physical chunks (and over 8 distinct chunk positions mod 8 per
// 16 lanes), where (r & 15) folded them onto 4.
__device__ __forceinline__ int chunk_at(int row, int chunk) { return row * kRowB + ((chunk ^ (row & 15)) << 4); }
__device__ __forceinline__ int vsw(int row) { return ((row & 1) << 2) ^ ((row & 2) ? 10 : 0); }
__device__ __forceinline__ int chunk_at_v(int row, int chunk) { return row * kRowB + ((chunk ^ vsw(row)) << 4); }

__device__ __forceinline__ v16f mfma_bf16(const bf16x8& a, const bf16x8& b, const v16f& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(const v4i& v) { return __builtin_bit_cast(bf16x8, v); }

// Combine a value with the one of lane ^ 32 without the LDS crossbar: v_permlane32_swap
// with both operands x returns {x[lane], x[lane ^ 32]} (in an order that depends on the
// half, measured on gfx950), and both halves add them in the same order.
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// QB query blocks of 32 per wave (workgroup = 4 waves x 32 QB queries): with QB = 2 every K
// fragment and every V^T operand read from LDS feeds two MFMAs.
template <int QB>
__global__ __launch_bounds__(256, QB == 1 ? 2 : 1) void attn_fwd_d128(AttnArgs a) {
  constexpr int BQ = 4 * 32 * QB;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][2][kTileB];  // [buffer][K, V]
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int head = blockIdx.y;
  const int ql = lane & 31, hf = lane >> 5;
  const int64_t Lq = a.q_len, Lk = a.k_len;
  int qrow[QB];
#pragma unroll
  for (int i = 0; i < QB; ++i) qrow[i] = blockIdx.x * BQ + (wave * QB + i) * 32 + ql;  // this lane's queries

  // Q as the B operand of S^T = K Q^T: lane holds Q[q][16 s + 8 hf .. +8], s = 0..7
  v4i qf[QB][8];
#pragma unroll
  for (int i = 0; i < QB; ++i) {
    const uint16_t* qp = a.q.ptr + (int64_t)min((int64_t)qrow[i], Lq - 1) * a.q.stride_token +
                         (int64_t)head * a.q.stride_head + 8 * hf;
#pragma unroll
    for (int st = 0; st < 8; ++st) qf[i][st] = *(const v4i*)(qp + 16 * st);
  }

  // K / V tiles reach LDS by direct-to-LDS DMA: one 16-byte load per lane and instruction
  // writes 1 KB = 4 LDS rows; lane l lands in row 4 i + l / 16, physical chunk l % 16, so it
  // fetches logical chunk (l % 16) ^ (row & 15) of that key row. Each wave moves 4 KB of K
  // and 4 KB of V per tile (16 rows each).
  // lane source pointers of the wave's 4 K and 4 V rows in the current tile, advanced by one
  // tile per iteration; the partial last tile recomputes them with the key clamped to Lk - 1
  const uint16_t* kbase = a.k.ptr + (int64_t)head * a.k.stride_head;
  const uint16_t* vbase = a.v.ptr + (int64_t)head * a.v.stride_head;
  const uint16_t* kp[4];
  const uint16_t* vp[4];
  auto set_ptrs = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = wave * 16 + i * 4 + (lane >> 4);
      const int64_t key = min(k0 + row, Lk - 1);
      kp[i] = kbase + key * a.k.stride_token + ((lane & 15) ^ (row & 15)) * 8;
      vp[i] = vbase + key * a.v.stride_token + ((lane & 15) ^ vsw(row)) * 8;
    }
  };
  auto dma_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      __builtin_amdgcn_global_load_lds((const void*)kp[i], (lds_void*)(&lds[buf][0][(wave * 16 + i * 4) * kRowB]),
                                       16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)vp[i], (lds_void*)(&lds[buf][1][(wave * 16 + i * 4) * kRowB]),
                                       16, 0, 0);
    }
  };
  const int64_t k_step = (int64_t)kBK * a.k.stride_token, v_step = (int64_t)kBK * a.v.stride_token;
  auto next_tile = [&](int64_t k0) {  // pointers of the tile starting at key k0 (= previous + kBK)
    if (k0 + kBK <= Lk) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kp[i] += k_step;
        vp[i] += v_step;
      }
    } else {
      set_ptrs(k0);
    }
  };

  // V^T A-operand addresses (transpose reads): lane (group g = lane / 16, a = lane % 16)
  // reads key row 16 b + 8 r + 4 hf + a / 4 of a 32-key block, columns d0 + 16 (g % 2) + 4 (a % 4)
  const int tg = lane >> 4, ta = lane & 15;
  const int tr_row = 4 * hf + (ta >> 2);
  const int tr_col = 16 * (tg & 1) + 4 * (ta & 3);  // element column within a 32-wide d block

  v16f o[QB][4];
#pragma unroll
  for (int i = 0; i < QB; ++i)
#pragma unroll
    for (int db = 0; db < 4; ++db) o[i][db] = (v16f){};
  float m_run[QB], l_run[QB];
#pragma unroll
  for (int i = 0; i < QB; ++i) m_run[i] = -INFINITY, l_run[i] = 0.f;
  const float sl2 = a.scale_log2e;

  const int64_t ntiles = (Lk + kBK - 1) / kBK;
  set_ptrs(0);
  dma_tile(0);
  // one tile; the buffer index is a template constant (the loop runs two tiles per trip), so
  // every LDS address is a loop-invariant lane offset plus an immediate
  auto tile = [&](auto bufc, int64_t t) {
    constexpr int buf = decltype(bufc)::value;
    // own DMAs of tile t landed (nothing else is outstanding); after the barrier every wave's
    // have, and every wave has finished tile t-1, whose buffer the next DMA overwrites
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0), lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (t + 1 < ntiles) {
      next_tile((t + 1) * kBK);
      dma_tile(buf ^ 1);
    }
    const uint8_t* kt = lds[buf][0];
    const uint8_t* vt = lds[buf][1];

    // raw scores S^T for two 32-key blocks; each K fragment feeds the QB query blocks
    // (the MFMA blocks run at raised wave priority, so that of the two waves on a SIMD the
    // one with MFMAs to issue gets the pipe while the other works through its softmax)
    __builtin_amdgcn_s_setprio(1);
    v16f s[QB][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int i = 0; i < QB; ++i) s[i][kb] = (v16f){};
      const int row = kb * 32 + ql;
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        const v4i kf = *(const v4i*)(kt + chunk_at(row, 2 * st + hf));
#pragma unroll
        for (int i = 0; i < QB; ++i) s[i][kb] = mfma_bf16(as_bf16x8(kf), as_bf16x8(qf[i][st]), s[i][kb]);
      }
    }

    __builtin_amdgcn_s_setprio(0);
    // online softmax in log2 units (scale folded into one fma); keys past Lk get -inf
    const int64_t k0 = t * kBK;
    if (k0 + kBK > Lk) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t key = k0 + kb * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
          if (key >= Lk)
#pragma unroll
            for (int i = 0; i < QB; ++i) s[i][kb][r] = -INFINITY;
        }
    }
    v4i pb[QB][4];  // P^T B operands, 16 keys each: chunk 2 kb + b = registers 8 b .. 8 b + 7 of s[kb]
#pragma unroll
    for (int i = 0; i < QB; ++i) {
      float mt = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[i][kb][r]);
      mt = xor32_max(mt);
      const float m_new = fmaxf(m_run[i], mt * sl2);
      const float alpha = __builtin_amdgcn_exp2f(m_run[i] - m_new);
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          float p[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            p[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i][kb][8 * b + j], sl2, -m_new));
            rs += p[j];
          }
          pb[i][2 * kb + b] = (v4i){(int)pack_bf16x2(p[0], p[1]), (int)pack_bf16x2(p[2], p[3]),
                                    (int)pack_bf16x2(p[4], p[5]), (int)pack_bf16x2(p[6], p[7])};
        }
      rs = xor32_sum(rs);
      l_run[i] = l_run[i] * alpha + rs;
      m_run[i] = m_new;
      // rescale only when some lane's running max moved (alpha == 1 otherwise)
      if (__builtin_amdgcn_read_exec() &&
          __builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
        for (int db = 0; db < 4; ++db) o[i][db] *= alpha;
      }
    }

    // O^T += V^T P^T; each V^T operand feeds the QB query blocks
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const int row0 = kb * 32 + 16 * b + tr_row;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const int col = db * 32 + tr_col;  // element column (4 consecutive)
          const int chunk = col >> 3, within = (col & 7) * 2;
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4*)(vt + chunk_at_v(row0, chunk) + within));
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4*)(vt + chunk_at_v(row0 + 8, chunk) + within));
          const v4i va = __builtin_bit_cast(v4i, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
          for (int i = 0; i < QB; ++i) o[i][db] = mfma_bf16(as_bf16x8(va), as_bf16x8(pb[i][2 * kb + b]), o[i][db]);
        }
      }
    __builtin_amdgcn_s_setprio(0);

  };
  int64_t t = 0;
  for (; t + 2 <= ntiles; t += 2) {
    tile(IC<0>{}, t);
    tile(IC<1>{}, t + 1);
  }
  if (t < ntiles) tile(IC<0>{}, t);
  __builtin_amdgcn_s_waitcnt(0x0070);  // (no DMA outstanding past the loop)

  // O = O^T / l: lane holds query q, d = 32 db + 8 (r / 4) + 4 hf + (r % 4)
#pragma unroll
  for (int i = 0; i < QB; ++i) {
    if (qrow[i] >= Lq) continue;
    const float inv = 1.0f / l_run[i];
    uint16_t* op = a.out + (int64_t)qrow[i] * a.out_stride_token + (int64_t)head * kD;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = db * 32 + 8 * r4 + 4 * hf;
        uint2 w;
        w.x = pack_bf16x2(o[i][db][4 * r4] * inv, o[i][db][4 * r4 + 1] * inv);
        w.y = pack_bf16x2(o[i][db][4 * r4 + 2] * inv, o[i][db][4 * r4 + 3] * inv);
        *(uint2*)(op + d) = w;
      }
  }
}

}  // namespace

// One query block per wave: with two, every K / V^T operand read feeds two MFMAs, but the
// registers spill and one workgroup fills a CU; measured at the cfg-4 joint shape (11312 x
// 32912 x 40 heads): 8.8 ms with QB = 1 against 15.3 ms with QB = 2.
hipError_t launch_attention_fwd(const AttnArgs& a, hipStream_t st) {
  constexpr int QB = 1;
  constexpr int BQ = 4 * 32 * QB;
  const dim3 grid((unsigned)((a.q_len + BQ - 1) / BQ), (unsigned)a.heads);
  hipLaunchKernelGGL(attn_fwd_d128<QB>, grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace joy
