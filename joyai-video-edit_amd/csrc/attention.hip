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
// K and V tiles travel global -> VGPR -> LDS (double-buffered, one barrier per
// tile); LDS rows of 256 bytes store 16-byte chunk c at c ^ (row & 15).
//
// ds_read_b64_tr_b16 lane layout (measured on gfx950): within each group of 16
// lanes, lane a points at 4 consecutive 16-bit values M[a][0..3] and lane i receives
// M[4j + i/4][i % 4] for j = 0..3.
#include "joy_common.hpp"
#include "joy_kernels.hpp"

namespace joy {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr int kD = 128;
constexpr int kBQ = 128;               // queries per workgroup
constexpr int kBK = 64;                // keys per tile
constexpr int kRowB = kD * 2;          // bytes per K / V row
constexpr int kTileB = kBK * kRowB;    // 16 KB per K or V tile

__device__ __forceinline__ int chunk_at(int row, int chunk) { return row * kRowB + ((chunk ^ (row & 15)) << 4); }

__device__ __forceinline__ v16f mfma_bf16(const bf16x8& a, const bf16x8& b, const v16f& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(const v4i& v) { return __builtin_bit_cast(bf16x8, v); }

__global__ __launch_bounds__(256, 2) void attn_fwd_d128(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][2][kTileB];  // [buffer][K, V]
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int head = blockIdx.y;
  const int ql = lane & 31, hf = lane >> 5;
  const int q = blockIdx.x * kBQ + wave * 32 + ql;  // this lane's query
  const int64_t Lq = a.q_len, Lk = a.k_len;

  // Q as the B operand of S^T = K Q^T: lane holds Q[q][16 s + 8 hf .. +8], s = 0..7
  v4i qf[8];
  {
    const uint16_t* qp = a.q.ptr + (int64_t)min((int64_t)q, Lq - 1) * a.q.stride_token +
                         (int64_t)head * a.q.stride_head + 8 * hf;
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = *(const v4i*)(qp + 16 * s);
  }

  // K / V tile loads: thread chunk c = tid + 256 i covers row c / 16, 16-byte chunk c % 16
  const uint16_t* kbase = a.k.ptr + (int64_t)head * a.k.stride_head;
  const uint16_t* vbase = a.v.ptr + (int64_t)head * a.v.stride_head;
  v4i ks[4], vs[4];
  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int64_t key = min(k0 + (c >> 4), Lk - 1);
      ks[i] = *(const v4i*)(kbase + key * a.k.stride_token + (c & 15) * 8);
      vs[i] = *(const v4i*)(vbase + key * a.v.stride_token + (c & 15) * 8);
    }
  };
  auto lwrite = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i;
      const int off = chunk_at(c >> 4, c & 15);
      *(v4i*)(&lds[buf][0][off]) = ks[i];
      *(v4i*)(&lds[buf][1][off]) = vs[i];
    }
  };

  // V^T A-operand addresses (transpose reads): lane (group g = lane / 16, a = lane % 16)
  // reads key row 16 b + 8 r + 4 hf + a / 4 of a 32-key block, columns d0 + 16 (g % 2) + 4 (a % 4)
  const int tg = lane >> 4, ta = lane & 15;
  const int tr_row = 4 * hf + (ta >> 2);
  const int tr_col = 16 * (tg & 1) + 4 * (ta & 3);  // element column within a 32-wide d block

  v16f o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = (v16f){};
  float m_run = -INFINITY, l_run = 0.f;
  const float sl2 = a.scale_log2e;

  const int64_t ntiles = (Lk + kBK - 1) / kBK;
  gload(0);
  lwrite(0);
  if (ntiles > 1) gload(kBK);
  for (int64_t t = 0; t < ntiles; ++t) {
    const int buf = (int)(t & 1);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): own LDS writes done
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* kt = lds[buf][0];
    const uint8_t* vt = lds[buf][1];

    // S^T for two 32-key blocks
    v16f s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      s[kb] = (v16f){};
      const int row = kb * 32 + ql;
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        const v4i kf = *(const v4i*)(kt + chunk_at(row, 2 * st + hf));
        s[kb] = mfma_bf16(as_bf16x8(kf), as_bf16x8(qf[st]), s[kb]);
      }
    }
    // online softmax; keys past Lk (only in the last tile) get -inf
    const int64_t k0 = t * kBK;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) s[kb] *= sl2;
    if (k0 + kBK > Lk) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t key = k0 + kb * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
          if (key >= Lk) s[kb][r] = -INFINITY;
        }
    }
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[kb][r]);
    mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
    const float m_new = fmaxf(m_run, mt);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    float rs = 0.f;
    v4i pb[4];  // P^T B operands, 16 keys each: chunk 2 kb + b = registers 8 b .. 8 b + 7 of s[kb]
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        float p[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          p[j] = __builtin_amdgcn_exp2f(s[kb][8 * b + j] - m_new);
          rs += p[j];
        }
        pb[2 * kb + b] = (v4i){(int)pack_bf16x2(p[0], p[1]), (int)pack_bf16x2(p[2], p[3]),
                               (int)pack_bf16x2(p[4], p[5]), (int)pack_bf16x2(p[6], p[7])};
      }
    rs += __shfl_xor(rs, 32, kWave);
    l_run = l_run * alpha + rs;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] *= alpha;

    // O^T += V^T P^T
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
              (lds_s16x4*)(vt + chunk_at(row0, chunk) + within));
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4*)(vt + chunk_at(row0 + 8, chunk) + within));
          const v4i va = __builtin_bit_cast(v4i, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
          o[db] = mfma_bf16(as_bf16x8(va), as_bf16x8(pb[2 * kb + b]), o[db]);
        }
      }

    // tile t+1 (in registers) into the other buffer; then start loading tile t+2
    if (t + 1 < ntiles) {
      lwrite(buf ^ 1);
      if (t + 2 < ntiles) gload((t + 2) * kBK);
    }
  }

  // O = O^T / l: lane holds query q, d = 32 db + 8 (r / 4) + 4 hf + (r % 4)
  if (q < Lq) {
    const float inv = 1.0f / l_run;
    uint16_t* op = a.out + (int64_t)q * a.out_stride_token + (int64_t)head * kD;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = db * 32 + 8 * r4 + 4 * hf;
        uint2 w;
        w.x = pack_bf16x2(o[db][4 * r4] * inv, o[db][4 * r4 + 1] * inv);
        w.y = pack_bf16x2(o[db][4 * r4 + 2] * inv, o[db][4 * r4 + 3] * inv);
        *(uint2*)(op + d) = w;
      }
  }
}

}  // namespace

hipError_t launch_attention_fwd(const AttnArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)((a.q_len + kBQ - 1) / kBQ), (unsigned)a.heads);
  hipLaunchKernelGGL(attn_fwd_d128, grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace joy
