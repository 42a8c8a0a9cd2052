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
// One wave = 32 queries of one head, 8 waves per workgroup (one workgroup per CU), one pass over
// the keys in tiles of 64 (flash attention with an online softmax), each tile as two 32-key
// halves with a softmax step each. Per half and wave:
//   * S^T = K Q^T: 8 v_mfma_f32_32x32x16_bf16 (K from LDS as the A operand, the wave's 32
//     queries kept in registers as the B operand). In the 32x32 output a lane holds 16 keys of
//     ONE query, so the row max / row sum are in-lane plus one exchange with lane ^ 32;
//   * online softmax in fp32 with exp2 (scale * log2 e folded into the scores), computed first
//     against the running max and redone with the half's row max only when a probability could
//     reach 2^7 (the first tile, or scores well above the running max);
//   * O^T += V^T P^T: 8 MFMAs; P^T is the B operand straight from the registers that hold the
//     scores (rounded to bf16), which fixes a permutation of the 16 keys of each MFMA; the A
//     operand (V^T) comes from the key-major V tile with two ds_read_b64_tr_b16 per MFMA, whose
//     addresses apply the same permutation. The O^T accumulator again gives each lane one
//     query, so the rescale by exp2(m_old - m_new) is per lane.
// The two halves are software-pipelined inside the wave: S(0); S(1) with the softmax of half 0
// on the VALU; PV(0) with the softmax of half 1; PV(1). The A operands of the tile's 32 MFMAs
// (K, then the transposed V) are fetched from LDS two MFMAs ahead of their use.
// K and V tiles reach LDS by buffer DMA straight into LDS (double-buffered, the next tile in
// flight during the current one, one barrier per tile); LDS rows of 256 bytes store 16-byte
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
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
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

// Buffer load of 16 bytes per lane (offset voff + soff within the descriptor's range, zeros past
// it) into LDS at m0 = lds_dst (wave-uniform) + lane * 16, as inline asm: the compiler then does
// not track these LDS writes, and the only wait on them is the explicit vmcnt(0) at the top of
// each key tile. (Through the builtin, the compiler cannot tell the transpose reads of the
// current tile from the DMA into the other buffer and waits for the in-flight next tile before
// them.) m0 is written only here in this file, and nothing else in the kernel reads it (checked in
// the generated code): the compiler's warning that a clobber of this reserved register is not
// preserved does not apply.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, int soff, lds_void* lds_dst) {
  const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_dst);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(m), "v"(voff), "s"(rsrc),
               "s"(soff)
               : "m0");
}
#pragma clang diagnostic pop

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

// One query block of 32 queries per wave, 8 waves per workgroup (one workgroup per CU, two waves
// per SIMD): the workgroup's 256 queries share every K / V tile it moves into LDS, half the DMA
// traffic per query of 128-query workgroups (measured 3.5 % faster at the cfg-4 shape). Each
// 64-key tile is processed as two 32-key halves with an online-softmax step each, so that within
// the wave the VALU work of one half overlaps the MFMAs of the other: S(0); S(1) with
// softmax(0); PV(0) with softmax(1); PV(1). A softmax step follows each MFMA in program order
// (sched_barrier keeps it there).
//
// Work split: the query blocks of all heads form one list (head-major, qb_per_head blocks per
// head) and workgroup w takes blocks 8 w .. 8 w + 7, so the grid has ceil(heads * qb_per_head / 8)
// workgroups whatever the query count per head (per-head workgroups would leave a nearly empty
// last round at 11312 queries: 45 x 40 = 1800 = 7.03 rounds of 256 CUs). A workgroup whose blocks
// straddle a head boundary moves the K / V tiles of both heads (LDS holds two heads' tiles);
// qb_per_head >= 8 keeps it to two heads. Blocks past the list (last workgroup) compute on the
// last valid block and store nothing.
constexpr int kWaves = 8;
__global__ __launch_bounds__(64 * kWaves, 1) void attn_fwd_d128(AttnArgs a, int qb_per_head) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][2][2][kTileB];  // [buffer][head slot][K, V]
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int ql = lane & 31, hf = lane >> 5;
  const int64_t Lq = a.q_len, Lk = a.k_len;
  const int nblocks = a.heads * qb_per_head;
  const int blk0 = (int)blockIdx.x * kWaves;
  const int head_lo = blk0 / qb_per_head;
  const int head_hi = (min(blk0 + kWaves, nblocks) - 1) / qb_per_head;  // blk0 < nblocks
  const bool straddle = head_hi != head_lo;
  const int blk = min(blk0 + wave, nblocks - 1);
  const bool active = blk0 + wave < nblocks;
  const int head = blk / qb_per_head;
  const int hslot = head == head_lo ? 0 : 1;
  const int qrow = (blk - head * qb_per_head) * 32 + ql;

  v4i qf[8];
  {
    const uint16_t* qp = a.q.ptr + (int64_t)min((int64_t)qrow, Lq - 1) * a.q.stride_token +
                         (int64_t)head * a.q.stride_head + 8 * hf;
#pragma unroll
    for (int st = 0; st < 8; ++st) qf[st] = *(const v4i*)(qp + 16 * st);
  }

  // K / V tiles by buffer DMA: wave w moves rows 8 w .. 8 w + 7 of each (two DMAs of 4 rows), for
  // the workgroup's first head and, when it straddles a head boundary, its second head.
  // The buffer descriptors are rebuilt per tile, based at the tile's first key and ending after
  // its last key below Lk: rows past Lk load zeros (their scores are -inf), and the offsets stay
  // below 64 rows whatever the sequence length.
  const int64_t ks = a.k.stride_token, vs = a.v.stride_token;
  auto dma_head = [&](int buf, int slot, int h, int64_t k0) {
    const uint16_t* kb = a.k.ptr + (int64_t)h * a.k.stride_head;
    const uint16_t* vb = a.v.ptr + (int64_t)h * a.v.stride_head;
    const int rows = (int)min((int64_t)kBK, Lk - k0);
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(kb + k0 * ks), 0, (int)(((rows - 1) * ks + kD) * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(vb + k0 * vs), 0, (int)(((rows - 1) * vs + kD) * 2), 0x00020000);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = wave * 8 + i * 4 + (lane >> 4);
      dma16_buf(krs, (uint32_t)(row * ks * 2 + ((lane & 15) ^ (row & 15)) * 16), 0,
                (lds_void*)&lds[buf][slot][0][(wave * 8 + i * 4) * kRowB]);
      dma16_buf(vrs, (uint32_t)(row * vs * 2 + ((lane & 15) ^ vsw(row)) * 16), 0,
                (lds_void*)&lds[buf][slot][1][(wave * 8 + i * 4) * kRowB]);
    }
  };
  auto dma_tile = [&](int buf, int64_t k0) {
    dma_head(buf, 0, head_lo, k0);
    if (straddle) dma_head(buf, 1, head_hi, k0);
  };

  const int tg = lane >> 4, ta = lane & 15;
  const int tr_row = 4 * hf + (ta >> 2);
  const int tr_col = 16 * (tg & 1) + 4 * (ta & 3);

  v16f o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = (v16f){};
  float m_run = -INFINITY, l_run = 0.f;
  const float sl2 = a.scale_log2e;

  // Softmax of one 32-key half (16 scores per lane), first against the running max m_run: steps 0-7
  // (one after each MFMA of the phase) compute 2 probabilities each, rounded to a bf16 pair for the
  // PV operand and summed as those bf16 values (v_dot2c_f32_bf16 against (1, 1)), so the row sum
  // normalises exactly the weights the MFMAs apply. The online softmax is exact for any reference
  // point, so the half needs no row max as long as its probabilities stay small: if every lane's sum
  // (16 keys of a query) is below 2^7, every probability is, and the half is done. Else (the first
  // tile, where m_run = -inf, or scores well above m_run) the wave redoes the half against the
  // larger of m_run and its row max (soft_max), and O is rescaled.
  struct Soft {
    float m_new, alpha, rs;
  };
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  // probabilities 2 e and 2 e + 1 against m_ref
  auto probs = [&](int e, const v16f& s, v4i (&pb)[2], float m_ref, float& rs) {
    const float q0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * e], sl2, -m_ref));
    const float q1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * e + 1], sl2, -m_ref));
    const uint32_t pk = pack_bf16x2(q0, q1);
    rs = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pk), one, rs, false);
    pb[e >> 2][e & 3] = (int)pk;
  };
  auto soft_step = [&](int step, const v16f& s, v4i (&pb)[2], Soft& st) {
    if (step == 0) st.rs = 0.f;
    probs(step, s, pb, m_run, st.rs);
  };
  // the same half against max(m_run, row max): its probabilities are then at most 1, and the later
  // halves pass the check unless their scores rise again
  auto soft_max = [&](const v16f& s, v4i (&pb)[2], Soft& st) {
    float m = fmaxf(fmaxf(s[0], s[1]), s[2]);
#pragma unroll
    for (int r = 3; r < 15; r += 2) m = fmaxf(fmaxf(m, s[r]), s[r + 1]);
    const float mt = xor32_max(fmaxf(m, s[15]));
    const float m_cand = mt * sl2;
    st.m_new = fmaxf(m_run, m_cand);
    st.alpha = __builtin_amdgcn_exp2f(m_run - st.m_new);
    st.rs = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) probs(e, s, pb, st.m_new, st.rs);
  };
  auto rescale = [&](float alpha) {
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;
    }
  };
  // Before the half's PV MFMAs: the check, on each lane's 16 keys (a sum below 2^7 there bounds every
  // probability as well), and where it fails the max-based redo and the rescale of O (the rare path,
  // laid out off the fall-through). The row sum over the 32 keys and the running sum follow after the
  // first PV MFMA (soft_sum).
  auto soft_end = [&](const v16f& s, v4i (&pb)[2], Soft& st) {
    st.alpha = 1.0f;
    // false for inf / NaN (m_run = -inf)
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(!(st.rs < 128.0f)) != 0, 0)) {
      soft_max(s, pb, st);
      m_run = st.m_new;
      rescale(st.alpha);
    }
  };
  auto soft_sum = [&](Soft& st) { l_run = l_run * st.alpha + xor32_sum(st.rs); };
  auto k_operand = [&](const uint8_t* kt, int kb, int st) -> v4i {
    return *(const v4i*)(kt + chunk_at(kb * 32 + ql, 2 * st + hf));
  };
  auto pv_operand = [&](const uint8_t* vt, int kb, int n) -> v4i {  // n = 4 b + db
    const int b = n >> 2, db = n & 3;
    const int row0 = kb * 32 + 16 * b + tr_row;
    const int col = db * 32 + tr_col;
    const int chunk = col >> 3, within = (col & 7) * 2;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vt + chunk_at_v(row0, chunk) + within));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vt + chunk_at_v(row0 + 8, chunk) + within));
    return __builtin_bit_cast(v4i, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  const int64_t ntiles = (Lk + kBK - 1) / kBK;
  dma_tile(0, 0);
  auto tile = [&](auto bufc, auto partc, int64_t t) {
    constexpr int buf = decltype(bufc)::value;
    constexpr bool partial = decltype(partc)::value;
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0), lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (t + 1 < ntiles) dma_tile(buf ^ 1, (t + 1) * kBK);
    const uint8_t* kt = lds[buf][hslot][0];
    const uint8_t* vt = lds[buf][hslot][1];
    const int64_t k0 = t * kBK;
    auto mask = [&](v16f& s, int kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t key = k0 + kb * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
        if (key >= Lk) s[r] = -INFINITY;
      }
    };
    v16f s0, s1;
    v4i p0[2], p1[2];
    Soft st0, st1;
    // The tile's 32 MFMAs read one stream of A operands -- K of half 0, K of half 1, V of half 0,
    // V of half 1 -- each fetched from LDS kOperandAhead MFMAs before it is used (one register set
    // per fetch in flight; with the 2 waves per SIMD this hides most of the LDS latency, and at
    // two fetches ahead the kernel still fits 256 registers without spilling).
    constexpr int kOperandAhead = 2;
    constexpr int NB = kOperandAhead + 1;
    v4i ob[NB];
    auto operand = [&](int i) -> v4i {
      if (i < 8) return k_operand(kt, 0, i);
      if (i < 16) return k_operand(kt, 1, i - 8);
      if (i < 24) return pv_operand(vt, 0, i - 16);
      return pv_operand(vt, 1, i - 24);
    };
#pragma unroll
    for (int i = 0; i < NB - 1; ++i) ob[i] = operand(i);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      if (i + NB - 1 < 32) ob[(i + NB - 1) % NB] = operand(i + NB - 1);
      const v4i op = ob[i % NB];
      if (i < 8) {  // S(0)
        s0 = mfma_bf16(as_bf16x8(op), as_bf16x8(qf[i]), i == 0 ? (v16f){} : s0);
      } else if (i < 16) {  // S(1) with softmax(0)
        s1 = mfma_bf16(as_bf16x8(op), as_bf16x8(qf[i - 8]), i == 8 ? (v16f){} : s1);
        __builtin_amdgcn_sched_barrier(0);
        soft_step(i - 8, s0, p0, st0);
      } else if (i < 24) {  // PV(0) with softmax(1)
        o[(i - 16) & 3] = mfma_bf16(as_bf16x8(op), as_bf16x8(p0[(i - 16) >> 2]), o[(i - 16) & 3]);
        __builtin_amdgcn_sched_barrier(0);
        if (i == 16) soft_sum(st0);
        soft_step(i - 16, s1, p1, st1);
      } else {  // PV(1)
        o[(i - 24) & 3] = mfma_bf16(as_bf16x8(op), as_bf16x8(p1[(i - 24) >> 2]), o[(i - 24) & 3]);
        if (i == 24) {
          __builtin_amdgcn_sched_barrier(0);
          soft_sum(st1);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (i == 7) {
        if constexpr (partial) mask(s0, 0);
        __builtin_amdgcn_sched_barrier(0);
      } else if (i == 15) {
        soft_end(s0, p0, st0);
        if constexpr (partial) mask(s1, 1);
        __builtin_amdgcn_sched_barrier(0);
      } else if (i == 23) {
        soft_end(s1, p1, st1);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  const int64_t nfull = Lk / kBK;
  int64_t t = 0;
  for (; t + 2 <= nfull; t += 2) {
    tile(IC<0>{}, std::false_type{}, t);
    tile(IC<1>{}, std::false_type{}, t + 1);
  }
  if (t < nfull) {
    tile(IC<0>{}, std::false_type{}, t);
    ++t;
    if (t < ntiles) tile(IC<1>{}, std::true_type{}, t);
  } else if (t < ntiles) {
    tile(IC<0>{}, std::true_type{}, t);
  }
  __builtin_amdgcn_s_waitcnt(0x0070);

  if (active && qrow < Lq) {
    const float inv = 1.0f / l_run;
    uint16_t* op = a.out + (int64_t)qrow * a.out_stride_token + (int64_t)head * kD;
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

// Tried and dropped (same inputs, cfg-4 joint shape): two query blocks per wave, pipelined inside
// the wave at one wave per SIMD (bit-identical outputs, 9.8 vs 8.2 ms: the scores no longer fit
// the architectural registers and every tile pays accumulator-register copies; rebuilt with two
// waves per workgroup it spills to scratch), and the same kernel without the half-tile split
// (MFMA busy 49 % at 1.94 GHz against 54 % at 1.83 GHz here: the part is power-limited, so the
// better overlap buys 2.6 %). A three-stage K / V ring (next-but-one tile in flight) measured no
// faster than two stages. Two query blocks per wave at one wave per SIMD with the output
// accumulators pinned in a0..a127 by inline asm (no accumulator copies, no spills, bit-identical):
// 3-5 % slower than this kernel -- half the LDS operand reads and a higher clock (2.1 against
// 1.87 GHz), but the single wave's own latencies exposed (MFMA busy 0.47 against 0.55).
hipError_t launch_attention_fwd(const AttnArgs& a, hipStream_t st) {
  // query blocks per head: at least kWaves, so a workgroup spans at most two heads
  const int qb = (int)max((a.q_len + 31) / 32, (int64_t)kWaves);
  const int64_t blocks = (int64_t)a.heads * qb;
  const dim3 grid((unsigned)((blocks + kWaves - 1) / kWaves));
  hipLaunchKernelGGL(attn_fwd_d128, grid, dim3(64 * kWaves), 0, st, a, qb);
  return hipGetLastError();
}

}  // namespace joy
