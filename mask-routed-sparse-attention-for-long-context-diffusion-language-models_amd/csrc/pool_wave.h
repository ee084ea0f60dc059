// Landmark pool of one (chunk, KV head), fused-kernel semantics
// (ops/chunk_attn_pool_gqa_tilelang.py:47-180), chunk_size 64, head_dim 128,
// up to 16 query heads per KV head, from the chunk's 64 key rows already in
// LDS.  Shared by the standalone matrix-core pool (one wave per chunk) and
// the kernel that lays out the K/V fragments and pools in one pass (four
// waves per chunk, one 16-key block each).
//   logits:  S^T = K . Q^T on the matrix cores (A: key rows, B: the query
//            heads as 16 columns, heads >= G zero); block mt, lane (grp, j):
//            keys 16 mt + 4 grp + r of head j; a masked slot gets -inf
//            except slot 0 (logit 0); an invalid chunk masks every slot;
//   softmax and entropy per column: each block's four values of a lane
//            summed as (x0 + x1) + (x2 + x3), then over the four lane groups,
//            and the four blocks as ((b0 + b1) + b2) + b3 -- the same order
//            for one wave and for four, so both give the same bits;
//   pooling: lmk^T = K^T . P^T with P rounded to bf16 and packed in the
//            tiled key order (reduction index 8 grp + e of k-step ks is key
//            32 ks + 16 (e >> 2) + 4 grp + (e & 3): blocks 2 ks and 2 ks + 1);
//            the K^T operand is read from the staged rows in the same order;
//            an invalid chunk writes zero keys and zero entropy.
#pragma once

#include "mrsa_device.h"

namespace mrsa {

// Rows: row16(key, blk) = the 16 bytes of dims 8 blk .. 8 blk + 7 of a key,
// elem(key, dim) = one bf16 of it.  Qb: the query heads' B operands (lane
// (grp, j): head j, dims 32 q4 + 8 grp ..).  real: bit k = key k is valid
// (the landmark slot 63 cleared).
template <class Rows>
__device__ __forceinline__ f32x4_t pool_logits(const Rows& rows, const u32x4_t (&Qb)[4],
                                               uint64_t real, float sm_scale, int mt, int lane) {
  const int j = lane & 15, grp = lane >> 4;
  f32x4_t S = zero4();
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) S = mfma_bf16_16x16x32(rows.row16(16 * mt + j, 4 * q4 + grp), Qb[q4], S);
  const bool chunk_valid = real != 0ull;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int sk = 16 * mt + 4 * grp + r;
    const bool rl = (real >> sk) & 1ull;
    S[r] = (rl && chunk_valid) ? S[r] * sm_scale : (sk == 0 ? 0.f : neg_inf());
  }
  return S;
}

__device__ __forceinline__ float pool_max4(const f32x4_t& x) {
  return fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
}

// x <- exp(x - mx) (0 for -inf); returns the block's column sum.
__device__ __forceinline__ float pool_exp(f32x4_t& x, float mx) {
#pragma unroll
  for (int r = 0; r < 4; ++r)
    x[r] = (mx != neg_inf() && x[r] != neg_inf()) ? exp2f((x[r] - mx) * kLog2e) : 0.f;
  return across4_sum((x[0] + x[1]) + (x[2] + x[3]));
}

// x <- x / sum (0 when sum is 0); returns the block's column sum of p ln p.
__device__ __forceinline__ float pool_prob(f32x4_t& x, float sum) {
  float t[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float pr = sum > 0.f ? x[r] / sum : 0.f;
    t[r] = pr > 0.f ? pr * logf(pr) : 0.f;
    x[r] = pr;
  }
  return across4_sum((t[0] + t[1]) + (t[2] + t[3]));
}

// Landmark dims 16 nt .. 16 nt + 15 of the G heads (rows lrow + 128 j) from
// the P^T operands Pb (k-step ks: blocks 2 ks, 2 ks + 1).
template <class Rows>
__device__ __forceinline__ void pool_lmk(const Rows& rows, const u32x4_t (&Pb)[2], int nt,
                                         bool chunk_valid, int G, uint16_t* __restrict__ lrow,
                                         int lane) {
  const int j = lane & 15, grp = lane >> 4;
  const int dim = 16 * nt + j;
  f32x4_t acc = zero4();
#pragma unroll
  for (int k2 = 0; k2 < 2; ++k2) {
    u32x4_t A;
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      uint32_t pr = 0u;
#pragma unroll
      for (int h1 = 0; h1 < 2; ++h1) {
        const int e = 2 * e2 + h1;
        const int key = 32 * k2 + 16 * (e >> 2) + 4 * grp + (e & 3);
        pr |= rows.elem(key, dim) << (16 * h1);
      }
      A[e2] = pr;
    }
    acc = mfma_bf16_16x16x32(A, Pb[k2], acc);
  }
  // lane (grp, j): dims 16 nt + 4 grp .. + 3 of head j
  if (j < G) {
    u32x2_t ov;
    ov[0] = chunk_valid ? pack_bf16x2(acc[0], acc[1]) : 0u;
    ov[1] = chunk_valid ? pack_bf16x2(acc[2], acc[3]) : 0u;
    *reinterpret_cast<u32x2_t*>(lrow + 128 * j + 16 * nt + 4 * grp) = ov;
  }
}

// Entropy (when `entropy` is given) and prior = entropy x bias_scale (when
// given) of the G heads from the column sum t of p ln p; o = (chunk * H + h)
// * G, bias_scale indexed by hG + head.
__device__ __forceinline__ void pool_stats(float t, bool chunk_valid, int G, int64_t o,
                                           const float* __restrict__ bias_scale, int hG,
                                           float* __restrict__ entropy, float* __restrict__ prior,
                                           int lane) {
  const int j = lane & 15, grp = lane >> 4;
  if (grp == 0 && j < G) {
    const float e_out = chunk_valid ? -t : 0.f;
    if (entropy) entropy[o + j] = e_out;
    if (prior) prior[o + j] = e_out * bias_scale[hG + j];
  }
}

// The whole pool on one wave.  o = (chunk * H + h) * G: the first of the G
// output rows; bias_scale / prior are optional (both or neither), and so is
// entropy.
template <class Rows>
__device__ __forceinline__ void pool_wave(const Rows& rows, const u32x4_t (&Qb)[4], uint64_t real,
                                          int G, float sm_scale, int64_t o,
                                          const float* __restrict__ bias_scale, int hG,
                                          uint16_t* __restrict__ lmk, float* __restrict__ entropy,
                                          float* __restrict__ prior, int lane) {
  const bool chunk_valid = real != 0ull;
  f32x4_t S[4];
  float mx = neg_inf();
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    S[mt] = pool_logits(rows, Qb, real, sm_scale, mt, lane);
    mx = fmaxf(mx, pool_max4(S[mt]));
  }
  mx = across4_max(mx);
  float part[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) part[mt] = pool_exp(S[mt], mx);
  const float sum = ((part[0] + part[1]) + part[2]) + part[3];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) part[mt] = pool_prob(S[mt], sum);
  pool_stats(((part[0] + part[1]) + part[2]) + part[3], chunk_valid, G, o, bias_scale, hG,
             entropy, prior, lane);
  u32x4_t Pb[2];
#pragma unroll
  for (int k2 = 0; k2 < 2; ++k2) {
    Pb[k2][0] = pack_bf16x2(S[2 * k2][0], S[2 * k2][1]);
    Pb[k2][1] = pack_bf16x2(S[2 * k2][2], S[2 * k2][3]);
    Pb[k2][2] = pack_bf16x2(S[2 * k2 + 1][0], S[2 * k2 + 1][1]);
    Pb[k2][3] = pack_bf16x2(S[2 * k2 + 1][2], S[2 * k2 + 1][3]);
  }
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) pool_lmk(rows, Pb, nt, chunk_valid, G, lmk + o * 128, lane);
}

}  // namespace mrsa
