// Route scoring and per-KV-group top-k chunk selection.
//
// Semantics follow ref_softmax_topk_max_pooling (ops/topk_head_softmax.py:15-156):
//   s[q,g,c]     = (q[q,g] . lmk[c,g]) * sm_scale        (causal-masked -> -inf)
//   x[q,g,c]     = s + bias[c,g]
//   post_softmax: y = x - logaddexp(lse_local[q,g], logsumexp_c x[q,g,:])
//   pre_softmax:  y = x
//   score[q,c]   = max_g y ; dropped chunks -> -inf
//   top-k over c; -inf picks become -1; indices sorted ascending with -1 last;
//   returned scores are s (no bias) at the picked chunks for every g.
// The logsumexp runs over every chunk, dropped ones included.  Ties in the
// selection score go to the lower chunk index (the rule of the reference's
// fused selection kernel, topk_head_softmax.py:614-626).
//
// Fast path (route_topk_fast_kernel): head_dim 128, chunks <= 256, bf16
// scores, 7 or 8 heads per KV group, no workspace.  A workgroup holds 128
// queries of one KV head (16 per wave); pass 1 computes every head's logits
// on the matrix cores and folds them into the running max over heads, the
// K-th largest score of each query is found by bisection on order-preserving
// integer keys (exact ties at the threshold broken by chunk index), and
// pass 2 recomputes the logits for the picks' raw scores.
//
// Short-block path (route_logits_kernel + route_select_kernel, with a caller
// workspace): logits of few query rows against up to 4096 chunks on the
// matrix cores, then one workgroup per (row, KV head) for LSE, scores and
// selection with the keys in registers.
//
// General path (route_topk_generic_kernel): one workgroup per (token, KV head)
// with scalar dot products; any head_dim / chunk count that fits LDS.
#include <mutex>
#include <type_traits>
#include <utility>

#include "block_select.h"
#include "mrsa_device.h"

using namespace mrsa;

namespace {

struct RouteArgs {
  const uint16_t* q;
  const uint16_t* lmk;
  const float* lse;
  const float* bias;
  const int32_t* drop;
  const uint8_t* key_valid;
  int64_t derive_window;
  int64_t B, L, C;
  int Hkv, G, D, K;
  int64_t block_size;
  int per_head_lmk;
  int is_causal;
  int64_t window_size;
  int64_t q_offset;
  int pre_softmax;
  float sm_scale;
  int32_t* indices;
  void* scores;
  int scores_fp32;
  int vec_out;  // K % 32 == 0, indices and scores 16-byte aligned: one 16-byte store per lane
};

__device__ __forceinline__ int64_t floor_div(int64_t a, int64_t b) {
  int64_t q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
  return q;
}

// First chunk index hidden by the causal mask for query row r (global offset applied).
__device__ __forceinline__ int64_t causal_limit(const RouteArgs& a, int64_t r) {
  const int64_t tq = r + a.q_offset;
  if (a.window_size > 0) return floor_div(tq - a.window_size + 1, a.block_size);
  return floor_div(tq, a.block_size);
}

// Whether a chunk has a valid real key: one of its first block_size - 1
// valid bytes (the last slot is the landmark) is set.  Four 16-byte loads
// for 64-key chunks at a 16-byte aligned address.
__device__ __forceinline__ bool chunk_has_valid_key(const uint8_t* kv, int64_t block_size) {
  if (block_size == 64 && ((uintptr_t)kv & 15) == 0) {
    u32x4_t acc = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const u32x4_t x = *reinterpret_cast<const u32x4_t*>(kv + 16 * v);
      acc[0] |= x[0];
      acc[1] |= x[1];
      acc[2] |= x[2];
      acc[3] |= v == 3 ? (x[3] & 0x00ffffffu) : x[3];
    }
    return (acc[0] | acc[1] | acc[2] | acc[3]) != 0u;
  }
  bool any = false;
  for (int64_t t = 0; t < block_size - 1; ++t) any |= kv[t] != 0;
  return any;
}

__device__ __forceinline__ const uint16_t* lmk_row(const RouteArgs& a, int64_t b, int64_t c, int h,
                                                   int g) {
  if (a.per_head_lmk) return a.lmk + ((b * a.C + c) * (int64_t)(a.Hkv * a.G) + h * a.G + g) * a.D;
  return a.lmk + ((b * a.C + c) * (int64_t)a.Hkv + h) * a.D;
}

// ---------------------------------------------------------------------------
// Fast path.
//
// A workgroup takes 128 queries of one KV head, 16 per wave; a wave keeps
// its queries' running max over heads M for all 256 chunks in registers.
// Logits are computed transposed, S^T = lmk . q^T (16 chunks x 16 queries
// per matrix product): lane (j, grp) holds query j's chunks 16 t + 4 grp + i
// (t = 0..15, i = 0..3), so every per-query reduction runs over the four
// lanes sharing j.
//   pass 1, heads 0..G-1: x = s * scale + bias, the head's LSE over all
//           chunks, M = max(M, x - logaddexp(local LSE, LSE));
//   selection: the K-th largest M per query by bisection on order keys
//           (ties at the threshold to the lower chunk), the ascending pick
//           list of each query in LDS;
//   pass 2, heads G-1..0: the raw logits again, rounded to bf16 into the
//           wave's [16][256] LDS tile, gathered at the picks.
// One head's landmark keys sit in LDS while the next head's stream in.
// ---------------------------------------------------------------------------
constexpr int kFastThreads = 512;  // 8 waves x 16 queries
constexpr int kFastQ = 128;        // queries per workgroup
constexpr int kFastMaxTopk = 64;

typedef __attribute__((address_space(3))) void lds_void_t;

// LDS carve-up.  Two landmark buffers ([256][128] bf16, 16-byte parts
// XOR-swizzled: part p of row c at unit 16 c + (p ^ (c & 15))); in pass 2
// the one pass 1 ends off holds the waves' raw-logit tiles.  Two bias rows
// (-inf past C), the chunk flags and the pick lists [128][K] int16.
struct FastLayout {
  static constexpr size_t lmk = 0;                    // [2][256][128] bf16
  static constexpr size_t bias = 2 * 256 * 128 * 2;   // [2][256] f32
  static constexpr size_t cbad = bias + 2 * 256 * 4;  // [256] u8
  static constexpr size_t picks = cbad + 256;         // [128][K] i16
  static size_t total(int K) { return picks + (size_t)kFastQ * K * 2; }
};

__device__ __forceinline__ int across4_sum_i(int v) {
  const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
  const int s = (int)r[0] + (int)r[1];
  const auto q = __builtin_amdgcn_permlane16_swap((uint32_t)s, (uint32_t)s, false, false);
  return (int)q[0] + (int)q[1];
}
__device__ __forceinline__ uint32_t across4_min_u(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  const uint32_t s = min((uint32_t)r[0], (uint32_t)r[1]);
  const auto q = __builtin_amdgcn_permlane16_swap(s, s, false, false);
  return min((uint32_t)q[0], (uint32_t)q[1]);
}
__device__ __forceinline__ uint32_t across4_max_u(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  const uint32_t s = max((uint32_t)r[0], (uint32_t)r[1]);
  const auto q = __builtin_amdgcn_permlane16_swap(s, s, false, false);
  return max((uint32_t)q[0], (uint32_t)q[1]);
}

// Position of chunk 16 t + 4 grp + i among the set bits of a query's four
// per-lane masks (bit 4 t + i of lane group grp'): the bits of all groups in
// tiles before t, of lower groups in tile t, and of lower i in this group.
__device__ __forceinline__ int chunk_rank(const uint64_t (&m)[4], int grp, int t, int i) {
  const uint64_t below = (1ull << (4 * t)) - 1ull;
  int r = 0;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    r += __popcll(m[g] & below);
    const int nib = (int)((m[g] >> (4 * t)) & 15u);
    r += g < grp ? __popc(nib) : (g == grp ? __popc(nib & ((1 << i) - 1)) : 0);
  }
  return r;
}

template <int G>
__global__ void __launch_bounds__(kFastThreads, 1) route_topk_fast_kernel(RouteArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int K = a.K;
  float* bias_s = reinterpret_cast<float*>(smem + FastLayout::bias);
  unsigned char* cbad = smem + FastLayout::cbad;
  int16_t* picks = reinterpret_cast<int16_t*>(smem + FastLayout::picks);
  auto lmk_buf = [&](int i) {
    return reinterpret_cast<uint16_t*>(smem + FastLayout::lmk) + i * 256 * 128;
  };

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int j = lane & 15, grp = lane >> 4;
  const int64_t b = blockIdx.z;
  const int h = blockIdx.y;
  const int64_t L = a.L, C = a.C;
  const int64_t q0 = (int64_t)blockIdx.x * kFastQ;
  const int ql = 16 * wave + j;            // this lane's query within the workgroup
  const int64_t r = q0 + ql;
  const bool rvalid = r < L;
  const int64_t rr = rvalid ? r : L - 1;   // rows past L re-read row L - 1
  const int64_t qrow = ((b * L + rr) * a.Hkv + h) * G;  // (row, head 0) of q, lse

  // Chunks with no valid real key (the last slot of a chunk is its landmark).
  if (a.derive_window >= 0) {
    for (int c = tid; c < 256; c += kFastThreads) {
      bool any = false;
      if (c < C) {
        if (a.key_valid) {
          const uint8_t* kv = a.key_valid + b * L + (int64_t)c * a.block_size;
          if (a.block_size == 64 && ((uintptr_t)kv & 15) == 0) {
            u32x4_t acc = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const u32x4_t x = *reinterpret_cast<const u32x4_t*>(kv + 16 * v);
              acc[0] |= x[0];
              acc[1] |= x[1];
              acc[2] |= x[2];
              acc[3] |= v == 3 ? (x[3] & 0x00ffffffu) : x[3];
            }
            any = (acc[0] | acc[1] | acc[2] | acc[3]) != 0u;
          } else {
            for (int64_t s = 0; s < a.block_size - 1; ++s) any |= kv[s] != 0;
          }
        } else {
          any = a.block_size > 1;
        }
      }
      cbad[c] = !any;
    }
  }

  // Head g's landmark keys into buffer i, instruction k (0..7) of this wave:
  // LDS units (8 wave + k) * 64 + lane = row 4 (8 wave + k) + lane / 16,
  // stored part lane & 15 (global part (lane & 15) ^ (row & 15)).  Rows >= C
  // re-read row C - 1; their logits are masked by the bias row.  The keys
  // of batch b are one buffer (chunk c's head slot s at element c rowlen +
  // 128 s, under 2 GB on this path): the lane's offset is a 24-bit multiply
  // and the head slot rides in the scalar offset.
  const uint32_t rowlen = (uint32_t)(a.per_head_lmk ? a.Hkv * G : a.Hkv) * 128u;
  const __amdgpu_buffer_rsrc_t lrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.lmk + b * C * (int64_t)rowlen), (short)0,
      (int)((uint32_t)C * rowlen * 2u), 0x00020000);
  auto stage_part = [&](int g, int i, int k) {
    const int row = 4 * (8 * wave + k) + (lane >> 4);
    const uint32_t part = (uint32_t)((lane & 15) ^ (row & 15));
    const uint32_t c = (uint32_t)min(row, (int)C - 1);
    const uint32_t slot = a.per_head_lmk ? (uint32_t)(h * G + g) : (uint32_t)h;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(lrs, (lds_void_t*)(lmk_buf(i) + (8 * wave + k) * 512),
                                             16, 2u * (__umul24(c, rowlen) + 8u * part),
                                             256u * slot, 0, 0);
  };
  // Bias of chunk tid for head g (-inf past C), loaded ahead of its LDS write.
  auto bias_of = [&](int g) {
    float v = neg_inf();
    if (tid < C) v = a.bias ? a.bias[((b * C + tid) * a.Hkv + h) * G + g] : 0.f;
    return v;
  };
  // This lane's Q^T operand (query j, dims 32 ks + 8 grp ..) of head g.
  auto load_q = [&](int g, u32x4_t (&Q)[4]) {
    const uint16_t* src = a.q + (qrow + g) * 128 + 8 * grp;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) Q[ks] = *reinterpret_cast<const u32x4_t*>(src + 32 * ks);
  };

  // An explicit drop mask, read before pass 1 while few registers are live,
  // so that its loads are in flight together: bit 4 t + e of this lane's
  // word is chunk 16 t + 4 grp + e (chunks >= C dropped).
  uint64_t dropbits = 0ull;
  if (a.derive_window < 0 && a.drop) {
    const int32_t* drow = a.drop + (b * L + rr) * C;
    if (C == 256 && ((uintptr_t)a.drop & 15) == 0) {
      u32x4_t d[16];
#pragma unroll
      for (int t = 0; t < 16; ++t) d[t] = *reinterpret_cast<const u32x4_t*>(drow + 16 * t + 4 * grp);
#pragma unroll
      for (int t = 0; t < 16; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) dropbits |= (uint64_t)(d[t][e] != 0u) << (4 * t + e);
    } else {
      int32_t d[16][4];
#pragma unroll
      for (int t = 0; t < 16; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) d[t][e] = drow[min(16 * t + 4 * grp + e, (int)C - 1)];
#pragma unroll
      for (int t = 0; t < 16; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          dropbits |= (uint64_t)((16 * t + 4 * grp + e >= C) | (d[t][e] != 0)) << (4 * t + e);
    }
  }

  // ---- pass 1 -------------------------------------------------------------
  float M[16][4];
#pragma unroll
  for (int t = 0; t < 16; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) M[t][e] = neg_inf();
  u32x4_t Qc[4], Qn[4];
  float lse_c = 0.f, lse_n = 0.f;
  load_q(0, Qc);
  if (!a.pre_softmax) lse_c = a.lse[qrow];
#pragma unroll
  for (int k = 0; k < 8; ++k) stage_part(0, 0, k);
  if (tid < 256) bias_s[tid] = bias_of(0);
  for (int g = 0; g < G; ++g) {
    // Head g landed (this wave's DMA; the barrier covers the others') and
    // every wave is done with the other buffer.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const bool more = g + 1 < G;
    float bnext = 0.f;
    if (more) {
      load_q(g + 1, Qn);
      if (!a.pre_softmax) lse_n = a.lse[qrow + g + 1];
      if (tid < 256) bnext = bias_of(g + 1);
    }
    // x = s * scale + bias (bias -inf past C), tile by tile after its
    // products, with the running max for the LSE.
    f32x4_t S[16];
    float mx = neg_inf();
    {
      const uint16_t* lmk_s = lmk_buf(g & 1);
      const float* brow = bias_s + 256 * (g & 1) + 4 * grp;
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        f32x4_t acc = zero4();
        const uint16_t* arow = lmk_s + (16 * t + j) * 128;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const u32x4_t A =
              *reinterpret_cast<const u32x4_t*>(arow + (((4 * ks + grp) ^ j) * 8));
          acc = mfma_bf16_16x16x32(A, Qc[ks], acc);
        }
        if (more && (t & 1)) stage_part(g + 1, (g + 1) & 1, t >> 1);
        const f32x4_t bv = *reinterpret_cast<const f32x4_t*>(brow + 16 * t);
#pragma unroll
        for (int e = 0; e < 4; ++e) S[t][e] = __builtin_fmaf(acc[e], a.sm_scale, bv[e]);
        mx = max3_raw(mx, max_raw(S[t][0], S[t][1]), max_raw(S[t][2], S[t][3]));
      }
    }
    // LSE over all chunks in base 2 with the hardware exp2 / log2.
    const float m2 = across4_max(mx) * kLog2e;
    float sm = 0.f;
    if (m2 != neg_inf()) {
      float p[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 16; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) p[e] += exp2_hw(__builtin_fmaf(S[t][e], kLog2e, -m2));
      sm = (p[0] + p[1]) + (p[2] + p[3]);
    }
    const float s2 = across4_sum(sm);
    const float lse2 = m2 == neg_inf() ? neg_inf() : m2 + log2_hw(s2);
    float tot = 0.f;
    if (!a.pre_softmax) {
      // logaddexp(local LSE, LSE) in base 2, back to natural units.  A -inf
      // total (no visible logit at all) is clamped to -FLT_MAX: finite x - tot
      // then ties at the top like x - (-inf) = +inf would, and -inf stays.
      const float lv2 = lse_c * kLog2e;
      const float hi = fmaxf(lv2, lse2), lo = fminf(lv2, lse2);
      tot = hi == neg_inf() ? -__FLT_MAX__ : (hi + log2_hw(1.f + exp2_hw(lo - hi))) * kLn2;
    }
#pragma unroll
    for (int t = 0; t < 16; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) M[t][e] = max_raw(M[t][e], S[t][e] - tot);
    if (more) {
      if (tid < 256) bias_s[256 * ((g + 1) & 1) + tid] = bnext;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) Qc[ks] = Qn[ks];
      lse_c = lse_n;
    }
  }

  // ---- selection ----------------------------------------------------------
  // Order keys of M (dropped chunks and chunks >= C: -inf).
  const uint32_t kNeg = float_order_key(neg_inf());
  // One uniform branch per drop source; straight-line code per element.
  uint32_t key[16][4];
  if (a.derive_window >= 0) {
    const int lc = (int)(max(rr - a.derive_window, (int64_t)0) / a.block_size);
    const int rc = (int)(min(rr + a.derive_window, L - 1) / a.block_size);
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int c0 = 16 * t + 4 * grp;
      const uint32_t bad4 = *reinterpret_cast<const uint32_t*>(cbad + c0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c = c0 + e;
        const bool dropped =
            (c >= C) | ((c >= lc) & (c <= rc)) | (((bad4 >> (8 * e)) & 0xffu) != 0u);
        key[t][e] = dropped ? kNeg : float_order_key(M[t][e]);
      }
    }
  } else if (a.drop) {
#pragma unroll
    for (int t = 0; t < 16; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        key[t][e] = ((dropbits >> (4 * t + e)) & 1ull) ? kNeg : float_order_key(M[t][e]);
  } else {
#pragma unroll
    for (int t = 0; t < 16; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        key[t][e] = 16 * t + 4 * grp + e >= C ? kNeg : float_order_key(M[t][e]);
  }
  int nfin = 0;
  uint32_t kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
  for (int t = 0; t < 16; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool fin = key[t][e] > kNeg;
      nfin += fin ? 1 : 0;
      kmin = min(kmin, fin ? key[t][e] : 0xffffffffu);
      kmax = max(kmax, key[t][e]);  // -inf keys are below every finite key
    }
  nfin = across4_sum_i(nfin);
  kmin = across4_min_u(kmin);
  kmax = across4_max_u(kmax);
  // Threshold: keys >= thr_hi are picked, plus the first `need` keys equal
  // to thr_tie in chunk order.  The search keeps count(key >= lo) = clo > K
  // and count(key >= hi) = chi < K and stops when a probe counts exactly K
  // (or hi = lo + 1: ties at lo).  Probes interpolate the count linearly in
  // key space; a probe that leaves more than half the interval is followed
  // by a bisection step, so the search never takes more than twice the
  // steps of plain bisection.
  uint32_t thr_hi, thr_tie = 0u, lo = kmin, hi = kmax + 1u;
  int clo = nfin, chi = 0;
  int need = 0;
  bool done = nfin <= K;
  thr_hi = done ? kNeg + 1u : 0u;
  bool bisect = false;
  for (int it = 0; it < 80; ++it) {
    if (!done && hi - lo <= 1u) done = true;
    if (!__any(!done)) break;
    uint32_t mid = lo + ((hi - lo) >> 1);
    if (!done && !bisect) {
      const float f = (float)(clo - K) / (float)(clo - chi);
      const uint32_t step = (uint32_t)((float)(hi - lo) * f);
      mid = min(max(lo + step, lo + 1u), hi - 1u);
    }
    int cnt = 0;
#pragma unroll
    for (int t = 0; t < 16; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) cnt += key[t][e] >= mid ? 1 : 0;
    cnt = across4_sum_i(cnt);
    if (!done) {
      const uint32_t width = hi - lo;
      if (cnt == K) {
        thr_hi = mid;
        done = true;
      } else if (cnt > K) {
        lo = mid;
        clo = cnt;
      } else {
        hi = mid;
        chi = cnt;
      }
      bisect = !bisect && (hi - lo) > (width >> 1);
    }
  }
  if (thr_hi == 0u) {  // hi = lo + 1: keys >= hi, then ties at lo
    thr_hi = hi;
    thr_tie = lo;
    need = K - chi;
  }
  // This lane's picks / ties as bit masks (bit 4 t + e), built per 32-bit half.
  uint32_t ph[2] = {0u, 0u}, th[2] = {0u, 0u};
  const uint32_t tie_key = need > 0 ? thr_tie : 0u;  // key 0 is never finite
#pragma unroll
  for (int t = 0; t < 16; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int bit = (4 * t + e) & 31;
      ph[t >> 3] |= (uint32_t)(key[t][e] >= thr_hi) << bit;
      th[t >> 3] |= (uint32_t)(key[t][e] == tie_key) << bit;
    }
  uint64_t pm = ((uint64_t)ph[1] << 32) | ph[0];
  const uint64_t tm = ((uint64_t)th[1] << 32) | th[0];
  // The four lanes' masks of this query, in lane-group order.
  auto gather4 = [&](uint64_t v, uint64_t (&m)[4]) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int src = j + 16 * g;
      const uint32_t lo32 = (uint32_t)__shfl((int)(uint32_t)v, src, 64);
      const uint32_t hi32 = (uint32_t)__shfl((int)(uint32_t)(v >> 32), src, 64);
      m[g] = ((uint64_t)hi32 << 32) | lo32;
    }
  };
  if (__any(need > 0)) {
    // Ties at the threshold: the first `need` in chunk order.
    uint64_t tall[4];
    gather4(tm, tall);
    uint64_t x = tm;
    while (x) {
      const int p = __builtin_ctzll(x);
      x &= x - 1ull;
      if (chunk_rank(tall, grp, p >> 2, p & 3) < need) pm |= 1ull << p;
    }
  }
  uint64_t pall[4];
  gather4(pm, pall);
  const int total = __popcll(pall[0]) + __popcll(pall[1]) + __popcll(pall[2]) + __popcll(pall[3]);
  int16_t* plist = picks + ql * K;  // this query's ascending pick list
  {
    uint64_t x = pm;
    while (x) {
      const int p = __builtin_ctzll(x);
      x &= x - 1ull;
      plist[chunk_rank(pall, grp, p >> 2, p & 3)] = (int16_t)(16 * (p >> 2) + 4 * grp + (p & 3));
    }
  }
  // The wave's own pick lists are read back below (LDS keeps one wave's
  // operations in order).
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  int32_t* irow = a.indices + ((b * L + r) * a.Hkv + h) * K;
  // Output slots: with vec_out a lane writes the K / 4 consecutive slots
  // s0 .. s0 + K / 4 - 1 of its query (one 16-byte store per 8 scores, per
  // 4 indices), its picks held as int16 pairs in pk; else slots grp + 4 i.
  const bool vec = a.vec_out != 0;
  const int per = K >> 2, nv = K >> 5, s0 = per * grp;
  uint32_t pk[8];
#pragma unroll
  for (int v = 0; v < 2; ++v) {
    u32x4_t x = {0u, 0u, 0u, 0u};
    if (vec && v < nv) x = *reinterpret_cast<const u32x4_t*>(plist + s0 + 8 * v);
#pragma unroll
    for (int e = 0; e < 4; ++e) pk[4 * v + e] = x[e];
  }
  // chunk of this lane's slot s0 + 8 v + e (0 past the picks)
  auto pick_at = [&](int v, int e) {
    const int c = (int)((pk[4 * v + (e >> 1)] >> (16 * (e & 1))) & 0xffffu);
    return s0 + 8 * v + e < total ? c : 0;
  };
  if (rvalid) {
    if (vec) {
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        if (v >= nv) break;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          u32x4_t o;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            o[e] = s0 + 8 * v + 4 * hh + e < total ? (uint32_t)pick_at(v, 4 * hh + e) : 0xffffffffu;
          *reinterpret_cast<u32x4_t*>(irow + s0 + 8 * v + 4 * hh) = o;
        }
      }
    } else {
      for (int s = grp; s < K; s += 4) irow[s] = s < total ? (int32_t)plist[s] : -1;
    }
  }

  // ---- pass 2 -------------------------------------------------------------
  // Raw logits bf16(s * scale) of the picks, heads G-1..0.  Pass 1 left head
  // G-1 in buffer pb; the other buffer holds the waves' tiles: query j's
  // chunk c at j * 256 + 4 ((c >> 2) ^ j) + (c & 3) (8-byte units swizzled
  // by query so a tile write touches distinct banks).
  const int pb = (G - 1) & 1;
  uint16_t* tile = lmk_buf(1 - pb) + wave * 16 * 256;
  uint16_t* sc16 = reinterpret_cast<uint16_t*>(a.scores);
  load_q(G - 1, Qc);
  for (int g = G - 1; g >= 0; --g) {
    if (g < G - 1) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();  // head g landed in buffer pb
    }
    if (g > 0) load_q(g - 1, Qn);
    // S^T tile by tile (S[e] = q_j . lmk[16 t + 4 grp + e]) into the LDS tile.
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      f32x4_t acc = zero4();
      const uint16_t* arow = lmk_buf(pb) + (16 * t + j) * 128;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const u32x4_t A = *reinterpret_cast<const u32x4_t*>(arow + (((4 * ks + grp) ^ j) * 8));
        acc = mfma_bf16_16x16x32(A, Qc[ks], acc);
      }
      u32x2_t w;
      w[0] = pack_bf16x2(acc[0] * a.sm_scale, acc[1] * a.sm_scale);
      w[1] = pack_bf16x2(acc[2] * a.sm_scale, acc[3] * a.sm_scale);
      *reinterpret_cast<u32x2_t*>(tile + j * 256 + 4 * ((4 * t + grp) ^ j)) = w;
    }
    if (g > 0) {
      __syncthreads();  // every wave is done with head g's keys
#pragma unroll
      for (int k = 0; k < 8; ++k) stage_part(g - 1, pb, k);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (rvalid) {
      uint16_t* orow = sc16 + (((b * L + r) * a.Hkv + h) * G + g) * K;
      if (vec) {
#pragma unroll
        for (int v = 0; v < 2; ++v) {
          if (v >= nv) break;
          uint32_t w[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int c = pick_at(v, e);
            const uint32_t x = tile[j * 256 + 4 * ((c >> 2) ^ j) + (c & 3)];
            w[e] = s0 + 8 * v + e < total ? x : 0xff80u;  // -inf past the picks
          }
          u32x4_t o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = w[2 * e] | (w[2 * e + 1] << 16);
          *reinterpret_cast<u32x4_t*>(orow + s0 + 8 * v) = o;
        }
      } else {
        for (int s = grp; s < K; s += 4) {
          uint16_t v = 0xff80u;  // -inf past the picks
          if (s < total) {
            const int c = plist[s];
            v = tile[j * 256 + 4 * ((c >> 2) ^ j) + (c & 3)];
          }
          orow[s] = v;
        }
      }
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) Qc[ks] = Qn[ks];
  }
}

// ---------------------------------------------------------------------------
// General path.
// ---------------------------------------------------------------------------
constexpr int kGenThreads = 256;

__device__ __forceinline__ float block_reduce_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < kGenThreads / 64; ++w) r = fmaxf(r, red[w]);
  return r;
}
__device__ __forceinline__ float block_reduce_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = 0.f;
  for (int w = 0; w < kGenThreads / 64; ++w) r += red[w];
  return r;
}
__device__ __forceinline__ int block_reduce_sum_i(int v, int* red) {
  v = wave_sum_i(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  int r = 0;
  for (int w = 0; w < kGenThreads / 64; ++w) r += red[w];
  return r;
}
// Exclusive prefix sum over the block (thread order), plus the total.
__device__ __forceinline__ int block_exclusive_scan(int v, int* scratch, int* total) {
  const int tid = threadIdx.x;
  __syncthreads();
  scratch[tid] = v;
  __syncthreads();
  for (int o = 1; o < kGenThreads; o <<= 1) {
    const int add = tid >= o ? scratch[tid - o] : 0;
    __syncthreads();
    scratch[tid] += add;
    __syncthreads();
  }
  const int incl = scratch[tid];
  *total = scratch[kGenThreads - 1];
  __syncthreads();
  return incl - v;
}

__global__ void __launch_bounds__(kGenThreads) route_topk_generic_kernel(RouteArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int64_t C = a.C, L = a.L;
  const int G = a.G, D = a.D, K = a.K;
  float* raw = reinterpret_cast<float*>(smem);  // [G][C]
  float* Ms = raw + (int64_t)G * C;             // [C]
  float* qs = Ms + C;                           // [G][D]
  float* tot = qs + G * D;                      // [G]
  float* redf = tot + G;                        // [8]
  int* redi = reinterpret_cast<int*>(redf + 8);  // [8]
  int* scan = redi + 8;                          // [256]

  const int tid = threadIdx.x;
  const int64_t r = blockIdx.x;
  const int h = blockIdx.y;
  const int64_t b = blockIdx.z;
  for (int e = tid; e < G * D; e += kGenThreads) {
    const int g = e / D, d = e - g * D;
    qs[e] = bf16_to_f32(a.q[(((b * L + r) * a.Hkv + h) * G + g) * D + d]);
  }
  __syncthreads();
  const int64_t climit = a.is_causal ? causal_limit(a, r) : C;
  for (int64_t p = tid; p < (int64_t)G * C; p += kGenThreads) {
    const int g = (int)(p / C);
    const int64_t c = p - (int64_t)g * C;
    const uint16_t* kr = lmk_row(a, b, c, h, g);
    const float* qr = qs + g * D;
    float acc = 0.f;
    for (int d = 0; d < D; ++d) acc = fmaf(qr[d], bf16_to_f32(kr[d]), acc);
    float x = acc * a.sm_scale;
    if (c >= climit) x = neg_inf();
    raw[p] = x;
  }
  __syncthreads();
  for (int g = 0; g < G; ++g) {
    float m = neg_inf();
    for (int64_t c = tid; c < C; c += kGenThreads) {
      const float bv = a.bias ? a.bias[((b * C + c) * a.Hkv + h) * G + g] : 0.f;
      m = fmaxf(m, raw[(int64_t)g * C + c] + bv);
    }
    m = block_reduce_max(m, redf);
    float s = 0.f;
    if (m != neg_inf())
      for (int64_t c = tid; c < C; c += kGenThreads) {
        const float bv = a.bias ? a.bias[((b * C + c) * a.Hkv + h) * G + g] : 0.f;
        s += expf(raw[(int64_t)g * C + c] + bv - m);
      }
    s = block_reduce_sum(s, redf);
    if (tid == 0) {
      const float lse_h = (m == neg_inf()) ? m : m + logf(s);
      const float lv = a.pre_softmax ? 0.f : a.lse[((b * L + r) * a.Hkv + h) * G + g];
      tot[g] = a.pre_softmax ? 0.f : logaddexp_f(lv, lse_h);
    }
  }
  __syncthreads();
  int64_t lc = 0, rc = -1;
  if (a.derive_window >= 0) {
    lc = max(r - a.derive_window, (int64_t)0) / a.block_size;
    rc = min(r + a.derive_window, L - 1) / a.block_size;
  }
  for (int64_t c = tid; c < C; c += kGenThreads) {
    float best = neg_inf();
    for (int g = 0; g < G; ++g) {
      const float bv = a.bias ? a.bias[((b * C + c) * a.Hkv + h) * G + g] : 0.f;
      const float xb = raw[(int64_t)g * C + c] + bv;
      best = fmaxf(best, xb == neg_inf() ? xb : xb - tot[g]);
    }
    bool dropped = false;
    if (a.derive_window >= 0) {
      bool any = false;
      if (a.key_valid) {
        const uint8_t* kv = a.key_valid + b * L + c * a.block_size;
        for (int64_t s = 0; s < a.block_size - 1; ++s) any |= kv[s] != 0;
      } else {
        any = a.block_size > 1;
      }
      dropped = (c >= lc && c <= rc) || !any;
    } else if (a.drop) {
      dropped = a.drop[(b * L + r) * C + c] != 0;
    }
    Ms[c] = dropped ? neg_inf() : best;
  }
  __syncthreads();

  // Threshold search on order keys (block-wide counts).
  const uint32_t kNeg = float_order_key(neg_inf());
  int nfin = 0;
  uint32_t kmin = 0xffffffffu, kmax = 0u;
  for (int64_t c = tid; c < C; c += kGenThreads) {
    const uint32_t key = float_order_key(Ms[c]);
    if (key > kNeg) {
      ++nfin;
      kmin = min(kmin, key);
      kmax = max(kmax, key);
    }
  }
  nfin = block_reduce_sum_i(nfin, redi);
  // min / max through float reductions on the key bits is not order-safe;
  // reduce the keys as ints instead.
  {
    int vmin = (int)(kmin ^ 0x80000000u), vmax = (int)(kmax ^ 0x80000000u);
    for (int o = 1; o < 64; o <<= 1) {
      vmin = min(vmin, __shfl_xor(vmin, o, 64));
      vmax = max(vmax, __shfl_xor(vmax, o, 64));
    }
    __syncthreads();
    if ((tid & 63) == 0) {
      redi[tid >> 6] = vmin;
      redi[4 + (tid >> 6)] = vmax;
    }
    __syncthreads();
    for (int w = 1; w < 4; ++w) {
      vmin = min(vmin, redi[w]);
      vmax = max(vmax, redi[4 + w]);
    }
    vmin = min(vmin, redi[0]);
    vmax = max(vmax, redi[4]);
    kmin = (uint32_t)vmin ^ 0x80000000u;
    kmax = (uint32_t)vmax ^ 0x80000000u;
  }
  uint32_t thr_hi, thr_tie = 0u;
  int need = 0;
  if (nfin <= K) {
    thr_hi = kNeg + 1u;
  } else {
    uint32_t lo = kmin, hi = kmax + 1u;
    bool exact = false;
    thr_hi = 0u;
    while (hi - lo > 1u) {
      const uint32_t mid = lo + ((hi - lo) >> 1);
      int cnt = 0;
      for (int64_t c = tid; c < C; c += kGenThreads) cnt += float_order_key(Ms[c]) >= mid ? 1 : 0;
      cnt = block_reduce_sum_i(cnt, redi);
      if (cnt == K) {
        thr_hi = mid;
        exact = true;
        break;
      }
      if (cnt > K) lo = mid; else hi = mid;
    }
    if (!exact) {
      int cnt_hi = 0;
      for (int64_t c = tid; c < C; c += kGenThreads) cnt_hi += float_order_key(Ms[c]) >= hi ? 1 : 0;
      cnt_hi = block_reduce_sum_i(cnt_hi, redi);
      thr_hi = hi;
      thr_tie = lo;
      need = K - cnt_hi;
    }
  }

  // Each thread owns a contiguous chunk range; scan counts for slots / tie ranks.
  const int64_t per = (C + kGenThreads - 1) / kGenThreads;
  const int64_t c0 = tid * per, c1 = min(C, c0 + per);
  int my_ties = 0;
  for (int64_t c = c0; c < c1; ++c) my_ties += (need > 0 && float_order_key(Ms[c]) == thr_tie) ? 1 : 0;
  int total_ties;
  int tie_base = block_exclusive_scan(my_ties, scan, &total_ties);
  int my_picks = 0;
  {
    int tr = tie_base;
    for (int64_t c = c0; c < c1; ++c) {
      const uint32_t key = float_order_key(Ms[c]);
      const bool tie = need > 0 && key == thr_tie;
      const bool pick = key >= thr_hi || (tie && tr < need);
      if (tie) ++tr;
      my_picks += pick ? 1 : 0;
    }
  }
  int total_picks;
  int slot = block_exclusive_scan(my_picks, scan, &total_picks);
  const int64_t row = (b * L + r) * a.Hkv + h;
  {
    int tr = tie_base;
    for (int64_t c = c0; c < c1; ++c) {
      const uint32_t key = float_order_key(Ms[c]);
      const bool tie = need > 0 && key == thr_tie;
      const bool pick = key >= thr_hi || (tie && tr < need);
      if (tie) ++tr;
      if (pick) {
        a.indices[row * K + slot] = (int32_t)c;
        for (int g = 0; g < G; ++g) {
          const float v = raw[(int64_t)g * C + c];
          if (a.scores_fp32)
            reinterpret_cast<float*>(a.scores)[(row * G + g) * K + slot] = v;
          else
            reinterpret_cast<uint16_t*>(a.scores)[(row * G + g) * K + slot] = (uint16_t)f32_to_bf16(v);
        }
        ++slot;
      }
    }
  }
  for (int s = total_picks + tid; s < K; s += kGenThreads) {
    a.indices[row * K + s] = -1;
    for (int g = 0; g < G; ++g) {
      if (a.scores_fp32)
        reinterpret_cast<float*>(a.scores)[(row * G + g) * K + s] = neg_inf();
      else
        reinterpret_cast<uint16_t*>(a.scores)[(row * G + g) * K + s] = 0xff80u;
    }
  }
}

// ---------------------------------------------------------------------------
// Short-block path: few query rows against many chunks (the cached block
// step: 32 rows, thousands of chunks).  Two kernels over a caller-provided
// fp32 workspace raw [B][L][Hkv][G][C] of scaled logits s = (q . lmk) * scale.
// ---------------------------------------------------------------------------
constexpr int kBlkQ = 32;        // query rows per logits workgroup
constexpr int kSelThreads = 512;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kSelMaxPer = 8;    // chunks per selection thread -> C <= 4096

// Logits: one workgroup per (16-chunk tile, 32-row tile, KV head, batch),
// one wave per query head g of the group.  S^T tiles on the matrix cores:
// A = 16 landmark rows, B = 16 query rows, both read straight from global
// memory (each landmark row is used by one wave only), all in one round trip.
__global__ void __launch_bounds__(512) route_logits_kernel(RouteArgs a, float* __restrict__ raw) {
  const int lane = threadIdx.x & 63, col = lane & 15, grp = lane >> 4;
  const int g = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t C = a.C, L = a.L;
  const int G = a.G;
  const int64_t c0 = (int64_t)blockIdx.x * 16;
  const int64_t q0 = (int64_t)blockIdx.y * kBlkQ;
  const int h = (int)(blockIdx.z % a.Hkv);
  const int64_t b = blockIdx.z / a.Hkv;
  const int64_t cl = min(c0 + col, C - 1);  // clamped: loads stay in bounds
  const int64_t qa = q0 + col, qb = q0 + 16 + col;
  const bool va = qa < L, vb = qb < L;
  const uint16_t* kr = lmk_row(a, b, cl, h, g) + 8 * grp;
  const uint16_t* qra = a.q + (((b * L + min(qa, L - 1)) * a.Hkv + h) * G + g) * 128 + 8 * grp;
  const uint16_t* qrb = a.q + (((b * L + min(qb, L - 1)) * a.Hkv + h) * G + g) * 128 + 8 * grp;
  u32x4_t A[4], Ba[4], Bb[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    A[j] = *reinterpret_cast<const u32x4_t*>(kr + 32 * j);
    Ba[j] = *reinterpret_cast<const u32x4_t*>(qra + 32 * j);
    Bb[j] = *reinterpret_cast<const u32x4_t*>(qrb + 32 * j);
  }
  f32x4_t Sa = zero4(), Sb = zero4();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    Sa = mfma_bf16_16x16x32(A[j], Ba[j], Sa);
    Sb = mfma_bf16_16x16x32(A[j], Bb[j], Sb);
  }
  // Sa[i]: chunk c0 + 4 grp + i, row qa (Sb: row qb).
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t c = c0 + 4 * grp + i;
    if (c < C) {
      if (va) raw[(((b * L + qa) * a.Hkv + h) * G + g) * C + c] = Sa[i] * a.sm_scale;
      if (vb) raw[(((b * L + qb) * a.Hkv + h) * G + g) * C + c] = Sb[i] * a.sm_scale;
    }
  }
}

// Block-wide reduction of one value per head (G <= 8) with a single barrier
// (`red` holds kSelWaves x 8 floats and must not be read by a previous
// reduction any more).
template <bool MAX>
__device__ __forceinline__ void block_reduce8(float (&v)[8], int G, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int g = 0; g < 8; ++g)
    if (g < G) v[g] = MAX ? wave_max(v[g]) : wave_sum(v[g]);
  if (lane == 0)
#pragma unroll
    for (int g = 0; g < 8; ++g)
      if (g < G) red[wave * 8 + g] = v[g];
  __syncthreads();
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    if (g >= G) continue;
    float r = red[g];
#pragma unroll
    for (int w = 1; w < kSelWaves; ++w) r = MAX ? fmaxf(r, red[w * 8 + g]) : r + red[w * 8 + g];
    v[g] = r;
  }
}

// The K largest keys of a selection workgroup's row (K <= kTwoLevelMaxK,
// C <= 4096; key[i] of thread tid is chunk tid + 512 i) in two levels with
// one barrier.  Each wave first picks the K largest of its own chunks
// (chunks 512 i + 64 wave + lane: the wave order index 64 i + lane follows
// the chunk order, so its ties go to the lower chunk) and lists them in LDS;
// wave 0 then selects the K largest of the <= 8 K candidates, the ties at
// the threshold going to the lowest chunks, and writes the picks in
// ascending chunk order.  Each chunk of the row's K largest is among its
// wave's K largest, so the result is the one-level selection's.
constexpr int kTwoLevelMaxK = 64;

template <int G>
__device__ void select_two_level(const RouteArgs& a, const uint32_t (&key)[kSelMaxPer], int n,
                                 int64_t row, const float* xr) {
  constexpr int kCand = kSelWaves * kTwoLevelMaxK / 64;  // candidate slots per lane
  __shared__ uint32_t ck_s[kSelWaves * kTwoLevelMaxK];
  __shared__ uint16_t cc_s[kSelWaves * kTwoLevelMaxK];
  __shared__ int cn_s[kSelWaves];
  __shared__ uint32_t cmask[128];  // chunk bit sets (C <= 4096)
  __shared__ uint32_t cpre[128];   // set bits below each word
  const int K = a.K;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint64_t below = (1ull << lane) - 1ull;
  {
    const uint64_t wp = WaveSelect<kSelMaxPer>::run(key, n, K);
    int base = 0;
#pragma unroll
    for (int i = 0; i < kSelMaxPer; ++i) {
      if (i >= n) continue;
      const bool p = (wp >> i) & 1ull;
      const uint64_t bl = __builtin_amdgcn_ballot_w64(p);
      if (p) {
        const int pos = wave * K + base + __builtin_popcountll(bl & below);
        ck_s[pos] = key[i];
        cc_s[pos] = (uint16_t)(tid + kSelThreads * i);
      }
      base += __builtin_popcountll(bl);
    }
    if (lane == 0) cn_s[wave] = base;
  }
  __syncthreads();
  if (wave != 0) return;
  // candidate e = 64 j + lane: entry e - w K of wave w = e / K
  const int n2 = (kSelWaves * K + 63) / 64;
  uint32_t ckey[kCand];
  int cch[kCand];
#pragma unroll
  for (int j = 0; j < kCand; ++j) {
    const int e = 64 * j + lane;
    const int w = e / K;
    const bool ok = j < n2 && w < kSelWaves && e - w * K < cn_s[w < kSelWaves ? w : 0];
    ckey[j] = ok ? ck_s[e] : 0u;
    cch[j] = ok ? (int)cc_s[e] : 0;
  }
  uint32_t thr_hi, thr_tie;
  int need;
  WaveSelect<kCand>::threshold(ckey, n2, K, thr_hi, thr_tie, need);
  // rank[j] = the members of the set below chunk cch[j] (for members), from
  // a chunk bit set in LDS and its per-word prefix counts (this wave only:
  // the LDS runs one wave's operations in order).
  auto ranks = [&](const bool (&in)[kCand], int (&rank)[kCand]) {
    asm volatile("" ::: "memory");
    cmask[lane] = 0u;
    cmask[lane + 64] = 0u;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int j = 0; j < kCand; ++j)
      if (in[j]) atomicOr(&cmask[cch[j] >> 5], 1u << (cch[j] & 31));
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const uint32_t w0 = cmask[2 * lane], w1 = cmask[2 * lane + 1];
    const int cnt = __popc(w0) + __popc(w1);
    int incl = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int t = __shfl_up(incl, o, 64);
      if (lane >= o) incl += t;
    }
    cpre[2 * lane] = (uint32_t)(incl - cnt);
    cpre[2 * lane + 1] = (uint32_t)(incl - cnt + __popc(w0));
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int j = 0; j < kCand; ++j) {
      rank[j] = 0;
      if (in[j]) {
        const int c = cch[j];
        rank[j] = (int)cpre[c >> 5] + __popc(cmask[c >> 5] & ((1u << (c & 31)) - 1u));
      }
    }
  };
  bool pick[kCand];
#pragma unroll
  for (int j = 0; j < kCand; ++j) pick[j] = j < n2 && ckey[j] >= thr_hi;
  if (need > 0) {  // wave-uniform: ties at the threshold to the lowest chunks
    bool tie[kCand];
    int tr[kCand];
#pragma unroll
    for (int j = 0; j < kCand; ++j) tie[j] = j < n2 && ckey[j] == thr_tie;
    ranks(tie, tr);
#pragma unroll
    for (int j = 0; j < kCand; ++j)
      if (tie[j] && tr[j] < need) pick[j] = true;
  }
  int slot[kCand];
  ranks(pick, slot);
  // The picks' chunks to lane slot order through the candidate area (free
  // now), then lane t writes output slot t with all its loads in flight.
  int total = 0;
#pragma unroll
  for (int j = 0; j < kCand; ++j) total += __builtin_popcountll(__builtin_amdgcn_ballot_w64(pick[j]));
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int j = 0; j < kCand; ++j)
    if (pick[j]) cc_s[slot[j]] = (uint16_t)cch[j];
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  if (lane < K) {
    const int t = lane;
    const bool live = t < total;
    const int64_t c = live ? (int64_t)cc_s[t] : 0;
    float v[G];
#pragma unroll
    for (int g = 0; g < G; ++g) v[g] = xr[(int64_t)g * a.C + c];
    a.indices[row * K + t] = live ? (int32_t)c : -1;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (a.scores_fp32)
        reinterpret_cast<float*>(a.scores)[(row * G + g) * K + t] = live ? v[g] : neg_inf();
      else
        reinterpret_cast<uint16_t*>(a.scores)[(row * G + g) * K + t] =
            live ? (uint16_t)f32_to_bf16(v[g]) : (uint16_t)0xff80u;
    }
  }
}

// Selection: one workgroup per (row, KV head, batch); chunk c = tid + 512 i.
// The row's logits and bias are read once into registers.  Same score, LSE,
// drop and tie rules as the general kernel.
template <int G>
__global__ void __launch_bounds__(kSelThreads) route_select_kernel(RouteArgs a,
                                                                   const float* __restrict__ raw) {
  using Select = BlockSelect<kSelThreads, kSelMaxPer>;
  __shared__ float redf[2][kSelWaves * 8];
  __shared__ typename Select::Lds sel;
  const int64_t C = a.C, L = a.L;
  const int K = a.K;
  const int tid = threadIdx.x;
  const int64_t r = blockIdx.x;
  const int h = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int n = (int)((C + kSelThreads - 1) / kSelThreads);  // <= kSelMaxPer
  const int64_t row = (b * L + r) * a.Hkv + h;
  const float* xr = raw + row * (int64_t)G * C;
  const int64_t climit = a.is_causal ? causal_limit(a, r) : C;

  // 1. x = s + bias (-inf past the causal limit or the last chunk).  The
  //    loads are unconditional (slots past the row read chunk 0), with no
  //    branch between them, so that they are all in flight at once: loads
  //    inside per-element branches were each waited for at the branch's end.
  float x[kSelMaxPer][G];
#pragma unroll
  for (int i = 0; i < kSelMaxPer; ++i) {
    const int64_t c = tid + (int64_t)kSelThreads * i;
    const int64_t cc = i < n && c < C ? c : 0;
#pragma unroll
    for (int g = 0; g < G; ++g) x[i][g] = xr[(int64_t)g * C + cc];
  }
  if (a.bias) {
    const float* brow = a.bias + (b * C * a.Hkv + h) * G;  // chunk c at c Hkv G
    const int64_t bstride = (int64_t)a.Hkv * G;
#pragma unroll
    for (int i = 0; i < kSelMaxPer; ++i) {
      const int64_t c = tid + (int64_t)kSelThreads * i;
      const int64_t cc = i < n && c < C ? c : 0;
#pragma unroll
      for (int g = 0; g < G; ++g) x[i][g] += brow[cc * bstride + g];
    }
  }
#pragma unroll
  for (int i = 0; i < kSelMaxPer; ++i) {
    const int64_t c = tid + (int64_t)kSelThreads * i;
    const bool ok = i < n && c < C && c < climit;
#pragma unroll
    for (int g = 0; g < G; ++g) x[i][g] = ok ? x[i][g] : neg_inf();
  }

  // 2. Per-head LSE over every chunk (dropped ones included).
  float m[8], sum[8];
#pragma unroll
  for (int g = 0; g < 8; ++g) {
    m[g] = neg_inf();
    sum[g] = 0.f;
  }
#pragma unroll
  for (int i = 0; i < kSelMaxPer; ++i)
#pragma unroll
    for (int g = 0; g < G; ++g) m[g] = fmaxf(m[g], x[i][g]);
  block_reduce8<true>(m, G, redf[0]);
#pragma unroll
  for (int i = 0; i < kSelMaxPer; ++i)
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (m[g] != neg_inf()) sum[g] += expf(x[i][g] - m[g]);
  block_reduce8<false>(sum, G, redf[1]);
  float tot[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float lse_h = m[g] == neg_inf() ? m[g] : m[g] + logf(sum[g]);
    const float lv = a.pre_softmax ? 0.f : a.lse[row * G + g];
    tot[g] = a.pre_softmax ? 0.f : logaddexp_f(lv, lse_h);
  }

  // 3. Selection keys: max over heads of x - tot, dropped chunks -inf.
  int64_t lc = 0, rc = -1;
  if (a.derive_window >= 0) {
    lc = max(r - a.derive_window, (int64_t)0) / a.block_size;
    rc = min(r + a.derive_window, L - 1) / a.block_size;
  }
  // Drop flags first, one uniform branch per drop source (loads batched as
  // in step 1).
  bool dropped[kSelMaxPer];
  if (a.derive_window >= 0) {
#pragma unroll
    for (int i = 0; i < kSelMaxPer; ++i) {
      const int64_t c = tid + (int64_t)kSelThreads * i;
      const int64_t cc = i < n && c < C ? c : 0;
      bool any = a.block_size > 1;
      if (a.key_valid) any = chunk_has_valid_key(a.key_valid + b * L + cc * a.block_size,
                                                 a.block_size);
      dropped[i] = (c >= lc && c <= rc) || !any;
    }
  } else if (a.drop) {
#pragma unroll
    for (int i = 0; i < kSelMaxPer; ++i) {
      const int64_t c = tid + (int64_t)kSelThreads * i;
      const int64_t cc = i < n && c < C ? c : 0;
      dropped[i] = a.drop[(b * L + r) * C + cc] != 0;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kSelMaxPer; ++i) dropped[i] = false;
  }
  uint32_t key[kSelMaxPer];
#pragma unroll
  for (int i = 0; i < kSelMaxPer; ++i) {
    const int64_t c = tid + (int64_t)kSelThreads * i;
    float best = neg_inf();
#pragma unroll
    for (int g = 0; g < G; ++g) best = fmaxf(best, x[i][g] == neg_inf() ? x[i][g] : x[i][g] - tot[g]);
    // 0 is below every real key: never picked
    key[i] = i < n && c < C ? float_order_key(dropped[i] ? neg_inf() : best) : 0u;
  }

  // 4. The K largest (ties to the lower chunk), in ascending chunk order.
  if (K <= kTwoLevelMaxK) {
    select_two_level<G>(a, key, n, row, xr);
    return;
  }
  bool pick[kSelMaxPer];
  int slot[kSelMaxPer];
  const int slot_base = Select::run(key, n, K, sel, pick, slot);
  // The picks' raw scores, all loaded before any store.
  float sv[kSelMaxPer][G];
#pragma unroll
  for (int i = 0; i < kSelMaxPer; ++i) {
    const int64_t c = tid + (int64_t)kSelThreads * i;
    const int64_t cc = i < n && c < C ? c : 0;
#pragma unroll
    for (int g = 0; g < G; ++g) sv[i][g] = xr[(int64_t)g * C + cc];
  }
#pragma unroll
  for (int i = 0; i < kSelMaxPer; ++i) {
    if (i >= n || !pick[i]) continue;
    const int64_t c = tid + (int64_t)kSelThreads * i;
    a.indices[row * K + slot[i]] = (int32_t)c;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float v = sv[i][g];
      if (a.scores_fp32)
        reinterpret_cast<float*>(a.scores)[(row * G + g) * K + slot[i]] = v;
      else
        reinterpret_cast<uint16_t*>(a.scores)[(row * G + g) * K + slot[i]] = (uint16_t)f32_to_bf16(v);
    }
  }
  for (int t = slot_base + tid; t < K; t += kSelThreads) {
    a.indices[row * K + t] = -1;
    for (int g = 0; g < G; ++g) {
      if (a.scores_fp32)
        reinterpret_cast<float*>(a.scores)[(row * G + g) * K + t] = neg_inf();
      else
        reinterpret_cast<uint16_t*>(a.scores)[(row * G + g) * K + t] = 0xff80u;
    }
  }
}

// Selection with one wave per (row, KV head, batch) and no barrier, for long
// sequences (many rows): chunk c = lane + 64 i, so the wave selection's order
// index is the chunk index and ties still go to the lower chunk.  The head
// LSEs come from one pass with a per-lane online max / sum; the keys are
// formed from the logits held in registers when PER * G <= 128 (C <= 1024 at
// G = 8) and from a second read of the row otherwise.  Same score, LSE, drop
// and tie rules as route_select_kernel.  Global loads are unconditional
// (slots past the row read chunk 0) and issued kB slots at a time with no
// branch between them: loads inside per-slot branches were each waited for
// at the branch's end.  topk <= 64: the picks' chunks pass through the
// wave's LDS row so that lane t writes output slot t.
template <int G, int PER>
__global__ void __launch_bounds__(256) route_select_wave_kernel(RouteArgs a,
                                                                const float* __restrict__ raw) {
  constexpr bool kHold = PER * G <= 128;
  constexpr int kB = kHold ? PER : 8;  // slots per batch of loads
  __shared__ int32_t pick_c[4][64];
  const int64_t C = a.C, L = a.L;
  const int K = a.K;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t r = (int64_t)blockIdx.x * 4 + wv;
  if (r >= L) return;  // wave-uniform
  const int h = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int n = (int)((C + 63) / 64);  // <= PER
  const int64_t row = (b * L + r) * a.Hkv + h;
  const float* xr = raw + row * (int64_t)G * C;
  const int64_t climit = a.is_causal ? causal_limit(a, r) : C;
  const float* bias = a.bias ? a.bias + (b * C * a.Hkv + h) * G : nullptr;  // + c * Hkv * G + g
  const int64_t bstride = (int64_t)a.Hkv * G;

  // x of slots i0 .. i0 + kB - 1: raw + bias, -inf past the row or the
  // causal limit.
  auto load_batch = [&](int i0, float (&v)[kB][G]) {
#pragma unroll
    for (int ii = 0; ii < kB; ++ii) {
      const int64_t c = lane + 64 * (int64_t)(i0 + ii);
      const int64_t cc = i0 + ii < n && c < C ? c : 0;
#pragma unroll
      for (int g = 0; g < G; ++g) v[ii][g] = xr[(int64_t)g * C + cc];
    }
    if (bias) {
#pragma unroll
      for (int ii = 0; ii < kB; ++ii) {
        const int64_t c = lane + 64 * (int64_t)(i0 + ii);
        const int64_t cc = i0 + ii < n && c < C ? c : 0;
#pragma unroll
        for (int g = 0; g < G; ++g) v[ii][g] += bias[cc * bstride + g];
      }
    }
#pragma unroll
    for (int ii = 0; ii < kB; ++ii) {
      const int64_t c = lane + 64 * (int64_t)(i0 + ii);
      const bool ok = i0 + ii < n && c < C && c < climit;
#pragma unroll
      for (int g = 0; g < G; ++g) v[ii][g] = ok ? v[ii][g] : neg_inf();
    }
  };

  float hold[kB][G];
  float m[G], sum[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = neg_inf();
    sum[g] = 0.f;
  }
#pragma unroll
  for (int i0 = 0; i0 < PER; i0 += kB) {
    if (i0 >= n) break;  // uniform
    load_batch(i0, hold);
#pragma unroll
    for (int ii = 0; ii < kB; ++ii)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float v = hold[ii][g];
        if (v > m[g]) {
          sum[g] = (m[g] == neg_inf() ? 0.f : sum[g] * expf(m[g] - v)) + 1.f;
          m[g] = v;
        } else if (v != neg_inf()) {
          sum[g] += expf(v - m[g]);
        }
      }
  }
  float tot[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float mm = wave_max(m[g]);
    const float ss = wave_sum(m[g] == neg_inf() ? 0.f : sum[g] * expf(m[g] - mm));
    const float lse_h = mm == neg_inf() ? mm : mm + logf(ss);
    tot[g] = a.pre_softmax ? 0.f : logaddexp_f(a.lse[row * G + g], lse_h);
  }

  // Drop flags (bit i: slot i), one uniform branch per drop source.
  uint64_t dropbits = 0ull;
  if (a.derive_window >= 0) {
    const int64_t lc = max(r - a.derive_window, (int64_t)0) / a.block_size;
    const int64_t rc = min(r + a.derive_window, L - 1) / a.block_size;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int64_t c = lane + 64 * (int64_t)i;
      const int64_t cc = i < n && c < C ? c : 0;
      bool any = a.block_size > 1;
      if (a.key_valid) any = chunk_has_valid_key(a.key_valid + b * L + cc * a.block_size,
                                                 a.block_size);
      dropbits |= (uint64_t)((c >= lc && c <= rc) || !any) << i;
    }
  } else if (a.drop) {
    const int32_t* drow = a.drop + (b * L + r) * C;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int64_t c = lane + 64 * (int64_t)i;
      dropbits |= (uint64_t)(drow[i < n && c < C ? c : 0] != 0) << i;
    }
  }
  uint32_t key[PER];
#pragma unroll
  for (int i0 = 0; i0 < PER; i0 += kB) {
    if (!kHold && i0 < n) load_batch(i0, hold);  // uniform
#pragma unroll
    for (int ii = 0; ii < kB; ++ii) {
      const int i = i0 + ii;
      const int64_t c = lane + 64 * (int64_t)i;
      float best = neg_inf();
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float x = hold[ii][g];
        best = fmaxf(best, x == neg_inf() ? x : x - tot[g]);
      }
      // 0 is below every real key: never picked
      key[i] = i < n && c < C ? float_order_key(((dropbits >> i) & 1ull) ? neg_inf() : best) : 0u;
    }
  }

  const uint64_t picks = WaveSelect<PER>::run(key, n, K);
  const uint64_t below = (1ull << lane) - 1ull;
  int base = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    if (i >= n) continue;  // uniform
    const bool p = (picks >> i) & 1ull;
    const uint64_t pb = __builtin_amdgcn_ballot_w64(p);
    if (p) pick_c[wv][base + __builtin_popcountll(pb & below)] = (int32_t)(lane + 64 * i);
    base += __builtin_popcountll(pb);
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's LDS row only
  // lane t writes output slot t (K <= 64)
  if (lane < K) {
    const int t = lane;
    const bool live = t < base;
    const int32_t c = live ? pick_c[wv][t] : 0;
    float v[G];
#pragma unroll
    for (int g = 0; g < G; ++g) v[g] = xr[(int64_t)g * C + c];
    a.indices[row * K + t] = live ? c : -1;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (a.scores_fp32)
        reinterpret_cast<float*>(a.scores)[(row * G + g) * K + t] = live ? v[g] : neg_inf();
      else
        reinterpret_cast<uint16_t*>(a.scores)[(row * G + g) * K + t] =
            live ? (uint16_t)f32_to_bf16(v[g]) : (uint16_t)0xff80u;
    }
  }
}

// Rows (token, KV head, batch) above which the wave selection replaces the
// workgroup selection: below it a workgroup per row spreads a short block's
// few rows over more of the chip.
constexpr int64_t kWaveSelectRows = 4096;

template <int G>
int launch_select_wave(const RouteArgs& a, const float* raw, hipStream_t s) {
  dim3 grid((unsigned)((a.L + 3) / 4), (unsigned)a.Hkv, (unsigned)a.B);
  if (a.C <= 1024)
    hipLaunchKernelGGL((route_select_wave_kernel<G, 16>), grid, dim3(256), 0, s, a, raw);
  else
    hipLaunchKernelGGL((route_select_wave_kernel<G, 64>), grid, dim3(256), 0, s, a, raw);
  return mrsa_launch_status();
}

template <int G>
int launch_select(const RouteArgs& a, const float* raw, hipStream_t s) {
  dim3 g2((unsigned)a.L, (unsigned)a.Hkv, (unsigned)a.B);
  hipLaunchKernelGGL(route_select_kernel<G>, g2, dim3(kSelThreads), 0, s, a, raw);
  return mrsa_launch_status();
}

int launch_block(const RouteArgs& a, float* raw, hipStream_t s) {
  dim3 g1((unsigned)((a.C + 15) / 16), (unsigned)((a.L + kBlkQ - 1) / kBlkQ),
          (unsigned)(a.Hkv * a.B));
  hipLaunchKernelGGL(route_logits_kernel, g1, dim3(64 * a.G), 0, s, a, raw);
  int st = mrsa_launch_status();
  if (st != MRSA_OK) return st;
  if (a.B * a.L * a.Hkv >= kWaveSelectRows && a.C <= 4096 && a.K <= 64 &&
      a.L <= 0x7ffffffc) {
    if (a.G == 7) return launch_select_wave<7>(a, raw, s);
    if (a.G == 8) return launch_select_wave<8>(a, raw, s);
  }
  switch (a.G) {
    case 1: return launch_select<1>(a, raw, s);
    case 2: return launch_select<2>(a, raw, s);
    case 3: return launch_select<3>(a, raw, s);
    case 4: return launch_select<4>(a, raw, s);
    case 5: return launch_select<5>(a, raw, s);
    case 6: return launch_select<6>(a, raw, s);
    case 7: return launch_select<7>(a, raw, s);
    default: return launch_select<8>(a, raw, s);
  }
}

// raw_ws: bf16 [B][L][Hkv][G][C] raw-score workspace (one pass), or null
// (a second pass recomputes the picks' raw scores).
template <int G>
int launch_fast(const RouteArgs& a, hipStream_t s) {
  const size_t smem = FastLayout::total(a.K);
  auto kern = route_topk_fast_kernel<G>;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess)
    return MRSA_ERR_LAUNCH;
  dim3 grid((unsigned)((a.L + kFastQ - 1) / kFastQ), (unsigned)a.Hkv, (unsigned)a.B);
  hipLaunchKernelGGL(kern, grid, dim3(kFastThreads), smem, s, a);
  return mrsa_launch_status();
}

}  // namespace

namespace {

// The one-pass matrix-core kernel (no workspace) serves the call.  Shared by
// the dispatcher and the no-allocation entry point, which must agree on
// which problems need the workspace.
bool fast_path(const void* q, const void* lmk, int64_t chunks, int64_t kv_heads, int64_t groups,
               int64_t head_dim, int64_t topk, int is_causal, int scores_fp32) {
  const bool aligned = ((uintptr_t)q % 16 == 0) && ((uintptr_t)lmk % 16 == 0);
  // (a batch's landmark keys, read through one buffer resource, stay under 2 GB)
  return !scores_fp32 && !is_causal && head_dim == 128 && chunks <= 256 &&
         topk <= kFastMaxTopk && aligned && (groups == 7 || groups == 8) &&
         chunks * kv_heads * groups * head_dim * 2 < ((int64_t)1 << 31);
}

int route_topk_dispatch(const void* q, const void* lmk, const float* lse_local, const float* bias,
                        const int32_t* drop_mask, const uint8_t* key_valid,
                        int64_t derive_window, int64_t batch, int64_t seq_len, int64_t chunks,
                        int64_t kv_heads, int64_t groups, int64_t head_dim, int64_t topk,
                        int64_t block_size, int per_head_lmk, int is_causal,
                        int64_t window_size, int64_t q_offset, int selection_mode,
                        float sm_scale, int32_t* indices, void* scores, int scores_fp32,
                        void* workspace, int64_t workspace_bytes, void* stream) {
  if (batch < 0 || seq_len < 0 || chunks <= 0 || kv_heads <= 0 || groups <= 0 ||
      head_dim <= 0 || topk <= 0 || block_size <= 0 || (selection_mode != 0 && selection_mode != 1))
    return MRSA_ERR_INVALID_ARGUMENT;
  if (batch == 0 || seq_len == 0) return MRSA_OK;
  if (!q || !lmk || !indices || !scores) return MRSA_ERR_INVALID_ARGUMENT;
  if (selection_mode == 0 && !lse_local) return MRSA_ERR_INVALID_ARGUMENT;
  if (derive_window >= 0 && chunks * block_size != seq_len) return MRSA_ERR_INVALID_ARGUMENT;
  if (kv_heads > 65535 || batch > 65535) return MRSA_ERR_UNSUPPORTED;

  RouteArgs a;
  a.q = (const uint16_t*)q;
  a.lmk = (const uint16_t*)lmk;
  a.lse = lse_local;
  a.bias = bias;
  a.drop = drop_mask;
  a.key_valid = key_valid;
  a.derive_window = derive_window;
  a.B = batch;
  a.L = seq_len;
  a.C = chunks;
  a.Hkv = (int)kv_heads;
  a.G = (int)groups;
  a.D = (int)head_dim;
  a.K = (int)topk;
  a.block_size = block_size;
  a.per_head_lmk = per_head_lmk;
  a.is_causal = is_causal;
  a.window_size = window_size;
  a.q_offset = q_offset;
  a.pre_softmax = selection_mode;
  a.sm_scale = sm_scale;
  a.indices = indices;
  a.scores = scores;
  a.scores_fp32 = scores_fp32;
  a.vec_out = topk % 32 == 0 && (uintptr_t)indices % 16 == 0 && (uintptr_t)scores % 16 == 0;
  hipStream_t s = (hipStream_t)stream;

  const bool aligned = ((uintptr_t)q % 16 == 0) && ((uintptr_t)lmk % 16 == 0);
  if (fast_path(q, lmk, chunks, kv_heads, groups, head_dim, topk, is_causal, scores_fp32)) return groups == 7 ? launch_fast<7>(a, s) : launch_fast<8>(a, s);
  const bool block = workspace && head_dim == 128 && groups <= 8 && aligned &&
                     chunks <= (int64_t)kSelThreads * kSelMaxPer && seq_len <= 0x7fffffff &&
                     (uintptr_t)workspace % 16 == 0 &&
                     workspace_bytes >= batch * seq_len * kv_heads * groups * chunks * 4;
  if (block) return launch_block(a, (float*)workspace, s);
  const size_t smem = ((size_t)groups * chunks + chunks + groups * head_dim + groups + 16) * 4 +
                      kGenThreads * 4;
  if (smem > 150 * 1024) return MRSA_ERR_UNSUPPORTED;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(&route_topk_generic_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess)
    return MRSA_ERR_LAUNCH;
  if (seq_len > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  dim3 grid((unsigned)seq_len, (unsigned)kv_heads, (unsigned)batch);
  hipLaunchKernelGGL(route_topk_generic_kernel, grid, dim3(kGenThreads), smem, s, a);
  return mrsa_launch_status();
}

}  // namespace

extern "C" int mrsa_route_topk_fwd(const void* q, const void* lmk, const float* lse_local,
                                   const float* bias, const int32_t* drop_mask,
                                   const uint8_t* key_valid, int64_t derive_window, int64_t batch,
                                   int64_t seq_len, int64_t chunks, int64_t kv_heads,
                                   int64_t groups, int64_t head_dim, int64_t topk,
                                   int64_t block_size, int per_head_lmk, int is_causal,
                                   int64_t window_size, int64_t q_offset, int selection_mode,
                                   float sm_scale, int32_t* indices, void* scores,
                                   int scores_fp32, void* stream) {
  return route_topk_dispatch(q, lmk, lse_local, bias, drop_mask, key_valid, derive_window, batch,
                             seq_len, chunks, kv_heads, groups, head_dim, topk, block_size,
                             per_head_lmk, is_causal, window_size, q_offset, selection_mode,
                             sm_scale, indices, scores, scores_fp32, nullptr, 0, stream);
}

extern "C" int64_t mrsa_route_topk_workspace_bytes(int64_t batch, int64_t seq_len, int64_t chunks,
                                                   int64_t kv_heads, int64_t groups) {
  if (batch < 0 || seq_len < 0 || chunks < 0 || kv_heads < 0 || groups < 0) return -1;
  return batch * seq_len * kv_heads * groups * chunks * 4;
}

// ---------------------------------------------------------------------------
// No-allocation variant: the workspace is a file-scope device array.
//
// `scratch` is one fixed buffer per GPU (each device holds its own copy for
// the life of the process).  Host code never passes the array's name to a
// kernel: its device address is looked up once per device with
// hipGetSymbolAddress (with that device current) and kept in scratch_ptr.
// Every call on one GPU shares the buffer, so calls that overlap on one GPU
// (two streams, two threads) race; the kernels write every byte they later
// read, so nothing needs clearing between calls.
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint8_t scratch[MRSA_ROUTE_TOPK_SCRATCH_BYTES];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// The current device's address of `scratch` (looked up on first use).
int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return MRSA_ERR_LAUNCH;
  if (dev < 0 || dev >= kMaxScratchDevices) return MRSA_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr)
      return MRSA_ERR_LAUNCH;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MRSA_OK;
}
}  // namespace

extern "C" int mrsa_route_topk_noalloc_fwd(
    const void* q, const void* lmk, const float* lse_local, const float* bias,
    const int32_t* drop_mask, const uint8_t* key_valid, int64_t derive_window, int64_t batch,
    int64_t seq_len, int64_t chunks, int64_t kv_heads, int64_t groups, int64_t head_dim,
    int64_t topk, int64_t block_size, int per_head_lmk, int is_causal, int64_t window_size,
    int64_t q_offset, int selection_mode, float sm_scale, int32_t* indices, void* scores,
    int scores_fp32, void* stream) {
  if (batch < 0 || seq_len < 0 || chunks <= 0 || kv_heads <= 0 || groups <= 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  // Workspace the workspace entry point takes for this problem: the fp32
  // logits [batch, seq_len, kv_heads, groups, chunks] of the short-block path.
  // The one-pass matrix-core path runs without one (the dispatcher's own
  // test decides).  A problem that needs more than the static buffer is
  // rejected.
  const int64_t need = fast_path(q, lmk, chunks, kv_heads, groups, head_dim, topk, is_causal, scores_fp32)
                           ? 0
                           : batch * seq_len * kv_heads * groups * chunks * 4;
  if (need > (int64_t)MRSA_ROUTE_TOPK_SCRATCH_BYTES) return MRSA_ERR_SCRATCH;
  void* ws = nullptr;
  if (need > 0) {
    const int st = scratch_address(&ws);
    if (st != MRSA_OK) return st;
  }
  return route_topk_dispatch(q, lmk, lse_local, bias, drop_mask, key_valid, derive_window, batch,
                             seq_len, chunks, kv_heads, groups, head_dim, topk, block_size,
                             per_head_lmk, is_causal, window_size, q_offset, selection_mode,
                             sm_scale, indices, scores, scores_fp32, ws, need, stream);
}

extern "C" int mrsa_route_topk_ws_fwd(const void* q, const void* lmk, const float* lse_local,
                                      const float* bias, const int32_t* drop_mask,
                                      const uint8_t* key_valid, int64_t derive_window,
                                      int64_t batch, int64_t seq_len, int64_t chunks,
                                      int64_t kv_heads, int64_t groups, int64_t head_dim,
                                      int64_t topk, int64_t block_size, int per_head_lmk,
                                      int is_causal, int64_t window_size, int64_t q_offset,
                                      int selection_mode, float sm_scale, int32_t* indices,
                                      void* scores, int scores_fp32, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace)) return MRSA_ERR_INVALID_ARGUMENT;
  return route_topk_dispatch(q, lmk, lse_local, bias, drop_mask, key_valid, derive_window, batch,
                             seq_len, chunks, kv_heads, groups, head_dim, topk, block_size,
                             per_head_lmk, is_causal, window_size, q_offset, selection_mode,
                             sm_scale, indices, scores, scores_fp32, workspace, workspace_bytes,
                             stream);
}
