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
// Fast path (route_topk_mfma_kernel): head_dim 128, chunks <= 256, bf16
// scores.  A workgroup holds 64 queries of one KV head (16 per wave).  For
// each query head g the landmark keys of that head are staged in LDS and the
// 16x256 logit tile of every wave is computed on the matrix cores, reduced to
// the head's LSE and folded into the running max over heads.  The logits of
// The 32nd-largest score of each row is found by bisection on
// order-preserving integer keys; exact ties at the threshold are broken by
// chunk index.  The returned raw scores of the picks come either from a
// second pass that recomputes every head's logits, or (with a caller
// workspace) from the bf16 raw scores pass 1 writes to HBM, gathered back at
// the picks after the selection.
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

__device__ __forceinline__ const uint16_t* lmk_row(const RouteArgs& a, int64_t b, int64_t c, int h,
                                                   int g) {
  if (a.per_head_lmk) return a.lmk + ((b * a.C + c) * (int64_t)(a.Hkv * a.G) + h * a.G + g) * a.D;
  return a.lmk + ((b * a.C + c) * (int64_t)a.Hkv + h) * a.D;
}

// ---------------------------------------------------------------------------
// Fast path.
// ---------------------------------------------------------------------------
constexpr int kFastThreads = 512;  // 8 waves: 4 query groups x 2 chunk halves
constexpr int kFastQ = 64;         // queries per workgroup
constexpr int kNT = 8;             // chunk tiles of 16 per wave (128 chunks)
constexpr int kFastMaxTopk = 64;

typedef __attribute__((address_space(3))) void lds_void_t;

// LDS carve-up.  Two buffers of one head's landmark keys ([256][128] bf16,
// 16-byte parts XOR-swizzled: part p of row c at unit c*16 + (p ^ (c & 15)))
// and two of its bias row alternate, so the next head streams in while the
// current one is computed.  The selection scores ([64][256] f32) reuse the
// buffer of the last first-pass head.
struct FastLayout {
  static constexpr size_t lmk = 0;                      // [2][256][128] bf16
  static constexpr size_t bias = 2 * 256 * 128 * 2;     // [2][256] f32
  static constexpr size_t cbad = bias + 2 * 256 * 4;    // [256] u8
  static constexpr size_t red_max = cbad + 256;         // [2][64] f32
  static constexpr size_t red_sum = red_max + 2 * 64 * 4;
  static constexpr size_t lse = red_sum + 2 * 64 * 4;  // [2][64] f32 local LSE rows
  static constexpr size_t slot = lse + 2 * 64 * 4;      // [64][256] i8
  static constexpr size_t ntot = slot + 64 * 256;        // [64] i32 picks per row
  static constexpr size_t sc = ntot + 64 * 4;            // [64][K] bf16, one head's picks
  static size_t total(int K) { return sc + (size_t)64 * K * 2; }
};

// Selection of the fast path.  The max-over-heads scores M go to LDS
// (row-major [64][256] f32, in the landmark buffer `ms_buf`), then wave w
// selects rows 8w..8w+7 with eight lanes per row, each lane owning the 32
// consecutive chunks 32*sub .. 32*sub+31: bisection on order-preserving keys
// for the K-th largest score, exact ties at the threshold broken toward the
// lower chunk index.  Writes the slot table (chunk -> list position or -1)
// the indices, the picks' chunks in list order (pick_s [64][K], when not
// null) and the per-row pick counts; slots past the picks get index -1
// (their scores are written as -inf by the emission of the scores).
template <int G>
__device__ __forceinline__ void select_step(const RouteArgs& a, const float (&M)[kNT][4],
                                            uint16_t* ms_buf, const unsigned char* cbad,
                                            int8_t* slot_s, int* ntot_s, int16_t* pick_s,
                                            int64_t q0, int64_t qbase, int64_t L,
                                            int64_t C, int h, int64_t b, int lane, int wave,
                                            int col, int grp, int qg, int cbase) {
  const int K = a.K;
  float* Ms = reinterpret_cast<float*>(ms_buf);
  __syncthreads();  // every wave is done with the landmark keys in ms_buf
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t r = qbase + 4 * grp + i;
    int64_t lc = 0, rc = -1;
    if (a.derive_window >= 0 && r < L) {
      lc = max(r - a.derive_window, (int64_t)0) / a.block_size;
      rc = min(r + a.derive_window, L - 1) / a.block_size;
    }
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
      const int c = cbase + 16 * t + col;
      bool dropped = (c >= C) || (r >= L);
      if (!dropped) {
        if (a.derive_window >= 0)
          dropped = (c >= lc && c <= rc) || cbad[c];
        else if (a.drop)
          dropped = a.drop[(b * L + r) * C + c] != 0;
      }
      Ms[(16 * qg + 4 * grp + i) * 256 + c] = dropped ? neg_inf() : M[t][i];
    }
  }
  __syncthreads();

  const int row = 8 * wave + (lane >> 3);
  const int sub = lane & 7;
  const int64_t r = q0 + row;
  uint32_t key[32];
#pragma unroll
  for (int e = 0; e < 32; e += 4) {
    const f32x4_t v = *reinterpret_cast<const f32x4_t*>(Ms + row * 256 + 32 * sub + e);
#pragma unroll
    for (int u = 0; u < 4; ++u) key[e + u] = float_order_key(v[u]);
  }
  const uint32_t kNeg = float_order_key(neg_inf());
  int nfin = 0;
  uint32_t kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
  for (int e = 0; e < 32; ++e)
    if (key[e] > kNeg) {
      ++nfin;
      kmin = min(kmin, key[e]);
      kmax = max(kmax, key[e]);
    }
  nfin = group8_sum_i(nfin);
  kmin = group8_min_u(kmin);
  kmax = group8_max_u(kmax);
  uint32_t thr_hi, thr_tie = 0u, lo = kmin, hi = kmax + 1u;
  int need = 0;
  bool done;
  if (nfin <= K) {
    thr_hi = kNeg + 1u;
    done = true;
  } else {
    thr_hi = 0u;
    done = false;
  }
  for (int it = 0; it < 40; ++it) {
    if (!__any(!done)) break;
    const uint32_t mid = lo + ((hi - lo) >> 1);
    int cnt = 0;
#pragma unroll
    for (int e = 0; e < 32; ++e) cnt += key[e] >= mid ? 1 : 0;
    cnt = group8_sum_i(cnt);
    if (!done) {
      if (hi - lo <= 1u) {
        done = true;
      } else if (cnt == K) {
        thr_hi = mid;
        done = true;
      } else if (cnt > K) {
        lo = mid;
      } else {
        hi = mid;
      }
    }
  }
  if (thr_hi == 0u) {
    int cnt_hi = 0;
#pragma unroll
    for (int e = 0; e < 32; ++e) cnt_hi += key[e] >= hi ? 1 : 0;
    cnt_hi = group8_sum_i(cnt_hi);
    thr_hi = hi;
    thr_tie = lo;
    need = K - cnt_hi;
  }
  // Exclusive prefix over the 8 lanes of the row (chunk order == lane order).
  auto excl8 = [&](int v) { return group8_excl_scan_i(v, sub); };
  int my_ties = 0;
#pragma unroll
  for (int e = 0; e < 32; ++e) my_ties += (need > 0 && key[e] == thr_tie) ? 1 : 0;
  int tie_rank = excl8(my_ties);
  int my_picks = 0;
  uint32_t pickbits = 0u;
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    const bool tie = need > 0 && key[e] == thr_tie;
    const bool pick = key[e] >= thr_hi || (tie && tie_rank < need);
    if (tie) ++tie_rank;
    if (pick) {
      pickbits |= 1u << e;
      ++my_picks;
    }
  }
  int slot = excl8(my_picks);
  int total = my_picks;
  total = group8_sum_i(total);
  const int64_t orow = (b * L + r) * a.Hkv + h;
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    const bool pick = (pickbits >> e) & 1u;
    slot_s[row * 256 + 32 * sub + e] = pick ? (int8_t)slot : (int8_t)-1;
    if (pick && r < L) a.indices[orow * K + slot] = 32 * sub + e;
    if (pick_s && pick) pick_s[row * K + slot] = (int16_t)(32 * sub + e);
    slot += pick ? 1 : 0;
  }
  if (r < L)
    for (int s = total + sub; s < K; s += 8) a.indices[orow * K + s] = -1;
  if (sub == 0) ntot_s[row] = total;
}

template <int G, bool WS>
__global__ void __launch_bounds__(kFastThreads, 1) route_topk_mfma_kernel(RouteArgs a,
                                                                         uint16_t* __restrict__ raw_ws) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int K = a.K;
  float* bias_s = reinterpret_cast<float*>(smem + FastLayout::bias);
  unsigned char* cbad = smem + FastLayout::cbad;
  float* red_max = reinterpret_cast<float*>(smem + FastLayout::red_max);
  float* red_sum = reinterpret_cast<float*>(smem + FastLayout::red_sum);
  float* lse_s = reinterpret_cast<float*>(smem + FastLayout::lse);
  int8_t* slot_s = reinterpret_cast<int8_t*>(smem + FastLayout::slot);
  int* ntot_s = reinterpret_cast<int*>(smem + FastLayout::ntot);
  uint16_t* sc_s = reinterpret_cast<uint16_t*>(smem + FastLayout::sc);
  auto lmk_buf = [&](int i) { return reinterpret_cast<uint16_t*>(smem + FastLayout::lmk) + i * 256 * 128; };

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int qg = wave & 3, half = wave >> 2;
  const int64_t b = blockIdx.z;
  const int h = blockIdx.y;
  const int64_t q0 = (int64_t)blockIdx.x * kFastQ;
  const int64_t qbase = q0 + 16 * qg;
  const int64_t qa = qbase + col;  // the A-operand row this lane supplies
  const int64_t L = a.L, C = a.C;
  const int cbase = 128 * half;
  const uint16_t* qb_base = a.q + b * L * (int64_t)(a.Hkv * G * 128);
  const float* lse_base = a.pre_softmax ? nullptr : a.lse + b * L * (int64_t)(a.Hkv * G);
  uint16_t* sc16 = reinterpret_cast<uint16_t*>(a.scores);

  if (a.derive_window >= 0) {
    for (int c = tid; c < 256; c += kFastThreads) {
      bool any = false;
      if (c < C) {
        if (a.key_valid) {
          const uint8_t* kv = a.key_valid + b * L + (int64_t)c * a.block_size;
          for (int64_t s = 0; s < a.block_size - 1; ++s) any |= kv[s] != 0;
        } else {
          any = a.block_size > 1;
        }
      }
      cbad[c] = !any;
    }
  }
  if (!a.bias)
    for (int e = tid; e < 512; e += kFastThreads) bias_s[e] = 0.f;

  // The walk is 2G steps: pass 1 over heads 0..G-1 (biased logits, LSE,
  // running max), then the selection, then pass 2 over heads G-1..0 (raw
  // logits of the picks).  Step s computes from buffer s & 1.
  auto head_of = [&](int s) { return s < G ? s : 2 * G - 1 - s; };
  // Global->LDS DMA of head g's landmark keys into buffer i: wave w,
  // instruction j moves units (8w + j) * 64 + lane = row 4(8w + j) + lane / 16,
  // stored part lane & 15 (global part (lane & 15) ^ (row & 15)).  Rows >= C
  // re-read row C - 1; their logits are masked to -inf.  Wave 0 also moves
  // the bias row (4-byte units, rows >= C re-read row C - 1 and are unused).
  // Instruction j (0..7) of the staging of head g into buffer i; j = 0
  // also moves the local LSE rows (wave 1) and the bias row (wave 0).
  auto stage_part = [&](int g, int i, int j, bool with_lse) {
    uint16_t* dst = lmk_buf(i);
    if (j == 0 && with_lse && lse_base && wave == 1) {
      // Local LSE of the tile's 64 rows for head g (rows >= L re-read L - 1).
      const int64_t r = min(q0 + lane, L - 1);
      __builtin_amdgcn_global_load_lds(lse_base + (r * a.Hkv + h) * G + g,
                                       (lds_void_t*)(lse_s + 64 * i), 4, 0, 0);
    }
    const int row = 4 * (8 * wave + j) + (lane >> 4);
    const int part = (lane & 15) ^ (row & 15);
    const int64_t c = min((int64_t)row, C - 1);
    __builtin_amdgcn_global_load_lds(lmk_row(a, b, c, h, g) + part * 8,
                                     (lds_void_t*)(dst + (8 * wave + j) * 512), 16, 0, 0);
    if (j == 0 && a.bias && wave == 0) {
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        const int64_t cb = min((int64_t)(64 * jb + lane), C - 1);
        __builtin_amdgcn_global_load_lds(a.bias + ((b * C + cb) * a.Hkv + h) * G + g,
                                         (lds_void_t*)(bias_s + 256 * i + 64 * jb), 4, 0, 0);
      }
    }
  };
  auto stage = [&](int g, int i, bool with_lse) {
#pragma unroll
    for (int j = 0; j < 8; ++j) stage_part(g, i, j, with_lse);
  };
  auto load_q = [&](int g, u32x4_t (&A)[4]) {
    const uint16_t* qrow = qb_base + (uint32_t)((((int)qa * a.Hkv + h) * G + g) * 128 + 8 * grp);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4_t z = {0u, 0u, 0u, 0u};
      A[j] = z;
      if (qa < L) A[j] = *reinterpret_cast<const u32x4_t*>(qrow + 32 * j);
    }
  };
  // S[t] = q_g (16 queries of this wave) . lmk (16 chunks of tile t).
  // The next head's staging is issued one instruction per tile, between the
  // products, so no wave stalls on a burst of DMA issue.
  // S[t] = q (16 rows) . lmk (16 chunks of tile t); with TRANSPOSED the same
  // operands give S^T: lane l holds query l % 16, chunks 16t + 4(l / 16) + i.
  auto logits = [&](auto transposed, const uint16_t* lmk_s, const u32x4_t (&A)[4],
                    f32x4_t (&S)[kNT], int next_g, int next_buf, bool with_lse) {
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
      f32x4_t acc = zero4();
      const uint16_t* brow = lmk_s + (cbase + 16 * t + col) * 128;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4_t B = *reinterpret_cast<const u32x4_t*>(brow + (((4 * j + grp) ^ col) * 8));
        if constexpr (decltype(transposed)::value)
          acc = mfma_bf16_16x16x32(B, A[j], acc);
        else
          acc = mfma_bf16_16x16x32(A[j], B, acc);
      }
      S[t] = acc;
      if (next_g >= 0) stage_part(next_g, next_buf, t, with_lse);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  float M[kNT][4];
#pragma unroll
  for (int t = 0; t < kNT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) M[t][i] = neg_inf();

  u32x4_t Acur[4], Anext[4];
  // Step prologue: head s landed (this wave's DMA and loads) and every wave
  // is done with the other buffer; then queue step s + 1's q operands.  Its
  // DMA follows inside the step's logits; nothing inside the step waits on
  // vector memory, so the prefetch is never drained early.
  auto begin_step = [&](int s, bool load_next_q) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (s + 1 < 2 * G && load_next_q) load_q(head_of(s + 1), Anext);
  };
  // Logits of step s, staging step s + 1's head meanwhile.
  constexpr int kSteps = WS ? G : 2 * G;
  auto step_logits = [&](auto transposed, int s, f32x4_t (&S)[kNT]) {
    const bool more = s + 1 < kSteps;
    logits(transposed, lmk_buf(s & 1), Acur, S, more ? head_of(s + 1) : -1, (s + 1) & 1,
           s + 1 < G);
  };
  // Pass-1 q tiles travel by DMA through the slot table's space (unused
  // until the selection): [64 rows][16 parts] of 16 bytes, part p of row r at
  // unit r * 16 + (p ^ (r & 15)); rows >= L re-read row L - 1 (their rows are
  // dropped).  Wave w moves units (2w + k) * 64 + lane, k = 0, 1.
  uint16_t* qstage = reinterpret_cast<uint16_t*>(slot_s);
  auto stage_q = [&](int g) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int row = 4 * (2 * wave + k) + (lane >> 4);
      const int part = (lane & 15) ^ (row & 15);
      const int64_t r = min(q0 + row, L - 1);
      __builtin_amdgcn_global_load_lds(qb_base + ((r * a.Hkv + h) * G + g) * 128 + part * 8,
                                       (lds_void_t*)(qstage + (2 * wave + k) * 512), 16, 0, 0);
    }
  };
  stage_q(0);
  stage(0, 0, true);

  // Raw scores bf16(s * sm_scale) of the previous head (WS), two rows per
  // register: Rp[t][p] holds rows 4grp + 2p, 4grp + 2p + 1 of chunk
  // cbase + 16t + col.  They are stored one step late, after the step's
  // vmcnt wait, so that the next wait (which covers stores too) finds them
  // long completed instead of stalling on their write latency.
  uint32_t Rp[kNT][2];
  // raw_ws [B][L][Hkv][G][C]: 16 lanes of a row cover 16 consecutive chunks
  // (2-byte stores; a quad transpose to 8-byte row stores measured slower).
  auto store_raw = [&](int gprev) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t r = qbase + 4 * grp + i;
      if (r < L) {
        uint16_t* wrow = raw_ws + (((b * L + r) * a.Hkv + h) * G + gprev) * C;
#pragma unroll
        for (int t = 0; t < kNT; ++t) {
          const int c = cbase + 16 * t + col;
          const uint32_t w = Rp[t][i >> 1];
          if (c < C) wrow[c] = (uint16_t)((i & 1) ? (w >> 16) : (w & 0xffffu));
        }
      }
    }
  };

  // Pass 1: biased logits, LSE over all chunks, running max over heads.
  for (int s = 0; s < G; ++s) {
    const int g = s;
    begin_step(s, false);
    if constexpr (WS) {
      if (s > 0) store_raw(s - 1);
    }
    // This lane's A operand rows: query 16qg + col (row & 15 == col).
#pragma unroll
    for (int j = 0; j < 4; ++j)
      Acur[j] = *reinterpret_cast<const u32x4_t*>(
          qstage + ((16 * qg + col) * 16 + ((4 * j + grp) ^ col)) * 8);
    f32x4_t S[kNT];
    step_logits(std::false_type{}, s, S);
    if constexpr (WS) {
#pragma unroll
      for (int t = 0; t < kNT; ++t) {
        Rp[t][0] = pack_bf16x2(S[t][0] * a.sm_scale, S[t][1] * a.sm_scale);
        Rp[t][1] = pack_bf16x2(S[t][2] * a.sm_scale, S[t][3] * a.sm_scale);
      }
    }
    const float* bias_g = bias_s + 256 * (s & 1);
    // x = s * scale + bias, -inf past C.
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
      const int c = cbase + 16 * t + col;
      const float bv = c < C ? bias_g[c] : neg_inf();
#pragma unroll
      for (int i = 0; i < 4; ++i) S[t][i] = __builtin_fmaf(S[t][i], a.sm_scale, bv);
    }
    float rmax[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      rmax[i] = max_raw(max3_raw(max3_raw(S[0][i], S[1][i], S[2][i]), S[3][i], S[4][i]),
                        max3_raw(S[5][i], S[6][i], S[7][i]));
    // Row LSE over both chunk halves, in base 2 with the hardware exp2/log2:
    // each half reduces (max, sum of exp2) over its 128 chunks; one LDS
    // exchange combines them with a rescale.
    float m2[4], s2[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      m2[i] = group16_max(rmax[i]) * kLog2e;
      float sm = 0.f;
      if (m2[i] != neg_inf()) {
#pragma unroll
        for (int t = 0; t < kNT; ++t) sm += exp2_hw(__builtin_fmaf(S[t][i], kLog2e, -m2[i]));
      }
      s2[i] = group16_sum(sm);
      if (col == 0) {
        const int row = 16 * qg + 4 * grp + i;
        red_max[half * 64 + row] = m2[i];
        red_sum[half * 64 + row] = s2[i];
      }
    }
    __syncthreads();
    // Every wave has read this head's q tile: stage the next one.
    if (s + 1 < G) stage_q(s + 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t r = qbase + 4 * grp + i;
      const int row = 16 * qg + 4 * grp + i;
      const float ma = red_max[row], mb = red_max[64 + row];
      const float mm = fmaxf(ma, mb);
      float lse2 = neg_inf();  // log2 sum_c 2^(x_c log2 e)
      if (mm != neg_inf())
        lse2 = mm + log2_hw((ma == neg_inf() ? 0.f : red_sum[row] * exp2_hw(ma - mm)) +
                            (mb == neg_inf() ? 0.f : red_sum[64 + row] * exp2_hw(mb - mm)));
      float tot = 0.f;
      if (!a.pre_softmax) {
        // logaddexp(local_lse, lse) in base 2, back to natural units.  A -inf
        // total (no visible logit at all) is clamped to -FLT_MAX: finite x - tot
        // then ties at the top like x - (-inf) = +inf would, and -inf stays.
        const float lv2 = r < L ? lse_s[64 * (s & 1) + row] * kLog2e : 0.f;
        const float hi = fmaxf(lv2, lse2), lo = fminf(lv2, lse2);
        tot = hi == neg_inf() ? -__FLT_MAX__ : (hi + log2_hw(1.f + exp2_hw(lo - hi))) * kLn2;
      }
#pragma unroll
      for (int t = 0; t < kNT; ++t) M[t][i] = max_raw(M[t][i], S[t][i] - tot);
    }
  }

  if constexpr (WS) store_raw(G - 1);
  int16_t* pick_s = WS ? reinterpret_cast<int16_t*>(lmk_buf(G & 1)) : nullptr;  // [64][K]
  select_step<G>(a, M, lmk_buf((G - 1) & 1), cbad, slot_s, ntot_s, pick_s, q0, qbase, L, C, h, b,
                 lane, wave, col, grp, qg, cbase);
  if constexpr (WS) {
    // Picks of every head from the workspace, gathered straight into the
    // [G][K] score rows: wave w emits rows 8w..8w+7, lane l value
    // e = 64 it + l (head e / K, slot e % K) of each row, with the reads of
    // all eight rows in flight before any is used.  All waves of the
    // workgroup share one CU (one L1): the barrier's workgroup-scope fence
    // (vmcnt(0) on the stores) makes every wave's raw scores visible to the
    // others.
    __syncthreads();  // pick lists and counts of every row, raw scores stored
    constexpr int kIt = (8 * kFastMaxTopk + 63) / 64;  // G * K <= 8 * 64 values per row
    const int gk = G * K;
    const int nit = (gk + 63) / 64;
    // Head and slot of value e of a row; es = K (never < a pick count) marks
    // e >= G * K, so the last partial iteration reads nothing past the row.
    int eg[kIt], es[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int e = 64 * it + lane;
      eg[it] = e < gk ? e / K : 0;
      es[it] = e < gk ? e - eg[it] * K : K;
    }
    const int64_t rstride = (int64_t)a.Hkv * G * C, ostride = (int64_t)a.Hkv * gk;
    const uint16_t* rbase = raw_ws + ((b * L + q0) * a.Hkv + h) * (int64_t)G * C;
    uint16_t* obase = sc16 + ((b * L + q0) * a.Hkv + h) * (int64_t)gk;
    for (int it0 = 0; it0 < nit; it0 += 2) {
      uint16_t v[8][2];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int row = 8 * wave + j;
        const int nt = row < 64 && q0 + row < L ? ntot_s[row] : 0;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int it = it0 + u;
          v[j][u] = 0xff80u;  // -inf past the picks
          if (it < nit && es[it] < nt)  // es < nt <= K implies e < G * K
            v[j][u] = rbase[row * rstride + eg[it] * C + pick_s[row * K + es[it]]];
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int row = 8 * wave + j;
        if (q0 + row >= L) continue;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int e = 64 * (it0 + u) + lane;
          if (it0 + u < nit && e < gk) obase[row * ostride + e] = v[j][u];
        }
      }
    }
    return;
  }
  load_q(head_of(G), Acur);

  // Pass 2: raw logit bf16(q.lmk * scale) of every picked chunk, heads G-1..0.
  // The picks of a head are gathered in list order in an LDS row buffer and
  // written out as contiguous K-slot row segments.
  const int nrows = (int)min((int64_t)kFastQ, L - q0);
  for (int s = G; s < 2 * G; ++s) {
    const int g = head_of(s);
    begin_step(s, true);
    f32x4_t S[kNT];
    step_logits(std::true_type{}, s, S);
    // S^T: this lane's row and 4 consecutive chunks per tile; one 4-byte read
    // of the slot table per tile, most of which hold no pick.
    const int row = 16 * qg + col;
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
      const uint32_t sw =
          *reinterpret_cast<const uint32_t*>(slot_s + row * 256 + cbase + 16 * t + 4 * grp);
      if (sw != 0xffffffffu) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int slot = (int)(int8_t)(sw >> (8 * i));
          if (slot >= 0) sc_s[row * K + slot] = (uint16_t)f32_to_bf16(S[t][i] * a.sm_scale);
        }
      }
    }
    __syncthreads();
    for (int e = tid; e < nrows * K; e += kFastThreads) {
      const int row = e / K, slot = e - row * K;
      sc16[(((b * L + q0 + row) * a.Hkv + h) * G + g) * K + slot] =
          slot < ntot_s[row] ? sc_s[e] : (uint16_t)0xff80u;  // -inf past the picks
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) Acur[j] = Anext[j];
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

  // 1. x = s + bias (-inf past the causal limit or the last chunk).
  float x[kSelMaxPer][G];
#pragma unroll
  for (int i = 0; i < kSelMaxPer; ++i) {
    const int64_t c = tid + (int64_t)kSelThreads * i;
    const bool ok = i < n && c < C;
    const int64_t cc = ok ? c : 0;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float v = neg_inf();
      if (ok) {
        v = xr[(int64_t)g * C + cc];
        if (a.bias) v += a.bias[((b * C + cc) * a.Hkv + h) * G + g];
      }
      x[i][g] = v;
    }
  }
#pragma unroll
  for (int i = 0; i < kSelMaxPer; ++i) {
    const int64_t c = tid + (int64_t)kSelThreads * i;
    if (c >= climit)
#pragma unroll
      for (int g = 0; g < G; ++g) x[i][g] = neg_inf();
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
  uint32_t key[kSelMaxPer];
#pragma unroll
  for (int i = 0; i < kSelMaxPer; ++i) {
    key[i] = 0u;  // below every real key: never picked
    const int64_t c = tid + (int64_t)kSelThreads * i;
    if (i >= n || c >= C) continue;
    float best = neg_inf();
#pragma unroll
    for (int g = 0; g < G; ++g) best = fmaxf(best, x[i][g] == neg_inf() ? x[i][g] : x[i][g] - tot[g]);
    bool dropped = false;
    if (a.derive_window >= 0) {
      bool any = false;
      if (a.key_valid) {
        const uint8_t* kv = a.key_valid + b * L + c * a.block_size;
        for (int64_t t = 0; t < a.block_size - 1; ++t) any |= kv[t] != 0;
      } else {
        any = a.block_size > 1;
      }
      dropped = (c >= lc && c <= rc) || !any;
    } else if (a.drop) {
      dropped = a.drop[(b * L + r) * C + c] != 0;
    }
    key[i] = float_order_key(dropped ? neg_inf() : best);
  }

  // 4. The K largest (ties to the lower chunk), in ascending chunk order.
  bool pick[kSelMaxPer];
  int slot[kSelMaxPer];
  const int slot_base = Select::run(key, n, K, sel, pick, slot);
#pragma unroll
  for (int i = 0; i < kSelMaxPer; ++i) {
    if (i >= n || !pick[i]) continue;
    const int64_t c = tid + (int64_t)kSelThreads * i;
    a.indices[row * K + slot[i]] = (int32_t)c;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float v = xr[(int64_t)g * C + c];
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
// and tie rules as route_select_kernel.
template <int G, int PER>
__global__ void __launch_bounds__(256) route_select_wave_kernel(RouteArgs a,
                                                                const float* __restrict__ raw) {
  constexpr bool kHold = PER * G <= 128;
  const int64_t C = a.C, L = a.L;
  const int K = a.K;
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= L) return;  // wave-uniform
  const int h = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int n = (int)((C + 63) / 64);  // <= PER
  const int64_t row = (b * L + r) * a.Hkv + h;
  const float* xr = raw + row * (int64_t)G * C;
  const int64_t climit = a.is_causal ? causal_limit(a, r) : C;
  const float* bias = a.bias ? a.bias + (b * C * a.Hkv + h) * G : nullptr;  // + c * Hkv * G + g

  auto logit = [&](int g, int64_t c) -> float {
    if (c >= climit) return neg_inf();
    float v = xr[(int64_t)g * C + c];
    if (bias) v += bias[c * a.Hkv * G + g];
    return v;
  };

  float hold[kHold ? PER : 1][G];
  float m[G], sum[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = neg_inf();
    sum[g] = 0.f;
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int64_t c = lane + 64 * (int64_t)i;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float v = (i < n && c < C) ? logit(g, c) : neg_inf();
      if (kHold) hold[i][g] = v;
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

  int64_t lc = 0, rc = -1;
  if (a.derive_window >= 0) {
    lc = max(r - a.derive_window, (int64_t)0) / a.block_size;
    rc = min(r + a.derive_window, L - 1) / a.block_size;
  }
  uint32_t key[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    key[i] = 0u;  // below every real key: never picked
    const int64_t c = lane + 64 * (int64_t)i;
    if (i >= n || c >= C) continue;
    float best = neg_inf();
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float x = kHold ? hold[i][g] : logit(g, c);
      best = fmaxf(best, x == neg_inf() ? x : x - tot[g]);
    }
    bool dropped = false;
    if (a.derive_window >= 0) {
      bool any = false;
      if (a.key_valid) {
        const uint8_t* kv = a.key_valid + b * L + c * a.block_size;
        for (int64_t t = 0; t < a.block_size - 1; ++t) any |= kv[t] != 0;
      } else {
        any = a.block_size > 1;
      }
      dropped = (c >= lc && c <= rc) || !any;
    } else if (a.drop) {
      dropped = a.drop[(b * L + r) * C + c] != 0;
    }
    key[i] = float_order_key(dropped ? neg_inf() : best);
  }

  const uint64_t picks = WaveSelect<PER>::run(key, n, K);
  const uint64_t below = (1ull << lane) - 1ull;
  int base = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    if (i >= n) continue;  // uniform
    const bool p = (picks >> i) & 1ull;
    const uint64_t pb = __builtin_amdgcn_ballot_w64(p);
    if (p) {
      const int slot = base + __builtin_popcountll(pb & below);
      const int64_t c = lane + 64 * (int64_t)i;
      a.indices[row * K + slot] = (int32_t)c;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float v = xr[(int64_t)g * C + c];
        if (a.scores_fp32)
          reinterpret_cast<float*>(a.scores)[(row * G + g) * K + slot] = v;
        else
          reinterpret_cast<uint16_t*>(a.scores)[(row * G + g) * K + slot] =
              (uint16_t)f32_to_bf16(v);
      }
    }
    base += __builtin_popcountll(pb);
  }
  for (int t = base + lane; t < K; t += 64) {
    a.indices[row * K + t] = -1;
    for (int g = 0; g < G; ++g) {
      if (a.scores_fp32)
        reinterpret_cast<float*>(a.scores)[(row * G + g) * K + t] = neg_inf();
      else
        reinterpret_cast<uint16_t*>(a.scores)[(row * G + g) * K + t] = 0xff80u;
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
  if (a.B * a.L * a.Hkv >= kWaveSelectRows && a.C <= 4096 && a.L <= 0x7ffffffc) {
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
int launch_fast(const RouteArgs& a, uint16_t* raw_ws, hipStream_t s) {
  const size_t smem = FastLayout::total(a.K);
  auto kern = raw_ws ? route_topk_mfma_kernel<G, true> : route_topk_mfma_kernel<G, false>;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess)
    return MRSA_ERR_LAUNCH;
  dim3 grid((unsigned)((a.L + kFastQ - 1) / kFastQ), (unsigned)a.Hkv, (unsigned)a.B);
  hipLaunchKernelGGL(kern, grid, dim3(kFastThreads), smem, s, a, raw_ws);
  return mrsa_launch_status();
}

}  // namespace

namespace {

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
  hipStream_t s = (hipStream_t)stream;

  const bool aligned = ((uintptr_t)q % 16 == 0) && ((uintptr_t)lmk % 16 == 0);
  const bool fast = !scores_fp32 && !is_causal && head_dim == 128 &&
                    seq_len * kv_heads * groups * head_dim < ((int64_t)1 << 31) && chunks <= 256 && topk <= kFastMaxTopk && aligned &&
                    (groups == 7 || groups == 8);
  if (fast) {
    uint16_t* raw_ws = nullptr;
    if (workspace && (uintptr_t)workspace % 16 == 0 &&
        workspace_bytes >= batch * seq_len * kv_heads * groups * chunks * 2)
      raw_ws = (uint16_t*)workspace;
    return groups == 7 ? launch_fast<7>(a, raw_ws, s) : launch_fast<8>(a, raw_ws, s);
  }
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
  // logits [batch, seq_len, kv_heads, groups, chunks] of the short-block path
  // (beyond 256 chunks).  The matrix-core path (<= 256 chunks) runs without
  // one.  A problem that needs more than the static buffer is rejected.
  const bool fast_shape = chunks <= 256 && head_dim == 128 && !scores_fp32 && !is_causal &&
                          (groups == 7 || groups == 8);
  const int64_t need = fast_shape ? 0 : batch * seq_len * kv_heads * groups * chunks * 4;
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
