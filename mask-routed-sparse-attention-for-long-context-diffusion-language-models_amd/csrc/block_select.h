// Block-wide (and wave-wide) top-K selection over order keys held in registers.
//
// Each of THREADS threads holds PER keys; element (i, tid) has order index
// i * THREADS + tid.  Keys above kFloor are candidates (kFloor is the order
// key of -inf; 0 marks "no element").  The K largest candidates are picked;
// at the threshold, equal keys go to the lowest order indices.  Picks get
// slots 0..total-1 in ascending order index.
//
// Method: the candidate count and key range first, then bisection on the key
// value, counting with wave ballots (one barrier per step, the count buffer
// alternating between two LDS slots so that a wave running ahead never
// overwrites counts a slower wave still reads), then tie ranks and pick slots
// from per-wave ballot prefix counts.
#pragma once

#include "mrsa_device.h"

namespace mrsa {

template <int THREADS, int PER>
struct BlockSelect {
  static constexpr int kWaves = THREADS / 64;
  struct Lds {
    int red[2][kWaves];
    int range[3][kWaves];
    int cnt[2][PER][kWaves];
  };

  __device__ static int count_ge(const uint32_t (&key)[PER], int n, uint32_t t, int* buf) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int c = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (i < n) c += __builtin_popcountll(__builtin_amdgcn_ballot_w64(key[i] >= t));
    if (lane == 0) buf[wave] = c;
    __syncthreads();
    int r = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) r += buf[w];
    return r;
  }

  // n: key slots in use per thread (<= PER, uniform).  Returns the pick count.
  __device__ static int run(const uint32_t (&key)[PER], int n, int K, Lds& s, bool (&pick)[PER],
                            int (&slot)[PER]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t kFloor = float_order_key(neg_inf());
    int nfin = 0;
    uint32_t kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (i < n && key[i] > kFloor) {
        ++nfin;
        kmin = min(kmin, key[i]);
        kmax = max(kmax, key[i]);
      }
    }
    {
      int vmin = (int)(kmin ^ 0x80000000u), vmax = (int)(kmax ^ 0x80000000u);
      for (int o = 1; o < 64; o <<= 1) {
        vmin = min(vmin, __shfl_xor(vmin, o, 64));
        vmax = max(vmax, __shfl_xor(vmax, o, 64));
        nfin += __shfl_xor(nfin, o, 64);
      }
      if (lane == 0) {
        s.range[0][wave] = nfin;
        s.range[1][wave] = vmin;
        s.range[2][wave] = vmax;
      }
      __syncthreads();
      nfin = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        nfin += s.range[0][w];
        vmin = min(vmin, s.range[1][w]);
        vmax = max(vmax, s.range[2][w]);
      }
      kmin = (uint32_t)vmin ^ 0x80000000u;
      kmax = (uint32_t)vmax ^ 0x80000000u;
    }

    // Threshold: keys >= thr_hi are picked, plus the `need` lowest-index
    // elements whose key equals thr_tie.
    uint32_t thr_hi, thr_tie = 0u;
    int need = 0, it = 0;
    if (nfin <= K) {
      thr_hi = kFloor + 1u;
    } else {
      uint32_t lo = kmin, hi = kmax + 1u;  // count(lo) > K > count(hi)
      bool exact = false;
      thr_hi = 0u;
      while (hi - lo > 1u) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        const int c = count_ge(key, n, mid, s.red[it++ & 1]);
        if (c == K) {
          thr_hi = mid;
          exact = true;
          break;
        }
        if (c > K) lo = mid; else hi = mid;
      }
      if (!exact) {
        const int cnt_hi = count_ge(key, n, hi, s.red[it++ & 1]);
        thr_hi = hi;
        thr_tie = lo;
        need = K - cnt_hi;
      }
    }

    // Tie ranks, then pick slots, in ascending order index.
    const uint64_t below = (1ull << lane) - 1ull;
    uint64_t tie_bits[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      tie_bits[i] = 0ull;
      if (i >= n) continue;
      tie_bits[i] = __builtin_amdgcn_ballot_w64(need > 0 && key[i] == thr_tie);
      if (lane == 0) s.cnt[0][i][wave] = __builtin_popcountll(tie_bits[i]);
    }
    __syncthreads();
    {
      int base = 0;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        pick[i] = false;
        if (i >= n) continue;
        int before = base;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          const int v = s.cnt[0][i][w];
          before += w < wave ? v : 0;
          base += v;
        }
        const bool tie = (tie_bits[i] >> lane) & 1ull;
        const int tr = before + __builtin_popcountll(tie_bits[i] & below);
        pick[i] = key[i] >= thr_hi || (tie && tr < need);
        const uint64_t pb = __builtin_amdgcn_ballot_w64(pick[i]);
        if (lane == 0) s.cnt[1][i][wave] = __builtin_popcountll(pb);
      }
    }
    __syncthreads();
    int total = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      slot[i] = -1;
      if (i >= n) continue;
      const uint64_t pb = __builtin_amdgcn_ballot_w64(pick[i]);
      int before = total;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const int v = s.cnt[1][i][w];
        before += w < wave ? v : 0;
        total += v;
      }
      if (pick[i]) slot[i] = before + __builtin_popcountll(pb & below);
    }
    return total;
  }
};

// The same selection by one wave with no barrier: element (i, lane) has
// order index i * 64 + lane; every count is a sum of ballot popcounts, so
// the whole search runs on scalar registers after each compare.
template <int PER>
struct WaveSelect {
  __device__ static uint32_t wave_min_u(uint32_t v) {
    for (int o = 1; o < 64; o <<= 1) v = min(v, (uint32_t)__shfl_xor((int)v, o, 64));
    return v;
  }
  __device__ static uint32_t wave_max_u(uint32_t v) {
    for (int o = 1; o < 64; o <<= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, 64));
    return v;
  }
  // Ballots in groups of 8 with a scheduling fence between groups: the
  // scheduler would otherwise keep all PER ballot masks live in SGPRs.
  __device__ static int count_ge(const uint32_t (&key)[PER], int n, uint32_t t) {
    int c = 0;
#pragma unroll
    for (int i0 = 0; i0 < PER; i0 += 8) {
#pragma unroll
      for (int i = i0; i < i0 + 8 && i < PER; ++i)
        if (i < n) c += __builtin_popcountll(__builtin_amdgcn_ballot_w64(key[i] >= t));
      __builtin_amdgcn_sched_barrier(0);
    }
    return c;
  }

  // The threshold of the K largest candidates: keys >= thr_hi are picked,
  // plus `need` of the keys equal to thr_tie (need = 0: no tie to break).
  // n: key slots in use per lane (<= PER, uniform).
  __device__ static void threshold(const uint32_t (&key)[PER], int n, int K, uint32_t& thr_hi,
                                   uint32_t& thr_tie, int& need) {
    const uint32_t kFloor = float_order_key(neg_inf());
    int nfin = 0;
    uint32_t kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (i >= n) continue;
      const bool f = key[i] > kFloor;
      nfin += f ? 1 : 0;
      if (f) {
        kmin = min(kmin, key[i]);
        kmax = max(kmax, key[i]);
      }
    }
    for (int o = 1; o < 64; o <<= 1) nfin += __shfl_xor(nfin, o, 64);
    kmin = wave_min_u(kmin);
    kmax = wave_max_u(kmax);
    thr_tie = 0u;
    need = 0;
    if (nfin <= K) {
      thr_hi = kFloor + 1u;
    } else {
      uint32_t lo = kmin, hi = kmax + 1u;  // count(lo) > K > count(hi)
      bool exact = false;
      thr_hi = 0u;
      while (hi - lo > 1u) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        const int c = count_ge(key, n, mid);
        if (c == K) {
          thr_hi = mid;
          exact = true;
          break;
        }
        if (c > K) lo = mid; else hi = mid;
      }
      if (!exact) {
        thr_hi = hi;
        thr_tie = lo;
        need = K - count_ge(key, n, hi);
      }
    }
  }

  // n: key slots in use per lane (<= PER <= 64, uniform).  Returns this
  // lane's picks as bits (bit i: element (i, lane)); per-lane bits keep the
  // picks in vector registers (an array of bools would take a scalar mask
  // pair per element).
  __device__ static uint64_t run(const uint32_t (&key)[PER], int n, int K) {
    static_assert(PER <= 64, "one pick bit per key slot");
    const int lane = threadIdx.x & 63;
    uint32_t thr_hi, thr_tie;
    int need;
    threshold(key, n, K, thr_hi, thr_tie, need);
    const uint64_t below = (1ull << lane) - 1ull;
    int base = 0;
    uint64_t picks = 0ull;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (i >= n) continue;
      bool p = key[i] >= thr_hi;
      if (need > 0) {  // uniform
        const uint64_t tb = __builtin_amdgcn_ballot_w64(key[i] == thr_tie);
        p = p || (((tb >> lane) & 1ull) && base + __builtin_popcountll(tb & below) < need);
        base += __builtin_popcountll(tb);
      }
      picks |= p ? 1ull << i : 0ull;
      if ((i & 7) == 7) __builtin_amdgcn_sched_barrier(0);
    }
    return picks;
  }
};

}  // namespace mrsa
