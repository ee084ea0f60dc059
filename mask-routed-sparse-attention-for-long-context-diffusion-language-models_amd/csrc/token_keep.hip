// Global token keep of the remote-token refinement:
// select_global_token_keep (dream_dllm_hils/token_refinement.py:112-148)
// without training noise.  In each row of n = K * S candidate scores
// ([B, L, Hkv, K, S] flattened per (b, l, h)), the min(budget, n) largest are
// kept when finite; ties at the threshold go to the lower flat index.  -inf
// (and NaN) scores are never kept.
//
// One wave per row (four rows per workgroup): element e = lane + 64 i lives
// in registers as an order key and the wave-level bisection of
// block_select.h finds the threshold without a barrier.  HBM-bound: n * 4
// bytes read and n bytes written per row.
#include "block_select.h"

#include <cmath>
#include "mrsa_device.h"

using namespace mrsa;

namespace {

constexpr int kRowsPerBlock = 4;

template <int PER>
__global__ void __launch_bounds__(64 * kRowsPerBlock)
    token_keep_kernel(const float* __restrict__ scores, int64_t rows, int64_t n, int budget,
                      uint8_t* __restrict__ keep) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole waves only
  const float* sr = scores + row * n;
  // Slot rows i < per are in use (uniform); only the last one may be partial
  // (lanes >= last are past the row).  Loads are unconditional at clamped
  // addresses so that none of them waits alone inside a branch.
  const int per = (int)((n + 63) / 64);
  const int last = (int)(n - 64 * (int64_t)(per - 1));
  float v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) v[i] = sr[min(lane + 64 * (int64_t)i, n - 1)];
  uint32_t key[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    key[i] = i < per ? float_order_key(v[i] == v[i] ? v[i] : neg_inf()) : 0u;
    if (i == per - 1 && lane >= last) key[i] = 0u;
  }
  const uint64_t picks = WaveSelect<PER>::run(key, per, budget);
  uint8_t* kr = keep + row * n;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    if (i >= per) break;
    if (i < per - 1 || lane < last) kr[lane + 64 * (int64_t)i] = (uint8_t)((picks >> i) & 1ull);
  }
}

template <int PER>
void launch_keep(const float* scores, int64_t rows, int64_t n, int budget, uint8_t* keep,
                 hipStream_t s) {
  hipLaunchKernelGGL(token_keep_kernel<PER>,
                     dim3((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock)),
                     dim3(64 * kRowsPerBlock), 0, s, scores, rows, n, budget, keep);
}

// ---- entropy-adaptive token keep -------------------------------------------
// refine_remote_tokens_entropy_g7 (dream_dllm_hils/token_refinement.py:396-438)
// without training noise:
//   e_k   selected entropy of slot k: the group mean of entropy[b, c, h, :]
//         at c = clamp(idx_k, 0, C - 1), 0 for idx_k < 0
//         (gather_selected_chunk_entropy, :244-284);
//   a_k   allocate_entropy_token_budget(e, capacity, budget, min) (:150-241):
//         target = min(sum capacity, budget), baseline min(capacity, min),
//         then K + 1 rounds of capped largest-remainder apportionment by
//         support exp(clamp(e, 0, ln budget)) (0 for empty chunks);
//   keep  in chunk k the a_k largest scores (ties to the lower key index),
//         finite only (select_entropy_adaptive_token_keep, :287-333).
// One wave per (b, l, h) row: lane k < K holds slot k through the
// apportionment; a chunk's S scores are read with one lane per key for the
// capacities and again for the per-chunk wave selects.  The support sum is formed
// exactly (in double; the supports lie in [1, budget]) and rounded once, so
// it does not depend on the summation order.  A round that leaves nothing
// to apportion ends the loop (the remaining rounds change nothing).
struct EntropyKeepArgs {
  const float* scores;        // [rows, K, S] ranking scores, or null
  const int64_t* capacity;    // [rows, K], or null: finite scores per chunk
  const float* sel_entropy;   // [rows, K], or null: gathered from entropy
  const float* entropy;       // [B, C, Hkv, G]
  const int32_t* indices;     // [B, L, Hkv, K]
  int64_t rows, L, C;
  int Hkv, G, K, S;
  int64_t budget, min_tokens;
  float max_entropy;          // fp32(ln(max(budget, 1)))
  uint8_t* keep;              // [rows, K, S] or null
  int64_t* allocation;        // [rows, K]
};

__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int lo = __shfl_xor((int)(uint32_t)v, o, 64);
    const int hi = __shfl_xor((int)(uint32_t)((uint64_t)v >> 32), o, 64);
    v += (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
  }
  return v;
}
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t x = (uint64_t)__double_as_longlong(v);
    const int lo = __shfl_xor((int)(uint32_t)x, o, 64);
    const int hi = __shfl_xor((int)(uint32_t)(x >> 32), o, 64);
    v += __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
  }
  return v;
}

__global__ void __launch_bounds__(64 * kRowsPerBlock) token_keep_entropy_kernel(EntropyKeepArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= a.rows) return;  // whole waves only
  const int K = a.K, S = a.S;
  const bool lk = lane < K;
  // capacities: finite scores per chunk (chunk k's S scores, lane = key)
  int64_t cap = 0;
  const float* sr = a.scores ? a.scores + row * K * S : nullptr;
  if (sr && !a.capacity) {
    for (int k = 0; k < K; ++k) {
      const float x = lane < S ? sr[k * S + lane] : neg_inf();
      const int n = __builtin_popcountll(__builtin_amdgcn_ballot_w64(__builtin_isfinite(x)));
      if (lane == k) cap = n;
    }
  }
  if (a.capacity) cap = lk ? a.capacity[row * K + lane] : 0;
  // selected entropy and support of slot `lane`
  float e = 0.f;
  if (lk) {
    if (a.sel_entropy) {
      e = a.sel_entropy[row * K + lane];
    } else {
      const int64_t h = row % a.Hkv;
      const int64_t b = row / a.Hkv / a.L;
      const int32_t c = a.indices[row * K + lane];
      if (c >= 0) {
        const int64_t cc = c < a.C ? c : a.C - 1;
        const float* er = a.entropy + ((b * a.C + cc) * a.Hkv + h) * a.G;
        float sum = 0.f;
        for (int g = 0; g < a.G; ++g) sum += er[g];
        e = sum / (float)a.G;
      }
    }
  }
  float x = e;
  if (x != x) x = 0.f;
  else if (x == __builtin_inff()) x = a.max_entropy;
  else if (x == -__builtin_inff()) x = 0.f;
  x = fminf(fmaxf(x, 0.f), a.max_entropy);
  const float support = (lk && cap > 0) ? expf(x) : 0.f;
  const int64_t sumcap = wave_sum_i64(cap);
  const int64_t target = sumcap < a.budget ? sumcap : a.budget;
  int64_t alloc = lk ? (cap < a.min_tokens ? cap : a.min_tokens) : 0;
  int64_t remaining = target - wave_sum_i64(alloc);
  for (int it = 0; it <= K; ++it) {
    if (remaining <= 0) break;  // uniform
    const bool act = lk && alloc < cap;
    const float as = act ? support : 0.f;
    const float den = (float)wave_sum_f64((double)as);
    const float quota = den > 0.f ? ((float)remaining * as) / fmaxf(den, 1e-12f) : 0.f;
    const float fq = floorf(quota);
    const int64_t room = cap - alloc;
    alloc += (int64_t)fq < room ? (int64_t)fq : room;
    remaining = target - wave_sum_i64(alloc);
    const bool act2 = lk && alloc < cap;
    const int64_t acnt = __builtin_popcountll(__builtin_amdgcn_ballot_w64(act2));
    const int64_t bonus_count = remaining < acnt ? remaining : acnt;
    if (bonus_count > 0) {
      // rank in the stable descending order of the fractional parts
      const float frac = act2 ? quota - fq : neg_inf();
      int rank = 0;
      for (int k2 = 0; k2 < K; ++k2) {
        const float f2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(frac), k2));
        rank += (f2 > frac || (f2 == frac && k2 < lane)) ? 1 : 0;
      }
      if (lk && rank < bonus_count && alloc < cap) alloc += 1;
      remaining = target - wave_sum_i64(alloc);
    }
  }
  if (lk) a.allocation[row * K + lane] = alloc;
  if (!a.keep || !a.scores) return;
  uint8_t* kr = a.keep + row * K * S;
  for (int k = 0; k < K; ++k) {
    const int ak = __builtin_amdgcn_readlane((int)alloc, k);
    float x = lane < S ? sr[k * S + lane] : neg_inf();
    if (x != x) x = neg_inf();
    uint32_t key[1] = {lane < S ? float_order_key(x) : 0u};
    uint64_t pick = 0ull;
    if (ak > 0) pick = WaveSelect<1>::run(key, 1, ak < S ? ak : S);
    if (lane < S) kr[k * S + lane] = (uint8_t)(pick & 1ull);
  }
}

// gather_selected_chunk_entropy (token_refinement.py:244-284): one thread
// per (row, slot).
__global__ void __launch_bounds__(256) gather_entropy_kernel(const float* entropy,
                                                             const int32_t* indices, int64_t n,
                                                             int64_t L, int64_t C, int Hkv,
                                                             int G, int K, float* out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t row = i / K;
  const int64_t h = row % Hkv;
  const int64_t b = row / Hkv / L;
  const int32_t c = indices[i];
  float e = 0.f;
  if (c >= 0) {
    const int64_t cc = c < C ? c : C - 1;
    const float* er = entropy + ((b * C + cc) * Hkv + h) * G;
    float sum = 0.f;
    for (int g = 0; g < G; ++g) sum += er[g];
    e = sum / (float)G;
  }
  out[i] = e;
}

}  // namespace

extern "C" int mrsa_token_keep_fwd(const float* scores, int64_t rows, int64_t n,
                                   int64_t token_budget, uint8_t* keep, void* stream) {
  if (rows < 0 || n < 0 || token_budget <= 0) return MRSA_ERR_INVALID_ARGUMENT;
  if (rows == 0 || n == 0) return MRSA_OK;
  if (!scores || !keep) return MRSA_ERR_INVALID_ARGUMENT;
  if (n > 4096 || rows > ((int64_t)1 << 32)) return MRSA_ERR_UNSUPPORTED;
  const int budget = (int)(token_budget < n ? token_budget : n);
  hipStream_t s = (hipStream_t)stream;
  if (n <= 512) launch_keep<8>(scores, rows, n, budget, keep, s);
  else if (n <= 1024) launch_keep<16>(scores, rows, n, budget, keep, s);
  else if (n <= 2048) launch_keep<32>(scores, rows, n, budget, keep, s);
  else launch_keep<64>(scores, rows, n, budget, keep, s);
  return mrsa_launch_status();
}

extern "C" int mrsa_token_keep_entropy_fwd(const float* scores, const int64_t* capacity,
                                           const float* selected_entropy, const float* entropy,
                                           const int32_t* indices, int64_t batch,
                                           int64_t seq_len, int64_t kv_heads, int64_t groups,
                                           int64_t chunks, int64_t topk, int64_t chunk_size,
                                           int64_t token_budget, int64_t min_tokens_per_chunk,
                                           uint8_t* keep, int64_t* allocation, void* stream) {
  if (batch < 0 || seq_len < 0 || kv_heads <= 0 || topk <= 0 || chunk_size <= 0 ||
      token_budget <= 0 || min_tokens_per_chunk < 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (token_budget < topk * min_tokens_per_chunk) return MRSA_ERR_INVALID_ARGUMENT;
  if (topk > 64 || chunk_size > 64) return MRSA_ERR_UNSUPPORTED;
  if (!allocation || (!capacity && !scores)) return MRSA_ERR_INVALID_ARGUMENT;
  if (!selected_entropy && (!entropy || !indices || groups <= 0 || chunks <= 0))
    return MRSA_ERR_INVALID_ARGUMENT;
  const int64_t rows = batch * seq_len * kv_heads;
  if (rows == 0) return MRSA_OK;
  EntropyKeepArgs a;
  a.scores = scores;
  a.capacity = capacity;
  a.sel_entropy = selected_entropy;
  a.entropy = entropy;
  a.indices = indices;
  a.rows = rows;
  a.L = seq_len;
  a.C = chunks;
  a.Hkv = (int)kv_heads;
  a.G = (int)groups;
  a.K = (int)topk;
  a.S = (int)chunk_size;
  a.budget = token_budget;
  a.min_tokens = min_tokens_per_chunk;
  a.max_entropy = (float)log((double)(token_budget > 1 ? token_budget : 1));
  a.keep = keep;
  a.allocation = allocation;
  const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  if (blocks > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(token_keep_entropy_kernel, dim3((unsigned)blocks),
                     dim3(64 * kRowsPerBlock), 0, (hipStream_t)stream, a);
  return mrsa_launch_status();
}

extern "C" int mrsa_gather_selected_chunk_entropy(const float* entropy, const int32_t* indices,
                                                  int64_t batch, int64_t seq_len,
                                                  int64_t chunks, int64_t kv_heads,
                                                  int64_t groups, int64_t topk, float* out,
                                                  void* stream) {
  if (batch < 0 || seq_len < 0 || chunks <= 0 || kv_heads <= 0 || groups <= 0 || topk <= 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  const int64_t n = batch * seq_len * kv_heads * topk;
  if (n == 0) return MRSA_OK;
  if (!entropy || !indices || !out) return MRSA_ERR_INVALID_ARGUMENT;
  if ((n + 255) / 256 > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(gather_entropy_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, entropy, indices, n, seq_len, chunks, (int)kv_heads,
                     (int)groups, (int)topk, out);
  return mrsa_launch_status();
}
