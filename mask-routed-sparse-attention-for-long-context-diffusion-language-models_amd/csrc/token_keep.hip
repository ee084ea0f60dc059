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
