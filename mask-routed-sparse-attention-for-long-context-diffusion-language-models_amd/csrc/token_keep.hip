// Global token keep of the remote-token refinement:
// select_global_token_keep (dream_dllm_hils/token_refinement.py:112-148)
// without training noise.  In each row of n = K * S candidate scores
// ([B, L, Hkv, K, S] flattened per (b, l, h)), the min(budget, n) largest are
// kept when finite; ties at the threshold go to the lower flat index.  -inf
// (and NaN) scores are never kept.
//
// One 512-thread workgroup per row; element e = tid + 512 i lives in
// registers as an order key, and the block-wide bisection of block_select.h
// finds the threshold.  HBM-bound: n * 4 bytes read and n bytes written per
// row.
#include "block_select.h"
#include "mrsa_device.h"

using namespace mrsa;

namespace {

constexpr int kKeepThreads = 512;
constexpr int kKeepPer = 8;  // n <= 4096

__global__ void __launch_bounds__(kKeepThreads)
    token_keep_kernel(const float* __restrict__ scores, int64_t n, int budget,
                      uint8_t* __restrict__ keep) {
  using Select = BlockSelect<kKeepThreads, kKeepPer>;
  __shared__ typename Select::Lds sel;
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const float* sr = scores + row * n;
  const int per = (int)((n + kKeepThreads - 1) / kKeepThreads);
  uint32_t key[kKeepPer];
#pragma unroll
  for (int i = 0; i < kKeepPer; ++i) {
    key[i] = 0u;
    const int64_t e = tid + (int64_t)kKeepThreads * i;
    if (i < per && e < n) {
      const float v = sr[e];
      key[i] = float_order_key(v == v ? v : neg_inf());
    }
  }
  bool pick[kKeepPer];
  int slot[kKeepPer];
  Select::run(key, per, budget, sel, pick, slot);
  uint8_t* kr = keep + row * n;
#pragma unroll
  for (int i = 0; i < kKeepPer; ++i) {
    const int64_t e = tid + (int64_t)kKeepThreads * i;
    if (i < per && e < n) kr[e] = pick[i] ? 1 : 0;
  }
}

}  // namespace

extern "C" int mrsa_token_keep_fwd(const float* scores, int64_t rows, int64_t n,
                                   int64_t token_budget, uint8_t* keep, void* stream) {
  if (rows < 0 || n < 0 || token_budget <= 0) return MRSA_ERR_INVALID_ARGUMENT;
  if (rows == 0 || n == 0) return MRSA_OK;
  if (!scores || !keep) return MRSA_ERR_INVALID_ARGUMENT;
  if (n > (int64_t)kKeepThreads * kKeepPer || rows > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  const int budget = (int)(token_budget < n ? token_budget : n);
  hipLaunchKernelGGL(token_keep_kernel, dim3((unsigned)rows), dim3(kKeepThreads), 0,
                     (hipStream_t)stream, scores, n, budget, keep);
  return mrsa_launch_status();
}
