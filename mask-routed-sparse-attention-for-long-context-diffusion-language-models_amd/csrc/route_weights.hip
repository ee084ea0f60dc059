// Route weights: one lane per (token, query head) normalises the topk routed
// chunk logits together with the local-branch LSE.
//
// Semantics: _route_weights_torch (dream_dllm_hils/attention.py:126-235):
//   remote_k = valid(idx_k) ? float(score_k) + prior_bias[idx_k] : -inf
//   local    = local_lse (- gate_offset in the plain form when given)
//   logits   = [remote, local] / temperature; all -inf -> both outputs 0
//   plain form:  softmax(logits)
//   affine form: mass = sigmoid(gate_scale * (lse(remote) - local) + gate_offset),
//                remote_w = softmax(remote) * mass, local_w = 1 - mass
// The TileLang route_weights kernel (ops/hils_bidir_route_weights_tilelang.py:15-94)
// computes the plain form with temperature 1.
#include "mrsa_device.h"

using namespace mrsa;

namespace {

constexpr int kMaxTopk = 64;

__global__ void __launch_bounds__(256)
    route_weights_kernel(const uint16_t* __restrict__ scores, const int32_t* __restrict__ indices,
                         const float* __restrict__ bias, const float* __restrict__ lse,
                         int64_t rows, int64_t L, int64_t C, int Hkv, int G, int K, float inv_t,
                         int has_off, float off, int affine, float gscale,
                         uint16_t* __restrict__ rw, uint16_t* __restrict__ lw) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int Hq = Hkv * G;
  const int hq = (int)(r % Hq);
  const int64_t bl = r / Hq;
  const int64_t b = bl / L;
  const int hk = hq / G, g = hq - hk * G;
  const uint16_t* sc = scores + r * K;
  const int32_t* ix = indices + (bl * Hkv + hk) * K;

  float x[kMaxTopk];
  float rmax = neg_inf();
#pragma unroll
  for (int k = 0; k < kMaxTopk; ++k) {
    if (k < K) {
      const int32_t c = ix[k];
      float v = neg_inf();
      if (c >= 0 && c < C) v = bf16_to_f32(sc[k]) + bias[((b * C + c) * Hkv + hk) * G + g];
      x[k] = v * inv_t;
      rmax = fmaxf(rmax, x[k]);
    }
  }
  float local = lse[r];
  if (has_off && !affine) local -= off;
  local *= inv_t;

  uint16_t* out = rw + r * K;
  const float m = fmaxf(rmax, local);
  if (m == neg_inf()) {  // every logit masked
    for (int k = 0; k < K; ++k) out[k] = 0;
    lw[r] = 0;
    return;
  }
  if (!affine) {
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxTopk; ++k)
      if (k < K) {
        x[k] = x[k] == neg_inf() ? 0.f : expf(x[k] - m);
        sum += x[k];
      }
    const float el = local == neg_inf() ? 0.f : expf(local - m);
    sum += el;
#pragma unroll
    for (int k = 0; k < kMaxTopk; ++k)
      if (k < K) out[k] = (uint16_t)f32_to_bf16(x[k] / sum);
    lw[r] = (uint16_t)f32_to_bf16(el / sum);
    return;
  }
  // Affine-sigmoid gate.
  float mass;
  if (rmax == neg_inf()) {
    // No routed chunk: softmax of the remote part is zeroed, gate -> local.
    mass = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxTopk; ++k)
      if (k < K) x[k] = 0.f;
  } else {
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxTopk; ++k)
      if (k < K) {
        x[k] = x[k] == neg_inf() ? 0.f : expf(x[k] - rmax);
        sum += x[k];
      }
    const float remote_lse = rmax + logf(sum);
    const float gate = gscale * (remote_lse - local) + (has_off ? off : 0.f);
    mass = 1.f / (1.f + expf(-gate));
#pragma unroll
    for (int k = 0; k < kMaxTopk; ++k)
      if (k < K) x[k] = x[k] / sum;
  }
#pragma unroll
  for (int k = 0; k < kMaxTopk; ++k)
    if (k < K) out[k] = (uint16_t)f32_to_bf16(x[k] * mass);
  lw[r] = (uint16_t)f32_to_bf16(1.f - mass);
}

}  // namespace

extern "C" int mrsa_route_weights_fwd(const void* scores, const int32_t* indices,
                                      const float* prior_bias, const float* local_lse,
                                      int64_t batch, int64_t seq_len, int64_t chunks,
                                      int64_t kv_heads, int64_t groups, int64_t topk,
                                      float temperature, int has_gate_offset, float gate_offset,
                                      int has_gate_scale, float gate_scale, void* remote_weights,
                                      void* local_weight, void* stream) {
  if (batch < 0 || seq_len < 0 || chunks <= 0 || kv_heads <= 0 || groups <= 0 || topk <= 0 ||
      !(temperature > 0.f))
    return MRSA_ERR_INVALID_ARGUMENT;
  if (topk > kMaxTopk) return MRSA_ERR_UNSUPPORTED;
  const int64_t rows = batch * seq_len * kv_heads * groups;
  if (rows == 0) return MRSA_OK;
  if (!scores || !indices || !prior_bias || !local_lse || !remote_weights || !local_weight)
    return MRSA_ERR_INVALID_ARGUMENT;
  const int64_t blocks = (rows + 255) / 256;
  if (blocks > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(route_weights_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)scores, indices, prior_bias, local_lse,
                     rows, seq_len, chunks, (int)kv_heads, (int)groups, (int)topk,
                     1.f / temperature, has_gate_offset, gate_offset, has_gate_scale, gate_scale,
                     (uint16_t*)remote_weights, (uint16_t*)local_weight);
  return mrsa_launch_status();
}
