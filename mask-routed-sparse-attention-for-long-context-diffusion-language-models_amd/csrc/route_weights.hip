// Route weights: the topk routed chunk logits of each (token, query head) are
// normalised together with the local-branch LSE.
//
// Semantics: _route_weights_torch (dream_dllm_hils/attention.py:126-235):
//   remote_k = valid(idx_k) ? float(score_k) + prior_bias[idx_k]
//              (+ value_bonus_k) (+ selected_gumbel_k) : -inf
//   local    = local_lse (- gate_offset in the plain form when given)
//   logits   = [remote, local] / temperature; all -inf -> both outputs 0
//   plain form:  softmax(logits)
//   affine form: mass = sigmoid(gate_scale * (lse(remote) - local) + gate_offset),
//                remote_w = softmax(remote) * mass, local_w = 1 - mass
// The TileLang route_weights kernel (ops/hils_bidir_route_weights_tilelang.py:15-94)
// computes the plain form with temperature 1.
//
// Work split: LPR lanes cooperate on one (token, query head) row, 8
// consecutive slots per lane.  Score, index and weight rows move as 16-byte
// vectors when topk % 8 == 0, so a wave reads or writes 1 KB per instruction;
// the row max / sum are reduced across the LPR lanes.
#include "mrsa_device.h"

#include <type_traits>

using namespace mrsa;

namespace {

constexpr int kMaxTopk = 64;

// Max / sum over the LPR lanes of a row (aligned groups of 1, 2, 4 or 8
// lanes) with DPP lane moves: swap neighbours, swap pairs, then mirror the
// two quads of an 8-lane half-row.  The same operand pairs as xor shuffles
// by 1, 2, 4, so the same bits.  Every lane of the row must be active.
template <int LPR>
__device__ __forceinline__ float row_lanes_max(float v) {
  if constexpr (LPR >= 2) v = fmaxf(v, dpp_mov<0xb1>(v));   // quad_perm [1,0,3,2]
  if constexpr (LPR >= 4) v = fmaxf(v, dpp_mov<0x4e>(v));   // quad_perm [2,3,0,1]
  if constexpr (LPR >= 8) v = fmaxf(v, dpp_mov<0x141>(v));  // row_half_mirror
  return v;
}
template <int LPR>
__device__ __forceinline__ float row_lanes_sum(float v) {
  if constexpr (LPR >= 2) v += dpp_mov<0xb1>(v);
  if constexpr (LPR >= 4) v += dpp_mov<0x4e>(v);
  if constexpr (LPR >= 8) v += dpp_mov<0x141>(v);
  return v;
}

// I: the index type (uint32_t when every index of the call fits 32 bits,
// which turns the row decode's divisions into 32-bit ones).  VEC: topk is a
// multiple of 8 (every lane's 8 slots are real).  UNIT_T: temperature 1 (no
// 1 / T products).  EX: the optional additive terms e1 (value bonus) and e2
// (selected Gumbel noise), fp32 in the scores' layout, may be given.
template <int LPR, bool VEC, bool UNIT_T, class I, bool EX = false>
__device__ __forceinline__ void route_weights_row(
    int64_t t64, const uint16_t* __restrict__ scores,
    const int32_t* __restrict__ indices, const float* __restrict__ bias,
    const float* __restrict__ lse, int64_t rows64, int64_t L64, int64_t C64, int Hkv, int G, int K,
    float inv_t, int has_off, int affine, float off, float gscale, uint16_t* __restrict__ rw,
    uint16_t* __restrict__ lw, float* __restrict__ gate_logit, const float* __restrict__ e1,
    const float* __restrict__ e2) {
  const I t = (I)t64, rows = (I)rows64, L = (I)L64, C = (I)C64;
  const int part = (int)(t % LPR);
  const I r0 = t / LPR;
  const bool live = r0 < rows;
  const I r = live ? r0 : rows - 1;  // lanes past the end still join the row reductions
  const I Hq = (I)(Hkv * G);
  const I bl = r / Hq;
  const int hq = (int)(r - bl * Hq);
  const I b = bl / L;
  const int hk = hq / G, g = hq - hk * G;
  const int k0 = part * 8;
  const uint16_t* sc = scores + r * (I)K + k0;
  const int32_t* ix = indices + (bl * (I)Hkv + hk) * (I)K + k0;

  // lanes past the last slot (8 LPR > K, e.g. K = 24 or 40) keep chunk -1:
  // masked slots
  uint32_t sv[4] = {0u, 0u, 0u, 0u};
  int32_t iv[8] = {-1, -1, -1, -1, -1, -1, -1, -1};
  if (VEC && k0 < K) {
    const u32x4_t s4 = *reinterpret_cast<const u32x4_t*>(sc);
    const u32x4_t i0 = *reinterpret_cast<const u32x4_t*>(ix);
    const u32x4_t i1 = *reinterpret_cast<const u32x4_t*>(ix + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sv[j] = s4[j];
      iv[j] = (int32_t)i0[j];
      iv[4 + j] = (int32_t)i1[j];
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const bool in = k0 + j < K;
      const uint32_t h = in ? sc[j] : 0u;
      sv[j >> 1] |= (j & 1) ? (h << 16) : h;
      iv[j] = in ? ix[j] : -1;
    }
  }
  // The bias of every slot is loaded (chunk 0 for a masked slot), so the
  // gathers need no divergent branches.
  float x[8];
  float rmax = neg_inf();
  const float* brow = bias + (b * C * (I)Hkv + hk) * (I)G + g;  // chunk c at c * Hkv * G
  const I cstride = (I)(Hkv * G);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int32_t c = iv[j];
    const bool ok = (VEC || k0 + j < K) && c >= 0 && (I)c < C;
    const float bv = brow[(ok ? (I)c : (I)0) * cstride];
    const float s = (j & 1) ? bf16_hi(sv[j >> 1]) : bf16_lo(sv[j >> 1]);
    float y = s + bv;
    if constexpr (EX) {
      // clamped slots: every load unconditional (see the backward kernel)
      const I kk = r * (I)K + (I)min(k0 + j, K - 1);
      const float t1 = e1 ? e1[kk] : 0.f;
      const float t2 = e2 ? e2[kk] : 0.f;
      if (e1) y += t1;
      if (e2) y += t2;
    }
    x[j] = ok ? (UNIT_T ? y : y * inv_t) : neg_inf();
    rmax = fmaxf(rmax, x[j]);
  }
  rmax = row_lanes_max<LPR>(rmax);
  float local = lse[r];
  if (has_off && !affine) local -= off;
  if (!UNIT_T) local *= inv_t;

  // Every lane of a row takes the same branch (m and rmax are row-uniform),
  // so the reductions inside the branches stay within active lanes.
  float lw_val = 0.f;
  // gate_logit (attention.py:196-235): lse(remote logits) - local logit, then
  // gate_scale * (.) + gate_offset in the affine form; 0 when every logit is
  // masked.  -inf (or its affine image) when only the remote ones are.
  // Exponentials and logarithms run in base 2 on the hardware instructions
  // (exp(y) = 2^(y log2 e)), quotients as products with the hardware
  // reciprocal: within a few fp32 ulps of the exact softmax.
  float gl_val = 0.f;
  const float m = fmaxf(rmax, local);
  if (m == neg_inf()) {  // every logit masked: both outputs zero
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = 0.f;
  } else if (!affine) {
    if (gate_logit) {
      // Remote LSE against its own max (torch.logsumexp's form), so a local
      // logit far above the remote ones cannot underflow it.
      float rs = 0.f;
      const float rb = rmax * kLog2e;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        rs += x[j] == neg_inf() ? 0.f : exp2_hw(__builtin_fmaf(x[j], kLog2e, -rb));
      rs = row_lanes_sum<LPR>(rs);
      gl_val = (rmax == neg_inf() ? neg_inf() : rmax + log2_hw(rs) * kLn2) - local;
    }
    const float mb = m * kLog2e;
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      x[j] = exp2_hw(__builtin_fmaf(x[j], kLog2e, -mb));  // -inf -> 0
      sum += x[j];
    }
    sum = row_lanes_sum<LPR>(sum);
    const float el = exp2_hw(__builtin_fmaf(local, kLog2e, -mb));
    sum += el;
    const float inv = rcp_hw(sum);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] *= inv;
    lw_val = el * inv;
  } else if (rmax == neg_inf()) {
    // Affine gate with no routed chunk: remote softmax zeroed, gate -> local.
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = 0.f;
    lw_val = 1.f;
    gl_val = gscale * (neg_inf() - local) + off;
  } else {
    const float rb = rmax * kLog2e;
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      x[j] = exp2_hw(__builtin_fmaf(x[j], kLog2e, -rb));  // -inf -> 0
      sum += x[j];
    }
    sum = row_lanes_sum<LPR>(sum);
    const float remote_lse = rmax + log2_hw(sum) * kLn2;
    const float gate = gscale * (remote_lse - local) + off;
    const float mass = rcp_hw(1.f + exp2_hw(-gate * kLog2e));
    const float f = rcp_hw(sum) * mass;
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] *= f;
    lw_val = 1.f - mass;
    gl_val = gate;
  }
  if (!live) return;
  if (gate_logit && part == 0) gate_logit[r] = gl_val;
  uint16_t* out = rw + r * (I)K + k0;
  if (VEC && k0 < K) {
    u32x4_t o4;
#pragma unroll
    for (int j = 0; j < 4; ++j) o4[j] = pack_bf16x2(x[2 * j], x[2 * j + 1]);
    *reinterpret_cast<u32x4_t*>(out) = o4;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (k0 + j < K) out[j] = (uint16_t)f32_to_bf16(x[j]);
  }
  if (part == 0) lw[r] = (uint16_t)f32_to_bf16(lw_val);
}

template <int LPR, bool VEC, bool UNIT_T, class I, bool EX>
__global__ void __launch_bounds__(256)
    route_weights_kernel(const uint16_t* __restrict__ scores, const int32_t* __restrict__ indices,
                         const float* __restrict__ bias, const float* __restrict__ lse,
                         int64_t rows, int64_t L, int64_t C, int Hkv, int G, int K, float inv_t,
                         const float* __restrict__ goff, const float* __restrict__ gsc,
                         uint16_t* __restrict__ rw, uint16_t* __restrict__ lw,
                         float* __restrict__ gate_logit, const float* __restrict__ e1,
                         const float* __restrict__ e2) {
  // Gate parameters are device scalars (the layer's parameters, read in
  // place: no host round trip); a null pointer means "not given".
  const int has_off = goff != nullptr, affine = gsc != nullptr;
  const float off = has_off ? *goff : 0.f;
  const float gscale = affine ? *gsc : 1.f;
  route_weights_row<LPR, VEC, UNIT_T, I, EX>((int64_t)blockIdx.x * blockDim.x + threadIdx.x, scores,
                                             indices, bias, lse, rows, L, C, Hkv, G, K, inv_t,
                                             has_off, affine, off, gscale, rw, lw, gate_logit, e1,
                                             e2);
}

template <int LPR>
int launch_rw(bool vec, hipStream_t s, const uint16_t* scores, const int32_t* indices,
              const float* bias, const float* lse, int64_t rows, int64_t L, int64_t C, int Hkv,
              int G, int K, float inv_t, const float* goff, const float* gsc, uint16_t* rw,
              uint16_t* lw, float* gate_logit, const float* e1, const float* e2) {
  const int64_t blocks = (rows * LPR + 255) / 256;
  if (blocks > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  // 32-bit indices when the largest flat index of the call fits
  const bool small = rows * LPR < ((int64_t)1 << 31) && rows * K < ((int64_t)1 << 31) &&
                     (rows / (Hkv * G) / L + 1) * C * Hkv * G < ((int64_t)1 << 31);
  // the common call (32-bit indices, vectors, temperature 1) has an
  // instance of its own
  // instance of its own; the additive terms take the general one
  auto kern = (e1 || e2) ? route_weights_kernel<LPR, false, false, int64_t, true>
              : small ? (vec ? (inv_t == 1.f ? route_weights_kernel<LPR, true, true, uint32_t, false>
                                             : route_weights_kernel<LPR, true, false, uint32_t, false>)
                             : route_weights_kernel<LPR, false, false, uint32_t, false>)
                      : (vec ? route_weights_kernel<LPR, true, false, int64_t, false>
                             : route_weights_kernel<LPR, false, false, int64_t, false>);
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, s, scores, indices, bias, lse,
                     rows, L, C, Hkv, G, K, inv_t, goff, gsc, rw, lw, gate_logit, e1, e2);
  return mrsa_launch_status();
}

}  // namespace

namespace {

int route_weights_fwd(const void* scores, const int32_t* indices, const float* prior_bias,
                      const float* local_lse, int64_t batch, int64_t seq_len, int64_t chunks,
                      int64_t kv_heads, int64_t groups, int64_t topk, float temperature,
                      const float* gate_offset, const float* gate_scale,
                      const float* value_bonus, const float* selected_gumbel,
                      void* remote_weights, void* local_weight, float* gate_logit,
                      void* stream) {
  if (batch < 0 || seq_len < 0 || chunks <= 0 || kv_heads <= 0 || groups <= 0 || topk <= 0 ||
      !(temperature > 0.f))
    return MRSA_ERR_INVALID_ARGUMENT;
  if (topk > kMaxTopk) return MRSA_ERR_UNSUPPORTED;
  const int64_t rows = batch * seq_len * kv_heads * groups;
  if (rows == 0) return MRSA_OK;
  if (!scores || !indices || !prior_bias || !local_lse || !remote_weights || !local_weight)
    return MRSA_ERR_INVALID_ARGUMENT;
  const bool vec = topk % 8 == 0 && ((uintptr_t)scores | (uintptr_t)indices |
                                     (uintptr_t)remote_weights) % 16 == 0;
  hipStream_t s = (hipStream_t)stream;
  const int lanes = (int)((topk + 7) / 8);
  auto go = [&](auto lpr) {
    return launch_rw<decltype(lpr)::value>(
        vec, s, (const uint16_t*)scores, indices, prior_bias, local_lse, rows, seq_len, chunks,
        (int)kv_heads, (int)groups, (int)topk, 1.f / temperature, gate_offset, gate_scale,
        (uint16_t*)remote_weights, (uint16_t*)local_weight, gate_logit, value_bonus,
        selected_gumbel);
  };
  if (lanes <= 1) return go(std::integral_constant<int, 1>{});
  if (lanes <= 2) return go(std::integral_constant<int, 2>{});
  if (lanes <= 4) return go(std::integral_constant<int, 4>{});
  return go(std::integral_constant<int, 8>{});
}

}  // namespace

extern "C" int mrsa_route_weights_fwd(const void* scores, const int32_t* indices,
                                      const float* prior_bias, const float* local_lse,
                                      int64_t batch, int64_t seq_len, int64_t chunks,
                                      int64_t kv_heads, int64_t groups, int64_t topk,
                                      float temperature, const float* gate_offset,
                                      const float* gate_scale, void* remote_weights,
                                      void* local_weight, float* gate_logit, void* stream) {
  return route_weights_fwd(scores, indices, prior_bias, local_lse, batch, seq_len, chunks,
                           kv_heads, groups, topk, temperature, gate_offset, gate_scale, nullptr,
                           nullptr, remote_weights, local_weight, gate_logit, stream);
}

extern "C" int mrsa_route_weights_extra_fwd(
    const void* scores, const int32_t* indices, const float* prior_bias, const float* local_lse,
    int64_t batch, int64_t seq_len, int64_t chunks, int64_t kv_heads, int64_t groups,
    int64_t topk, float temperature, const float* gate_offset, const float* gate_scale,
    const float* value_bonus, const float* selected_gumbel, void* remote_weights,
    void* local_weight, float* gate_logit, void* stream) {
  return route_weights_fwd(scores, indices, prior_bias, local_lse, batch, seq_len, chunks,
                           kv_heads, groups, topk, temperature, gate_offset, gate_scale,
                           value_bonus, selected_gumbel, remote_weights, local_weight, gate_logit,
                           stream);
}

namespace {

// Backward of the route weights with the forward's work split (LPR lanes per
// (token, query head) row, 8 slots per lane); the row's logits and
// probabilities are recomputed rather than saved.
//   plain form (the TileLang backward, ops/hils_bidir_route_weights_tilelang.py:97-166,
//   generalised to temperature T):  dz = p (g - sum p g),  d logit = dz / T,
//     d local_lse = dz_local / T, d gate_offset = -d local_lse
//   affine form (autograd of _route_weights_torch, attention.py:180-214):
//     q = softmax(remote / T), mass = sigmoid(s (lse(remote / T) - local / T) + o)
//     dm = sum g_j q_j - g_local,  dgate = dm mass (1 - mass)
//     dz_j = q_j (g_j mass - sum_k q_k g_k mass) + dgate s q_j,  d remote_j = dz_j / T
//     d local_lse = -dgate s / T,  d s = sum dgate (lse - local / T),  d o = sum dgate
// With an upstream gradient gG of the gate logit (attention.py:196-235) the
// plain form adds gG q_j / T to d remote_j (q = softmax of the remote logits)
// and -gG / T to d local_lse; the affine form adds gG to dgate.
// Rows whose outputs are constant (every logit masked; affine form with no
// routed chunk) get zero gradients.  Gradients of the selected bias entries
// are added atomically into d_bias, and the gate gradients into d_gate[0..1]
// once per wave; both are zeroed by the caller.
template <int LPR>
__global__ void __launch_bounds__(256)
    route_weights_bwd_kernel(const uint16_t* __restrict__ scores,
                             const int32_t* __restrict__ indices, const float* __restrict__ bias,
                             const float* __restrict__ lse, const uint16_t* __restrict__ g_rw,
                             const uint16_t* __restrict__ g_lw, const float* __restrict__ g_gl,
                             int64_t rows, int64_t L, int64_t C, int Hkv, int G, int K,
                             float inv_t, const float* __restrict__ goff,
                             const float* __restrict__ gsc, const float* __restrict__ e1,
                             const float* __restrict__ e2, float* __restrict__ d_scores,
                             float* __restrict__ d_bias, float* __restrict__ d_lse,
                             float* __restrict__ d_gate) {
  const int has_off = goff != nullptr, affine = gsc != nullptr;
  const float off = has_off ? *goff : 0.f;
  const float gscale = affine ? *gsc : 1.f;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int part = (int)(t % LPR);
  const int64_t r0 = t / LPR;
  const bool live = r0 < rows;
  const int64_t r = live ? r0 : rows - 1;  // lanes past the end join the reductions
  const int Hq = Hkv * G;
  const int hq = (int)(r % Hq);
  const int64_t bl = r / Hq;
  const int64_t b = bl / L;
  const int hk = hq / G, g = hq - hk * G;
  const int k0 = part * 8;
  const int32_t* ix = indices + (bl * Hkv + hk) * K + k0;

  // Loads are unconditional (clamped slots and chunks) and issued together:
  // loads inside per-slot branches were each waited for at the branch end.
  int32_t iv[8];
  float x[8], gr[8];
  float rmax = neg_inf();
  const int64_t kl = K - 1;
#pragma unroll
  for (int j = 0; j < 8; ++j) iv[j] = ix[min((int64_t)j, kl - k0)];
  float sc[8], bv[8], ex1[8], ex2[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t kk = r * K + min((int64_t)(k0 + j), kl);
    const bool ok = iv[j] >= 0 && iv[j] < C;
    gr[j] = bf16_to_f32(g_rw[kk]);
    sc[j] = bf16_to_f32(scores[kk]);
    bv[j] = bias[((b * C + (ok ? iv[j] : 0)) * Hkv + hk) * G + g];
    ex1[j] = e1 ? e1[kk] : 0.f;
    ex2[j] = e2 ? e2[kk] : 0.f;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const bool in = k0 + j < K;
    if (!in) iv[j] = -1;
    if (!in) gr[j] = 0.f;
    float y = sc[j] + bv[j];
    if (e1) y += ex1[j];
    if (e2) y += ex2[j];
    const float v = in && iv[j] >= 0 && iv[j] < C ? y * inv_t : neg_inf();
    x[j] = v;
    rmax = fmaxf(rmax, v);
  }
#pragma unroll
  for (int o = 1; o < LPR; o <<= 1) rmax = fmaxf(rmax, __shfl_xor(rmax, o, 64));
  float local = lse[r];
  if (has_off && !affine) local -= off;
  local *= inv_t;
  const float gl = g_lw ? bf16_to_f32(g_lw[r]) : 0.f;
  const float gG = g_gl ? g_gl[r] : 0.f;

  // Branches are row-uniform, so the lane reductions inside stay within
  // active lanes.
  float dloc = 0.f, dscale = 0.f, doff = 0.f;
  const float m = fmaxf(rmax, local);
  if (m == neg_inf() || (affine && rmax == neg_inf())) {
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = 0.f;
  } else if (!affine) {
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      x[j] = x[j] == neg_inf() ? 0.f : expf(x[j] - m);
      sum += x[j];
    }
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) sum += __shfl_xor(sum, o, 64);
    const float el = local == neg_inf() ? 0.f : expf(local - m);
    sum += el;
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      x[j] /= sum;
      dot += x[j] * gr[j];
    }
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) dot += __shfl_xor(dot, o, 64);
    const float pl = el / sum;
    dot += pl * gl;
    // q_j = e_j / sum_remote e = x_j * sum / (sum - el); no remote chunk: 0.
    const float rs = sum - el;
    const float qf = rs > 0.f ? sum / rs : 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = (x[j] * (gr[j] - dot) + gG * x[j] * qf) * inv_t;
    dloc = (pl * (gl - dot) - gG) * inv_t;
    doff = has_off ? -dloc : 0.f;
  } else {
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      x[j] = x[j] == neg_inf() ? 0.f : expf(x[j] - rmax);
      sum += x[j];
    }
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) sum += __shfl_xor(sum, o, 64);
    const float rl = rmax + logf(sum);
    const float gate = gscale * (rl - local) + (has_off ? off : 0.f);
    const float mass = 1.f / (1.f + expf(-gate));
    float qg = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      x[j] /= sum;
      qg += x[j] * gr[j];
    }
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) qg += __shfl_xor(qg, o, 64);
    const float dgate = (qg - gl) * mass * (1.f - mass) + gG;
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = x[j] * ((gr[j] - qg) * mass + dgate * gscale) * inv_t;
    dloc = -dgate * gscale * inv_t;
    dscale = dgate * (rl - local);
    doff = has_off ? dgate : 0.f;
  }
  if (live) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (k0 + j >= K) continue;
      const bool valid = iv[j] >= 0 && iv[j] < C;
      d_scores[r * K + k0 + j] = valid ? x[j] : 0.f;
      if (valid && x[j] != 0.f) atomicAdd(&d_bias[((b * C + iv[j]) * Hkv + hk) * G + g], x[j]);
    }
    if (part == 0) d_lse[r] = dloc;
  }
  if (d_gate) {
    const bool mine = live && part == 0;
    dscale = wave_sum(mine ? dscale : 0.f);
    doff = wave_sum(mine ? doff : 0.f);
    if ((threadIdx.x & 63) == 0) {
      if (affine) atomicAdd(&d_gate[0], dscale);
      if (has_off) atomicAdd(&d_gate[1], doff);
    }
  }
}

}  // namespace

namespace {

int route_weights_bwd(const void* scores, const int32_t* indices, const float* prior_bias,
                      const float* local_lse, const void* grad_remote, const void* grad_local,
                      const float* grad_gate_logit, int64_t batch, int64_t seq_len,
                      int64_t chunks, int64_t kv_heads, int64_t groups, int64_t topk,
                      float temperature, const float* gate_offset, const float* gate_scale,
                      const float* value_bonus, const float* selected_gumbel, float* d_scores,
                      float* d_bias, float* d_local_lse, float* d_gate, void* stream) {
  if (batch < 0 || seq_len < 0 || chunks <= 0 || kv_heads <= 0 || groups <= 0 || topk <= 0 ||
      !(temperature > 0.f))
    return MRSA_ERR_INVALID_ARGUMENT;
  if (topk > kMaxTopk) return MRSA_ERR_UNSUPPORTED;
  const int64_t rows = batch * seq_len * kv_heads * groups;
  if (rows == 0) return MRSA_OK;
  if (!scores || !indices || !prior_bias || !local_lse || !grad_remote || !d_scores || !d_bias ||
      !d_local_lse || ((gate_scale || gate_offset) && !d_gate))
    return MRSA_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  const int lanes = (int)((topk + 7) / 8);
  auto go = [&](auto lpr) {
    constexpr int LPR = decltype(lpr)::value;
    const int64_t blocks = (rows * LPR + 255) / 256;
    if (blocks > 0x7fffffff) return (int)MRSA_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(route_weights_bwd_kernel<LPR>, dim3((unsigned)blocks), dim3(256), 0, s,
                       (const uint16_t*)scores, indices, prior_bias, local_lse,
                       (const uint16_t*)grad_remote, (const uint16_t*)grad_local,
                       grad_gate_logit, rows, seq_len, chunks, (int)kv_heads, (int)groups,
                       (int)topk, 1.f / temperature, gate_offset, gate_scale, value_bonus,
                       selected_gumbel, d_scores, d_bias, d_local_lse,
                       (gate_scale || gate_offset) ? d_gate : nullptr);
    return mrsa_launch_status();
  };
  if (lanes <= 1) return go(std::integral_constant<int, 1>{});
  if (lanes <= 2) return go(std::integral_constant<int, 2>{});
  if (lanes <= 4) return go(std::integral_constant<int, 4>{});
  return go(std::integral_constant<int, 8>{});
}

}  // namespace

extern "C" int mrsa_route_weights_bwd(const void* scores, const int32_t* indices,
                                      const float* prior_bias, const float* local_lse,
                                      const void* grad_remote, const void* grad_local,
                                      const float* grad_gate_logit, int64_t batch,
                                      int64_t seq_len, int64_t chunks, int64_t kv_heads,
                                      int64_t groups, int64_t topk, float temperature,
                                      const float* gate_offset, const float* gate_scale,
                                      float* d_scores, float* d_bias, float* d_local_lse,
                                      float* d_gate, void* stream) {
  return route_weights_bwd(scores, indices, prior_bias, local_lse, grad_remote, grad_local,
                           grad_gate_logit, batch, seq_len, chunks, kv_heads, groups, topk,
                           temperature, gate_offset, gate_scale, nullptr, nullptr, d_scores,
                           d_bias, d_local_lse, d_gate, stream);
}

extern "C" int mrsa_route_weights_extra_bwd(
    const void* scores, const int32_t* indices, const float* prior_bias, const float* local_lse,
    const void* grad_remote, const void* grad_local, const float* grad_gate_logit,
    int64_t batch, int64_t seq_len, int64_t chunks, int64_t kv_heads, int64_t groups,
    int64_t topk, float temperature, const float* gate_offset, const float* gate_scale,
    const float* value_bonus, const float* selected_gumbel, float* d_scores, float* d_bias,
    float* d_local_lse, float* d_gate, void* stream) {
  return route_weights_bwd(scores, indices, prior_bias, local_lse, grad_remote, grad_local,
                           grad_gate_logit, batch, seq_len, chunks, kv_heads, groups, topk,
                           temperature, gate_offset, gate_scale, value_bonus, selected_gumbel,
                           d_scores, d_bias, d_local_lse, d_gate, stream);
}
