// Decoder-layer glue around the attention path of the Dream-7B-shaped model:
// residual add + RMSNorm, rotary embedding of the fused QKV projection (with
// the Q-Cal routing-query finish), and the SwiGLU activation.  The GEMMs run
// on hipBLASLt through torch; these kernels are the elementwise passes
// between them, each a single HBM stream.
//
// Rounding points follow the reference modules (bf16 storage between ops):
//   * Qwen2 RMSNorm: fp32 normalisation, rounded to bf16, then the bf16
//     weight product rounded again; the residual sum is a bf16 add.
//   * rotary embedding: fp32 products with fp32 cos/sin tables (the YaRN
//     attention factor already folded in), one bf16 rounding per element.
//   * Q-Cal (dream_dllm_hils/attention.py:477-511, qcal.py:22-26):
//     route_q = rope(rms_norm(q_unrotated + delta) * w) with an fp32 weight
//     product; q_unrotated is the pre-rotation projection itself.
//   * SwiGLU: bf16(silu(gate)) * up, rounded to bf16.
#include "mrsa_device.h"

using namespace mrsa;

namespace {

constexpr int kNormThreads = 256;

template <int MAXV>
__global__ void __launch_bounds__(kNormThreads)
    add_rms_norm_kernel(const u32x4_t* __restrict__ x, const u32x4_t* __restrict__ res,
                        const uint16_t* __restrict__ w, int V, float inv_h, float eps,
                        u32x4_t* __restrict__ sum_out, u32x4_t* __restrict__ out) {
  __shared__ float red[kNormThreads / 64];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  float val[MAXV][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int v = tid + i * kNormThreads;
    if (v >= V) continue;
    const u32x4_t a = x[row * V + v];
    u32x4_t s = a;
    if (res) {
      const u32x4_t b = res[row * V + v];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        s[j] = pack_bf16x2(bf16_lo(a[j]) + bf16_lo(b[j]), bf16_hi(a[j]) + bf16_hi(b[j]));
      if (sum_out) sum_out[row * V + v] = s;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      val[i][2 * j] = bf16_lo(s[j]);
      val[i][2 * j + 1] = bf16_hi(s[j]);
      ss = fmaf(val[i][2 * j], val[i][2 * j], ss);
      ss = fmaf(val[i][2 * j + 1], val[i][2 * j + 1], ss);
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) tot += red[i];
  const float r = rsqrtf(tot * inv_h + eps);
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int v = tid + i * kNormThreads;
    if (v >= V) continue;
    const u32x4_t wv = reinterpret_cast<const u32x4_t*>(w)[v];
    u32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float n0 = bf16_to_f32(f32_to_bf16(val[i][2 * j] * r));
      const float n1 = bf16_to_f32(f32_to_bf16(val[i][2 * j + 1] * r));
      o[j] = pack_bf16x2(bf16_lo(wv[j]) * n0, bf16_hi(wv[j]) * n1);
    }
    out[row * V + v] = o;
  }
}

// One wave per (token, head) of the fused projection [L, (Hq + 2 Hkv) * 128]:
// lane i holds elements i and i + 64, the pair rotate_half couples.
__global__ void __launch_bounds__(256)
    rope_qkv_kernel(const uint16_t* __restrict__ qkv, const float* __restrict__ cos_t,
                    const float* __restrict__ sin_t, const uint16_t* __restrict__ delta,
                    const float* __restrict__ qnorm_w, float qnorm_eps, int64_t L, int Hq,
                    int Hkv, uint16_t* __restrict__ q, uint16_t* __restrict__ k,
                    uint16_t* __restrict__ v, uint16_t* __restrict__ route_q) {
  constexpr int D = 128;
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  const int heads = Hq + 2 * Hkv;
  if (wave >= L * heads) return;  // wave-uniform
  const int64_t t = wave / heads;
  const int h = (int)(wave - t * heads);
  const uint16_t* src = qkv + wave * D;
  const float x0 = bf16_to_f32(src[lane]), x1 = bf16_to_f32(src[lane + 64]);
  if (h >= Hq + Hkv) {  // value head: copy
    uint16_t* dst = v + (t * Hkv + (h - Hq - Hkv)) * D;
    dst[lane] = src[lane];
    dst[lane + 64] = src[lane + 64];
    return;
  }
  const float c = cos_t[t * 64 + lane], s = sin_t[t * 64 + lane];
  uint16_t* dst = h < Hq ? q + (t * Hq + h) * D : k + (t * Hkv + (h - Hq)) * D;
  dst[lane] = (uint16_t)f32_to_bf16(x0 * c - x1 * s);
  dst[lane + 64] = (uint16_t)f32_to_bf16(x1 * c + x0 * s);
  if (h < Hq && delta) {
    const uint16_t* dr = delta + (t * Hq + h) * D;
    const float c0 = bf16_to_f32(f32_to_bf16(x0 + bf16_to_f32(dr[lane])));
    const float c1 = bf16_to_f32(f32_to_bf16(x1 + bf16_to_f32(dr[lane + 64])));
    const float r = rsqrtf(wave_sum(c0 * c0 + c1 * c1) * (1.f / D) + qnorm_eps);
    const float n0 = bf16_to_f32(f32_to_bf16(qnorm_w[lane] * (c0 * r)));
    const float n1 = bf16_to_f32(f32_to_bf16(qnorm_w[lane + 64] * (c1 * r)));
    uint16_t* rq = route_q + (t * Hq + h) * D;
    rq[lane] = (uint16_t)f32_to_bf16(n0 * c - n1 * s);
    rq[lane + 64] = (uint16_t)f32_to_bf16(n1 * c + n0 * s);
  }
}

__global__ void __launch_bounds__(256)
    swiglu_kernel(const u32x4_t* __restrict__ gate_up, int64_t rows, int Vi,
                  u32x4_t* __restrict__ out) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= rows * Vi) return;
  const int64_t row = e / Vi;
  const int c = (int)(e - row * Vi);
  const u32x4_t g = gate_up[row * 2 * Vi + c];
  const u32x4_t u = gate_up[row * 2 * Vi + Vi + c];
  u32x4_t o;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float g0 = bf16_lo(g[j]), g1 = bf16_hi(g[j]);
    const float a0 = bf16_to_f32(f32_to_bf16(g0 / (1.f + expf(-g0))));
    const float a1 = bf16_to_f32(f32_to_bf16(g1 / (1.f + expf(-g1))));
    o[j] = pack_bf16x2(a0 * bf16_lo(u[j]), a1 * bf16_hi(u[j]));
  }
  out[e] = o;
}

}  // namespace

extern "C" int mrsa_add_rms_norm_fwd(const void* x, const void* residual, const void* weight,
                                     int64_t rows, int64_t hidden, float eps, void* sum_out,
                                     void* out, void* stream) {
  if (rows < 0 || hidden <= 0 || hidden % 8 != 0 || !(eps >= 0.f))
    return MRSA_ERR_INVALID_ARGUMENT;
  if (rows == 0) return MRSA_OK;
  if (!x || !weight || !out || (sum_out && !residual)) return MRSA_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)x | (uintptr_t)residual | (uintptr_t)weight | (uintptr_t)sum_out |
       (uintptr_t)out) % 16 != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (hidden > 8 * 4 * kNormThreads) return MRSA_ERR_UNSUPPORTED;
  if (rows > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  const int V = (int)(hidden / 8);
  auto kern = V <= 2 * kNormThreads ? add_rms_norm_kernel<2> : add_rms_norm_kernel<4>;
  hipLaunchKernelGGL(kern, dim3((unsigned)rows), dim3(kNormThreads), 0, (hipStream_t)stream,
                     (const u32x4_t*)x, (const u32x4_t*)residual, (const uint16_t*)weight, V,
                     1.f / (float)hidden, eps, (u32x4_t*)sum_out, (u32x4_t*)out);
  return mrsa_launch_status();
}

extern "C" int mrsa_rope_qkv_fwd(const void* qkv, const float* cos_table, const float* sin_table,
                                 const void* qcal_delta, const float* qcal_norm_weight,
                                 float qcal_eps, int64_t tokens, int64_t q_heads,
                                 int64_t kv_heads, int64_t head_dim, void* q, void* k, void* v,
                                 void* route_q, void* stream) {
  if (tokens < 0 || q_heads <= 0 || kv_heads <= 0) return MRSA_ERR_INVALID_ARGUMENT;
  if (head_dim != 128) return MRSA_ERR_UNSUPPORTED;
  if (tokens == 0) return MRSA_OK;
  if (!qkv || !cos_table || !sin_table || !q || !k || !v) return MRSA_ERR_INVALID_ARGUMENT;
  if (qcal_delta && (!qcal_norm_weight || !route_q)) return MRSA_ERR_INVALID_ARGUMENT;
  const int64_t waves = tokens * (q_heads + 2 * kv_heads);
  const int64_t blocks = (waves + 3) / 4;
  if (blocks > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(rope_qkv_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)qkv, cos_table, sin_table, (const uint16_t*)qcal_delta,
                     qcal_norm_weight, qcal_eps, tokens, (int)q_heads, (int)kv_heads,
                     (uint16_t*)q, (uint16_t*)k, (uint16_t*)v, (uint16_t*)route_q);
  return mrsa_launch_status();
}

extern "C" int mrsa_swiglu_fwd(const void* gate_up, int64_t rows, int64_t intermediate, void* out,
                               void* stream) {
  if (rows < 0 || intermediate <= 0 || intermediate % 8 != 0) return MRSA_ERR_INVALID_ARGUMENT;
  if (rows == 0) return MRSA_OK;
  if (!gate_up || !out || ((uintptr_t)gate_up | (uintptr_t)out) % 16 != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  const int64_t n = rows * (intermediate / 8);
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const u32x4_t*)gate_up, rows, (int)(intermediate / 8), (u32x4_t*)out);
  return mrsa_launch_status();
}
