// Landmark (mask-token) chunk-summary attention pool.
//
// One workgroup per (chunk, KV head).  The chunk's keys are staged in LDS once
// and shared by the `groups` query heads of that KV group.  Semantics follow
// the fused reference kernel ops/chunk_attn_pool_gqa_tilelang.py:47-180:
//   * the chunk counts as valid iff any of its first chunk_size-1 keys is valid
//     (:94-99);
//   * logits = (mu_q . k) * sm_scale over the chunk_size-1 real keys; a masked
//     slot gets -inf, except slot 0, which gets logit 0 (:118-129);
//   * probabilities are normalised in fp32; the entropy -sum p ln p uses the
//     fp32 probabilities (:142-149), the pooled key uses them rounded to bf16
//     (P_shared is bf16, :151-158), accumulated in fp32 and rounded to bf16;
//   * an invalid chunk writes zero keys and zero entropy (:161-178).
// With dense_torch_semantics the compiled torch twin _compact_pool_torch
// (:17-37) is followed instead: every masked slot is -inf, a fully masked
// chunk gives zero probabilities (nan_to_num) and the pooling uses fp32
// probabilities.
#include "mrsa_device.h"
#include "pool_wave.h"

using namespace mrsa;

namespace {

constexpr int kThreads = 256;

__global__ void __launch_bounds__(kThreads)
    pool_kernel(const uint16_t* __restrict__ mu_q, int64_t mu_stride,
                const uint16_t* __restrict__ kc, const uint8_t* __restrict__ key_valid, int S,
                int H, int G, int D,
                float sm_scale, int dense, const float* __restrict__ bias_scale,
                uint16_t* __restrict__ lmk, float* __restrict__ entropy,
                float* __restrict__ prior) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int64_t bc = blockIdx.x;
  const int h = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;

  uint16_t* ks = reinterpret_cast<uint16_t*>(smem);    // [S][D] bf16
  float* qs = reinterpret_cast<float*>(ks + S * D);     // [G][D]
  float* ps = qs + G * D;                               // [G][S] logits -> probabilities
  float* pw = ps + G * S;                               // [G][S] pooling weights
  int* flag = reinterpret_cast<int*>(pw + G * S);
  unsigned char* vs = reinterpret_cast<unsigned char*>(flag + 1);  // [S]

  const int vec_per_row = D / 8;
  for (int v = tid; v < S * vec_per_row; v += kThreads) {
    const int s = v / vec_per_row, c = v - s * vec_per_row;
    const u32x4_t* src =
        reinterpret_cast<const u32x4_t*>(kc + ((bc * S + s) * H + h) * (int64_t)D) + c;
    reinterpret_cast<u32x4_t*>(ks + s * D)[c] = *src;
  }
  for (int e = tid; e < G * D; e += kThreads)
    qs[e] = bf16_to_f32(mu_q[bc * mu_stride + (int64_t)(h * G) * D + e]);
  if (tid == 0) flag[0] = 0;
  for (int s = tid; s < S; s += kThreads) vs[s] = key_valid[bc * S + s] != 0;
  __syncthreads();
  if (tid < S - 1 && vs[tid]) flag[0] = 1;
  __syncthreads();
  const bool chunk_valid = flag[0] != 0;

  // Logits: each thread owns (g, s) pairs; the start of the reduction over d
  // is staggered by s (in units of 8) so neighbouring threads hit different
  // LDS banks.  K and q move as 16-byte LDS reads, 8 elements at a time,
  // accumulated one by one in d order (D % 8 == 0).
  for (int p = tid; p < G * S; p += kThreads) {
    const int g = p / S, s = p - g * S;
    const float* qr = qs + g * D;
    const uint16_t* kr = ks + s * D;
    int d = (s * 8) % D;
    float acc = 0.f;
    for (int i = 0; i < D; i += 8) {
      const u32x4_t w = *reinterpret_cast<const u32x4_t*>(kr + d);
      const f32x4_t qa = *reinterpret_cast<const f32x4_t*>(qr + d);
      const f32x4_t qb = *reinterpret_cast<const f32x4_t*>(qr + d + 4);
      acc = fmaf(qa[0], bf16_lo(w[0]), acc);
      acc = fmaf(qa[1], bf16_hi(w[0]), acc);
      acc = fmaf(qa[2], bf16_lo(w[1]), acc);
      acc = fmaf(qa[3], bf16_hi(w[1]), acc);
      acc = fmaf(qb[0], bf16_lo(w[2]), acc);
      acc = fmaf(qb[1], bf16_hi(w[2]), acc);
      acc = fmaf(qb[2], bf16_lo(w[3]), acc);
      acc = fmaf(qb[3], bf16_hi(w[3]), acc);
      d += 8;
      if (d >= D) d -= D;
    }
    const bool real = (s < S - 1) && vs[s];
    float logit;
    if (dense) {
      logit = real ? acc * sm_scale : neg_inf();
    } else {
      logit = (real && chunk_valid) ? acc * sm_scale : (s == 0 ? 0.f : neg_inf());
    }
    ps[p] = logit;
  }
  __syncthreads();

  // Softmax + entropy per query head: one wave per head.
  for (int g = wave; g < G; g += kThreads / 64) {
    const float v0 = lane < S ? ps[g * S + lane] : neg_inf();
    const float v1 = lane + 64 < S ? ps[g * S + lane + 64] : neg_inf();
    const float m = wave_max(fmaxf(v0, v1));
    float e0 = 0.f, e1 = 0.f;
    if (m != neg_inf()) {
      e0 = (lane < S && v0 != neg_inf()) ? exp2f((v0 - m) * kLog2e) : 0.f;
      e1 = (lane + 64 < S && v1 != neg_inf()) ? exp2f((v1 - m) * kLog2e) : 0.f;
    }
    const float sum = wave_sum(e0 + e1);
    const float p0 = sum > 0.f ? e0 / sum : 0.f;
    const float p1 = sum > 0.f ? e1 / sum : 0.f;
    const float t = (p0 > 0.f ? p0 * logf(p0) : 0.f) + (p1 > 0.f ? p1 * logf(p1) : 0.f);
    const float ent = -wave_sum(t);
    if (lane < S) pw[g * S + lane] = dense ? p0 : bf16_to_f32(f32_to_bf16(p0));
    if (lane + 64 < S) pw[g * S + lane + 64] = dense ? p1 : bf16_to_f32(f32_to_bf16(p1));
    if (lane == 0) {
      const float e_out = (dense || chunk_valid) ? ent : 0.f;
      const int64_t o = (bc * H + h) * G + g;
      entropy[o] = e_out;
      if (prior) prior[o] = e_out * bias_scale[h * G + g];
    }
  }
  __syncthreads();

  // Pooled key: lmk[g][d] = sum_s w[g][s] * k[s][d], fp32 accumulation in s
  // order; each thread owns 8 consecutive d of one head (16-byte K reads).
  const int dv = D / 8;
  uint16_t* lbase = lmk + ((bc * H + h) * G) * (int64_t)D;
  const bool lvec = ((uintptr_t)lmk & 15) == 0;
  for (int p = tid; p < G * dv; p += kThreads) {
    const int g = p / dv, c = p - g * dv;
    const float* wr = pw + g * S;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < S; ++s) {
      const u32x4_t kv = *reinterpret_cast<const u32x4_t*>(ks + s * D + 8 * c);
      const float w = wr[s];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] = fmaf(w, bf16_lo(kv[j]), acc[2 * j]);
        acc[2 * j + 1] = fmaf(w, bf16_hi(kv[j]), acc[2 * j + 1]);
      }
    }
    if (!dense && !chunk_valid)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = 0.f;
    uint16_t* dst = lbase + g * D + 8 * c;
    if (lvec) {
      u32x4_t o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = pack_bf16x2(acc[2 * j], acc[2 * j + 1]);
      *reinterpret_cast<u32x4_t*>(dst) = o;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) dst[j] = (uint16_t)f32_to_bf16(acc[j]);
    }
  }
}


// Matrix-core pool for the fused semantics at chunk_size 64, head_dim 128 and
// up to 16 query heads per KV head: one wave per (chunk, KV head), four per
// workgroup, the same formulas as pool_kernel above (pool_wave).  The
// chunk's 64 key rows are staged in the wave's LDS rows (256 bytes per key;
// 16-byte block b of a row stored at b ^ (key & 15)).
constexpr int kPoolWaves = 4;

__device__ __forceinline__ int pool_blk(int key, int blk) { return blk ^ (key & 15); }

struct SwizzledRows {
  const uint16_t* ks;
  __device__ u32x4_t row16(int key, int blk) const {
    return *reinterpret_cast<const u32x4_t*>(ks + key * 128 + 8 * pool_blk(key, blk));
  }
  __device__ uint32_t elem(int key, int dim) const {
    return ks[key * 128 + 8 * pool_blk(key, dim >> 3) + (dim & 7)];
  }
};

__global__ void __launch_bounds__(64 * kPoolWaves)
    pool_mfma_kernel(const uint16_t* __restrict__ mu_q, int64_t mu_stride,
                     const uint16_t* __restrict__ kc, const uint8_t* __restrict__ key_valid,
                     int H, int G, int64_t units, float sm_scale,
                     const float* __restrict__ bias_scale, uint16_t* __restrict__ lmk,
                     float* __restrict__ entropy, float* __restrict__ prior) {
  __shared__ __attribute__((aligned(16))) uint16_t ks_all[kPoolWaves][64 * 128];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t unit = (int64_t)blockIdx.x * kPoolWaves + wave;
  if (unit >= units) return;  // wave-uniform; no workgroup barrier below
  const int64_t bc = unit / H;
  const int h = (int)(unit - bc * H);
  const int j = lane & 15, grp = lane >> 4;
  uint16_t* ks = ks_all[wave];
  // key rows -> LDS: segment 64 i + lane = key 4 i + grp, dims 8 j ..
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int key = 4 * i + grp;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(kc + ((bc * 64 + key) * H + h) * 128 + 8 * j);
    *reinterpret_cast<u32x4_t*>(ks + key * 128 + 8 * pool_blk(key, j)) = v;
  }
  u32x4_t Qb[4];
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    Qb[q4] = u32x4_t{0u, 0u, 0u, 0u};
    if (j < G)
      Qb[q4] = *reinterpret_cast<const u32x4_t*>(mu_q + bc * mu_stride + (int64_t)(h * G + j) * 128 +
                                                 32 * q4 + 8 * grp);
  }
  const uint64_t vbits = __builtin_amdgcn_ballot_w64(key_valid[bc * 64 + lane] != 0);
  // The staged rows are read by this wave only (LDS keeps its order).
  pool_wave(SwizzledRows{ks}, Qb, vbits & ~(1ull << 63), G, sm_scale, (bc * H + h) * G,
            bias_scale, h * G, lmk, entropy, prior, lane);
}

// Landmark refresh of listed chunks of a K/V cache in place (the cached block
// step, fastdllm_attention.py:236-292): for listed chunk c of batch b, the
// routing query row whose position is c * 64 + 63 (found by a binary search
// of the sorted query positions), the chunk's 64 key rows and valid bytes
// read straight from the cache, the pool written into the cache's landmark
// keys and prior bias at chunk c.  One wave per (batch, listed chunk, KV
// head), the same wave math as pool_mfma_kernel.  A listed chunk outside
// [0, C) or whose landmark position is not a query position is skipped.
__global__ void __launch_bounds__(64 * kPoolWaves)
    pool_cached_kernel(const uint16_t* __restrict__ route_q, const int64_t* __restrict__ qpos,
                       int64_t Lq, const uint16_t* __restrict__ key,
                       const uint8_t* __restrict__ key_valid, int64_t L,
                       const int64_t* __restrict__ chunks, int64_t n, int H, int G,
                       int64_t units, float sm_scale, const float* __restrict__ bias_scale,
                       uint16_t* __restrict__ lmk, float* __restrict__ prior) {
  __shared__ __attribute__((aligned(16))) uint16_t ks_all[kPoolWaves][64 * 128];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t unit = (int64_t)blockIdx.x * kPoolWaves + wave;
  if (unit >= units) return;  // wave-uniform; no workgroup barrier below
  const int64_t bi = unit / H;
  const int h = (int)(unit - bi * H);
  const int64_t b = bi / n;
  const int64_t c = chunks[bi - b * n];
  const int64_t C = L / 64;
  if (c < 0 || c >= C) return;
  const int64_t pos = c * 64 + 63;
  int64_t lo = 0, hi = Lq;  // first query position >= pos
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (qpos[mid] < pos)
      lo = mid + 1;
    else
      hi = mid;
  }
  if (lo == Lq || qpos[lo] != pos) return;
  const int j = lane & 15, grp = lane >> 4;
  uint16_t* ks = ks_all[wave];
  const int64_t bc = b * C + c;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int kk = 4 * i + grp;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(key + ((bc * 64 + kk) * H + h) * 128 + 8 * j);
    *reinterpret_cast<u32x4_t*>(ks + kk * 128 + 8 * pool_blk(kk, j)) = v;
  }
  u32x4_t Qb[4];
  const uint16_t* qrow = route_q + ((b * Lq + lo) * H * G + (int64_t)h * G) * 128;
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    Qb[q4] = u32x4_t{0u, 0u, 0u, 0u};
    if (j < G) Qb[q4] = *reinterpret_cast<const u32x4_t*>(qrow + j * 128 + 32 * q4 + 8 * grp);
  }
  const uint64_t vbits = __builtin_amdgcn_ballot_w64(key_valid[bc * 64 + lane] != 0);
  pool_wave(SwizzledRows{ks}, Qb, vbits & ~(1ull << 63), G, sm_scale, bc * H * G + h * G,
            bias_scale, h * G, lmk, nullptr, prior, lane);
}
}  // namespace

namespace {

int pool_forward(const void* mu_q, int64_t mu_row_stride, const void* k_chunked,
                 const uint8_t* key_valid, int64_t batch_chunks, int64_t chunk_size,
                 int64_t kv_heads, int64_t groups, int64_t head_dim, float sm_scale,
                 int dense_torch_semantics, const float* bias_scale, void* landmark_keys,
                 float* entropy, float* prior_bias, void* stream) {
  if (batch_chunks < 0 || chunk_size < 2 || chunk_size > 128 || kv_heads <= 0 || groups <= 0 ||
      groups > 16 || head_dim <= 0 || head_dim > 256 || head_dim % 8 != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (mu_row_stride < kv_heads * groups * head_dim) return MRSA_ERR_INVALID_ARGUMENT;
  if ((prior_bias != nullptr) != (bias_scale != nullptr)) return MRSA_ERR_INVALID_ARGUMENT;
  if (batch_chunks == 0) return MRSA_OK;
  if (!mu_q || !k_chunked || !key_valid || !landmark_keys || !entropy)
    return MRSA_ERR_INVALID_ARGUMENT;
  if ((uintptr_t)k_chunked % 16 != 0) return MRSA_ERR_INVALID_ARGUMENT;
  if (batch_chunks > 0x7fffffff || kv_heads > 65535) return MRSA_ERR_UNSUPPORTED;
  const int S = (int)chunk_size, G = (int)groups, D = (int)head_dim;
  if (!dense_torch_semantics && S == 64 && D == 128 && G <= 16 &&
      ((uintptr_t)mu_q | (uintptr_t)landmark_keys) % 16 == 0 && mu_row_stride % 8 == 0) {
    const int64_t units = batch_chunks * kv_heads;
    const int64_t blocks = (units + kPoolWaves - 1) / kPoolWaves;
    if (blocks > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(pool_mfma_kernel, dim3((unsigned)blocks), dim3(64 * kPoolWaves), 0,
                       (hipStream_t)stream, (const uint16_t*)mu_q, mu_row_stride,
                       (const uint16_t*)k_chunked, key_valid, (int)kv_heads, G, units, sm_scale,
                       bias_scale, (uint16_t*)landmark_keys, entropy, prior_bias);
    return mrsa_launch_status();
  }
  const size_t smem = (size_t)S * D * 2 + (size_t)G * D * 4 + 2 * (size_t)G * S * 4 + 4 + S;
  if (smem > 64 * 1024) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&pool_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess)
      return MRSA_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL(pool_kernel, dim3((unsigned)batch_chunks, (unsigned)kv_heads), dim3(kThreads),
                     smem, (hipStream_t)stream, (const uint16_t*)mu_q, mu_row_stride,
                     (const uint16_t*)k_chunked, key_valid, S, (int)kv_heads, G, D, sm_scale,
                     dense_torch_semantics, bias_scale, (uint16_t*)landmark_keys, entropy,
                     prior_bias);
  return mrsa_launch_status();
}

}  // namespace

extern "C" int mrsa_chunk_attn_pool_gqa_fwd(const void* mu_q, const void* k_chunked,
                                            const uint8_t* key_valid, int64_t batch_chunks,
                                            int64_t chunk_size, int64_t kv_heads, int64_t groups,
                                            int64_t head_dim, float sm_scale,
                                            int dense_torch_semantics, const float* bias_scale,
                                            void* landmark_keys, float* entropy,
                                            float* prior_bias, void* stream) {
  return pool_forward(mu_q, kv_heads * groups * head_dim, k_chunked, key_valid, batch_chunks,
                      chunk_size, kv_heads, groups, head_dim, sm_scale, dense_torch_semantics,
                      bias_scale, landmark_keys, entropy, prior_bias, stream);
}

extern "C" int mrsa_chunk_attn_pool_gqa_strided_fwd(
    const void* mu_q, int64_t mu_row_stride, const void* k_chunked, const uint8_t* key_valid,
    int64_t batch_chunks, int64_t chunk_size, int64_t kv_heads, int64_t groups, int64_t head_dim,
    float sm_scale, int dense_torch_semantics, const float* bias_scale, void* landmark_keys,
    float* entropy, float* prior_bias, void* stream) {
  return pool_forward(mu_q, mu_row_stride, k_chunked, key_valid, batch_chunks, chunk_size,
                      kv_heads, groups, head_dim, sm_scale, dense_torch_semantics, bias_scale,
                      landmark_keys, entropy, prior_bias, stream);
}

extern "C" int mrsa_pool_cached_chunks_fwd(const void* route_q, const int64_t* query_positions,
                                           int64_t query_len, const void* key,
                                           const uint8_t* key_valid, int64_t batch,
                                           int64_t cache_len, const int64_t* chunks,
                                           int64_t count, int64_t kv_heads, int64_t groups,
                                           int64_t head_dim, int64_t chunk_size, float sm_scale,
                                           const float* bias_scale, void* landmark_keys,
                                           float* prior_bias, void* stream) {
  if (batch < 0 || query_len < 0 || cache_len < 0 || count < 0 || kv_heads <= 0 || groups <= 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (chunk_size != 64 || head_dim != 128 || groups > 16 || cache_len % 64 != 0)
    return MRSA_ERR_UNSUPPORTED;
  if (batch == 0 || count == 0 || query_len == 0 || cache_len == 0) return MRSA_OK;
  if (!route_q || !query_positions || !key || !key_valid || !chunks || !bias_scale ||
      !landmark_keys || !prior_bias)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)route_q | (uintptr_t)key | (uintptr_t)landmark_keys) % 16 != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (kv_heads > 65535) return MRSA_ERR_UNSUPPORTED;
  const int64_t units = batch * count * kv_heads;
  const int64_t blocks = (units + kPoolWaves - 1) / kPoolWaves;
  if (blocks > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(pool_cached_kernel, dim3((unsigned)blocks), dim3(64 * kPoolWaves), 0,
                     (hipStream_t)stream, (const uint16_t*)route_q, query_positions, query_len,
                     (const uint16_t*)key, key_valid, cache_len, chunks, count, (int)kv_heads,
                     (int)groups, units, sm_scale, bias_scale, (uint16_t*)landmark_keys,
                     prior_bias);
  return mrsa_launch_status();
}

namespace {

// Backward of the pool, one workgroup per (chunk, KV head) like the forward;
// the probabilities are recomputed from mu_q and K rather than saved.
// Fused-kernel semantics (_pool_gqa_bwd, ops/chunk_attn_pool_gqa_tilelang.py:183-325):
//   pb = bf16(p) for a valid chunk, else 0;  dP = gK . k;  delta = sum_s pb dP
//   dlogit = pb ((dP - delta) - gH (ln pb + H))  (0 where pb = 0), rounded to
//   bf16 after the sm_scale factor;  d_mu = dlogit . K;  d_k = dlogit^T q + pb^T gK
//   (a masked slot 0, whose logit is the constant 0, still gets its term, as
//   in the reference kernel).
// Dense semantics (autograd of _compact_pool_torch, :17-37): fp32 p,
//   dp = dP - gH (ln p + 1) for p > 0, dz = p (dp - sum p dp), dlogit = dz sm_scale.
__global__ void __launch_bounds__(kThreads)
    pool_bwd_kernel(const uint16_t* __restrict__ mu_q, const uint16_t* __restrict__ kc,
                    const uint8_t* __restrict__ key_valid, const uint16_t* __restrict__ g_lmk,
                    const float* __restrict__ g_ent, int S, int H, int G, int D, float sm_scale,
                    int dense, uint16_t* __restrict__ d_mu, uint16_t* __restrict__ d_k) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int64_t bc = blockIdx.x;
  const int h = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;

  uint16_t* ks = reinterpret_cast<uint16_t*>(smem);  // [S][D] bf16
  float* qs = reinterpret_cast<float*>(ks + S * D);   // [G][D]
  float* gs = qs + G * D;                             // [G][D] grad of the pooled key
  float* ps = gs + G * D;                             // [G][S] logits -> pb
  float* dq = ps + G * S;                             // [G][S] dP -> dlogit
  int* flag = reinterpret_cast<int*>(dq + G * S);
  unsigned char* vs = reinterpret_cast<unsigned char*>(flag + 1);  // [S]

  const int vec_per_row = D / 8;
  for (int v = tid; v < S * vec_per_row; v += kThreads) {
    const int s = v / vec_per_row, c = v - s * vec_per_row;
    reinterpret_cast<u32x4_t*>(ks + s * D)[c] =
        reinterpret_cast<const u32x4_t*>(kc + ((bc * S + s) * H + h) * (int64_t)D)[c];
  }
  const int64_t qbase = ((bc * H + h) * G) * (int64_t)D;
  for (int e = tid; e < G * D; e += kThreads) {
    qs[e] = bf16_to_f32(mu_q[qbase + e]);
    gs[e] = g_lmk ? bf16_to_f32(g_lmk[qbase + e]) : 0.f;
  }
  if (tid == 0) flag[0] = 0;
  for (int s = tid; s < S; s += kThreads) vs[s] = key_valid[bc * S + s] != 0;
  __syncthreads();
  if (tid < S - 1 && vs[tid]) flag[0] = 1;
  __syncthreads();
  const bool chunk_valid = flag[0] != 0;

  for (int p = tid; p < G * S; p += kThreads) {
    const int g = p / S, s = p - g * S;
    const float* qr = qs + g * D;
    const float* gr = gs + g * D;
    const uint16_t* kr = ks + s * D;
    int d = (s * 8) % D;
    float acc = 0.f, dacc = 0.f;
    for (int i = 0; i < D; i += 2) {
      const uint32_t w = *reinterpret_cast<const uint32_t*>(kr + d);
      acc = fmaf(qr[d], bf16_lo(w), acc);
      acc = fmaf(qr[d + 1], bf16_hi(w), acc);
      dacc = fmaf(gr[d], bf16_lo(w), dacc);
      dacc = fmaf(gr[d + 1], bf16_hi(w), dacc);
      d += 2;
      if (d >= D) d -= D;
    }
    const bool real = (s < S - 1) && vs[s];
    float logit;
    if (dense) {
      logit = real ? acc * sm_scale : neg_inf();
    } else {
      logit = (real && chunk_valid) ? acc * sm_scale : (s == 0 ? 0.f : neg_inf());
    }
    ps[p] = logit;
    dq[p] = dacc;
  }
  __syncthreads();

  for (int g = wave; g < G; g += kThreads / 64) {
    const bool in0 = lane < S, in1 = lane + 64 < S;
    const float v0 = in0 ? ps[g * S + lane] : neg_inf();
    const float v1 = in1 ? ps[g * S + lane + 64] : neg_inf();
    const float dp0 = in0 ? dq[g * S + lane] : 0.f;
    const float dp1 = in1 ? dq[g * S + lane + 64] : 0.f;
    const float m = wave_max(fmaxf(v0, v1));
    float e0 = 0.f, e1 = 0.f;
    if (m != neg_inf()) {
      e0 = (in0 && v0 != neg_inf()) ? exp2f((v0 - m) * kLog2e) : 0.f;
      e1 = (in1 && v1 != neg_inf()) ? exp2f((v1 - m) * kLog2e) : 0.f;
    }
    const float sum = wave_sum(e0 + e1);
    const float p0 = sum > 0.f ? e0 / sum : 0.f;
    const float p1 = sum > 0.f ? e1 / sum : 0.f;
    const float gh = g_ent ? g_ent[(bc * H + h) * G + g] : 0.f;
    float b0, b1, l0, l1;
    if (!dense) {
      const float ent =
          -wave_sum((p0 > 0.f ? p0 * logf(p0) : 0.f) + (p1 > 0.f ? p1 * logf(p1) : 0.f));
      b0 = chunk_valid ? bf16_to_f32(f32_to_bf16(p0)) : 0.f;
      b1 = chunk_valid ? bf16_to_f32(f32_to_bf16(p1)) : 0.f;
      const float delta = wave_sum(b0 * dp0 + b1 * dp1);
      l0 = b0 > 0.f ? b0 * ((dp0 - delta) - gh * (logf(b0) + ent)) : 0.f;
      l1 = b1 > 0.f ? b1 * ((dp1 - delta) - gh * (logf(b1) + ent)) : 0.f;
      l0 = bf16_to_f32(f32_to_bf16(l0 * sm_scale));
      l1 = bf16_to_f32(f32_to_bf16(l1 * sm_scale));
    } else {
      b0 = p0;
      b1 = p1;
      const float q0 = p0 > 0.f ? dp0 - gh * (logf(fmaxf(p0, 1e-30f)) + (p0 >= 1e-30f ? 1.f : 0.f))
                                : dp0;
      const float q1 = p1 > 0.f ? dp1 - gh * (logf(fmaxf(p1, 1e-30f)) + (p1 >= 1e-30f ? 1.f : 0.f))
                                : dp1;
      const float delta = wave_sum(p0 * q0 + p1 * q1);
      l0 = p0 * (q0 - delta) * sm_scale;
      l1 = p1 * (q1 - delta) * sm_scale;
    }
    if (in0) {
      ps[g * S + lane] = b0;
      dq[g * S + lane] = l0;
    }
    if (in1) {
      ps[g * S + lane + 64] = b1;
      dq[g * S + lane + 64] = l1;
    }
  }
  __syncthreads();

  for (int p = tid; p < G * D; p += kThreads) {
    const int g = p / D, d = p - g * D;
    const float* lr = dq + g * S;
    float acc = 0.f;
    for (int s = 0; s < S; ++s) acc = fmaf(lr[s], bf16_to_f32(ks[s * D + d]), acc);
    d_mu[qbase + p] = (uint16_t)f32_to_bf16(acc);
  }
  for (int p = tid; p < S * D; p += kThreads) {
    const int s = p / D, d = p - s * D;
    float acc = 0.f;
    for (int g = 0; g < G; ++g) {
      acc = fmaf(dq[g * S + s], qs[g * D + d], acc);
      acc = fmaf(ps[g * S + s], gs[g * D + d], acc);
    }
    d_k[((bc * S + s) * H + h) * (int64_t)D + d] = (uint16_t)f32_to_bf16(acc);
  }
}

}  // namespace

extern "C" int mrsa_chunk_attn_pool_gqa_bwd(const void* mu_q, const void* k_chunked,
                                            const uint8_t* key_valid, const void* grad_landmark,
                                            const float* grad_entropy, int64_t batch_chunks,
                                            int64_t chunk_size, int64_t kv_heads, int64_t groups,
                                            int64_t head_dim, float sm_scale,
                                            int dense_torch_semantics, void* d_mu_q,
                                            void* d_k_chunked, void* stream) {
  if (batch_chunks < 0 || chunk_size < 2 || chunk_size > 128 || kv_heads <= 0 || groups <= 0 ||
      groups > 16 || head_dim <= 0 || head_dim > 256 || head_dim % 8 != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (batch_chunks == 0) return MRSA_OK;
  if (!mu_q || !k_chunked || !key_valid || !d_mu_q || !d_k_chunked)
    return MRSA_ERR_INVALID_ARGUMENT;
  if ((uintptr_t)k_chunked % 16 != 0) return MRSA_ERR_INVALID_ARGUMENT;
  if (batch_chunks > 0x7fffffff || kv_heads > 65535) return MRSA_ERR_UNSUPPORTED;
  const int S = (int)chunk_size, G = (int)groups, D = (int)head_dim;
  const size_t smem = (size_t)S * D * 2 + 2 * (size_t)G * D * 4 + 2 * (size_t)G * S * 4 + 4 + S;
  if (smem > 64 * 1024) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&pool_bwd_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess)
      return MRSA_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL(pool_bwd_kernel, dim3((unsigned)batch_chunks, (unsigned)kv_heads),
                     dim3(kThreads), smem, (hipStream_t)stream, (const uint16_t*)mu_q,
                     (const uint16_t*)k_chunked, key_valid, (const uint16_t*)grad_landmark,
                     grad_entropy, S, (int)kv_heads, G, D, sm_scale, dense_torch_semantics,
                     (uint16_t*)d_mu_q, (uint16_t*)d_k_chunked);
  return mrsa_launch_status();
}
