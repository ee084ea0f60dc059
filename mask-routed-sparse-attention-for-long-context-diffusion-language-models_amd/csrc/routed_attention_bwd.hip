// Backward of the routed (selected-chunk) attention.
//
// Forward: out[q, g] = sum_k w[q, g, k] * softmax_{s in chunk idx[q, k], s visible}(q_g . k_s * scale) . V
// (the forward kernel's semantics: a list ends at its first negative entry,
// entries >= kv_len / 64 are skipped, the landmark slot and invalid / dropped
// keys are not visible).  The backward follows the reference kernel
// ops/hils_fwd_bwd_head.py:573-910 and its rounding points:
//   P      = 2^(s c - lse) over the visible keys (lse = log2-sum-exp of the
//            chunk, recomputed here), rounded to bf16;
//   dP     = dO . V^T (fp32);  di = sum_s P dP  ->  dW[q, g, k] = di (bf16);
//   dS     = bf16(scale * w * P * (dP - di));
//   dQ    += dS . K            (fp32, summed over the query's chunks);
//   dK    += dS^T . Q,  dV += P^T . bf16(w * dO)  (fp32 atomic adds, like the
//            reference's atomic_add into DK / DV).
// A chunk listed twice is processed once per slot (its gradient terms add,
// as the weights do in the forward).
//
// Work split: one wave per (batch, query, KV head), four per workgroup.  The
// wave's 16 matrix columns are the group's heads (columns >= G are zero).
// Operands come from two fragment layouts of the same K / V:
//   fwd = mrsa_kv_fragments(k, v): K images (keys x dims) for S^T = K . Q^T;
//   bwd = mrsa_kv_fragments(v, k): V images (keys x dims) for dP^T = V . dO^T
//         and K^T images (dims x keys, tiled order) for dQ^T = K^T . dS^T.
// dK and dV (keys x dims) run as 16x16x32 products whose reduction is the
// 16 columns (lane groups 2 and 3 supply zeros), with dS^T / P^T and Q^T /
// dO^T staged through per-wave LDS tiles.
#include "mrsa_device.h"

using namespace mrsa;

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxTopk = 64;
constexpr uint32_t kFragBytes = 32768;

struct BwdArgs {
  const uint16_t* q;
  const uint16_t* dout;
  const uint16_t* fwd;       // [B, Hkv, Ck, 16384]: K images | V^T images
  const uint16_t* bwd;       // [B, Hkv, Ck, 16384]: V images | K^T images
  const uint16_t* w;
  const int32_t* idx;
  const uint8_t* key_valid;
  const int8_t* keep;        // [B, Lq, Hkv, K, 64] or null
  int64_t B, Lq, Lk, Ck;
  int Hq, Hkv, G, K;
  int mask_last;
  float scale, scale_log2;
  float* dq;                 // [B, Lq, Hq, 128] fp32
  float* dk;                 // [B, Lk, Hkv, 128] fp32, accumulated
  float* dv;                 // [B, Lk, Hkv, 128] fp32, accumulated
  uint16_t* dw;              // [B, Lq, Hq, K] bf16
};

// Per-wave LDS tiles (bf16): Q^T and dO^T as [128 dims][16 columns], and the
// transposes of P and dS as [64 keys][16 columns].
struct WaveTiles {
  uint16_t qt[128 * 16];
  uint16_t dt[128 * 16];
  uint16_t ps[64 * 16];
  uint16_t ds[64 * 16];
  float wcol[16];
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           (int)0x00020000);
}
__device__ __forceinline__ u32x4_t bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
}
// First-half images (K or V, keys x dims): image 4 mt + ks at 1024 (4 mt + ks).
__device__ __forceinline__ void load_rows(u32x4_t (&x)[4][4], __amdgpu_buffer_rsrc_t r,
                                          uint32_t lo, uint32_t cb) {
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) x[mt][ks] = bload(r, lo + 1024u * ks, cb + 4096u * mt);
}
// Second-half images (V^T or K^T, dims x keys): image 2 nt + ks at 16384 + 1024 (2 nt + ks).
__device__ __forceinline__ void load_cols(u32x4_t (&x)[8][2], __amdgpu_buffer_rsrc_t r,
                                          uint32_t lo, uint32_t cb) {
#pragma unroll
  for (int nt = 0; nt < 8; ++nt)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int i = 2 * nt + ks;
      x[nt][ks] = bload(r, lo + 1024u * (i & 3), cb + 16384u + 4096u * (i >> 2));
    }
}

// Bits of the nonzero bytes (bit j = byte j) of one 64-byte keep / key-valid
// row: one byte per lane and a wave ballot (every lane must be active).
__device__ __forceinline__ uint64_t nonzero_bits(const int8_t* row) {
  return __builtin_amdgcn_ballot_w64(row[threadIdx.x & 63] != 0);
}

__global__ void __launch_bounds__(kThreads) routed_attn_bwd_kernel(BwdArgs a) {
  __shared__ WaveTiles tiles[kWaves];
  __shared__ int32_t list_s[kWaves][kMaxTopk];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int j = lane & 15, grp = lane >> 4;
  // (b, q, h): KV head fastest so the four waves of a workgroup share q rows.
  const int64_t unit = (int64_t)blockIdx.x * kWaves + wave;
  const int64_t units = a.B * a.Lq * a.Hkv;
  if (unit >= units) return;  // wave-uniform; no workgroup barrier follows
  const int h = (int)(unit % a.Hkv);
  const int64_t bq = unit / a.Hkv;
  const int64_t b = bq / a.Lq;
  const int64_t q = bq % a.Lq;
  const int G = a.G, K = a.K;
  const bool cvalid = j < G;
  WaveTiles& T = tiles[wave];

  // ---- this query's rows: Q^T / dO^T operands (columns j = heads) and the
  // transposed tiles [dim][column]
  const int64_t row0 = (b * a.Lq + q) * a.Hq + (int64_t)h * G;  // (query, head 0) row
  u32x4_t Qb[4], Db[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    u32x4_t z = {0u, 0u, 0u, 0u};
    Qb[ks] = z;
    Db[ks] = z;
    if (cvalid) {
      Qb[ks] = *reinterpret_cast<const u32x4_t*>(a.q + (row0 + j) * 128 + 32 * ks + 8 * grp);
      Db[ks] = *reinterpret_cast<const u32x4_t*>(a.dout + (row0 + j) * 128 + 32 * ks + 8 * grp);
    }
  }
  for (int e = lane; e < 128 * 16; e += 64) {
    const int d = e >> 4, col = e & 15;
    uint16_t qv = 0, dv = 0;
    if (col < G) {
      qv = a.q[(row0 + col) * 128 + d];
      dv = a.dout[(row0 + col) * 128 + d];
    }
    T.qt[d * 16 + col] = qv;
    T.dt[d * 16 + col] = dv;
  }
  // the index list (ends at the first negative entry)
  const int32_t* irow = a.idx + ((b * a.Lq + q) * a.Hkv + h) * K;
  if (lane < K) list_s[wave][lane] = irow[lane];
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  int n = K;
  for (int k = 0; k < K; ++k)
    if (list_s[wave][k] < 0) {
      n = k;
      break;
    }

  const uint32_t lo = 16u * lane;
  const __amdgpu_buffer_rsrc_t frs =
      make_rsrc(a.fwd + (b * a.Hkv + h) * a.Ck * 16384, (uint32_t)a.Ck * kFragBytes);
  const __amdgpu_buffer_rsrc_t brs =
      make_rsrc(a.bwd + (b * a.Hkv + h) * a.Ck * 16384, (uint32_t)a.Ck * kFragBytes);
  const float c2 = a.scale_log2;
  f32x4_t dq[8];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) dq[nt] = zero4();
  uint16_t* dwrow = a.dw + row0 * K;

  for (int k = 0; k < K; ++k) {
    const int32_t c = list_s[wave][k];
    float di_out = 0.f;
    const bool active = k < n && c >= 0 && c < a.Ck;
    if (active) {
      const float wv = cvalid ? bf16_to_f32(a.w[(row0 + j) * K + k]) : 0.f;
      if (lane < 16) T.wcol[lane] = lane < G ? bf16_to_f32(a.w[(row0 + lane) * K + k]) : 0.f;
      // excluded keys: landmark slot, invalid keys, dropped by the keep row
      uint64_t excl = a.mask_last ? (1ull << 63) : 0ull;
      if (a.key_valid)
        excl |= ~nonzero_bits(reinterpret_cast<const int8_t*>(a.key_valid + b * a.Lk + (int64_t)c * 64));
      if (a.keep)
        excl |= ~nonzero_bits(a.keep + (((b * a.Lq + q) * a.Hkv + h) * K + k) * 64);
      const uint64_t msh = excl >> (4 * grp);  // bit 16 mt + r: key 16 mt + 4 grp + r
      const uint32_t cb = (uint32_t)c * kFragBytes;

      // S^T = K . Q^T and dP^T = V . dO^T (lane (grp, j): keys 16 mt + 4 grp + r, column j)
      f32x4_t S[4], dP[4];
      {
        u32x4_t kb[4][4];
        load_rows(kb, frs, lo, cb);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          S[mt] = zero4();
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) S[mt] = mfma_bf16_16x16x32(kb[mt][ks], Qb[ks], S[mt]);
        }
        load_rows(kb, brs, lo, cb);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          dP[mt] = zero4();
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) dP[mt] = mfma_bf16_16x16x32(kb[mt][ks], Db[ks], dP[mt]);
        }
      }
      // P = 2^(s c - lse) over the visible keys, rounded to bf16
      float mx = neg_inf();
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (!((msh >> (16 * mt + r)) & 1ull)) mx = fmaxf(mx, S[mt][r] * c2);
      mx = across4_max(mx);
      float sum = 0.f;
      if (mx != neg_inf()) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (!((msh >> (16 * mt + r)) & 1ull)) sum += exp2_hw(S[mt][r] * c2 - mx);
      }
      sum = across4_sum(sum);
      const float lse = mx == neg_inf() ? neg_inf() : mx + log2_hw(sum);
      float P[4][4];
      float di = 0.f;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const bool vis = !((msh >> (16 * mt + r)) & 1ull) && lse != neg_inf();
          const float p = vis ? bf16_to_f32(f32_to_bf16(exp2_hw(S[mt][r] * c2 - lse))) : 0.f;
          P[mt][r] = p;
          di += p * dP[mt][r];
        }
      di = across4_sum(di);
      di_out = di;
      // dS = bf16(scale w P (dP - di)); both transposes into the wave's tiles
      float dS[4][4];
      const float sw = a.scale * wv;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          dS[mt][r] = bf16_to_f32(f32_to_bf16(sw * P[mt][r] * (dP[mt][r] - di)));
          const int key = 16 * mt + 4 * grp + r;
          T.ps[key * 16 + j] = (uint16_t)f32_to_bf16(P[mt][r]);
          T.ds[key * 16 + j] = (uint16_t)f32_to_bf16(dS[mt][r]);
        }
      // dQ^T += K^T . dS^T (K^T images; reduction index 8 grp + e of k-step
      // ks is key 32 ks + 16 (e >> 2) + 4 grp + (e & 3), the tiled order)
      {
        u32x4_t kt[8][2];
        load_cols(kt, brs, lo, cb);
        u32x4_t Sb[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          Sb[ks][0] = pack_bf16x2(dS[2 * ks][0], dS[2 * ks][1]);
          Sb[ks][1] = pack_bf16x2(dS[2 * ks][2], dS[2 * ks][3]);
          Sb[ks][2] = pack_bf16x2(dS[2 * ks + 1][0], dS[2 * ks + 1][1]);
          Sb[ks][3] = pack_bf16x2(dS[2 * ks + 1][2], dS[2 * ks + 1][3]);
        }
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) {
          dq[nt] = mfma_bf16_16x16x32(kt[nt][0], Sb[0], dq[nt]);
          dq[nt] = mfma_bf16_16x16x32(kt[nt][1], Sb[1], dq[nt]);
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // dK (keys x dims) = dS^T . Q and dV = P^T . bf16(w dO): A = the key row
      // of the transposed tile (columns 8 grp .. + 7; groups 2, 3 zero), B = the
      // dim row of Q^T / dO^T.
      const u32x4_t zero = {0u, 0u, 0u, 0u};
      float* dkb = a.dk + ((b * a.Lk + (int64_t)c * 64) * a.Hkv + h) * 128;
      float* dvb = a.dv + ((b * a.Lk + (int64_t)c * 64) * a.Hkv + h) * 128;
      const int64_t krow = (int64_t)a.Hkv * 128;  // floats between keys
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const u32x4_t As = grp < 2 ? *reinterpret_cast<const u32x4_t*>(&T.ds[(16 * mt + j) * 16 + 8 * grp]) : zero;
        const u32x4_t Ap = grp < 2 ? *reinterpret_cast<const u32x4_t*>(&T.ps[(16 * mt + j) * 16 + 8 * grp]) : zero;
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) {
          const u32x4_t Bq = grp < 2 ? *reinterpret_cast<const u32x4_t*>(&T.qt[(16 * nt + j) * 16 + 8 * grp]) : zero;
          u32x4_t Bd = zero;
          if (grp < 2) {
            const u32x4_t x = *reinterpret_cast<const u32x4_t*>(&T.dt[(16 * nt + j) * 16 + 8 * grp]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float w0 = T.wcol[8 * grp + 2 * i], w1 = T.wcol[8 * grp + 2 * i + 1];
              Bd[i] = pack_bf16x2(w0 * bf16_lo(x[i]), w1 * bf16_hi(x[i]));
            }
          }
          const f32x4_t ck = mfma_bf16_16x16x32(As, Bq, zero4());
          const f32x4_t cv = mfma_bf16_16x16x32(Ap, Bd, zero4());
          // lane (grp, j): keys 16 mt + 4 grp + r, dim 16 nt + j
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int64_t off = (int64_t)(16 * mt + 4 * grp + r) * krow + 16 * nt + j;
            atomicAdd(dkb + off, ck[r]);
            atomicAdd(dvb + off, cv[r]);
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (cvalid && grp == 0) dwrow[(int64_t)j * K + k] = (uint16_t)f32_to_bf16(di_out);
  }
  // dQ rows (lane (grp, j): column j, dims 16 nt + 4 grp + r)
  if (cvalid) {
    float* dqr = a.dq + (row0 + j) * 128;
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
      *reinterpret_cast<f32x4_t*>(dqr + 16 * nt + 4 * grp) = dq[nt];
  }
}

}  // namespace

extern "C" int mrsa_selected_attention_bwd(
    const void* q, const void* grad_out, const void* kv_frags, const void* kv_frags_bwd,
    const void* weights, const int32_t* indices, const uint8_t* key_valid,
    const int8_t* token_keep, int64_t batch, int64_t q_len, int64_t kv_len, int64_t q_heads,
    int64_t kv_heads, int64_t head_dim, int64_t topk, int64_t chunk_size, int mask_last_token,
    float sm_scale, float* grad_q, float* grad_k, float* grad_v, void* grad_weights,
    void* stream) {
  if (batch < 0 || q_len < 0 || kv_len < 0 || q_heads <= 0 || kv_heads <= 0 ||
      q_heads % kv_heads != 0 || head_dim <= 0 || topk <= 0 || chunk_size <= 0 ||
      !(sm_scale > 0.f) || sm_scale == __builtin_inff())
    return MRSA_ERR_INVALID_ARGUMENT;
  if (kv_len % chunk_size != 0) return MRSA_ERR_INVALID_ARGUMENT;
  if (chunk_size != 64 || head_dim != 128 || q_heads / kv_heads > 16 || topk > kMaxTopk)
    return MRSA_ERR_UNSUPPORTED;
  if (kv_len / 64 >= 131072) return MRSA_ERR_UNSUPPORTED;
  if (batch == 0 || q_len == 0) return MRSA_OK;
  if (!q || !grad_out || !kv_frags || !kv_frags_bwd || !weights || !indices || !grad_q ||
      !grad_k || !grad_v || !grad_weights)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)q | (uintptr_t)grad_out | (uintptr_t)kv_frags | (uintptr_t)kv_frags_bwd |
       (uintptr_t)grad_q) % 16 != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  BwdArgs a;
  a.q = (const uint16_t*)q;
  a.dout = (const uint16_t*)grad_out;
  a.fwd = (const uint16_t*)kv_frags;
  a.bwd = (const uint16_t*)kv_frags_bwd;
  a.w = (const uint16_t*)weights;
  a.idx = indices;
  a.key_valid = key_valid;
  a.keep = token_keep;
  a.B = batch;
  a.Lq = q_len;
  a.Lk = kv_len;
  a.Ck = kv_len / 64;
  a.Hq = (int)q_heads;
  a.Hkv = (int)kv_heads;
  a.G = (int)(q_heads / kv_heads);
  a.K = (int)topk;
  a.mask_last = mask_last_token;
  a.scale = sm_scale;
  a.scale_log2 = sm_scale * kLog2e;
  a.dq = grad_q;
  a.dk = grad_k;
  a.dv = grad_v;
  a.dw = (uint16_t*)grad_weights;
  const int64_t units = batch * q_len * kv_heads;
  const int64_t blocks = (units + kWaves - 1) / kWaves;
  if (blocks > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(routed_attn_bwd_kernel, dim3((unsigned)blocks), dim3(kThreads), 0,
                     (hipStream_t)stream, a);
  return mrsa_launch_status();
}
