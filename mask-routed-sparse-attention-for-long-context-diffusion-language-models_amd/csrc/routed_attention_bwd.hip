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
//   dK    += dS^T . Q,  dV += P^T . bf16(w * dO)  (fp32, summed over the
//            (query, slot) pairs that route to the chunk).
// A chunk listed twice is processed once per slot (its gradient terms add,
// as the weights do in the forward).
//
// Work split (chunk-major).  A list of the (query, slot) pairs of every
// chunk is built first (count, scan, fill); a workgroup then owns one chunk
// (or a segment of kSegEntries of its pairs) and recomputes each pair's
// chunk softmax:
//   dK / dV  stay in the workgroup's registers and are written once per
//            chunk (added with atomics when the chunk's pairs span several
//            segments) -- the reference instead adds each query block's
//            dK / dV into global memory with atomics;
//   dS       each pair's bf16 dS tile is stored as a record (128 bytes per
//            (query, head, slot));
//   dW       written directly (one pair = one slot).
// dQ is then the forward kernel's walk over each query tile's chunks
// (routed_attention.hip, mrsa::routed_dq_walk): the tiles take the records
// as their P^T operand and K^T where the forward reads V, and the rows are
// summed in LDS and added into dQ once -- no atomics.
// Operands come from two fragment layouts of the same K / V:
//   fwd = mrsa_kv_fragments(k, v): K images (keys x dims) for S^T = K . Q^T;
//   bwd = mrsa_kv_fragments(v, k): V images (keys x dims) for dP^T = V . dO^T
//         and K^T images (dims x keys, tiled order) for the walk's dS . K.
#include "mrsa_device.h"

#include <algorithm>

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
  // chunk-major pass: pair lists (entry = query | slot << 24), per chunk
  // (b, h, c) the list start and the first work unit
  const int32_t* list;
  const int32_t* start;      // [B * Hkv * Ck + 1]
  const int32_t* ustart;     // [B * Hkv * Ck + 1]
  const float* slope;        // [Hq] ALiBi slopes or null
  // dS records [B, Lq, Hq, K] x 64 bf16 (lane group g's 16 keys at 16 g, in
  // the packed P^T order of the forward's tiles), one per listed slot, for
  // the dQ walk.
  uint16_t* ds_rec;
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
// Bits of the nonzero bytes (bit j = byte j) of one 64-byte keep / key-valid
// row: one byte per lane and a wave ballot (every lane must be active).
__device__ __forceinline__ uint64_t nonzero_bits(const int8_t* row) {
  return __builtin_amdgcn_ballot_w64(row[threadIdx.x & 63] != 0);
}

// One column tile's chunk gradient, in place.  S^T / dP^T lane (grp, j):
// keys 16 mt + 4 grp + r of column j; msh bit 16 mt + r set = key excluded.
//   S  <- P  = bf16(2^(s c - lse)) over the visible keys (0 when none is)
//   dP <- dS = bf16(sw P (dP - di)),  di = sum P dP per column (returned)
// With ALiBi (alibi, wave-uniform) the exp2-domain logit is s c + sl
// max(0, 62 - key), sl = -slope[head] c for this lane's column
// (ops/hils_fwd_bwd_head.py:755-760, the backward's bias term).
__device__ __forceinline__ float chunk_grad(f32x4_t (&S)[4], f32x4_t (&dP)[4], uint64_t msh,
                                            float c2, float sw, bool alibi = false,
                                            float sl = 0.f, int grp = 0) {
  if (alibi) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        S[mt][r] = __builtin_fmaf(
            S[mt][r], c2, sl * fmaxf(0.f, (float)(62 - 16 * mt - r) - 4.f * (float)grp));
    c2 = 1.f;
  }
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
  float di = 0.f;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool vis = !((msh >> (16 * mt + r)) & 1ull) && lse != neg_inf();
      const float p = vis ? bf16_to_f32(f32_to_bf16(exp2_hw(S[mt][r] * c2 - lse))) : 0.f;
      S[mt][r] = p;
      di += p * dP[mt][r];
    }
  di = across4_sum(di);
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      dP[mt][r] = bf16_to_f32(f32_to_bf16(sw * S[mt][r] * (dP[mt][r] - di)));
  return di;
}

// ---- chunk-major dK / dV ---------------------------------------------------
constexpr int kListBlock = 256;       // queries per list workgroup (one per thread)
constexpr int kMaxListChunks = 8192;  // LDS counters of the list kernels (32 KB)
constexpr int kSegEntries = 1024;     // (query, slot) pairs per dK / dV work unit

// The valid slots of one index row: up to the first negative entry, chunks
// below Ck.
template <class F>
__device__ __forceinline__ void for_each_slot(const int32_t* row, int K, int64_t Ck, F&& f) {
  for (int k = 0; k < K; ++k) {
    const int32_t c = row[k];
    if (c < 0) break;
    if (c < Ck) f(k, c);
  }
}

// 1. Pairs per (chunk, query block) in LDS; each block's run of a chunk's
//    list is reserved with one global add (blkbase = its offset).
__global__ void __launch_bounds__(kListBlock) list_count_kernel(BwdArgs a, int32_t* count,
                                                                int32_t* blkbase, int nqb) {
  __shared__ int32_t hist[kMaxListChunks];
  const int tid = threadIdx.x;
  const int qb = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int64_t b = bh / a.Hkv;
  const int h = (int)(bh % a.Hkv);
  for (int64_t c = tid; c < a.Ck; c += kListBlock) hist[c] = 0;
  __syncthreads();
  const int64_t q = (int64_t)qb * kListBlock + tid;
  if (q < a.Lq)
    for_each_slot(a.idx + ((b * a.Lq + q) * a.Hkv + h) * a.K, a.K, a.Ck,
                  [&](int, int32_t c) { atomicAdd(&hist[c], 1); });
  __syncthreads();
  for (int64_t c = tid; c < a.Ck; c += kListBlock) {
    const int n = hist[c];
    blkbase[(bh * nqb + qb) * a.Ck + c] = n ? atomicAdd(&count[bh * a.Ck + c], n) : 0;
  }
}

// 2. Exclusive scans over the chunks (b, h, c): list starts and work-unit
//    starts (ceil(count / kSegEntries) units per chunk).  One workgroup.
__global__ void __launch_bounds__(1024) list_scan_kernel(const int32_t* count, int64_t N,
                                                         int32_t* start, int32_t* ustart) {
  __shared__ int32_t s1[1024], s2[1024];
  const int tid = threadIdx.x;
  const int64_t per = (N + 1023) / 1024;
  const int64_t lo = min(N, tid * per), hi = min(N, lo + per);
  int32_t t1 = 0, t2 = 0;
  for (int64_t i = lo; i < hi; ++i) {
    t1 += count[i];
    t2 += (count[i] + kSegEntries - 1) / kSegEntries;
  }
  s1[tid] = t1;
  s2[tid] = t2;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const int32_t u1 = tid >= o ? s1[tid - o] : 0, u2 = tid >= o ? s2[tid - o] : 0;
    __syncthreads();
    s1[tid] += u1;
    s2[tid] += u2;
    __syncthreads();
  }
  int32_t r1 = s1[tid] - t1, r2 = s2[tid] - t2;
  for (int64_t i = lo; i < hi; ++i) {
    start[i] = r1;
    ustart[i] = r2;
    r1 += count[i];
    r2 += (count[i] + kSegEntries - 1) / kSegEntries;
  }
  if (tid == 1023) {
    start[N] = s1[1023];
    ustart[N] = s2[1023];
  }
}

// 3. Pairs written into their chunk's list: query | slot << 24.
__global__ void __launch_bounds__(kListBlock) list_fill_kernel(BwdArgs a, const int32_t* blkbase,
                                                               int nqb, int32_t* list) {
  __shared__ int32_t cur[kMaxListChunks];
  const int tid = threadIdx.x;
  const int qb = blockIdx.x;
  const int64_t bh = blockIdx.y;
  const int64_t b = bh / a.Hkv;
  const int h = (int)(bh % a.Hkv);
  for (int64_t c = tid; c < a.Ck; c += kListBlock) cur[c] = 0;
  __syncthreads();
  const int64_t q = (int64_t)qb * kListBlock + tid;
  if (q < a.Lq)
    for_each_slot(a.idx + ((b * a.Lq + q) * a.Hkv + h) * a.K, a.K, a.Ck, [&](int k, int32_t c) {
      const int p = atomicAdd(&cur[c], 1);
      const int64_t bhc = bh * a.Ck + c;
      list[(int64_t)a.start[bhc] + blkbase[(bh * nqb + qb) * a.Ck + c] + p] =
          (int32_t)(q | ((int64_t)k << 24));
    });
}

// Kept-key bits (bit j = key j kept) of one 64-byte token-keep row, per lane.
__device__ __forceinline__ uint64_t keep_row_bits(const int8_t* kr) {
  uint64_t bits = 0ull;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const u32x4_t x = *reinterpret_cast<const u32x4_t*>(kr + 16 * v);
#pragma unroll
    for (int w = 0; w < 4; ++w)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        bits |= ((x[w] >> (8 * i)) & 0xffu) ? 1ull << (16 * v + 4 * w + i) : 0ull;
  }
  return bits;
}

// LDS of the chunk-major kernel (bytes): the chunk's V images (16 KB, lane
// l's 16 bytes of image i at 1024 i + 16 l) and one round's tiles, bf16
// [row][64 columns] with 128-byte rows whose 16-byte block b sits at
// b ^ ((row >> 1) & 7): P^T and dS^T (64 key rows), Q^T and bf16(w dO)^T
// (128 dim rows).
constexpr uint32_t kKvV = 0;
constexpr uint32_t kKvPt = 16384;
constexpr uint32_t kKvDs = kKvPt + 8192;
constexpr uint32_t kKvQt = kKvDs + 8192;
constexpr uint32_t kKvWd = kKvQt + 16384;
constexpr uint32_t kKvBytes = kKvWd + 16384;

__device__ __forceinline__ uint32_t tile_off(uint32_t base, int row, int col) {
  return base + row * 128 + ((((col >> 3) ^ ((row >> 1) & 7))) << 4) + (col & 7) * 2;
}
__device__ __forceinline__ u32x4_t tile_read(const unsigned char* sm, uint32_t base, int row,
                                             int blk) {
  return *reinterpret_cast<const u32x4_t*>(sm + base + row * 128 +
                                           ((blk ^ ((row >> 1) & 7)) << 4));
}
__device__ __forceinline__ void tile_put(unsigned char* sm, uint32_t base, int row, int col,
                                         uint32_t v16) {
  *reinterpret_cast<uint16_t*>(sm + tile_off(base, row, col)) = (uint16_t)v16;
}

// One workgroup per work unit: chunk (b, h, c) and a segment of its pairs.
// A round takes 8 pairs, two per wave (16 columns: pair 8 j >> 3, head j & 7):
//   phase 1 (per wave): S^T = K . Q^T (K images in registers), dP^T = V . dO^T
//     (V images from LDS), the chunk gradient, and the columns of P^T, dS^T,
//     Q^T, bf16(w dO)^T into the round's tiles;
//   phase 2 (wave w: dims 32 w .. + 31): dK += dS^T . Q, dV += P^T . bf16(w dO)
//     over the round's 64 columns (two k-steps).
template <bool ALIBI>
__global__ void __launch_bounds__(kThreads, 2) routed_attn_dkv_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char sm[kKvBytes];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int j = lane & 15, grp = lane >> 4;
  const int64_t N = a.B * a.Hkv * a.Ck;
  const int64_t u = blockIdx.x;
  if (u >= (int64_t)a.ustart[N]) return;  // workgroup-uniform
  // the chunk whose units hold u: ustart[lo] <= u < ustart[lo + 1]
  int64_t lo = 0, hi = N;
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)a.ustart[mid] <= u) lo = mid;
    else hi = mid;
  }
  const int64_t bhc = lo;
  const int64_t cs = a.start[bhc], ce = a.start[bhc + 1];
  const int64_t e0 = cs + (u - a.ustart[bhc]) * kSegEntries;
  const int64_t e1 = min(ce, e0 + kSegEntries);
  const bool whole = ce - cs <= kSegEntries;
  const int64_t c = bhc % a.Ck;
  const int64_t bh = bhc / a.Ck;
  const int h = (int)(bh % a.Hkv);
  const int64_t b = bh / a.Hkv;
  const int G = a.G, K = a.K;

  uint64_t excl = a.mask_last ? (1ull << 63) : 0ull;
  if (a.key_valid)
    excl |= ~nonzero_bits(reinterpret_cast<const int8_t*>(a.key_valid + b * a.Lk + c * 64));
  const uint32_t l16 = 16u * lane;
  const uint32_t cb = (uint32_t)c * kFragBytes;
  u32x4_t kb[4][4];
  load_rows(kb, make_rsrc(a.fwd + (b * a.Hkv + h) * a.Ck * 16384, (uint32_t)a.Ck * kFragBytes),
            l16, cb);
  {
    // the V images: the first half of the chunk's bwd fragment (16 KB)
    const unsigned char* vsrc =
        reinterpret_cast<const unsigned char*>(a.bwd + (b * a.Hkv + h) * a.Ck * 16384) + cb;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int o = 16 * (tid + kThreads * i);
      *reinterpret_cast<u32x4_t*>(sm + kKvV + o) = *reinterpret_cast<const u32x4_t*>(vsrc + o);
    }
  }
  f32x4_t dk[4][2], dv[4][2];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      dk[mt][dt] = zero4();
      dv[mt][dt] = zero4();
    }
  const float c2 = a.scale_log2;
  const int g = j & 7;
  const int col = 16 * wave + j;
  __syncthreads();  // V images staged

  for (int64_t r0 = e0; r0 < e1; r0 += 8) {
    // The tile addresses derive from lane values redefined each round, so
    // they are formed where used rather than held in registers across rounds.
    int lj = j, lg = grp, lc = col;
    asm volatile("" : "+v"(lj), "+v"(lg), "+v"(lc));
    // ---- phase 1
    const int64_t e = r0 + 2 * wave + (j >> 3);
    const bool have = e < e1;
    const bool cvalid = have && g < G;
    int64_t q = 0;
    int k = 0;
    if (have) {
      const int32_t v = a.list[e];
      q = v & 0xffffff;
      k = (v >> 24) & 63;
    }
    const int64_t row = (b * a.Lq + q) * a.Hq + (int64_t)h * G + g;
    u32x4_t Qb[4], Db[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const u32x4_t z = {0u, 0u, 0u, 0u};
      Qb[ks] = z;
      Db[ks] = z;
      if (cvalid) {
        Qb[ks] = *reinterpret_cast<const u32x4_t*>(a.q + row * 128 + 32 * ks + 8 * grp);
        Db[ks] = *reinterpret_cast<const u32x4_t*>(a.dout + row * 128 + 32 * ks + 8 * grp);
      }
    }
    const float wv = cvalid ? bf16_to_f32(a.w[row * K + k]) : 0.f;
    uint64_t ex = excl;
    if (a.keep && have) ex |= ~keep_row_bits(a.keep + (((b * a.Lq + q) * a.Hkv + h) * K + k) * 64);
    const uint64_t msh = ex >> (4 * grp);
    f32x4_t S[4], dP[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      S[mt] = zero4();
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) S[mt] = mfma_bf16_16x16x32(kb[mt][ks], Qb[ks], S[mt]);
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      dP[mt] = zero4();
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const u32x4_t vi =
            *reinterpret_cast<const u32x4_t*>(sm + kKvV + 1024 * (4 * mt + ks) + l16);
        dP[mt] = mfma_bf16_16x16x32(vi, Db[ks], dP[mt]);
      }
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int e8 = 0; e8 < 8; ++e8) {
        const int dim = 32 * ks + 8 * lg + e8;
        const uint32_t qv = (Qb[ks][e8 >> 1] >> (16 * (e8 & 1))) & 0xffffu;
        const float dov = bf16_to_f32((Db[ks][e8 >> 1] >> (16 * (e8 & 1))) & 0xffffu);
        tile_put(sm, kKvQt, dim, lc, qv);
        tile_put(sm, kKvWd, dim, lc, f32_to_bf16(wv * dov));
      }
    const float sl = ALIBI && cvalid ? -a.slope[(int64_t)h * G + g] * c2 : 0.f;
    const float di = chunk_grad(S, dP, msh, c2, a.scale * wv, ALIBI, sl, lg);  // S <- P, dP <- dS
    if (cvalid && grp == 0) a.dw[row * K + k] = (uint16_t)f32_to_bf16(di);
    // dS of this lane's column packed in the tiled key order (reduction
    // index 8 grp + e of k-step ks is key 32 ks + 16 (e >> 2) + 4 grp +
    // (e & 3)), the P^T operand order of the forward's tiles: stored as the
    // column's record for the dQ walk.
    {
      u32x4_t Sb[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        Sb[ks][0] = pack_bf16x2(dP[2 * ks][0], dP[2 * ks][1]);
        Sb[ks][1] = pack_bf16x2(dP[2 * ks][2], dP[2 * ks][3]);
        Sb[ks][2] = pack_bf16x2(dP[2 * ks + 1][0], dP[2 * ks + 1][1]);
        Sb[ks][3] = pack_bf16x2(dP[2 * ks + 1][2], dP[2 * ks + 1][3]);
      }
      // The dS record of this lane's column (pair e, head g): its 16 keys
      // (the dQ walk adds dS . K afterwards).
      if (cvalid) {
        uint16_t* rec =
            a.ds_rec + ((((b * a.Lq + q) * a.Hq + (int64_t)h * G + g) * K + k) * 64 + 16 * lg);
        *reinterpret_cast<u32x4_t*>(rec) = Sb[0];
        *reinterpret_cast<u32x4_t*>(rec + 8) = Sb[1];
      }
    }
    // this wave's columns of the tiles (columns without a pair or head hold
    // zeros in dS^T and bf16(w dO)^T, so they add nothing)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = 16 * mt + 4 * lg + r;
        tile_put(sm, kKvPt, key, lc, f32_to_bf16(S[mt][r]));
        tile_put(sm, kKvDs, key, lc, f32_to_bf16(dP[mt][r]));
      }
    __syncthreads();
    // ---- phase 2: keys x dims 32 wave .. + 31, reduction over the columns
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      u32x4_t bq[2], bw[2];
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const int dim = 32 * wave + 16 * dt + lj;
        bq[dt] = tile_read(sm, kKvQt, dim, 4 * ks + lg);
        bw[dt] = tile_read(sm, kKvWd, dim, 4 * ks + lg);
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const u32x4_t ad = tile_read(sm, kKvDs, 16 * mt + lj, 4 * ks + lg);
        const u32x4_t ap = tile_read(sm, kKvPt, 16 * mt + lj, 4 * ks + lg);
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
          dk[mt][dt] = mfma_bf16_16x16x32(ad, bq[dt], dk[mt][dt]);
          dv[mt][dt] = mfma_bf16_16x16x32(ap, bw[dt], dv[mt][dt]);
        }
      }
    }
    __syncthreads();
  }
  // lane (grp, j) of tile (mt, dt): keys 16 mt + 4 grp + r, dim 32 wave + 16 dt + j
  float* dkb = a.dk + ((b * a.Lk + c * 64) * a.Hkv + h) * 128;
  float* dvb = a.dv + ((b * a.Lk + c * 64) * a.Hkv + h) * 128;
  const int64_t krow = (int64_t)a.Hkv * 128;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t off = (int64_t)(16 * mt + 4 * grp + r) * krow + 32 * wave + 16 * dt + j;
        if (whole) {
          dkb[off] = dk[mt][dt][r];
          dvb[off] = dv[mt][dt][r];
        } else {
          atomicAdd(dkb + off, dk[mt][dt][r]);
          atomicAdd(dvb + off, dv[mt][dt][r]);
        }
      }
}

__global__ void __launch_bounds__(256) fill_zero_i32(int32_t* p, int64_t n) {
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0;
}

struct ListPlan {
  int nqb;
  int64_t n;  // chunks B * Hkv * Ck
  int64_t count, blkbase, start, ustart, list, records, total;  // byte offsets / size
  int64_t max_units;
};

ListPlan list_plan(int64_t B, int64_t Lq, int64_t Hkv, int64_t K, int64_t Ck, int64_t Hq) {
  ListPlan p;
  p.nqb = (int)((Lq + kListBlock - 1) / kListBlock);
  p.n = B * Hkv * Ck;
  const int64_t pairs = B * Lq * Hkv * K;
  int64_t o = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = o;
    o += (bytes + 255) / 256 * 256;
    return at;
  };
  p.count = take(p.n * 4);
  p.blkbase = take(B * Hkv * p.nqb * Ck * 4);
  p.start = take((p.n + 1) * 4);
  p.ustart = take((p.n + 1) * 4);
  p.list = take(pairs * 4);
  p.records = take(B * Lq * Hq * K * 64 * 2);  // dS records of the dQ walk
  p.total = o;
  p.max_units = (pairs + kSegEntries - 1) / kSegEntries + p.n;
  return p;
}

}  // namespace

namespace {

int selected_backward(
    const void* q, const void* grad_out, const void* kv_frags, const void* kv_frags_bwd,
    const void* weights, const int32_t* indices, const uint8_t* key_valid,
    const int8_t* token_keep, int64_t batch, int64_t q_len, int64_t kv_len, int64_t q_heads,
    int64_t kv_heads, int64_t head_dim, int64_t topk, int64_t chunk_size, int mask_last_token,
    float sm_scale, float* grad_q, float* grad_k, float* grad_v, void* grad_weights,
    void* workspace, int64_t workspace_bytes, void* stream, const float* slope) {
  if (batch < 0 || q_len < 0 || kv_len < 0 || q_heads <= 0 || kv_heads <= 0 ||
      q_heads % kv_heads != 0 || head_dim <= 0 || topk <= 0 || chunk_size <= 0 ||
      !(sm_scale > 0.f) || sm_scale == __builtin_inff())
    return MRSA_ERR_INVALID_ARGUMENT;
  if (kv_len % chunk_size != 0) return MRSA_ERR_INVALID_ARGUMENT;
  if (chunk_size != 64 || head_dim != 128 || q_heads / kv_heads > 8 || topk > kMaxTopk)
    return MRSA_ERR_UNSUPPORTED;
  if (kv_len / 64 > kMaxListChunks || q_len >= (1 << 24)) return MRSA_ERR_UNSUPPORTED;
  if (batch * q_len * kv_heads * topk >= 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  if (batch == 0 || q_len == 0) return MRSA_OK;
  if (!q || !grad_out || !kv_frags || !kv_frags_bwd || !weights || !indices || !grad_q ||
      !grad_k || !grad_v || !grad_weights || !workspace)
    return MRSA_ERR_INVALID_ARGUMENT;
  const ListPlan lp = list_plan(batch, q_len, kv_heads, topk, kv_len / 64, q_heads);
  if (workspace_bytes < lp.total || (uintptr_t)workspace % 256 != 0)
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
  a.slope = slope;
  if (lp.max_units > 0x7fffffff || lp.nqb > 0x7fffffff || batch * kv_heads > 65535)
    return MRSA_ERR_UNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  // pair lists, then the chunk-major pass
  char* ws = (char*)workspace;
  int32_t* count = (int32_t*)(ws + lp.count);
  int32_t* blkbase = (int32_t*)(ws + lp.blkbase);
  int32_t* start = (int32_t*)(ws + lp.start);
  int32_t* ustart = (int32_t*)(ws + lp.ustart);
  int32_t* list = (int32_t*)(ws + lp.list);
  hipLaunchKernelGGL(fill_zero_i32, dim3((unsigned)std::min<int64_t>((lp.n + 255) / 256, 4096)),
                     dim3(256), 0, st, count, lp.n);
  const dim3 lgrid((unsigned)lp.nqb, (unsigned)(batch * kv_heads));
  hipLaunchKernelGGL(list_count_kernel, lgrid, dim3(kListBlock), 0, st, a, count, blkbase, lp.nqb);
  hipLaunchKernelGGL(list_scan_kernel, dim3(1), dim3(1024), 0, st, (const int32_t*)count, lp.n,
                     start, ustart);
  a.start = start;
  a.ustart = ustart;
  hipLaunchKernelGGL(list_fill_kernel, lgrid, dim3(kListBlock), 0, st, a,
                     (const int32_t*)blkbase, lp.nqb, list);
  a.list = list;
  a.ds_rec = (uint16_t*)(ws + lp.records);
  if (slope)
    hipLaunchKernelGGL(routed_attn_dkv_kernel<true>, dim3((unsigned)lp.max_units), dim3(kThreads),
                       0, st, a);
  else
    hipLaunchKernelGGL(routed_attn_dkv_kernel<false>, dim3((unsigned)lp.max_units), dim3(kThreads),
                       0, st, a);
  const int s2 = mrsa_launch_status();
  if (s2 != MRSA_OK) return s2;
  // dQ: the forward's walk over each query tile's chunks, adding dS . K
  // into rows it owns (no atomics) from the records just written
  return mrsa::routed_dq_walk(kv_frags_bwd, a.ds_rec, indices, key_valid, batch, q_len, kv_len,
                              q_heads, kv_heads, topk, grad_q, stream);
}

}  // namespace

extern "C" int mrsa_selected_attention_bwd(
    const void* q, const void* grad_out, const void* kv_frags, const void* kv_frags_bwd,
    const void* weights, const int32_t* indices, const uint8_t* key_valid,
    const int8_t* token_keep, int64_t batch, int64_t q_len, int64_t kv_len, int64_t q_heads,
    int64_t kv_heads, int64_t head_dim, int64_t topk, int64_t chunk_size, int mask_last_token,
    float sm_scale, float* grad_q, float* grad_k, float* grad_v, void* grad_weights,
    void* workspace, int64_t workspace_bytes, void* stream) {
  return selected_backward(q, grad_out, kv_frags, kv_frags_bwd, weights, indices, key_valid,
                           token_keep, batch, q_len, kv_len, q_heads, kv_heads, head_dim, topk,
                           chunk_size, mask_last_token, sm_scale, grad_q, grad_k, grad_v,
                           grad_weights, workspace, workspace_bytes, stream, nullptr);
}

extern "C" int mrsa_selected_attention_alibi_bwd(
    const void* q, const void* grad_out, const void* kv_frags, const void* kv_frags_bwd,
    const void* weights, const int32_t* indices, const uint8_t* key_valid,
    const int8_t* token_keep, const float* slope, int64_t batch, int64_t q_len, int64_t kv_len,
    int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t topk, int64_t chunk_size,
    int mask_last_token, float sm_scale, float* grad_q, float* grad_k, float* grad_v,
    void* grad_weights, void* workspace, int64_t workspace_bytes, void* stream) {
  if (batch > 0 && q_len > 0 && !slope) return MRSA_ERR_INVALID_ARGUMENT;
  return selected_backward(q, grad_out, kv_frags, kv_frags_bwd, weights, indices, key_valid,
                           token_keep, batch, q_len, kv_len, q_heads, kv_heads, head_dim, topk,
                           chunk_size, mask_last_token, sm_scale, grad_q, grad_k, grad_v,
                           grad_weights, workspace, workspace_bytes, stream, slope);
}

extern "C" int64_t mrsa_selected_attention_bwd_workspace_bytes(int64_t batch, int64_t q_len,
                                                               int64_t kv_len, int64_t q_heads,
                                                               int64_t kv_heads, int64_t topk) {
  if (batch < 0 || q_len < 0 || kv_len < 0 || q_heads <= 0 || kv_heads <= 0 || topk <= 0 ||
      kv_len % 64 || q_heads % kv_heads)
    return -1;
  return list_plan(batch, q_len, kv_heads, topk, kv_len / 64, q_heads).total;
}
