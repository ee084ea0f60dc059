// Routed (selected-chunk) attention and candidate token scores.
//
// out[q, g] = sum_k w[q, g, k] * softmax_{s in chunk idx[q, k], s valid}(q_g . k_s * scale) . V
// Each routed chunk is normalised on its own (ops/hils_fwd_bwd_head.py:453-559;
// formula restated in the reference test test_hils_non_power_two_topk.py:122-138):
// the landmark slot (last key of the chunk, when mask_last_token) and invalid
// keys are excluded, P = bf16(p * w / sum p) feeds the PV product with fp32
// accumulation, and a chunk whose keys are all masked contributes nothing.
// Index lists are read like the reference kernel: a query's list ends at its
// first negative entry; entries >= kv_len / 64 are skipped.
//
// Work split.  A workgroup owns a tile of queries of one KV head; each of its 8
// waves owns a fixed set of those queries, whose output accumulators stay in
// registers for the whole kernel.  The workgroup walks the union of the tile's
// routed chunks in ascending order; every chunk's K and V are staged in LDS
// once and every wave that owns a query routed to that chunk consumes them:
//   S^T = K_chunk (64 x 128) . Q^T (2 queries x 8 head columns)   16 MFMAs
//   per-column softmax over the 64 keys, scaled by the routing weight
//   O^T += V_chunk^T (128 x 64) . P^T                            16 MFMAs
// Columns of queries that do not own the chunk get P = 0.  When every
// query's list is strictly ascending (what the router emits), the chunk walk
// comes from a bitmask union; otherwise a k-way merge over the lists (the
// reference's ownership merge, hils_fwd_bwd_head.py:346-409) produces it.
//
// Token-score mode (candidate_token_scores_gqa,
// ops/hils_token_score_gqa_tilelang.py:17-114) reuses the walk and the S^T
// product and writes, per routed (query, slot), max over the group of q.k
// times sm_scale for every key, -inf at the last slot and invalid keys.
#include "mrsa_device.h"

using namespace mrsa;

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kKPitch = 136;
constexpr int kVPitch = 72;
constexpr int kStageVecs = 2048;
constexpr int kPer = kStageVecs / kThreads;  // 4
constexpr int kMaxTopk = 64;

struct SelArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* vt;
  const uint16_t* w;
  const int32_t* idx;
  const uint8_t* key_valid;
  int64_t B, Lq, Lk;
  int Hq, Hkv, G, K;
  int64_t Ck;   // chunks in the cache
  int64_t NTk;  // 64-key tiles in the cache (== Ck)
  int mask_last;
  float scale_log2;
  float sm_scale;
  int token_mode;
  uint16_t* out;
  float* tscores;
};

// LDS carve-up of the selected-attention workgroup (byte offsets, 16-aligned).
struct SelLayout {
  size_t ks, vs, umask, ulist, omask, comp_idx, comp_slot, comp_len, misc, kvbits, wts, total;
};
__host__ __device__ inline size_t align16(size_t x) { return (x + 15) & ~(size_t)15; }
__host__ __device__ inline SelLayout sel_layout(int TQ, int K, int64_t Ck) {
  SelLayout l;
  const size_t n = (size_t)TQ * K;
  size_t o = 0;
  l.ks = o;        o = align16(o + 2 * (size_t)64 * kKPitch * 2);   // two buffers
  l.vs = o;        o = align16(o + 2 * (size_t)128 * kVPitch * 2);
  l.umask = o;     o = align16(o + n * 8);
  l.ulist = o;     o = align16(o + n * 4);
  l.omask = o;     o = align16(o + (size_t)Ck * 8);
  l.comp_idx = o;  o = align16(o + n * 4);
  l.comp_slot = o; o = align16(o + n);
  l.comp_len = o;  o = align16(o + (size_t)TQ * 4);
  l.misc = o;      o = align16(o + (size_t)(4 + kThreads) * 4);
  l.kvbits = o;    o = align16(o + (size_t)Ck * 8);   // per-chunk key-valid bits
  l.wts = o;       o = align16(o + (size_t)TQ * 8 * K * 2);  // [TQ][8][K] bf16 weights
  l.total = o;
  return l;
}

template <int NTILE, bool TOKEN>
__global__ void __launch_bounds__(kThreads) selected_attn_kernel(SelArgs a) {
  constexpr int QPW = 2 * NTILE;      // queries per wave
  constexpr int TQ = kWaves * QPW;    // queries per workgroup (<= 64)
  extern __shared__ __align__(16) unsigned char smem[];
  const int K = a.K;
  const int64_t Ck = a.Ck;
  const SelLayout lay = sel_layout(TQ, K, Ck);
  uint16_t* Ks = reinterpret_cast<uint16_t*>(smem + lay.ks);          // [64][136]
  uint16_t* Vs = reinterpret_cast<uint16_t*>(smem + lay.vs);          // [128][72]
  uint64_t* umask = reinterpret_cast<uint64_t*>(smem + lay.umask);    // [TQ*K]
  int32_t* ulist = reinterpret_cast<int32_t*>(smem + lay.ulist);      // [TQ*K]
  uint64_t* omask = reinterpret_cast<uint64_t*>(smem + lay.omask);    // [Ck]
  int32_t* comp_idx = reinterpret_cast<int32_t*>(smem + lay.comp_idx);  // [TQ][K]
  uint8_t* comp_slot = smem + lay.comp_slot;                           // [TQ][K]
  int32_t* comp_len = reinterpret_cast<int32_t*>(smem + lay.comp_len);  // [TQ]
  int32_t* misc = reinterpret_cast<int32_t*>(smem + lay.misc);  // [0] unsorted, [1] steps, [4..] scan
  uint64_t* kvbits = reinterpret_cast<uint64_t*>(smem + lay.kvbits);  // [Ck]
  uint16_t* wts = reinterpret_cast<uint16_t*>(smem + lay.wts);          // [TQ][8][K]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int64_t b = blockIdx.z;
  const int h = blockIdx.y;
  const int64_t q0 = (int64_t)blockIdx.x * TQ;
  const int G = a.G;

  // 1. Per-query compacted lists (thread per query).
  if (tid == 0) misc[0] = 0;
  __syncthreads();
  if (tid < TQ) {
    const int64_t qi = q0 + tid;
    int n = 0;
    bool sorted = true;
    int prev = -1;
    if (qi < a.Lq) {
      const int32_t* row = a.idx + ((b * a.Lq + qi) * a.Hkv + h) * K;
      for (int kk = 0; kk < K; ++kk) {
        const int32_t c = row[kk];
        if (c < 0) break;
        if (c >= Ck) {
          sorted = false;
          continue;
        }
        if (c <= prev) sorted = false;
        prev = c;
        comp_idx[tid * K + n] = c;
        comp_slot[tid * K + n] = (uint8_t)kk;
        ++n;
      }
    }
    comp_len[tid] = n;
    if (!sorted) misc[0] = 1;
  }
  __syncthreads();
  const bool merge_path = misc[0] != 0;

  // 2. The ordered chunk walk with owner masks.
  if (!merge_path) {
    for (int64_t c = tid; c < Ck; c += kThreads) omask[c] = 0ull;
    __syncthreads();
    for (int e = tid; e < TQ * K; e += kThreads) {
      const int qq = e / K, r = e - qq * K;
      if (r < comp_len[qq]) atomicOr((unsigned long long*)&omask[comp_idx[e]], 1ull << qq);
    }
    __syncthreads();
    // Compaction: thread t scans a contiguous chunk range.
    const int64_t per = (Ck + kThreads - 1) / kThreads;
    const int64_t c0 = tid * per, c1 = min(Ck, c0 + per);
    int cnt = 0;
    for (int64_t c = c0; c < c1; ++c) cnt += omask[c] != 0ull;
    int* scan = misc + 4;
    scan[tid] = cnt;
    __syncthreads();
    for (int o = 1; o < kThreads; o <<= 1) {
      const int add = tid >= o ? scan[tid - o] : 0;
      __syncthreads();
      scan[tid] += add;
      __syncthreads();
    }
    int pos = scan[tid] - cnt;
    if (tid == kThreads - 1) misc[1] = scan[tid];
    for (int64_t c = c0; c < c1; ++c) {
      const uint64_t m = omask[c];
      if (m) {
        ulist[pos] = (int32_t)c;
        umask[pos] = m;
        ++pos;
      }
    }
  } else if (wave == 0) {
    int ptr = 0;
    const int len = lane < TQ ? comp_len[lane] : 0;
    int n = 0;
    for (int step = 0; step < TQ * K; ++step) {
      const int cur = ptr < len ? comp_idx[lane * K + ptr] : 0x7fffffff;
      const int m = wave_min_i(cur);
      if (m == 0x7fffffff) break;
      const bool own = cur == m && lane < TQ;
      const uint64_t om = __ballot(own);
      if (own) ++ptr;
      if (lane == 0) {
        ulist[n] = m;
        umask[n] = om;
      }
      ++n;
    }
    if (lane == 0) misc[1] = n;
  }
  __syncthreads();
  const int nsteps = misc[1];

  // Per-chunk key-valid bits and this tile's routing weights, staged once.
  for (int64_t c = wave; c < Ck; c += kWaves) {
    const bool ok = a.key_valid ? a.key_valid[b * a.Lk + c * 64 + lane] != 0 : true;
    const uint64_t vb = __ballot(ok);
    if (lane == 0) kvbits[c] = vb;
  }
  if (!TOKEN) {
    for (int e = tid; e < TQ * 8 * K; e += kThreads) {
      const int qq = e / (8 * K), rem = e - qq * 8 * K;
      const int gg = rem / K, kk = rem - gg * K;
      const int64_t qi = q0 + qq;
      wts[e] = (qi < a.Lq && gg < G) ? a.w[((b * a.Lq + qi) * a.Hq + h * G + gg) * K + kk] : 0;
    }
  }

  // 3. Q^T operands for this wave's queries (2 per column tile, 8 columns each).
  u32x4_t Qb[NTILE][4];
  f32x4_t acc[NTILE][8];
  int rank[NTILE];
#pragma unroll
  for (int nt = 0; nt < NTILE; ++nt) {
    const int ql = wave * QPW + 2 * nt + (col >> 3);
    const int gg = col & 7;
    const int64_t qi = q0 + ql;
    rank[nt] = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4_t z = {0u, 0u, 0u, 0u};
      Qb[nt][j] = z;
      if (qi < a.Lq && gg < G)
        Qb[nt][j] = *reinterpret_cast<const u32x4_t*>(
            a.q + ((b * a.Lq + qi) * a.Hq + h * G + gg) * 128 + 32 * j + 8 * grp);
    }
#pragma unroll
    for (int td = 0; td < 8; ++td) acc[nt][td] = zero4();
  }

  // Staging: uniform (scalar) chunk bases plus per-lane 32-bit offsets.
  const uint16_t* kbase = a.k + (b * a.Lk) * (int64_t)a.Hkv * 128 + (int64_t)h * 128;
  const uint16_t* vbase =
      TOKEN ? nullptr : a.vt + ((b * a.Hkv + h) * a.NTk) * (int64_t)(128 * 64);
  const int kstride = a.Hkv * 128;
  u32x4_t pre[kPer];
  auto prefetch = [&](int64_t c) {
    const uint16_t* kc = kbase + c * 64 * (int64_t)kstride;
    const uint16_t* vc = TOKEN ? nullptr : vbase + c * (128 * 64);
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const int v = tid + p * kThreads;
      if (v < 1024) {
        pre[p] = *reinterpret_cast<const u32x4_t*>(kc + (v >> 4) * kstride + (v & 15) * 8);
      } else if (!TOKEN) {
        pre[p] = *reinterpret_cast<const u32x4_t*>(vc + (v - 1024) * 8);
      } else {
        u32x4_t z = {0u, 0u, 0u, 0u};
        pre[p] = z;
      }
    }
  };
  auto commit = [&](int buf) {
    uint16_t* Kb = Ks + buf * (64 * kKPitch);
    uint16_t* Vb = Vs + buf * (128 * kVPitch);
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const int v = tid + p * kThreads;
      if (v < 1024)
        *reinterpret_cast<u32x4_t*>(Kb + (v >> 4) * kKPitch + (v & 15) * 8) = pre[p];
      else
        *reinterpret_cast<u32x4_t*>(Vb + ((v - 1024) >> 3) * kVPitch + ((v - 1024) & 7) * 8) = pre[p];
    }
  };
  if (nsteps > 0) {
    prefetch(ulist[0]);
    commit(0);
  }
  __syncthreads();

  const uint64_t last_mask = a.mask_last ? (1ull << 63) : 0ull;
  for (int st = 0; st < nsteps; ++st) {
    const int buf = st & 1;
    const uint64_t om = umask[st];
    const uint64_t masked = (~kvbits[ulist[st]]) | last_mask;  // keys excluded from the softmax
    if (st + 1 < nsteps) prefetch(ulist[st + 1]);
    const uint16_t* Kb = Ks + buf * (64 * kKPitch);
    const uint16_t* Vb = Vs + buf * (128 * kVPitch);
    const uint32_t wbits = (uint32_t)((om >> (wave * QPW)) & ((1ull << QPW) - 1ull));

#pragma unroll
    for (int nt = 0; nt < NTILE; ++nt) {
      const uint32_t pair = (wbits >> (2 * nt)) & 3u;
      if (pair == 0u) continue;
      const int half = col >> 3, gg = col & 7;
      const bool owns = (pair >> half) & 1u;
      const int ql = wave * QPW + 2 * nt + half;
      const int64_t qi = q0 + ql;
      // Opaque zero: keeps the compiler from hoisting this tile's K / V operand
      // reads out of the tile loop (that would pin 128 extra registers).
      int zoff = 0;
      asm volatile("" : "+v"(zoff));
      const uint16_t* Kt = Kb + zoff;
      const uint16_t* Vt = Vb + zoff;

      f32x4_t S[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) S[t] = zero4();
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const u32x4_t Ka =
              *reinterpret_cast<const u32x4_t*>(Kt + (16 * t + col) * kKPitch + 32 * j + 8 * grp);
          S[t] = mfma_bf16_16x16x32(Ka, Qb[nt][j], S[t]);
        }
      }
      int slot = 0;
      if (owns) {
        slot = comp_slot[ql * K + rank[nt]];
        ++rank[nt];
      }

      if constexpr (TOKEN) {
        // max over the query's G head columns (lanes sharing col >> 3).
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float v = gg < G ? S[t][i] : neg_inf();
            v = fmaxf(v, __shfl_xor(v, 1, 64));
            v = fmaxf(v, __shfl_xor(v, 2, 64));
            v = fmaxf(v, __shfl_xor(v, 4, 64));
            S[t][i] = v;
          }
        if (owns && gg == 0) {
          float* dst = a.tscores + (((b * a.Lq + qi) * a.Hkv + h) * K + slot) * 64;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            f32x4_t o;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int s = 16 * t + 4 * grp + i;
              o[i] = ((masked >> s) & 1ull) ? neg_inf() : S[t][i] * a.sm_scale;
            }
            *reinterpret_cast<f32x4_t*>(dst + 16 * t + 4 * grp) = o;
          }
        }
        continue;
      }

      const float wv = owns ? bf16_to_f32(wts[(ql * 8 + gg) * K + slot]) : 0.f;
      float mx = neg_inf();
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int s = 16 * t + 4 * grp + i;
          float v = S[t][i] * a.scale_log2;
          if ((masked >> s) & 1ull) v = neg_inf();
          S[t][i] = v;
          mx = fmaxf(mx, v);
        }
      mx = across4_max(mx);
      float sum = 0.f;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = (mx == neg_inf()) ? 0.f : exp2f(S[t][i] - mx);
          S[t][i] = p;
          sum += p;
        }
      sum = across4_sum(sum);
      const float f = (sum > 0.f) ? wv / sum : 0.f;
      u32x4_t Pb[2];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        Pb[jj][0] = pack_bf16x2(S[2 * jj][0] * f, S[2 * jj][1] * f);
        Pb[jj][1] = pack_bf16x2(S[2 * jj][2] * f, S[2 * jj][3] * f);
        Pb[jj][2] = pack_bf16x2(S[2 * jj + 1][0] * f, S[2 * jj + 1][1] * f);
        Pb[jj][3] = pack_bf16x2(S[2 * jj + 1][2] * f, S[2 * jj + 1][3] * f);
      }
#pragma unroll
      for (int td = 0; td < 8; ++td) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const uint16_t* vrow = Vt + (16 * td + col) * kVPitch + 32 * jj + 4 * grp;
          const u32x2_t v0 = *reinterpret_cast<const u32x2_t*>(vrow);
          const u32x2_t v1 = *reinterpret_cast<const u32x2_t*>(vrow + 16);
          u32x4_t Va = {v0[0], v0[1], v1[0], v1[1]};
          acc[nt][td] = mfma_bf16_16x16x32(Va, Pb[jj], acc[nt][td]);
        }
      }
    }
    if (st + 1 < nsteps) commit(buf ^ 1);
    __syncthreads();
  }

  if constexpr (TOKEN) return;
#pragma unroll
  for (int nt = 0; nt < NTILE; ++nt) {
    const int ql = wave * QPW + 2 * nt + (col >> 3);
    const int gg = col & 7;
    const int64_t qi = q0 + ql;
    if (qi >= a.Lq || gg >= G) continue;
    uint16_t* orow = a.out + ((b * a.Lq + qi) * a.Hq + h * G + gg) * 128;
#pragma unroll
    for (int td = 0; td < 8; ++td) {
      u32x2_t o;
      o[0] = pack_bf16x2(acc[nt][td][0], acc[nt][td][1]);
      o[1] = pack_bf16x2(acc[nt][td][2], acc[nt][td][3]);
      *reinterpret_cast<u32x2_t*>(orow + 16 * td + 4 * grp) = o;
    }
  }
}

// Token-score mode fills every (query, slot) row first with -inf so that
// slots without a routed chunk read as fully masked.
__global__ void __launch_bounds__(256) fill_neg_inf(float* p, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += stride)
    p[e] = neg_inf();
}

constexpr int kNtile = 3;

int launch_selected(SelArgs& a, hipStream_t s) {
  constexpr int TQ = kWaves * 2 * kNtile;
  const size_t smem = sel_layout(TQ, a.K, a.Ck).total;
  if (smem > 160 * 1024) return MRSA_ERR_UNSUPPORTED;
  auto kern = a.token_mode ? selected_attn_kernel<kNtile, true> : selected_attn_kernel<kNtile, false>;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess)
    return MRSA_ERR_LAUNCH;
  dim3 grid((unsigned)((a.Lq + TQ - 1) / TQ), (unsigned)a.Hkv, (unsigned)a.B);
  hipLaunchKernelGGL(kern, grid, dim3(kThreads), smem, s, a);
  return mrsa_launch_status();
}

int check_common(const void* q, const void* k, const int32_t* indices, int64_t batch,
                 int64_t q_len, int64_t kv_len, int64_t q_heads, int64_t kv_heads,
                 int64_t head_dim, int64_t topk, int64_t chunk_size) {
  if (batch < 0 || q_len < 0 || kv_len < 0 || q_heads <= 0 || kv_heads <= 0 ||
      q_heads % kv_heads != 0 || head_dim <= 0 || topk <= 0 || chunk_size <= 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (kv_len % chunk_size != 0) return MRSA_ERR_INVALID_ARGUMENT;
  if (chunk_size != 64 || head_dim != 128 || q_heads / kv_heads > 8 || topk > kMaxTopk)
    return MRSA_ERR_UNSUPPORTED;
  if (kv_heads > 65535 || batch > 65535) return MRSA_ERR_UNSUPPORTED;
  if (batch > 0 && q_len > 0 && (!q || !k || !indices)) return MRSA_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)q | (uintptr_t)k) % 16 != 0) return MRSA_ERR_INVALID_ARGUMENT;
  return MRSA_OK;
}

}  // namespace

extern "C" int mrsa_selected_attention_fwd(const void* q, const void* k, const void* v_tiles,
                                           const void* weights, const int32_t* indices,
                                           const uint8_t* key_valid, int64_t batch,
                                           int64_t q_len, int64_t kv_len, int64_t q_heads,
                                           int64_t kv_heads, int64_t head_dim, int64_t topk,
                                           int64_t chunk_size, int mask_last_token,
                                           float sm_scale, void* out, void* stream) {
  int st = check_common(q, k, indices, batch, q_len, kv_len, q_heads, kv_heads, head_dim, topk,
                        chunk_size);
  if (st != MRSA_OK) return st;
  if (batch == 0 || q_len == 0) return MRSA_OK;
  if (!v_tiles || !weights || !out || (uintptr_t)v_tiles % 16 != 0 || (uintptr_t)out % 8 != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  SelArgs a;
  a.q = (const uint16_t*)q;
  a.k = (const uint16_t*)k;
  a.vt = (const uint16_t*)v_tiles;
  a.w = (const uint16_t*)weights;
  a.idx = indices;
  a.key_valid = key_valid;
  a.B = batch;
  a.Lq = q_len;
  a.Lk = kv_len;
  a.Hq = (int)q_heads;
  a.Hkv = (int)kv_heads;
  a.G = (int)(q_heads / kv_heads);
  a.K = (int)topk;
  a.Ck = kv_len / 64;
  a.NTk = (kv_len + 63) / 64;
  a.mask_last = mask_last_token;
  a.scale_log2 = sm_scale * kLog2e;
  a.sm_scale = sm_scale;
  a.token_mode = 0;
  a.out = (uint16_t*)out;
  a.tscores = nullptr;
  return launch_selected(a, (hipStream_t)stream);
}

extern "C" int mrsa_candidate_token_scores_fwd(const void* q, const void* k,
                                               const int32_t* indices, const uint8_t* key_valid,
                                               int64_t batch, int64_t q_len, int64_t kv_len,
                                               int64_t q_heads, int64_t kv_heads,
                                               int64_t head_dim, int64_t topk,
                                               int64_t chunk_size, float sm_scale,
                                               float* scores, void* stream) {
  int st = check_common(q, k, indices, batch, q_len, kv_len, q_heads, kv_heads, head_dim, topk,
                        chunk_size);
  if (st != MRSA_OK) return st;
  if (batch == 0 || q_len == 0) return MRSA_OK;
  if (!scores || (uintptr_t)scores % 16 != 0) return MRSA_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  const int64_t n = batch * q_len * kv_heads * topk * chunk_size;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 8192);
  hipLaunchKernelGGL(fill_neg_inf, dim3((unsigned)blocks), dim3(256), 0, s, scores, n);
  st = mrsa_launch_status();
  if (st != MRSA_OK) return st;
  SelArgs a;
  a.q = (const uint16_t*)q;
  a.k = (const uint16_t*)k;
  a.vt = nullptr;
  a.w = nullptr;
  a.idx = indices;
  a.key_valid = key_valid;
  a.B = batch;
  a.Lq = q_len;
  a.Lk = kv_len;
  a.Hq = (int)q_heads;
  a.Hkv = (int)kv_heads;
  a.G = (int)(q_heads / kv_heads);
  a.K = (int)topk;
  a.Ck = kv_len / 64;
  a.NTk = (kv_len + 63) / 64;
  a.mask_last = 1;
  a.scale_log2 = sm_scale * kLog2e;
  a.sm_scale = sm_scale;
  a.token_mode = 1;
  a.out = nullptr;
  a.tscores = scores;
  return launch_selected(a, s);
}
