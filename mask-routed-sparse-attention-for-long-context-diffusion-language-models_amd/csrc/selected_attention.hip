// Routed (selected-chunk) attention and candidate token scores.
//
// out[q, g] = sum_k w[q, g, k] * softmax_{s in chunk idx[q, k], s valid}(q_g . k_s * scale) . V
// Each routed chunk is normalised on its own (ops/hils_fwd_bwd_head.py:453-559;
// formula restated in the reference test test_hils_non_power_two_topk.py:122-138):
// the landmark slot (last key of the chunk, when mask_last_token) and invalid
// keys are excluded, P = bf16(p * w / sum p) feeds the PV product with fp32
// accumulation, and a chunk whose keys are all masked contributes nothing.
// Index lists are read like the reference kernel: a query's list ends at its
// first negative entry; entries >= kv_len / 64 are skipped.  A chunk listed
// twice contributes twice (its weights are summed before use).
//
// Work split.  A workgroup owns a tile of 48 queries of one KV head; each of
// its 8 waves owns 6 of those queries (3 column tiles of 2 queries x 8 head
// columns), whose output accumulators stay in registers for the whole
// kernel.  The workgroup walks the union of the tile's routed chunks in
// ascending order.  Each chunk's K and V^T (32 KB) arrive in a 3-slot LDS ring
// by asynchronous global->LDS DMA issued two chunks ahead, so the only
// per-chunk synchronisation is one workgroup barrier.  Every wave with a query
// routed to the chunk consumes it:
//   S^T = K_chunk (64 x 128) . Q^T (2 queries x 8 head columns)   16 MFMAs
//   per-column softmax over the 64 keys, scaled by the routing weight
//   O^T += V_chunk^T (128 x 64) . P^T                            16 MFMAs
// Columns of queries that do not own the chunk get P = 0.
//
// Ring slot layout (16-byte units, XOR-swizzled so the matrix-operand reads of
// 16 consecutive rows hit distinct banks):
//   K   row r (64 keys),  part p (8 dims):  unit r*16 + (p ^ (r & 15))
//   V^T row d (128 dims), part p (8 keys):  unit 1024 + d*8 + (p ^ (d & 7))
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
constexpr int kNtile = 3;               // column tiles per wave
constexpr int kQPW = 2 * kNtile;        // queries per wave
constexpr int kTQ = kWaves * kQPW;      // queries per workgroup
constexpr int kSlotBytes = 32768;       // one chunk: K (16 KB) + V^T (16 KB)
constexpr int kRing = 3;
constexpr int kMaxTopk = 64;

typedef __attribute__((address_space(3))) void lds_void_t;

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

// LDS carve-up (byte offsets, 16-aligned).  comp_idx lives inside the ring: it
// is only needed before the first chunk is loaded.
struct SelLayout {
  size_t ring, wts, kvbits, omask, ulist, umask, comp_slot, comp_len, misc, total;
  size_t comp_idx;
  int cap;
};
__host__ __device__ inline size_t align16(size_t x) { return (x + 15) & ~(size_t)15; }
__host__ __device__ inline SelLayout sel_layout(int K, int64_t Ck) {
  SelLayout l;
  const size_t n = (size_t)kTQ * K;
  l.cap = (int)(Ck < (int64_t)n ? Ck : (int64_t)n);
  size_t o = 0;
  l.ring = o;      o = align16(o + (size_t)kRing * kSlotBytes);
  l.wts = o;       o = align16(o + (size_t)kTQ * 8 * K * 2);   // [TQ][8][K] bf16
  l.kvbits = o;    o = align16(o + (size_t)Ck * 8);
  l.omask = o;     o = align16(o + (size_t)Ck * 8);
  l.ulist = o;     o = align16(o + (size_t)l.cap * 4);
  l.umask = o;     o = align16(o + (size_t)l.cap * 8);
  l.comp_slot = o; o = align16(o + n);
  l.comp_len = o;  o = align16(o + (size_t)kTQ * 4);
  l.misc = o;      o = align16(o + (size_t)(4 + kThreads) * 4);
  l.total = o;
  l.comp_idx = l.ring;
  return l;
}

// Barrier for the chunk ring.  __syncthreads() would also wait for every
// outstanding global access of the wave (vmcnt(0)), including the DMA of the
// chunk being prefetched; this waits only for this wave's DMA of the chunk
// about to be consumed (each wave issues 4 DMA instructions per chunk) and for
// its LDS accesses, then synchronises the workgroup.
__device__ __forceinline__ void ring_barrier(bool leave_one_chunk) {
  if (leave_one_chunk)
    asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <bool TOKEN>
__global__ void __launch_bounds__(kThreads) selected_attn_kernel(SelArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int K = a.K;
  const int64_t Ck = a.Ck;
  const SelLayout lay = sel_layout(K, Ck);
  unsigned char* ring = smem + lay.ring;
  uint16_t* wts = reinterpret_cast<uint16_t*>(smem + lay.wts);          // [TQ][8][K]
  uint64_t* kvbits = reinterpret_cast<uint64_t*>(smem + lay.kvbits);    // [Ck]
  uint64_t* omask = reinterpret_cast<uint64_t*>(smem + lay.omask);      // [Ck]
  int32_t* ulist = reinterpret_cast<int32_t*>(smem + lay.ulist);        // [cap]
  uint64_t* umask = reinterpret_cast<uint64_t*>(smem + lay.umask);      // [cap]
  uint8_t* comp_slot = smem + lay.comp_slot;                            // [TQ][K]
  int32_t* comp_len = reinterpret_cast<int32_t*>(smem + lay.comp_len);  // [TQ]
  int32_t* misc = reinterpret_cast<int32_t*>(smem + lay.misc);          // [1] steps, [4..] scan
  int32_t* comp_idx = reinterpret_cast<int32_t*>(smem + lay.comp_idx);  // [TQ][K] (prologue)

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int64_t b = blockIdx.z;
  const int h = blockIdx.y;
  const int64_t q0 = (int64_t)blockIdx.x * kTQ;
  const int G = a.G;

  // 1. Routing weights of the tile ([TQ][8][K], head columns >= G zero) and
  //    per-chunk key-valid bits.
  if constexpr (!TOKEN) {
    for (int e = tid; e < kTQ * 8 * K; e += kThreads) {
      const int qq = e / (8 * K), rem = e - qq * 8 * K;
      const int gg = rem / K, kk = rem - gg * K;
      const int64_t qi = q0 + qq;
      wts[e] = (qi < a.Lq && gg < G) ? a.w[((b * a.Lq + qi) * a.Hq + h * G + gg) * K + kk] : 0;
    }
  }
  for (int64_t c = wave; c < Ck; c += kWaves) {
    const bool ok = a.key_valid ? a.key_valid[b * a.Lk + c * 64 + lane] != 0 : true;
    const uint64_t vb = __ballot(ok);
    if (lane == 0) kvbits[c] = vb;
  }
  __syncthreads();

  // 2. Per-query lists (thread per query): keep the entries before the first
  //    negative one that are < Ck, sort them by chunk, fold duplicates into one
  //    entry by summing their weights.  comp_slot maps list rank -> original slot.
  if (tid < kTQ) {
    const int64_t qi = q0 + tid;
    int32_t* ci = comp_idx + tid * K;
    uint8_t* cs = comp_slot + tid * K;
    int n = 0;
    bool sorted = true;
    if (qi < a.Lq) {
      const int32_t* row = a.idx + ((b * a.Lq + qi) * a.Hkv + h) * K;
      for (int kk = 0; kk < K; ++kk) {
        const int32_t c = row[kk];
        if (c < 0) break;
        if (c >= Ck) continue;
        if (n > 0 && c <= ci[n - 1]) sorted = false;
        ci[n] = c;
        cs[n] = (uint8_t)kk;
        ++n;
      }
    }
    if (!sorted) {
      for (int i = 1; i < n; ++i) {  // stable insertion sort by chunk id
        const int32_t c = ci[i];
        const uint8_t sl = cs[i];
        int j = i - 1;
        while (j >= 0 && ci[j] > c) {
          ci[j + 1] = ci[j];
          cs[j + 1] = cs[j];
          --j;
        }
        ci[j + 1] = c;
        cs[j + 1] = sl;
      }
      int m = 0;
      for (int i = 0; i < n; ++i) {
        if (m > 0 && ci[i] == ci[m - 1]) {
          if constexpr (!TOKEN) {
            uint16_t* wq = wts + tid * 8 * K;
            for (int gg = 0; gg < G; ++gg) {
              const float s = bf16_to_f32(wq[gg * K + cs[m - 1]]) + bf16_to_f32(wq[gg * K + cs[i]]);
              wq[gg * K + cs[m - 1]] = (uint16_t)f32_to_bf16(s);
            }
          }
          continue;
        }
        ci[m] = ci[i];
        cs[m] = cs[i];
        ++m;
      }
      n = m;
    }
    comp_len[tid] = n;
  }
  for (int64_t c = tid; c < Ck; c += kThreads) omask[c] = 0ull;
  __syncthreads();
  for (int e = tid; e < kTQ * K; e += kThreads) {
    const int qq = e / K, r = e - qq * K;
    if (r < comp_len[qq]) atomicOr((unsigned long long*)&omask[comp_idx[e]], 1ull << qq);
  }
  __syncthreads();

  // 3. Ascending chunk walk: compaction of the non-empty owner masks.
  {
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
  }
  __syncthreads();
  const int nsteps = misc[1];

  // 4. Q^T operands and accumulators of this wave's queries.
  u32x4_t Qb[kNtile][4];
  f32x4_t acc[kNtile][8];
  int rank[kNtile];
#pragma unroll
  for (int nt = 0; nt < kNtile; ++nt) {
    const int ql = wave * kQPW + 2 * nt + (col >> 3);
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

  // 5. DMA of one chunk into a ring slot: wave w issues instructions for units
  //    (4w + i) * 64 + lane; waves 0-3 fetch K rows, waves 4-7 fetch V^T rows.
  const uint16_t* kbase = a.k + (b * a.Lk) * (int64_t)a.Hkv * 128 + (int64_t)h * 128;
  const uint16_t* vbase =
      TOKEN ? nullptr : a.vt + ((b * a.Hkv + h) * a.NTk) * (int64_t)(128 * 64);
  const int kstride = a.Hkv * 128;
  // Per-lane element offsets of this wave's 4 DMA instructions within a chunk.
  uint32_t dma_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int unit = (4 * wave + i) * 64 + lane;
    if (wave < 4) {
      const int r = unit >> 4, p = (unit & 15) ^ (r & 15);
      dma_off[i] = (uint32_t)(r * kstride + p * 8);
    } else {
      const int u = unit - 1024, d = u >> 3, p = (u & 7) ^ (d & 7);
      dma_off[i] = (uint32_t)(d * 64 + p * 8);
    }
  }
  auto issue = [&](int st) {
    const int64_t c = ulist[st];
    unsigned char* slot = ring + (st % kRing) * kSlotBytes + wave * 4096;
    if (TOKEN && wave >= 4) return;
    const uint16_t* base = wave < 4 ? kbase + c * 64 * (int64_t)kstride : vbase + c * (128 * 64);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds(base + dma_off[i], (lds_void_t*)(slot + i * 1024), 16, 0, 0);
  };
  if (nsteps > 0) issue(0);
  if (nsteps > 1) issue(1);

  const uint64_t last_mask = a.mask_last ? (1ull << 63) : 0ull;
  for (int st = 0; st < nsteps; ++st) {
    ring_barrier(st + 1 < nsteps && !TOKEN);
    if (st + 2 < nsteps) issue(st + 2);
    const uint64_t om = umask[st];
    const uint64_t masked = (~kvbits[ulist[st]]) | last_mask;  // keys excluded from the softmax
    const uint16_t* Kb = reinterpret_cast<const uint16_t*>(ring + (st % kRing) * kSlotBytes);
    const uint16_t* Vb = Kb + 8192;
    const uint32_t wbits = (uint32_t)((om >> (wave * kQPW)) & ((1ull << kQPW) - 1ull));

#pragma unroll
    for (int nt = 0; nt < kNtile; ++nt) {
      const uint32_t pair = (wbits >> (2 * nt)) & 3u;
      if (pair == 0u) continue;
      const int half = col >> 3, gg = col & 7;
      const bool owns = (pair >> half) & 1u;
      const int ql = wave * kQPW + 2 * nt + half;
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
        const int p = 4 * j + grp;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int r = 16 * t + col;
          const u32x4_t Ka = *reinterpret_cast<const u32x4_t*>(Kt + (r * 16 + (p ^ col)) * 8);
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
      } else {
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
          const int d = 16 * td + col;
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) {
            const int p1 = 4 * jj + (grp >> 1), p2 = p1 + 2;
            const int sub = (grp & 1) * 4;
            const u32x2_t v0 =
                *reinterpret_cast<const u32x2_t*>(Vt + (d * 8 + (p1 ^ (d & 7))) * 8 + sub);
            const u32x2_t v1 =
                *reinterpret_cast<const u32x2_t*>(Vt + (d * 8 + (p2 ^ (d & 7))) * 8 + sub);
            u32x4_t Va = {v0[0], v0[1], v1[0], v1[1]};
            acc[nt][td] = mfma_bf16_16x16x32(Va, Pb[jj], acc[nt][td]);
          }
        }
      }
    }
  }

  if constexpr (!TOKEN) {
#pragma unroll
    for (int nt = 0; nt < kNtile; ++nt) {
      const int ql = wave * kQPW + 2 * nt + (col >> 3);
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
}

// Token-score mode fills every (query, slot) row first with -inf so that
// slots without a routed chunk read as fully masked.
__global__ void __launch_bounds__(256) fill_neg_inf(float* p, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += stride)
    p[e] = neg_inf();
}

int launch_selected(SelArgs& a, hipStream_t s) {
  const SelLayout lay = sel_layout(a.K, a.Ck);
  if (lay.total > 160 * 1024) return MRSA_ERR_UNSUPPORTED;
  auto kern = a.token_mode ? selected_attn_kernel<true> : selected_attn_kernel<false>;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lay.total) != hipSuccess)
    return MRSA_ERR_LAUNCH;
  dim3 grid((unsigned)((a.Lq + kTQ - 1) / kTQ), (unsigned)a.Hkv, (unsigned)a.B);
  hipLaunchKernelGGL(kern, grid, dim3(kThreads), lay.total, s, a);
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
