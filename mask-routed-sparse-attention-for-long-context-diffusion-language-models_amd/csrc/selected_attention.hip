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
// Work split.  A workgroup owns a tile of queries (48 with the default split)
// of one KV head; each of
// its waves owns a few query pairs (column tiles of 2 queries x 8 head
// columns), whose output accumulators stay in registers for the whole
// kernel.  The workgroup walks the union of the tile's routed chunks in
// ascending order.  Each chunk's K and V^T (32 KB) arrive in an R-slot LDS
// ring by asynchronous global->LDS DMA; waves synchronise per walk step
// through LDS counters, not workgroup barriers, so they drift apart by up to
// R chunks.  Every wave with a query routed to a chunk consumes it:
//   S^T = K_chunk (64 x 128) . Q^T (2 queries x 8 head columns)   16 MFMAs
//   per-column softmax over the 64 keys, scaled by the routing weight
//   O^T += V_chunk^T (128 x 64) . P^T                            16 MFMAs
// Columns of queries that do not own the chunk get P = 0.
//
// Ring slot layout (16-byte units, XOR-swizzled so that the matrix-operand
// reads of 8 consecutive lanes hit distinct banks):
//   K   row r (64 keys),  part p (8 dims):  unit r*16 + (p ^ (r & 15))
//   V^T row d (128 dims), part p (8 keys):  unit 1024 + d*8 + (p ^ (d & 7))
// V^T parts hold keys in the tiled-V operand order, so part 4*jj + g is
// exactly the 8 reduction keys lane group g feeds to the jj-th PV product.
//
// Token-score mode (candidate_token_scores_gqa,
// ops/hils_token_score_gqa_tilelang.py:17-114) reuses the walk and the S^T
// product and writes, per routed (query, slot), max over the group of q.k
// times sm_scale for every key, -inf at the last slot and invalid keys.
#include "chunk_tile.h"
#include "mrsa_device.h"

#include <type_traits>
#include <utility>

using namespace mrsa;

namespace {

constexpr int kSlotBytes = 32768;       // one chunk: K (16 KB) + V^T (16 KB)
constexpr int kMaxTopk = 64;
constexpr size_t kMaxLds = 160 * 1024;
constexpr int64_t kMaxParts = 64;       // walk split limit
constexpr int kSpinLimit = 1 << 16;     // bound on every wait for a ring slot (~4M clocks)
#ifndef MRSA_SEL_INTERLEAVE
#define MRSA_SEL_INTERLEAVE 1           // query pairs dealt round-robin over the waves
#endif
#ifndef MRSA_SEL_IDLE_HELP
#define MRSA_SEL_IDLE_HELP 2            // steps ahead a wave with no work still helps fetch
#endif
#ifndef MRSA_SEL_DEPTH
#define MRSA_SEL_DEPTH 0                // LDS operand reads in flight (0: by work split)
#endif
#ifndef MRSA_SEL_WAVES
#define MRSA_SEL_WAVES 12               // work split: 12 (12 waves x 2 tiles), 8 (8 x 3), 82 (8 x 2), 16 (16 x 1)
#endif

// Work split: NW waves, each owning NT column tiles of 2 queries x 8 head
// columns; TQ queries per workgroup (at most 64: owner sets are 64-bit masks).
template <int NW, int NT>
struct Split {
  static constexpr int kWaves = NW;
  static constexpr int kThreads = 64 * NW;
  static constexpr int kNtile = NT;
  static constexpr int kQPW = 2 * NT;
  static constexpr int kTQ = NW * 2 * NT;
  static_assert(kTQ <= 64, "work split");
};
using Split8 = Split<8, 3>;
using Split8x2 = Split<8, 2>;
using Split12 = Split<12, 2>;


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
  // Walk split: `parts` workgroups share each (query tile, KV head), each
  // taking an equal share of the walk's steps and writing fp32 partial
  // outputs [parts][B][Lq][Hq][128] to `partial` (parts == 1: bf16 `out`).
  int parts;
  float* partial;
  // Optional token keep mask int8 [B, Lq, Hkv, K, 64] (nonzero = key kept)
  // of the remote-token refinement; read only by the KEEP instantiation.
  const int8_t* keep;
  // Queries per tile actually used (<= the split's capacity): tile x covers
  // queries [x * tq, x * tq + tq).
  int tq;
  // Optional output fusion (both null or both set): out = bf16(bf16(routed)
  // + fuse_w[row] * fuse_local[row]) with local output bf16 [B, Lq, Hq, 128]
  // and local weight bf16 [B, Lq, Hq] -- fuse_hils_outputs folded into the
  // epilogue (or into the part sum).
  const uint16_t* fuse_local;
  const uint16_t* fuse_w;
};

// LDS carve-up (byte offsets, 16-aligned).  The p_* arrays are only used by
// the prologue and live inside the ring, which is free until the first DMA.
struct SelLayout {
  size_t ring, wr, s_chunk, s_own, s_mask, s_cnt, comp_slot, misc, s_rank, s_keep, total;
  size_t p_idx, p_omask, p_len, p_w, p_end;
  int cap;
};
__host__ __device__ inline size_t align16(size_t x) { return (x + 15) & ~(size_t)15; }
// The walk has at most min(Ck, queries x K) steps; a tile holds at most
// min(TQ, Lq) queries.
__host__ __device__ inline SelLayout sel_layout(int TQ, int NW, int K, int64_t Ck, int R,
                                                bool token, int64_t Lq, bool keep = false) {
  SelLayout l;
  const size_t n = (size_t)TQ * K;
  const size_t wbytes = token ? 0 : (size_t)TQ * 8 * K * 2;
  const int64_t steps = (Lq < (int64_t)TQ ? Lq : (int64_t)TQ) * (int64_t)K;
  l.cap = (int)(Ck < steps ? Ck : steps);
  size_t o = 0;
  l.ring = o;      o = align16(o + (size_t)R * kSlotBytes);
  l.wr = o;        o = align16(o + wbytes);                 // [TQ][K][8] bf16, list order
  l.s_chunk = o;   o = align16(o + (size_t)l.cap * 4);
  l.s_own = o;     o = align16(o + (size_t)l.cap * 8);
  l.s_mask = o;    o = align16(o + (size_t)l.cap * 8);
  l.s_cnt = o;     o = align16(o + (size_t)l.cap * 4);
  l.comp_slot = o; o = align16(o + n);
  l.misc = o;      o = align16(o + (size_t)(NW + 8) * 4);
  l.s_rank = o;    o = align16(o + (size_t)TQ * 4);         // [TQ] first list rank
  l.s_keep = o;    o = align16(o + (keep ? n * 8 : 0));       // [TQ][K] kept-key bits
  l.total = o;
  o = l.ring;
  l.p_idx = o;     o = align16(o + n * 4);
  l.p_omask = o;   o = align16(o + (size_t)Ck * 8);
  l.p_len = o;     o = align16(o + (size_t)TQ * 4);
  l.p_w = o;       o = align16(o + wbytes);                 // [TQ][8][K] bf16, slot order
  l.p_end = o;
  return l;
}
__host__ __device__ inline bool sel_layout_fits(const SelLayout& l, int R) {
  return l.total <= kMaxLds && l.p_end <= l.ring + (size_t)R * kSlotBytes;
}

// Walk counters in LDS, accessed with asm so the compiler does not order
// them behind the in-flight global->LDS DMA (it waits for vmcnt(0) before
// any LDS atomic that may alias a DMA destination).
__device__ __forceinline__ int lds_load_flag(uint32_t addr) {
  int v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
  return v;
}
__device__ __forceinline__ void lds_store_flag(uint32_t addr, int v) {
  asm volatile("ds_write_b32 %0, %1" ::"v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ int lds_fetch_add(uint32_t addr, int v) {
  int old;
  asm volatile("ds_add_rtn_u32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
               : "=v"(old)
               : "v"(addr), "v"(v)
               : "memory");
  return old;
}
__device__ __forceinline__ void lds_add(uint32_t addr, int v) {
  asm volatile("ds_add_u32 %0, %1" ::"v"(addr), "v"(v) : "memory");
}

// One LDS round trip per walk step (lane 0 only): count the wave done with
// a step (returns the previous count) and read the owner bits, excluded-key
// bits and ring-slot tag of the next step.
__device__ __forceinline__ void step_exchange(uint32_t done_addr, uint32_t own_addr,
                                              uint32_t mask_addr, uint32_t tag_addr,
                                              uint32_t cur_addr, int& old, uint64_t& own,
                                              uint64_t& mask, int& tag, int& cur) {
  const int one = 1;
  asm volatile(
      "ds_add_rtn_u32 %0, %5, %10\n\t"
      "ds_read_b64 %1, %6\n\t"
      "ds_read_b64 %2, %7\n\t"
      "ds_read_b32 %3, %8\n\t"
      "ds_read_b32 %4, %9\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(old), "=&v"(own), "=&v"(mask), "=&v"(tag), "=&v"(cur)
      : "v"(done_addr), "v"(own_addr), "v"(mask_addr), "v"(tag_addr), "v"(cur_addr), "v"(one)
      : "memory");
}
__device__ __forceinline__ void step_read(uint32_t own_addr, uint32_t mask_addr,
                                          uint32_t tag_addr, uint64_t& own, uint64_t& mask,
                                          int& tag) {
  asm volatile(
      "ds_read_b64 %0, %3\n\t"
      "ds_read_b64 %1, %4\n\t"
      "ds_read_b32 %2, %5\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(own), "=&v"(mask), "=&v"(tag)
      : "v"(own_addr), "v"(mask_addr), "v"(tag_addr)
      : "memory");
}


// LDS arrays the prologue fills (s_*, wr, comp_slot, misc) or uses as
// scratch (p_*).
struct WalkLds {
  uint16_t* wr;         // [TQ][K][8] bf16 weights in list order (attention mode)
  uint16_t* wts;        // [TQ][8][K] bf16 staged weights (scratch)
  int32_t* s_chunk;     // [cap] chunk of each walk step
  uint64_t* s_own;      // [cap] owner bits (query i of the tile -> bit i)
  uint64_t* s_mask;     // [cap] excluded-key bits (invalid keys, landmark slot)
  uint8_t* comp_slot;   // [TQ][K] list position -> original slot
  int32_t* misc;        // [waves] scan, [waves] step count, first chunk
  int32_t* s_rank;      // [TQ] list rank of each query at the first step
  uint64_t* s_keep;     // [TQ][K] kept-key bits in list order (keep mode)
  int32_t* p_idx;       // [TQ][K] staged / compacted index rows (scratch)
  uint64_t* p_omask;    // [Ck] owner bits by chunk (scratch)
  int32_t* p_len;       // [TQ] list lengths (scratch)
};

// Excluded-key bits of one 64-key chunk from its 64 key-valid bytes (bit j
// set: key j invalid).
__device__ __forceinline__ uint64_t invalid_key_bits(const uint8_t* kv, bool al16) {
  uint64_t m = 0;
  if (al16) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const u32x4_t x = *reinterpret_cast<const u32x4_t*>(kv + 16 * v);
#pragma unroll
      for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          m |= ((x[w] >> (8 * j)) & 0xffu) ? 0ull : 1ull << (16 * v + 4 * w + j);
    }
  } else {
    for (int j = 0; j < 64; ++j) m |= kv[j] ? 0ull : 1ull << j;
  }
  return m;
}

// Prologue shared by both routed-attention kernels: stages the tile's index
// rows and weights, compacts each query's list the way the reference kernel
// reads it (stop at the first negative entry, skip >= Ck, sort, merge
// duplicates by summing weights), builds the ascending walk over the union of
// the tile's chunks with their excluded keys, and (attention mode) the
// weights in list order.  With the walk split over a.parts workgroups, part
// `part` keeps steps [total * part / parts, total * (part + 1) / parts) and
// each query's list rank at its first kept step (W.s_rank).  Returns the
// number of kept steps.  Ends with a workgroup barrier.
template <bool TOKEN, class SP, bool KEEP = false>
__device__ int build_walk(const SelArgs& a, const WalkLds& W, int64_t b, int h, int64_t q0,
                          int64_t nq, int part) {
  constexpr int kWaves = SP::kWaves, kThreads = SP::kThreads, kTQ = SP::kTQ;
  const int K = a.K;
  const int64_t Ck = a.Ck;
  const int G = a.G;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  uint16_t* wr = W.wr;
  uint16_t* wts = W.wts;
  int32_t* s_chunk = W.s_chunk;
  uint64_t* s_own = W.s_own;
  uint64_t* s_mask = W.s_mask;
  uint8_t* comp_slot = W.comp_slot;
  int32_t* misc = W.misc;
  int32_t* p_idx = W.p_idx;
  uint64_t* p_omask = W.p_omask;
  int32_t* p_len = W.p_len;

  // 1. Stage the tile's index rows (-1 past the end of the sequence) and
  //    routing weights ([TQ][8][K], head columns >= G zero).
  for (int e = tid; e < kTQ * K; e += kThreads) {
    const int qq = e / K, kk = e - qq * K;
    p_idx[e] = qq < nq ? a.idx[((b * a.Lq + q0 + qq) * a.Hkv + h) * K + kk] : -1;
  }
  if constexpr (!TOKEN) {
    const uint16_t* wrow0 = a.w + ((b * a.Lq + q0) * a.Hq + (int64_t)h * G) * K;
    const int64_t qstride = (int64_t)a.Hq * K;
    if ((K & 7) == 0 && ((uintptr_t)a.w & 15) == 0) {
      const int vpr = K >> 3;  // 16-byte vectors per (query, head) row
      for (int e = tid; e < kTQ * 8 * vpr; e += kThreads) {
        const int row = e / vpr, v = e - row * vpr;
        const int qq = row >> 3, gg = row & 7;
        u32x4_t x = {0u, 0u, 0u, 0u};
        if (qq < nq && gg < G)
          x = *reinterpret_cast<const u32x4_t*>(wrow0 + qq * qstride + gg * K + 8 * v);
        *reinterpret_cast<u32x4_t*>(wts + row * K + 8 * v) = x;
      }
    } else {
      for (int e = tid; e < kTQ * 8 * K; e += kThreads) {
        const int row = e / K, kk = e - row * K;
        const int qq = row >> 3, gg = row & 7;
        wts[e] = (qq < nq && gg < G) ? wrow0[qq * qstride + gg * K + kk] : (uint16_t)0;
      }
    }
  }
  for (int64_t c = tid; c < Ck; c += kThreads) p_omask[c] = 0ull;
  __syncthreads();

  // 2. Per-query lists (thread per query): keep the entries before the first
  //    negative one that are < Ck, sort them by chunk, fold duplicates into one
  //    entry by summing their weights.  comp_slot maps list rank -> original
  //    slot; the compacted chunk ids overwrite the staged index row.
  if (tid < kTQ) {
    int32_t* ci = p_idx + tid * K;
    uint8_t* cs = comp_slot + tid * K;
    int n = 0;
    bool sorted = true;
    for (int kk = 0; kk < K; ++kk) {
      const int32_t c = ci[kk];
      if (c < 0) break;
      if (c >= Ck) continue;
      if (n > 0 && c <= ci[n - 1]) sorted = false;
      ci[n] = c;
      cs[n] = (uint8_t)kk;
      ++n;
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
    p_len[tid] = n;
  }
  __syncthreads();
  for (int e = tid; e < kTQ * K; e += kThreads) {
    const int qq = e / K, r = e - qq * K;
    if (r < p_len[qq]) atomicOr((unsigned long long*)&p_omask[p_idx[e]], 1ull << qq);
  }
  if constexpr (!TOKEN) {
    // Weights in list order: wr[q][r][g] = weight of the r-th listed chunk.
    for (int e = tid; e < kTQ * K * 8; e += kThreads) {
      const int qq = e / (K * 8), rem = e - qq * K * 8;
      const int r = rem >> 3, gg = rem & 7;
      wr[e] = r < p_len[qq] ? wts[(qq * 8 + gg) * K + comp_slot[qq * K + r]] : (uint16_t)0;
    }
  }
  if constexpr (KEEP) {
    // Kept-key bits of each listed (query, chunk), bit j = key j, from the
    // keep row of the chunk's original slot (a merged duplicate uses its
    // first slot's row).
    for (int e = tid; e < kTQ * K; e += kThreads) {
      const int qq = e / K, r = e - qq * K;
      uint64_t bits = 0ull;
      if (r < p_len[qq]) {
        const int8_t* kr =
            a.keep + (((b * a.Lq + q0 + qq) * a.Hkv + h) * K + comp_slot[qq * K + r]) * 64;
        if (((uintptr_t)a.keep & 15) == 0) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const u32x4_t x = *reinterpret_cast<const u32x4_t*>(kr + 16 * v);
#pragma unroll
            for (int w = 0; w < 4; ++w)
#pragma unroll
              for (int j = 0; j < 4; ++j)
                bits |= ((x[w] >> (8 * j)) & 0xffu) ? 1ull << (16 * v + 4 * w + j) : 0ull;
          }
        } else {
          for (int j = 0; j < 64; ++j) bits |= kr[j] ? 1ull << j : 0ull;
        }
      }
      W.s_keep[e] = bits;
    }
  }
  __syncthreads();

  // 3. Walk list: the chunks with at least one owner, ascending, with their
  //    owner bits and excluded-key bits (invalid keys, the landmark slot);
  //    this part's share of it.
  {
    const uint64_t last_mask = a.mask_last ? (1ull << 63) : 0ull;
    const int64_t per = (Ck + kThreads - 1) / kThreads;
    const int64_t c0 = min(Ck, tid * per), c1 = min(Ck, c0 + per);
    int cnt = 0;
    for (int64_t c = c0; c < c1; ++c) cnt += p_omask[c] != 0ull;
    int incl = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int up = __shfl_up(incl, o, 64);
      if (lane >= o) incl += up;
    }
    if (lane == 63) misc[wave] = incl;
    __syncthreads();
    int pos = incl - cnt, total = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const int x = misc[w];
      pos += w < wave ? x : 0;
      total += x;
    }
    const int st_lo = (int)((int64_t)part * total / a.parts);
    const int st_hi = (int)((int64_t)(part + 1) * total / a.parts);
    const uint8_t* kv = a.key_valid ? a.key_valid + b * a.Lk : nullptr;
    const bool al16 = ((uintptr_t)kv & 15) == 0;
    for (int64_t c = c0; c < c1; ++c) {
      const uint64_t m = p_omask[c];
      if (m) {
        if (pos >= st_lo && pos < st_hi) {
          const uint64_t bad = kv ? invalid_key_bits(kv + 64 * c, al16) : 0ull;
          s_chunk[pos - st_lo] = (int32_t)c;
          s_own[pos - st_lo] = m;
          s_mask[pos - st_lo] = bad | last_mask;
          if (pos == st_lo) misc[kWaves + 1] = (int32_t)c;
        }
        ++pos;
      }
    }
    if (tid == 0) misc[kWaves] = st_hi - st_lo;
  }
  __syncthreads();
  if (a.parts > 1) {
    // Rank of the first kept step in each query's list: its listed chunks
    // below that step's chunk (lists are ascending and duplicate-free).
    const int nkept = misc[kWaves];
    const int32_t c_lo = nkept > 0 ? misc[kWaves + 1] : (int32_t)Ck;
    if (tid < kTQ) {
      const int32_t* ci = p_idx + tid * K;
      const int n = p_len[tid];
      int r = 0;
      for (int i = 0; i < n; ++i) r += ci[i] < c_lo ? 1 : 0;
      W.s_rank[tid] = r;
    }
    __syncthreads();
  }
  return misc[kWaves];
}

template <bool TOKEN, int R, class SP, bool KEEP>
__global__ void __launch_bounds__(SP::kThreads) selected_attn_kernel(SelArgs a) {
  constexpr int kWaves = SP::kWaves, kThreads = SP::kThreads, kNtile = SP::kNtile;
  constexpr int kTQ = SP::kTQ;
  // LDS operand reads in flight: 8 when registers allow, 4 for 12 waves.
  constexpr int kDepth = MRSA_SEL_DEPTH > 0 ? MRSA_SEL_DEPTH : (kWaves > 8 ? 4 : 8);
  static_assert(R >= 2, "ring depth");
  extern __shared__ __align__(16) unsigned char smem[];
  const int K = a.K;
  const int64_t Ck = a.Ck;
  const SelLayout lay = sel_layout(kTQ, kWaves, K, Ck, R, TOKEN, a.Lq, KEEP);
  unsigned char* ring = smem + lay.ring;
  uint16_t* wr = reinterpret_cast<uint16_t*>(smem + lay.wr);            // [TQ][K][8]
  uint16_t* wts = reinterpret_cast<uint16_t*>(smem + lay.p_w);          // [TQ][8][K]
  int32_t* s_chunk = reinterpret_cast<int32_t*>(smem + lay.s_chunk);    // [cap] walk order
  uint64_t* s_own = reinterpret_cast<uint64_t*>(smem + lay.s_own);      // [cap] owner bits
  uint64_t* s_mask = reinterpret_cast<uint64_t*>(smem + lay.s_mask);    // [cap] masked keys
  uint8_t* comp_slot = smem + lay.comp_slot;                            // [TQ][K]
  int32_t* misc = reinterpret_cast<int32_t*>(smem + lay.misc);          // [kWaves] scan, [kWaves] n
  // Walk counters per step: waves done with it, DMA portions of its chunk
  // claimed and landed.
  // One word per step: waves done with it (bits 0-7), DMA portions of its
  // chunk claimed (bits 8-15) and landed (bits 16-23).  No field overflows:
  // at most 16 waves, and claims stop at kPortions plus one late claim per
  // wave.
  int32_t* s_cnt = reinterpret_cast<int32_t*>(smem + lay.s_cnt);         // [cap]
  int32_t* cursor = misc + kWaves + 4;  // oldest chunk with unclaimed portions
  int32_t* s_rank = reinterpret_cast<int32_t*>(smem + lay.s_rank);      // [TQ]
  uint64_t* s_keep = reinterpret_cast<uint64_t*>(smem + lay.s_keep);    // [TQ][K]
  int32_t* p_idx = reinterpret_cast<int32_t*>(smem + lay.p_idx);        // [TQ][K]
  uint64_t* p_omask = reinterpret_cast<uint64_t*>(smem + lay.p_omask);  // [Ck]
  int32_t* p_len = reinterpret_cast<int32_t*>(smem + lay.p_len);        // [TQ]

  const int tid = threadIdx.x;
  // The wave index is uniform: kept in a scalar register so that per-wave
  // decisions (tile ownership, DMA duty) are scalar branches.
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int64_t b = blockIdx.z % a.B;
  const int part = (int)(blockIdx.z / a.B);
  const int h = blockIdx.y;
  const int64_t q0 = (int64_t)blockIdx.x * a.tq;
  const int G = a.G;
  const int64_t nq = min((int64_t)a.tq, a.Lq - q0);  // queries of this tile that exist

  // Zeroed counters, published by the prologue's barriers.
  if (tid == 0) *cursor = 0;
  for (int i = tid; i < lay.cap; i += kThreads) s_cnt[i] = 0;
  const int nsteps = build_walk<TOKEN, SP, KEEP>(
      a,
      WalkLds{wr, wts, s_chunk, s_own, s_mask, comp_slot, misc, s_rank, s_keep, p_idx, p_omask,
              p_len},
      b, h, q0, nq, part);

  // 4. Q^T operands and accumulators of this wave's queries.
  //    Column tile nt of wave w holds query pair qpair(w, nt), i.e. queries
  //    2 qpair and 2 qpair + 1 of the tile.  Neighbouring queries tend to route
  //    to the same chunks, so dealing pairs round-robin over the waves spreads
  //    each chunk's work over more waves than consecutive blocks would.
  auto qpair = [&](int nt) { return MRSA_SEL_INTERLEAVE ? nt * kWaves + wave : wave * kNtile + nt; };
  u32x4_t Qb[kNtile][4];
  f32x4_t acc[kNtile][8];
  int rank[kNtile];
#pragma unroll
  for (int nt = 0; nt < kNtile; ++nt) {
    const int ql = 2 * qpair(nt) + (col >> 3);
    const int gg = col & 7;
    rank[nt] = a.parts > 1 ? s_rank[ql] : 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4_t z = {0u, 0u, 0u, 0u};
      Qb[nt][j] = z;
      if (ql < nq && gg < G)
        Qb[nt][j] = *reinterpret_cast<const u32x4_t*>(
            a.q + ((b * a.Lq + q0 + ql) * a.Hq + h * G + gg) * 128 + 32 * j + 8 * grp);
    }
#pragma unroll
    for (int td = 0; td < 8; ++td) acc[nt][td] = zero4();
  }

  // 5. Chunk sources: K rows of this KV head, V^T tiles.
  const uint16_t* kbase = a.k + (b * a.Lk) * (int64_t)a.Hkv * 128 + (int64_t)h * 128;
  const uint16_t* vbase =
      TOKEN ? nullptr : a.vt + ((b * a.Hkv + h) * a.NTk) * (int64_t)(128 * 64);
  const int kstride = a.Hkv * 128;

  // Per-lane element offsets of the matrix-operand reads inside a slot:
  // K row 16t + col, part (4j + grp) ^ col  -> kofs0 ^ 32j + 2048t;
  // V^T row 16td + col, part (4jj + grp) ^ (col & 7) -> vofs0 ^ 32jj + 1024td.
  const uint32_t kofs0 = (uint32_t)(col * 128 + ((grp ^ col) * 8));
  const uint32_t vofs0 = (uint32_t)(8192 + col * 64 + ((grp ^ (col & 7)) * 8));
  auto kofs = [&](int j) { return kofs0 ^ (uint32_t)(32 * j); };
  auto vofs = [&](int jj) { return vofs0 ^ (uint32_t)(32 * jj); };

  const float c2 = a.scale_log2;
  const int half = col >> 3, gg = col & 7;
  float ninf_v = neg_inf();
  asm volatile("" : "+v"(ninf_v));  // kept in a register for set_where

  auto consume = [&](int st, uint64_t om, uint64_t msk) {
    const uint16_t* Kb = reinterpret_cast<const uint16_t*>(ring + (st % R) * kSlotBytes);
    // This lane's excluded-key bits: bit 16t + i of msh is key 16t + 4grp + i.
    const uint64_t msh = msk >> (4 * grp);

#pragma unroll
    for (int nt = 0; nt < kNtile; ++nt) {
      const uint32_t pair = (uint32_t)(om >> (2 * qpair(nt))) & 3u;
      if (pair == 0u) continue;
      const bool owns = (pair >> half) & 1u;
      const int ql = 2 * qpair(nt) + half;
      // List position of this chunk for the owning column; reads are made
      // unconditional (clamped index) so they do not split the block.
      const int pos = min(rank[nt], K - 1);
      rank[nt] += owns ? 1 : 0;
      int slot = 0;
      if constexpr (TOKEN) slot = comp_slot[ql * K + pos];
      // Routing weight of the lane's column, read with the K operands (LDS
      // reads complete in order, so it has landed once the S^T product has).
      uint32_t wbits = 0u;
      if constexpr (!TOKEN)
        asm volatile("ds_read_u16 %0, %1" : "=v"(wbits) : "v"(lds_addr(&wr[(ql * K + pos) * 8 + gg])));
      // Kept-key bits of the column's (query, chunk), read the same way.
      uint64_t kbits = ~0ull;
      if constexpr (KEEP)
        asm volatile("ds_read_b64 %0, %1" : "=v"(kbits) : "v"(lds_addr(&s_keep[ql * K + pos])));
      // Opaque zero: keeps the compiler from hoisting this tile's K / V operand
      // reads out of the tile loop (that would pin 128 extra registers).
      int zoff = 0;
      asm volatile("" : "+v"(zoff));
      const uint16_t* Kt = Kb + zoff;

      const uint32_t kaddr[4] = {lds_addr(Kt + kofs(0)), lds_addr(Kt + kofs(1)),
                                 lds_addr(Kt + kofs(2)), lds_addr(Kt + kofs(3))};
      f32x4_t S[4];
      qk_tile<kDepth>(kaddr, Qb[nt], S);
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(wbits));  // already satisfied
      if constexpr (KEEP) asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(kbits));
      const float wv = owns ? bf16_to_f32(wbits) : 0.f;
      // The first V^T operands do not depend on P: read them now so they land
      // during the softmax.  PV operand o = 8 * jj + td.
      const uint32_t vaddr[2] = {lds_addr(Kt + vofs(0)), lds_addr(Kt + vofs(1))};
      u32x4_t vb[16];
      if constexpr (!TOKEN) {
        static_for<4>([&](auto oc) {
          constexpr int o = decltype(oc)::value;
          vb[o] = lds_read_b128<(o & 7) * 2048>(vaddr[o >> 3]);
        });
      }

      if constexpr (TOKEN) {
        // max over the query's G head columns (lanes sharing col >> 3).
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) S[t][i] = group8_max_f(gg < G ? S[t][i] : neg_inf());
        if (owns && gg == 0) {
          const int64_t qi = q0 + ql;
          float* dst = a.tscores + (((b * a.Lq + qi) * a.Hkv + h) * K + slot) * 64;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            f32x4_t o;
#pragma unroll
            for (int i = 0; i < 4; ++i)
              o[i] = ((msh >> (16 * t + i)) & 1ull) ? neg_inf() : S[t][i] * a.sm_scale;
            *reinterpret_cast<f32x4_t*>(dst + 16 * t + 4 * grp) = o;
          }
        }
      } else {
        u32x4_t Pb[2];
        // Excluded keys -> -inf, in place.  Key 63 (the landmark slot, the
        // usual only exclusion) is S[3][3] of lane group 3 (lanes 48-63);
        // any other excluded key takes the rare per-bit path.
        S[3][3] = set_where(S[3][3], (msk >> 63) ? 0xFFFF000000000000ull : 0ull, ninf_v);
        if (msk & ~(1ull << 63)) {
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              S[t][i] = set_where(
                  S[t][i], __builtin_amdgcn_ballot_w64((msh >> (16 * t + i)) & 1ull), ninf_v);
        }
        if constexpr (KEEP) {
          // Keys the column's keep row drops -> -inf (bit 16t + i of kb is
          // key 16t + 4grp + i, as for msh).
          const uint64_t kb = kbits >> (4 * grp);
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              S[t][i] = set_where(
                  S[t][i], __builtin_amdgcn_ballot_w64(!((kb >> (16 * t + i)) & 1ull)), ninf_v);
        }
        const float mx = across4_max(max16_raw(S));
        const float mb = mx == neg_inf() ? 0.f : mx * c2;
        float part[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
          for (int i = 0; i < 4; ++i) S[t][i] = exp2_hw(__builtin_fmaf(S[t][i], c2, -mb));
          part[t] = (S[t][0] + S[t][1]) + (S[t][2] + S[t][3]);
        }
        const float sum = across4_sum((part[0] + part[1]) + (part[2] + part[3]));
        const float f = sum > 0.f ? wv * rcp_hw(sum) : 0.f;
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          Pb[jj][0] = pack_bf16x2(S[2 * jj][0] * f, S[2 * jj][1] * f);
          Pb[jj][1] = pack_bf16x2(S[2 * jj][2] * f, S[2 * jj][3] * f);
          Pb[jj][2] = pack_bf16x2(S[2 * jj + 1][0] * f, S[2 * jj + 1][1] * f);
          Pb[jj][3] = pack_bf16x2(S[2 * jj + 1][2] * f, S[2 * jj + 1][3] * f);
        }
        // O^T += V^T . P^T with eight reads in flight; consecutive products go
        // to different accumulators.
        static_for<kDepth - 4>([&](auto oc) {
          constexpr int o = decltype(oc)::value + 4;
          vb[o] = lds_read_b128<(o & 7) * 2048>(vaddr[o >> 3]);
        });
        static_for<16>([&](auto oc) {
          constexpr int o = decltype(oc)::value;
          lds_wait<(15 - o < kDepth - 1 ? 15 - o : kDepth - 1)>(vb[o]);
          acc[nt][o & 7] = mfma_bf16_16x16x32(vb[o], Pb[o >> 3], acc[nt][o & 7]);
          if constexpr (o + kDepth < 16)
            vb[o + kDepth] = lds_read_b128<((o + kDepth) & 7) * 2048>(vaddr[(o + kDepth) >> 3]);
          __builtin_amdgcn_sched_barrier(0);
        });
      }
    }
  };

  // 6. The walk, synchronised through per-step LDS counters instead of
  //    workgroup barriers, so that waves drift apart by up to R chunks and
  //    the imbalance of their work evens out over that window.
  //    * Chunk n lives in ring slot n % R; it may be fetched once every wave
  //      has counted itself done with step n - R (s_cnt bits 0-7).
  //    * Its DMA is split into kPortions portions of 4 KB.  Waves that would
  //      otherwise idle (waiting for a chunk to land, or with no query routed
  //      to the current step) claim the oldest fetchable portions (bits 8-15,
  //      chunk order kept by `cursor`), issue them, wait for their own DMA
  //      (vmcnt) and count them landed (bits 16-23).  The slowest wave, which
  //      frees each slot, thus rarely spends time issuing fetches.
  //    * A wave consumes chunk st once all its portions have landed; a wave
  //      with no query routed to it neither waits for it nor reads it.
  //    Liveness: the first wave to reach step n helps until chunk n is
  //    claimed, and chunk n becomes fetchable once every wave finished step
  //    n - R, which depends only on earlier chunks.  The spin bound keeps
  //    every wave finite regardless.
  constexpr int kPortions = TOKEN ? 4 : 8;
  const uint32_t kc = (uint32_t)((col ^ grp) * 8);
  const uint32_t v0 = (uint32_t)((lane >> 3) * 64 + ((lane ^ (lane >> 3)) & 7) * 8);
  // Portion p < 4: K DMA instructions j = 4p + i (units 64j + lane: row
  // 4j + grp, part (col ^ grp) ^ 4i); portion 4 + p: V^T instructions
  // j = 4p + i (units 1024 + 64j + lane: row 8j + lane / 8, part
  // (lane ^ (lane / 8)) & 7).
  auto issue_portion = [&](int n, int p) {
    const int64_t c = __builtin_amdgcn_readfirstlane(s_chunk[n]);
    unsigned char* slot = ring + (n % R) * kSlotBytes;
    if (TOKEN || p < 4) {
      const uint16_t* kc0 = kbase + c * 64 * (int64_t)kstride + grp * kstride;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = 4 * p + i;
        __builtin_amdgcn_global_load_lds(kc0 + (4 * j) * kstride + (kc ^ (uint32_t)(32 * i)),
                                         (lds_void_t*)(slot + j * 1024), 16, 0, 0);
      }
    } else {
      const uint16_t* vc0 = vbase + c * (128 * 64) + v0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = 4 * (p - 4) + i;
        __builtin_amdgcn_global_load_lds(vc0 + 512 * j, (lds_void_t*)(slot + (16 + j) * 1024),
                                         16, 0, 0);
      }
    }
  };
  // Claims and fetches fetchable portions of chunks below `limit`, oldest
  // first, until none is left.
  auto help = [&](int limit) {
    limit = min(limit, nsteps);
    for (int guard = 0; guard < R * kPortions + 2; ++guard) {
      const int n = __builtin_amdgcn_readfirstlane(lds_load_flag(lds_addr(cursor)));
      if (n >= limit) return;
      if (n >= R &&
          (__builtin_amdgcn_readfirstlane(lds_load_flag(lds_addr(&s_cnt[n - R]))) & 0xff) < kWaves)
        return;
      int k = 0;
      if (lane == 0) k = lds_fetch_add(lds_addr(&s_cnt[n]), 1 << 8);
      k = (__builtin_amdgcn_readfirstlane(k) >> 8) & 0xff;
      if (k >= kPortions) continue;  // chunk taken meanwhile; the cursor moves on
      if (k == kPortions - 1 && lane == 0) lds_store_flag(lds_addr(cursor), n + 1);
      issue_portion(n, k);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      if (lane == 0) lds_add(lds_addr(&s_cnt[n]), 1 << 16);
    }
  };
  // Queries of this wave as owner bits.
  uint64_t my_bits = 0;
#pragma unroll
  for (int nt = 0; nt < kNtile; ++nt) my_bits |= 3ull << (2 * qpair(nt));

  // Words of the current step: owner bits, excluded-key bits, landed portions.
  uint64_t om = 0, msk = 0;
  int land = 0, old = 0, cur = 0;
  if (nsteps > 0 && lane == 0)
    step_read(lds_addr(&s_own[0]), lds_addr(&s_mask[0]), lds_addr(&s_cnt[0]), om, msk, land);
  for (int st = 0; st < nsteps; ++st) {
    om = uniform_u64(om);
    msk = uniform_u64(msk);
    const bool mine = (om & my_bits) != 0;
    // A wave with no work here helps only when the oldest unclaimed chunk
    // (cursor, read with the step words) is needed within a few steps.
    const bool helpful = __builtin_amdgcn_readfirstlane(cur) < st + MRSA_SEL_IDLE_HELP;
    if (mine ? ((__builtin_amdgcn_readfirstlane(land) >> 16) & 0xff) < kPortions : helpful) {
      // Idle: fetch what can be fetched; with work at this step, also wait
      // until its chunk has landed.
      for (int spins = 0; spins < kSpinLimit; ++spins) {
        help(st + R);
        if (!mine ||
            ((__builtin_amdgcn_readfirstlane(lds_load_flag(lds_addr(&s_cnt[st]))) >> 16) & 0xff) >=
                kPortions)
          break;
        __builtin_amdgcn_s_sleep(1);
      }
      asm volatile("" ::: "memory");
    }
    if (mine) consume(st, om, msk);
    // Count this wave done with step st (its reads of the slot have
    // completed: LDS instructions of a wave execute in order) and read the
    // next step's words in the same round trip.  The count is per step: a
    // wave with no work runs ahead and may count itself done with chunk
    // st + R before a slower wave is done with st.  A landed count read
    // here stays valid: the slot is not refetched before this wave is done
    // with the step.
    asm volatile("" ::: "memory");
    const int nx = min(st + 1, nsteps - 1);
    if (lane == 0)
      step_exchange(lds_addr(&s_cnt[st]), lds_addr(&s_own[nx]), lds_addr(&s_mask[nx]),
                    lds_addr(&s_cnt[nx]), lds_addr(cursor), old, om, msk, land, cur);
  }

  if constexpr (!TOKEN) {
#pragma unroll
    for (int nt = 0; nt < kNtile; ++nt) {
      const int ql = 2 * qpair(nt) + half;
      if (ql >= nq || gg >= G) continue;
      const int64_t row = (b * a.Lq + q0 + ql) * a.Hq + h * G + gg;
      if (a.parts > 1) {
        float* prow = a.partial + ((int64_t)part * a.B * a.Lq * a.Hq + row) * 128;
#pragma unroll
        for (int td = 0; td < 8; ++td)
          *reinterpret_cast<f32x4_t*>(prow + 16 * td + 4 * grp) = acc[nt][td];
        continue;
      }
      uint16_t* orow = a.out + row * 128;
      if (a.fuse_local) {
        const float wl = bf16_to_f32(a.fuse_w[row]);
        const uint16_t* lrow = a.fuse_local + row * 128;
        u32x2_t l[8];
#pragma unroll
        for (int td = 0; td < 8; ++td) l[td] = *reinterpret_cast<const u32x2_t*>(lrow + 16 * td + 4 * grp);
#pragma unroll
        for (int td = 0; td < 8; ++td) {
          u32x2_t o;
          o[0] = fuse_bf16x2(pack_bf16x2(acc[nt][td][0], acc[nt][td][1]), l[td][0], wl);
          o[1] = fuse_bf16x2(pack_bf16x2(acc[nt][td][2], acc[nt][td][3]), l[td][1], wl);
          *reinterpret_cast<u32x2_t*>(orow + 16 * td + 4 * grp) = o;
        }
        continue;
      }
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

// Sum of the walk parts' fp32 partial outputs, rounded to bf16 once (and
// fused with the local branch when fuse_local is set: 32 groups of 4 per
// 128-wide row).
__global__ void __launch_bounds__(256) sum_parts_kernel(const float* __restrict__ partial,
                                                        int parts, int64_t n4,
                                                        uint16_t* __restrict__ out,
                                                        const uint16_t* __restrict__ fuse_local,
                                                        const uint16_t* __restrict__ fuse_w) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n4; e += stride) {
    f32x4_t s = reinterpret_cast<const f32x4_t*>(partial)[e];
    for (int p = 1; p < parts; ++p) {
      const f32x4_t x = reinterpret_cast<const f32x4_t*>(partial)[(int64_t)p * n4 + e];
#pragma unroll
      for (int i = 0; i < 4; ++i) s[i] += x[i];
    }
    u32x2_t o;
    o[0] = pack_bf16x2(s[0], s[1]);
    o[1] = pack_bf16x2(s[2], s[3]);
    if (fuse_local) {
      const float wl = bf16_to_f32(fuse_w[e >> 5]);
      const u32x2_t l = reinterpret_cast<const u32x2_t*>(fuse_local)[e];
      o[0] = fuse_bf16x2(o[0], l[0], wl);
      o[1] = fuse_bf16x2(o[1], l[1], wl);
    }
    reinterpret_cast<u32x2_t*>(out)[e] = o;
  }
}

// Token-score mode fills every (query, slot) row first with -inf so that
// slots without a routed chunk read as fully masked.
__global__ void __launch_bounds__(256) fill_neg_inf(float* p, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += stride)
    p[e] = neg_inf();
}

template <bool TOKEN, int R, class SP, bool KEEP>
int launch_variant(SelArgs& a, const SelLayout& lay, hipStream_t s) {
  auto kern = selected_attn_kernel<TOKEN, R, SP, KEEP>;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lay.total) != hipSuccess)
    return MRSA_ERR_LAUNCH;
  dim3 grid((unsigned)((a.Lq + a.tq - 1) / a.tq), (unsigned)a.Hkv, (unsigned)(a.B * a.parts));
  hipLaunchKernelGGL(kern, grid, dim3(SP::kThreads), lay.total, s, a);
  return mrsa_launch_status();
}

// Compute units of the current device (cached per device).
int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
      cus[dev] = n;
  }
  return cus[dev];
}

// Queries per tile.  One workgroup fills a CU (its LDS ring), so workgroups
// run in rounds of `cus`.  Tiles of `cap` queries would leave the last round
// partly empty (configuration 2: 1368 workgroups = 5.3 rounds of 256); the
// smallest tile that needs no more rounds spreads the same work evenly over
// them, which shortens every workgroup instead.
int64_t tile_queries(int64_t Lq, int64_t groups, int cap, int cus) {
  if (cus <= 0 || Lq <= cap || groups <= 0) return cap;
  const int64_t tiles = (Lq + cap - 1) / cap;
  const int64_t rounds = (tiles * groups + cus - 1) / cus;
  const int64_t tiles_max = rounds * cus / groups;
  if (tiles_max <= tiles) return cap;
  const int64_t tq = (Lq + tiles_max - 1) / tiles_max;
  return tq < 1 ? 1 : (tq > cap ? cap : tq);
}

// Deepest ring that fits in LDS: 4 slots, else 3.
template <bool TOKEN, bool KEEP = false>
int launch_selected(SelArgs& a, hipStream_t s) {
  using SP = std::conditional_t<
      MRSA_SEL_WAVES == 16, Split<16, 1>,
      std::conditional_t<MRSA_SEL_WAVES == 12, Split12,
                         std::conditional_t<MRSA_SEL_WAVES == 82, Split8x2, Split8>>>;
  a.tq = (int)tile_queries(a.Lq, a.B * a.Hkv * a.parts, SP::kTQ, device_cus());
  const SelLayout l4 = sel_layout(SP::kTQ, SP::kWaves, a.K, a.Ck, 4, TOKEN, a.Lq, KEEP);
  if (sel_layout_fits(l4, 4)) return launch_variant<TOKEN, 4, SP, KEEP>(a, l4, s);
  const SelLayout l3 = sel_layout(SP::kTQ, SP::kWaves, a.K, a.Ck, 3, TOKEN, a.Lq, KEEP);
  if (sel_layout_fits(l3, 3)) return launch_variant<TOKEN, 3, SP, KEEP>(a, l3, s);
  return MRSA_ERR_UNSUPPORTED;
}

int check_common(const void* q, const void* k, const int32_t* indices, int64_t batch,
                 int64_t q_len, int64_t kv_len, int64_t q_heads, int64_t kv_heads,
                 int64_t head_dim, int64_t topk, int64_t chunk_size, float sm_scale) {
  if (batch < 0 || q_len < 0 || kv_len < 0 || q_heads <= 0 || kv_heads <= 0 ||
      q_heads % kv_heads != 0 || head_dim <= 0 || topk <= 0 || chunk_size <= 0 ||
      !(sm_scale > 0.f) || sm_scale == __builtin_inff())
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
                        chunk_size, sm_scale);
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
  a.parts = 1;
  a.partial = nullptr;
  a.keep = nullptr;
  a.fuse_local = nullptr;
  a.fuse_w = nullptr;
  return launch_selected<false>(a, (hipStream_t)stream);
}

extern "C" int mrsa_candidate_token_scores_fwd(const void* q, const void* k,
                                               const int32_t* indices, const uint8_t* key_valid,
                                               int64_t batch, int64_t q_len, int64_t kv_len,
                                               int64_t q_heads, int64_t kv_heads,
                                               int64_t head_dim, int64_t topk,
                                               int64_t chunk_size, float sm_scale,
                                               float* scores, void* stream) {
  int st = check_common(q, k, indices, batch, q_len, kv_len, q_heads, kv_heads, head_dim, topk,
                        chunk_size, sm_scale);
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
  a.parts = 1;
  a.partial = nullptr;
  a.keep = nullptr;
  a.fuse_local = nullptr;
  a.fuse_w = nullptr;
  return launch_selected<true>(a, s);
}

namespace {

// Routed attention with an optional walk split (parts > 1: fp32 partials in
// `partial`, summed into `out`) and an optional token keep mask.
int selected_forward(const void* q, const void* k, const void* v_tiles, const void* weights,
                     const int32_t* indices, const uint8_t* key_valid, const int8_t* keep,
                     int64_t batch, int64_t q_len, int64_t kv_len, int64_t q_heads,
                     int64_t kv_heads, int64_t head_dim, int64_t topk, int64_t chunk_size,
                     int mask_last_token, float sm_scale, int64_t parts, float* partial,
                     const void* fuse_local, const void* fuse_w, void* out, void* stream) {
  int st = check_common(q, k, indices, batch, q_len, kv_len, q_heads, kv_heads, head_dim, topk,
                        chunk_size, sm_scale);
  if (st != MRSA_OK) return st;
  if (parts < 1 || parts > kMaxParts) return MRSA_ERR_INVALID_ARGUMENT;
  if (batch * parts > 65535) return MRSA_ERR_UNSUPPORTED;
  if (batch == 0 || q_len == 0) return MRSA_OK;
  if (!v_tiles || !weights || !out || (uintptr_t)v_tiles % 16 != 0 || (uintptr_t)out % 8 != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (parts > 1 && (!partial || (uintptr_t)partial % 16 != 0)) return MRSA_ERR_INVALID_ARGUMENT;
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
  a.out = parts > 1 ? nullptr : (uint16_t*)out;
  a.tscores = nullptr;
  a.parts = (int)parts;
  a.partial = parts > 1 ? partial : nullptr;
  a.keep = keep;
  if ((fuse_local == nullptr) != (fuse_w == nullptr)) return MRSA_ERR_INVALID_ARGUMENT;
  if (fuse_local && (uintptr_t)fuse_local % 8 != 0) return MRSA_ERR_INVALID_ARGUMENT;
  a.fuse_local = (const uint16_t*)fuse_local;
  a.fuse_w = (const uint16_t*)fuse_w;
  hipStream_t s = (hipStream_t)stream;
  st = keep ? launch_selected<false, true>(a, s) : launch_selected<false>(a, s);
  if (st != MRSA_OK || parts == 1) return st;
  const int64_t n4 = batch * q_len * q_heads * 128 / 4;
  const int64_t blocks = std::min<int64_t>((n4 + 255) / 256, 4096);
  hipLaunchKernelGGL(sum_parts_kernel, dim3((unsigned)blocks), dim3(256), 0, s, partial,
                     (int)parts, n4, (uint16_t*)out, (const uint16_t*)fuse_local,
                     (const uint16_t*)fuse_w);
  return mrsa_launch_status();
}

}  // namespace

extern "C" int mrsa_selected_attention_split_fwd(
    const void* q, const void* k, const void* v_tiles, const void* weights,
    const int32_t* indices, const uint8_t* key_valid, int64_t batch, int64_t q_len,
    int64_t kv_len, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t topk,
    int64_t chunk_size, int mask_last_token, float sm_scale, int64_t parts, float* partial,
    void* out, void* stream) {
  return selected_forward(q, k, v_tiles, weights, indices, key_valid, nullptr, batch, q_len,
                          kv_len, q_heads, kv_heads, head_dim, topk, chunk_size, mask_last_token,
                          sm_scale, parts, partial, nullptr, nullptr, out, stream);
}

extern "C" int mrsa_selected_attention_keep_fwd(
    const void* q, const void* k, const void* v_tiles, const void* weights,
    const int32_t* indices, const uint8_t* key_valid, const int8_t* token_keep, int64_t batch,
    int64_t q_len, int64_t kv_len, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
    int64_t topk, int64_t chunk_size, int mask_last_token, float sm_scale, int64_t parts,
    float* partial, void* out, void* stream) {
  if (batch > 0 && q_len > 0 && !token_keep) return MRSA_ERR_INVALID_ARGUMENT;
  return selected_forward(q, k, v_tiles, weights, indices, key_valid, token_keep, batch, q_len,
                          kv_len, q_heads, kv_heads, head_dim, topk, chunk_size, mask_last_token,
                          sm_scale, parts, partial, nullptr, nullptr, out, stream);
}

extern "C" int mrsa_selected_attention_fused_fwd(
    const void* q, const void* k, const void* v_tiles, const void* weights,
    const int32_t* indices, const uint8_t* key_valid, const int8_t* token_keep,
    const void* local_output, const void* local_weight, int64_t batch, int64_t q_len,
    int64_t kv_len, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t topk,
    int64_t chunk_size, int mask_last_token, float sm_scale, int64_t parts, float* partial,
    void* out, void* stream) {
  if (batch > 0 && q_len > 0 && (!local_output || !local_weight))
    return MRSA_ERR_INVALID_ARGUMENT;
  return selected_forward(q, k, v_tiles, weights, indices, key_valid, token_keep, batch, q_len,
                          kv_len, q_heads, kv_heads, head_dim, topk, chunk_size, mask_last_token,
                          sm_scale, parts, partial, local_output, local_weight, out, stream);
}
