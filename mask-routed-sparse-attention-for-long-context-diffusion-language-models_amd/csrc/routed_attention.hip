// Routed (selected-chunk) attention and candidate token scores: the gather walk.
//
// out[q, g] = sum_k w[q, g, k] * softmax_{s in chunk idx[q, k], s valid}(q_g . k_s * scale) . V
// Each routed chunk is normalised on its own (ops/hils_fwd_bwd_head.py:453-559;
// formula restated in the reference test test_hils_non_power_two_topk.py:122-138):
// the landmark slot (last key of the chunk, when mask_last_token) and invalid
// keys are excluded, P = bf16(p * w / sum p) feeds the PV product with fp32
// accumulation, and a chunk whose keys are all masked contributes nothing.
// Index lists are read like the reference kernel: a query's list ends at its
// first negative entry; entries >= kv_len / 64 are skipped.  A chunk listed
// twice contributes once with the two weights summed (rounded to bf16).
//
// Work split.  A workgroup owns a tile of TQ (<= 32) queries of one KV head
// and keeps their fp32 outputs in LDS (a slot of 8 head rows of 128 floats
// per query, heads >= G padding).  Its prologue turns the tile's index lists
// into a walk: the ascending list of the chunks any of its queries routes
// to, and for each such chunk (a step) the items (query, weights) that own
// it.  The first 8 steps go to the 8 waves, each later one to the wave that
// claims it first (an LDS counter), and a wave processes a step on its own:
//   K and V of the chunk straight into registers from the chunk's
//   fragments (mrsa_kv_fragments: the operands' register images, so each of
//   the 32 load instructions reads 1 KB contiguous); the step's owners are
//   packed two per 16-column tile (column j: owner j >> 3, head j & 7);
//   per tile
//     S^T = K . Q^T                 16 MFMAs (16x16x32 bf16)
//     per-column softmax over the 64 keys, P = bf16(p w / sum p)
//     the owners' LDS rows read into the accumulators (lane (grp, j):
//     column j, dims 16 nt + 4 grp .. + 3), O^T += V^T . P^T (16 MFMAs)
//     and the rows written back
// The next tile's Q and the next step's K / V are loaded into the same
// registers as soon as the current ones are consumed.  The epilogue barrier
// turns the LDS outputs into bf16 rows (fused with the local branch when
// asked) or fp32 partial sums of a walk split.
//
// Adding a tile.  Two waves may hold tiles of the same query at once.  LDS
// float atomics (ds_add_f32) run at about two cycles per lane, so instead a
// wave takes both owners' bits of a per-workgroup lock word, reads the
// rows, accumulates onto them and writes them back with 16-byte accesses,
// and clears the bits.
// The first try is a ds_or_rtn of both bits, issued right after the QK
// product and read after the softmax.  On a conflict the wave gives back
// what the try took and sets the tile aside (its P^T stays in registers, up
// to two tiles) while it runs the step's other tiles; the step's last tile
// then adds the set-aside ones, waiting if need be: a fresh try of both
// bits, and on a conflict the wave keeps the lower bit if that try took it,
// gives the other back and takes the missing bits one at a time, lowest
// first, with one-bit ORs (which change nothing while the bit is taken).  A
// wave only waits while holding bits below the one it waits for, so no cycle
// of waits forms, and no failed try leaves a bit set.  (Retrying both bits with OR and undo let two waves that want the
// same bits block each other with their momentary bits in lockstep for as
// long as they kept retrying.)  LDS operations of one wave complete in issue
// order, so its writes land before its release and after another wave's
// acquire.  The order of the fp32 additions into a row depends on timing, so
// the last bit of an output can differ between runs.  Past `spin_limit`
// tries (about 6 ms; a guard that ends the wait, never reached while every
// holder finishes its tile) the wave gives its bits back and defers the tile:
// it appends (step, tile) to a per-workgroup queue and moves on.  After the
// walk's barrier, when no wave holds a row, wave 0 replays the queued tiles
// one by one (chunk, Q and softmax recomputed) onto the rows, so a deferred
// tile costs time but never terms.
//
// LDS output rows: row (q, g) of slot q at (8 q + g) * 128 floats; the
// 16-byte block b of dims 4 b .. 4 b + 3 sits at block b ^ g, so the eight
// lanes of one 16-byte access per row group (heads 0..7 of one owner) hit
// eight different bank groups.
//
// Token-score mode (candidate_token_scores_gqa,
// ops/hils_token_score_gqa_tilelang.py:17-114) runs the same walk and writes,
// per routed (query, slot), the max over the group of q.k times sm_scale for
// every key, -inf at the last slot and invalid keys.
#include "mrsa_device.h"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

using namespace mrsa;

// Tiles whose bounded lock wait ran out since the last read (each was
// deferred and replayed after the walk: the output stays exact; the count
// only reports the slow path).  One word per device, shared by every stream,
// read and cleared through mrsa_routed_lock_giveups.
__device__ unsigned long long g_lock_giveups;

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxTopk = 64;
constexpr int kMaxTQ = 32;                 // owner sets and the lock are 32-bit masks
constexpr int kMaxItems = 1024;            // TQ * K per workgroup
constexpr int64_t kMaxParts = 64;          // walk split limit
constexpr size_t kLdsBytes = 160 * 1024;
constexpr int kDefaultSpinLimit = 65536;   // lock tries before a tile is deferred

struct RaArgs {
  const uint16_t* q;
  const uint16_t* qf;        // [B, Hkv, Lq, 1024] Q operand images (mrsa_q_fragments) or null
  const uint16_t* kvf;       // [B, Hkv, Ck, 16384] K / V fragments
  const uint16_t* w;
  const int32_t* idx;
  const uint8_t* key_valid;
  const int8_t* keep;        // [B, Lq, Hkv, K, 64] nonzero = key kept (KEEP only)
  int64_t B, Lq, Lk;
  int Hq, Hkv, G, K;
  int64_t Ck;                // chunks in the cache
  int mask_last;
  float scale_log2;
  float sm_scale;
  uint16_t* out;
  float* tscores;
  int parts;
  float* partial;            // [parts][B][Lq][Hq][128] fp32 when parts > 1
  const uint16_t* fuse_local;
  const uint16_t* fuse_w;
  int tq;                    // queries per tile
  int64_t ntiles;            // ceil(Lq / tq)
  int64_t units;             // B * Hkv * parts * ntiles workgroups of work
  int spin_limit;            // lock tries before a tile is deferred (<= 0: every tile)
  int det;                   // fixed accumulation order (per-query tickets instead of the lock)
  const float* slope;        // [Hq] ALiBi slopes (ALIBI instances only)
  // EXT instances (the routed backward's dQ walk): P^T tiles read from
  // ext_p [B, Lq, Hq, K] records of 64 bf16 (lane group g's 16 keys at 16 g,
  // in the order tile_P packs them), the fragments' V half being K^T, and
  // the fp32 rows added into ext_out [B, Lq, Hq, 128].
  const uint16_t* ext_p;
  float* ext_out;
};

__host__ __device__ inline size_t al16(size_t x) { return (x + 15) & ~(size_t)15; }

// LDS carve-up (byte offsets).  The output region -- query slots of 8 head
// rows of 128 floats (heads >= G padding), one more slot taking the adds of
// a tile's missing second owner -- doubles as the prologue's scratch (raw
// index rows, list flags, staged weights, per-chunk owner bits and step
// numbers), which is dead once the items are built.
struct RaLayout {
  size_t o, o_bytes;
  size_t raw, qlen, qflag, wst, omask, step_of, scratch_end;
  size_t rec, iq, islot, iw, ikeep, dq, irank, tick, misc, total;
  int items, cap;
};

__host__ __device__ inline RaLayout ra_layout(int tq, int G, int K, int64_t Ck, bool token,
                                              bool keep, bool det) {
  RaLayout l;
  l.items = tq * K;
  l.cap = (int)(Ck < l.items ? Ck : l.items);
  l.o_bytes = token ? 0 : ((size_t)tq + 1) * 8 * 128 * 4;
  size_t s = 0;
  l.raw = s;     s = al16(s + (size_t)l.items * 4);
  l.qlen = s;    s = al16(s + (size_t)tq * 4);
  l.qflag = s;   s = al16(s + (size_t)tq * 4);
  l.wst = s;     s = al16(s + (token ? 0 : (size_t)tq * 8 * K * 2));
  l.omask = s;   s = al16(s + (size_t)Ck * 4);
  l.step_of = s; s = al16(s + (size_t)Ck * 2);
  l.scratch_end = s;
  l.o = 0;
  size_t o = al16(l.o_bytes > s ? l.o_bytes : s);
  l.rec = o;     o = al16(o + (size_t)l.cap * 16);
  l.iq = o;      o = al16(o + (size_t)l.items);
  l.islot = o;   o = al16(o + (size_t)l.items);
  l.iw = o;      o = al16(o + (token ? 0 : (size_t)l.items * 8 * 2));
  l.ikeep = o;   o = al16(o + (keep ? (size_t)l.items * 8 : 0));
  l.dq = o;      o = al16(o + (token ? 0 : (size_t)l.items * 2));
  l.irank = o;   o = al16(o + (det ? (size_t)l.items : 0));
  l.tick = o;    o = al16(o + (det ? ((size_t)tq + 1) * 4 : 0));
  l.misc = o;    o = al16(o + (size_t)(2 * kWaves + 8 + 64) * 4);
  l.total = o;
  return l;
}

__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}

// Kept-key bits (bit j = key j kept) of one 64-byte token-keep row.
__device__ __forceinline__ uint64_t kept_bits(const int8_t* kr) {
  uint64_t bits = 0ull;
  if (((uintptr_t)kr & 15) == 0) {
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
  return bits;
}

// Lock word accesses (lane 0 issues; results made wave-uniform).
__device__ __forceinline__ uint32_t lds_or_rtn(uint32_t addr, uint32_t v) {
  uint32_t old;
  asm volatile("ds_or_rtn_b32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
               : "=v"(old)
               : "v"(addr), "v"(v)
               : "memory");
  return old;
}
__device__ __forceinline__ uint32_t lds_read_rtn(uint32_t addr) {
  uint32_t v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
  return v;
}
__device__ __forceinline__ void lds_and(uint32_t addr, uint32_t v) {
  asm volatile("ds_and_b32 %0, %1" ::"v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Operand loads are buffer loads: one buffer resource per tensor (SGPRs),
// one per-lane byte offset (VGPR) and wave-uniform chunk offsets (SGPRs), so
// the 32 loads of a chunk need no 64-bit address registers.  Offsets past the
// resource's range read zero.
constexpr int64_t kFragElems = 16384;
constexpr uint32_t kFragBytes = 32768;
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw 32-bit dwords, no swizzle
constexpr uint32_t kZeroOffset = 0x7ffffff0u;  // past every range: reads zero

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           (int)kRsrcWord3);
}
__device__ __forceinline__ u32x4_t bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
}

// K operands (keys 16 mt + j, dims 32 ks + 8 grp..) and V operands (dims
// 16 nt + j, keys 32 ks + 8 grp.. in the tiled order) of the chunk whose
// fragments start at byte `cb`; `lo` = 16 * lane.  Instruction i of the
// chunk's 32 reads bytes 1024 i + lo: the part below 4 KB goes into the
// load's immediate offset, the rest into the SGPR offset.
__device__ __forceinline__ void load_k(u32x4_t (&kb)[4][4], __amdgpu_buffer_rsrc_t r,
                                       uint32_t lo, uint32_t cb) {
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) kb[mt][ks] = bload(r, lo + 1024u * ks, cb + 4096u * mt);
}
__device__ __forceinline__ void load_v(u32x4_t (&vb)[8][2], __amdgpu_buffer_rsrc_t r,
                                       uint32_t lo, uint32_t cb) {
#pragma unroll
  for (int nt = 0; nt < 8; ++nt)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int i = 2 * nt + ks;
      vb[nt][ks] = bload(r, lo + 1024u * (i & 3), cb + 16384u + 4096u * (i >> 2));
    }
}
// Q^T operand of one tile column: k-step ks at `off` + ks * `kstep` bytes
// (kZeroOffset for padding columns).  From q rows: off = the head row + 16
// grp, kstep 64.  From Q fragments: off = the query's image + 128 grp + 16
// head, kstep 512, so the 8 head columns of one lane group read one whole
// 128-byte line.
__device__ __forceinline__ void load_q(u32x4_t (&Qb)[4], __amdgpu_buffer_rsrc_t r, uint32_t off,
                                       uint32_t kstep) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) Qb[ks] = bload(r, off, kstep * ks);
}

template <bool TOKEN, bool KEEP, bool DET, bool ALIBI, bool EXT = false>
__global__ void __launch_bounds__(kThreads, 1) routed_attn_kernel(RaArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  // Workgroup -> work unit, XCD-aware: workgroups are dealt to the 8 XCDs
  // round-robin by linear id, so XCD x takes the contiguous unit range
  // [x * per, (x + 1) * per): one KV head's consecutive query tiles, whose
  // walks read the same chunks from that XCD's L2 at about the same time.
  const int64_t per = (int64_t)(gridDim.x >> 3);
  const int64_t unit = (int64_t)(blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (unit >= a.units) return;
  const int64_t tile = unit % a.ntiles;
  int64_t rest = unit / a.ntiles;
  const int part = (int)(rest % a.parts);
  rest /= a.parts;
  const int h = (int)(rest % a.Hkv);
  const int64_t b = rest / a.Hkv;

  const int K = a.K, G = a.G, tq = a.tq;
  const int64_t Ck = a.Ck;
  // (EXT items keep their duplicate slots' mask where KEEP keeps a keep row)
  const RaLayout L = ra_layout(tq, G, K, Ck, TOKEN, KEEP || EXT, DET);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t q0 = tile * tq;
  const int nq = (int)min((int64_t)tq, a.Lq - q0);
  const int items = L.items;

  int32_t* raw = reinterpret_cast<int32_t*>(smem + L.raw);         // [tq][K]
  int32_t* qlen = reinterpret_cast<int32_t*>(smem + L.qlen);       // [tq]
  uint32_t* qflag = reinterpret_cast<uint32_t*>(smem + L.qflag);   // [tq] list not strictly ascending
  uint16_t* wst = reinterpret_cast<uint16_t*>(smem + L.wst);       // [tq][8][K]
  uint32_t* omask = reinterpret_cast<uint32_t*>(smem + L.omask);   // [Ck]
  uint16_t* step_of = reinterpret_cast<uint16_t*>(smem + L.step_of);  // [Ck]
  float* O = reinterpret_cast<float*>(smem + L.o);                 // [tq + 1][8][128]
  // Step records [cap]: x = chunk | owners << 24, y = first item | the first
  // tile's two owner slots << 16, (z, w) = excluded keys of the chunk.
  u32x4_t* s_rec = reinterpret_cast<u32x4_t*>(smem + L.rec);
  uint8_t* it_q = smem + L.iq;                                     // [items]
  uint8_t* it_slot = smem + L.islot;                               // [items]
  uint16_t* it_w = reinterpret_cast<uint16_t*>(smem + L.iw);       // [items][8]
  uint64_t* it_keep = reinterpret_cast<uint64_t*>(smem + L.ikeep); // [items]
  int32_t* misc = reinterpret_cast<int32_t*>(smem + L.misc);
  uint32_t* lock = reinterpret_cast<uint32_t*>(misc + 2 * kWaves + 1);
  uint32_t* claim = reinterpret_cast<uint32_t*>(misc + 2 * kWaves + 2);  // steps claimed
  uint32_t* dcount = reinterpret_cast<uint32_t*>(misc + 2 * kWaves + 4);  // deferred tiles
  uint16_t* dq = reinterpret_cast<uint16_t*>(smem + L.dq);         // [items] step << 4 | tile
  uint8_t* it_rank = smem + L.irank;                               // [items] (det)
  uint32_t* tick = reinterpret_cast<uint32_t*>(smem + L.tick);     // [tq + 1] (det)
  uint32_t* idle_or = reinterpret_cast<uint32_t*>(misc + 2 * kWaves + 8);  // [64], never read

  // ---- prologue: the walk of this tile ----------------------------------
  // 1. Index rows (-1 past the sequence end), list lengths and flags, owner
  //    bits cleared, routing weights staged as [q][g][k] (heads >= G zero).
  for (int e = tid; e < items; e += kThreads) {
    const int qq = e / K, kk = e - qq * K;
    raw[e] = qq < nq ? a.idx[((b * a.Lq + q0 + qq) * a.Hkv + h) * K + kk] : -1;
  }
  for (int i = tid; i < tq; i += kThreads) {
    qlen[i] = K;
    qflag[i] = 0u;
  }
  if (DET)
    for (int i = tid; i <= tq; i += kThreads) tick[i] = 0u;
  if (tid == 0) {
    *lock = 0u;
    *claim = 0u;
    *dcount = 0u;
  }
  for (int64_t c = tid; c < Ck; c += kThreads) omask[c] = 0u;
  if constexpr (!TOKEN && !EXT) {
    const uint16_t* wrow0 = a.w + ((b * a.Lq + q0) * a.Hq + (int64_t)h * G) * K;
    const int64_t qstride = (int64_t)a.Hq * K;
    if ((K & 7) == 0 && ((uintptr_t)a.w & 15) == 0) {
      const int vpr = K >> 3;
      for (int e = tid; e < tq * 8 * vpr; e += kThreads) {
        const int row = e / vpr, v = e - row * vpr;
        const int qq = row >> 3, gg = row & 7;
        u32x4_t x = {0u, 0u, 0u, 0u};
        if (qq < nq && gg < G)
          x = *reinterpret_cast<const u32x4_t*>(wrow0 + qq * qstride + gg * K + 8 * v);
        *reinterpret_cast<u32x4_t*>(wst + row * K + 8 * v) = x;
      }
    } else {
      for (int e = tid; e < tq * 8 * K; e += kThreads) {
        const int row = e / K, kk = e - row * K;
        const int qq = row >> 3, gg = row & 7;
        wst[e] = (qq < nq && gg < G) ? wrow0[qq * qstride + gg * K + kk] : (uint16_t)0;
      }
    }
  }
  __syncthreads();
  // 2. A list ends at its first negative entry; a list that is not strictly
  //    ascending (up to its end) may hold duplicates.
  for (int e = tid; e < items; e += kThreads) {
    const int kk = e % K;
    const int32_t c = raw[e];
    if (c < 0) atomicMin(&qlen[e / K], kk);
    if (kk > 0 && c >= 0 && raw[e - 1] >= 0 && c <= raw[e - 1]) atomicOr(&qflag[e / K], 1u);
  }
  __syncthreads();
  // 3. Owner bits of every listed chunk.
  for (int e = tid; e < items; e += kThreads) {
    const int qq = e / K, kk = e - qq * K;
    const int32_t c = raw[e];
    if (kk < qlen[qq] && c < Ck) atomicOr(&omask[c], 1u << qq);
  }
  __syncthreads();
  // 4. Steps: owned chunks in ascending order, with the offset of their
  //    first item (items of a step are its owners in query order).
  {
    const int64_t cper = (Ck + kThreads - 1) / kThreads;
    const int64_t c0 = min(Ck, (int64_t)tid * cper), c1 = min(Ck, c0 + cper);
    int cnt = 0, pc = 0;
    for (int64_t c = c0; c < c1; ++c) {
      const uint32_t m = omask[c];
      cnt += m != 0u;
      pc += __popc(m);
    }
    int icnt = cnt, ipc = pc;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u1 = __shfl_up(icnt, o, 64), u2 = __shfl_up(ipc, o, 64);
      if (lane >= o) {
        icnt += u1;
        ipc += u2;
      }
    }
    if (lane == 63) {
      misc[wave] = icnt;
      misc[kWaves + wave] = ipc;
    }
    __syncthreads();
    int pos = icnt - cnt, item = ipc - pc, tsteps = 0, titems = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const int x = misc[w], y = misc[kWaves + w];
      pos += w < wave ? x : 0;
      item += w < wave ? y : 0;
      tsteps += x;
      titems += y;
    }
    for (int64_t c = c0; c < c1; ++c) {
      const uint32_t m = omask[c];
      if (m) {
        s_rec[pos][0] = (uint32_t)c;
        s_rec[pos][1] = (uint32_t)item;
        step_of[c] = (uint16_t)pos;
        ++pos;
        item += __popc(m);
      }
    }
    if (tid == 0) {
      misc[2 * kWaves] = tsteps;
      misc[2 * kWaves + 3] = titems;
    }
  }
  __syncthreads();
  const int st_lo = (int)((int64_t)part * misc[2 * kWaves] / a.parts);
  const int st_hi = (int)((int64_t)(part + 1) * misc[2 * kWaves] / a.parts);
  // 5. Items: the first occurrence of each chunk in a query's list (a later
  //    duplicate adds its weights to it).  Strictly ascending lists (what
  //    route scoring emits) have no duplicates and skip the scans.
  for (int e = tid; e < items; e += kThreads) {
    const int qq = e / K, kk = e - qq * K;
    const int32_t c = raw[e];
    const int n = qlen[qq];
    if (!(kk < n && c < Ck)) continue;
    const bool plain = qflag[qq] == 0u;
    if (!plain) {
      bool first = true;
      for (int k2 = 0; k2 < kk; ++k2) first &= raw[qq * K + k2] != c;
      if (!first) continue;
    }
    const uint32_t m = omask[c];
    const int pos = (int)s_rec[step_of[c]][1] + __popc(m & ((1u << qq) - 1u));
    it_q[pos] = (uint8_t)qq;
    it_slot[pos] = (uint8_t)kk;
    if (DET) {
      // Rank of the item in its query's walk order: the query's distinct
      // listed chunks below c (the slot itself for a strictly ascending
      // list, whose skipped entries >= Ck all come last).  A walk part
      // starts its query's ticket at the items of earlier steps.
      int rank = kk;
      if (!plain) {
        rank = 0;
        for (int k2 = 0; k2 < n; ++k2) {
          const int32_t c2 = raw[qq * K + k2];
          if (c2 >= c || c2 >= Ck) continue;
          bool first = true;
          for (int k3 = 0; k3 < k2; ++k3) first &= raw[qq * K + k3] != c2;
          rank += first ? 1 : 0;
        }
      }
      it_rank[pos] = (uint8_t)rank;
      if (step_of[c] < st_lo) atomicAdd(&tick[qq], 1u);
    }
    if constexpr (!TOKEN) {
      uint16_t wv[8];
#pragma unroll
      for (int gg = 0; gg < 8; ++gg) wv[gg] = wst[(qq * 8 + gg) * K + kk];
      if (!plain) {
        for (int k2 = kk + 1; k2 < n; ++k2) {
          if (raw[qq * K + k2] != c) continue;
#pragma unroll
          for (int gg = 0; gg < 8; ++gg)
            wv[gg] = (uint16_t)f32_to_bf16(bf16_to_f32(wv[gg]) +
                                           bf16_to_f32(wst[(qq * 8 + gg) * K + k2]));
        }
      }
      u32x4_t pk;
#pragma unroll
      for (int i = 0; i < 4; ++i) pk[i] = (uint32_t)wv[2 * i] | ((uint32_t)wv[2 * i + 1] << 16);
      *reinterpret_cast<u32x4_t*>(it_w + pos * 8) = pk;
    }
    if constexpr (KEEP)
      it_keep[pos] = kept_bits(a.keep + (((b * a.Lq + q0 + qq) * a.Hkv + h) * K + kk) * 64);
    if constexpr (EXT) {
      // the later slots of the list holding the same chunk: their dS records
      // add to the item's
      uint64_t dm = 0ull;
      if (!plain)
        for (int k2 = kk + 1; k2 < n; ++k2) dm |= (uint64_t)(raw[qq * K + k2] == c) << k2;
      it_keep[pos] = dm;
    }
  }
  // Excluded keys of every step (bit k = key k of its chunk): the landmark
  // slot and invalid keys.  One step per thread, its 64 valid bytes loaded
  // at once.
  const int nsteps = misc[2 * kWaves];
  const uint8_t* kvrow = a.key_valid ? a.key_valid + b * a.Lk : nullptr;
  for (int e = tid; e < nsteps; e += kThreads) {
    uint64_t m = a.mask_last ? (1ull << 63) : 0ull;
    if (kvrow) m |= ~kept_bits(reinterpret_cast<const int8_t*>(kvrow) + (int64_t)s_rec[e][0] * 64);
    s_rec[e][2] = (uint32_t)m;
    s_rec[e][3] = (uint32_t)(m >> 32);
  }
  __syncthreads();
  // Owner count and the first tile's owner slots of every step (a single
  // owner is listed twice).
  {
    const int titems = misc[2 * kWaves + 3];
    for (int e = tid; e < nsteps; e += kThreads) {
      const uint32_t i0 = s_rec[e][1];
      const uint32_t nx = e + 1 < nsteps ? (s_rec[e + 1][1] & 0xffffu) : (uint32_t)titems;
      const uint32_t cnt = nx - i0;
      s_rec[e][0] |= cnt << 24;
      s_rec[e][1] = i0 | ((uint32_t)it_q[i0] << 16) | ((uint32_t)it_q[i0 + (cnt > 1u)] << 24);
    }
  }
  // 6. Outputs start at zero (the scratch above is dead now).
  if constexpr (!TOKEN) {
    const int n4 = tq * 8 * 128 / 4;
    for (int i = tid; i < n4; i += kThreads) reinterpret_cast<f32x4_t*>(O)[i] = zero4();
  }
  __syncthreads();

  // ---- the walk ------------------------------------------------------------
  const int j = lane & 15, grp = lane >> 4;
  const int own = j >> 3, gcol = j & 7;  // this lane's tile column: owner, head
  const float c2 = a.scale_log2;
  // ALiBi (ops/hils_fwd_bwd_head.py:445-451, hils_torch_ref :68-76): the raw
  // logit of chunk key s gets -slope[head] * max(0, 62 - s) before the
  // scale, i.e. ab = -slope c2 max(0, 62 - s) in the exp2 domain; this
  // lane's keys are 16 mt + 4 grp + r of its column's head, fixed for the
  // whole walk.
  float ab[4][4];
  if constexpr (ALIBI) {
    const float sl = gcol < G ? -a.slope[h * G + gcol] * c2 : 0.f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        ab[mt][r] = sl * fmaxf(0.f, (float)(62 - 16 * mt - r) - 4.f * (float)grp);
  }
  const __amdgpu_buffer_rsrc_t frs =
      make_rsrc(a.kvf + (b * a.Hkv + h) * Ck * kFragElems, (uint32_t)Ck * kFragBytes);
  const uint32_t flo = 16u * lane;
  // Q of this tile.  From q rows: query qi's head gcol at byte qi * qrow +
  // 256 gcol; the range ends at the tile's last real row (head G - 1 of
  // query nq - 1): with a head offset h G the base is not row-aligned, so
  // nq * qrow would reach past the tensor at the sequence end.  From Q
  // fragments: query qi's 2 KB image at qi * 2048, lane bytes 128 grp + 16
  // gcol + 512 ks.
  const bool qfrag = a.qf != nullptr;
  const uint32_t qrow = qfrag ? 2048u : (uint32_t)a.Hq * 256u;
  const uint32_t qks = qfrag ? 512u : 64u;
  const __amdgpu_buffer_rsrc_t qrs =
      qfrag ? make_rsrc(a.qf + ((b * a.Hkv + h) * a.Lq + q0) * 1024, (uint32_t)nq * 2048u)
            : make_rsrc(a.q + ((b * a.Lq + q0) * a.Hq + (int64_t)h * G) * 128,
                        (uint32_t)(nq - 1) * qrow + (uint32_t)G * 256u);
  const uint32_t qcol = qfrag ? 128u * grp + 16u * gcol : 256u * gcol + 16u * grp;
  // Q offset of this lane's column in a tile whose owner slots are `own2`
  // (slot of owner 0 | slot of owner 1 << 8).
  auto qoff = [&](uint32_t own2, bool valid) {
    return valid ? __umul24((own2 >> (8 * own)) & 0xffu, qrow) + qcol : kZeroOffset;
  };
  const uint32_t lock_addr = lds_address(lock);
  const int sinkq = tq;  // query slot taking the adds of a missing second owner
  // This lane's output row is its column's (query slot, head gcol); its
  // accumulator nt holds dims 16 nt + 4 grp .. + 3, the 16-byte block
  // 4 nt + grp of the row, stored at block (4 nt + grp) ^ gcol.  Even nt:
  // lane_e + 16 nt floats into the slot, odd nt: lane_o + 16 (nt - 1).
  const int lane_c = gcol * 128 + 4 * ((grp ^ gcol) & 3);
  const int lane_e = lane_c + 16 * (gcol >> 2);
  const int lane_o = lane_c + 16 - 16 * (gcol >> 2);
  float ninf_v = neg_inf();
  asm volatile("" : "+v"(ninf_v));  // kept in a register for set_where

  // The wave's first two steps are fixed; later ones are claimed one step
  // ahead (an LDS counter), so a step's record is read a step before it runs.
  int st = st_lo + wave;
  int nst = st + kWaves;
  int64_t c = 0, cn = 0;
  int i0 = 0, n = 0, i0n = 0, nn = 0;
  uint32_t own2 = 0u, own2n = 0u;  // owner slots of the current / next tile
  bool more = false;
  uint64_t msk = 0, mskn = 0;
  u32x4_t kb[4][4], vb[8][2], Qb[4];
  u32x4_t Pn[2];  // EXT: the next tile's records
  // P^T operand of a tile from its S^T accumulators: excluded keys (the
  // chunk's `mskc`, bit k = key k; keys a keep row drops) -> -inf, the
  // chunk's softmax times the column's routing weight `wv`, rounded to bf16.
  // Row j of P is this lane's column; reduction index 8 grp + e of k-step ks
  // is key 32 ks + 16 (e >> 2) + 4 grp + (e & 3), the tiled-V order.
  auto tile_P = [&](f32x4_t (&S)[4], uint64_t mskc, float wv, uint64_t kept,
                    u32x4_t (&Pb)[2]) {
    const uint64_t msh = mskc >> (4 * grp);  // bit 16 mt + r: key 16 mt + 4 grp + r
    // Key 63 (the landmark slot, the usual only exclusion) is S[3][3] of
    // lane group 3; other excluded keys take the per-bit path.
    S[3][3] = set_where(S[3][3], (mskc >> 63) ? 0xFFFF000000000000ull : 0ull, ninf_v);
    if (mskc & ~(1ull << 63)) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          S[mt][r] = set_where(
              S[mt][r], __builtin_amdgcn_ballot_w64((msh >> (16 * mt + r)) & 1ull), ninf_v);
    }
    if constexpr (KEEP) {
      const uint64_t kbits = kept >> (4 * grp);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          S[mt][r] = set_where(
              S[mt][r], __builtin_amdgcn_ballot_w64(!((kbits >> (16 * mt + r)) & 1ull)), ninf_v);
    }
    // P = bf16(p w / sum p) does not depend on the stabiliser of p.  Without
    // one, p = 2^(s c) and sum p stay in fp32's range for any |s c| well
    // below 64: the per-column max (and its cross-lane reduction) is
    // skipped.  When some column's sum leaves [2^-64, 2^64] -- extreme
    // logits, or no key left (sum 0) -- the wave takes the max-stabilised
    // form, which handles both.
    f32x4_t E[4];
    auto exp_sum = [&](float mb) {
      float ps[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          E[mt][r] = exp2_hw(__builtin_fmaf(S[mt][r], c2, ALIBI ? ab[mt][r] - mb : -mb));
        ps[mt] = (E[mt][0] + E[mt][1]) + (E[mt][2] + E[mt][3]);
      }
      return across4_sum((ps[0] + ps[1]) + (ps[2] + ps[3]));
    };
    float sum = 0.f;
    bool stabilise = KEEP;  // keep rows often drop whole chunks (sum 0)
    if constexpr (!KEEP) {
      sum = exp_sum(0.f);
      stabilise = !__all(sum >= 0x1p-64f && sum <= 0x1p64f);
    }
    if (stabilise) {
      if constexpr (ALIBI) {
        float mx = neg_inf();
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r) mx = fmaxf(mx, __builtin_fmaf(S[mt][r], c2, ab[mt][r]));
        mx = across4_max(mx);
        sum = exp_sum(mx == neg_inf() ? 0.f : mx);
      } else {
        const float mx = across4_max(max16_raw(S));
        sum = exp_sum(mx == neg_inf() ? 0.f : mx * c2);
      }
    }
    const float f = sum > 0.f ? wv * rcp_hw(sum) : 0.f;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      Pb[ks][0] = pack_bf16x2(E[2 * ks][0] * f, E[2 * ks][1] * f);
      Pb[ks][1] = pack_bf16x2(E[2 * ks][2] * f, E[2 * ks][3] * f);
      Pb[ks][2] = pack_bf16x2(E[2 * ks + 1][0] * f, E[2 * ks + 1][1] * f);
      Pb[ks][3] = pack_bf16x2(E[2 * ks + 1][2] * f, E[2 * ks + 1][3] * f);
    }
  };
  // O^T rows += V^T . P^T: this lane's row blocks (pe: even nt, po: odd nt)
  // read into the accumulators, the 16 products, written back.
  auto add_rows = [&](float* pe, float* po, const u32x4_t (&Pb)[2]) {
    f32x4_t acc[8];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
      acc[nt] = *reinterpret_cast<const f32x4_t*>((nt & 1) ? po + 16 * (nt - 1) : pe + 16 * nt);
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      acc[nt] = mfma_bf16_16x16x32(vb[nt][0], Pb[0], acc[nt]);
      acc[nt] = mfma_bf16_16x16x32(vb[nt][1], Pb[1], acc[nt]);
    }
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
      *reinterpret_cast<f32x4_t*>((nt & 1) ? po + 16 * (nt - 1) : pe + 16 * nt) = acc[nt];
  };

  auto decode_next = [&](const u32x4_t r) {
    cn = (int64_t)(r[0] & 0xffffffu);
    nn = (int)(r[0] >> 24);
    i0n = (int)(r[1] & 0xffffu);
    own2n = r[1] >> 16;
    mskn = ((uint64_t)r[3] << 32) | r[2];
  };

  // Hands the owners' rows on after a tile's row writes (issued before it;
  // the LDS completes one wave's operations in order): the lock bits back,
  // or in the fixed-order mode each owner's ticket to its next rank.
  auto release = [&](uint32_t want, uint32_t dwant) {
    if (!DET) {
      if (lane == 0) lds_and(lock_addr, ~want);
    } else if (lane == 0) {
      __hip_atomic_store(tick + (dwant & 63u), ((dwant >> 12) & 63u) + 1u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_WORKGROUP);
      if ((dwant >> 24) & 1u)
        __hip_atomic_store(tick + ((dwant >> 6) & 63u), ((dwant >> 18) & 63u) + 1u,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  };
  // Adds a tile's P^T onto its owners' rows (srow: this lane's row slot)
  // under the lock, waiting for it: the first try takes both bits at once;
  // on a conflict the wave keeps the lower bit if that try took it, gives
  // back the other and takes the missing bits one at a time, lowest first,
  // with one-bit ORs (which change nothing while the bit is taken).  A wave
  // only waits while holding bits below the one it waits for, so no cycle
  // of waits forms, and no failed try leaves a bit set.  In the fixed-order
  // mode (`want` packed as in do_tile) the wave waits until both owners'
  // tickets reach the tile's ranks: every earlier item of those queries
  // belongs to an earlier step, and the earliest step in flight always has
  // its tickets, so the waits end.  When the bounded wait runs out, the
  // tile (step st, tile t) is queued for the replay after the walk.
  auto add_locked = [&](float* srow, uint32_t want, int t, const u32x4_t (&Pb)[2]) {
    bool locked = false;
    if (a.spin_limit > 0 && DET) {
      const uint32_t ia = want & 63u, ib = (want >> 6) & 63u;
      const uint32_t ra = (want >> 12) & 63u, rb = (want >> 18) & 63u;
      const bool hb2 = (want >> 24) & 1u;
      for (int spin = 0; spin < a.spin_limit; ++spin) {
        const uint32_t ta = __builtin_amdgcn_readfirstlane(
            lds_read_rtn(lds_address(tick + ia)));
        const uint32_t tb = hb2 ? __builtin_amdgcn_readfirstlane(
                                      lds_read_rtn(lds_address(tick + ib)))
                                : rb;
        if (ta == ra && tb == rb) {
          locked = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    } else if (a.spin_limit > 0) {
      uint32_t seen = 0u;
      if (lane == 0) seen = lds_or_rtn(lock_addr, want);
      seen = __builtin_amdgcn_readfirstlane(seen);
      const uint32_t low = want & (0u - want);
      const uint32_t keep = want & ~seen & low;
      const uint32_t back = want & ~seen & ~keep;
      if ((seen & want) != 0u && lane == 0 && back) lds_and(lock_addr, ~back);
      uint32_t need = (seen & want) == 0u ? 0u : want & ~keep;
      for (int spin = 1; need != 0u && spin < a.spin_limit; ++spin) {
        const uint32_t bit = need & (0u - need);
        __builtin_amdgcn_s_sleep(1);
        uint32_t old = 0u;
        if (lane == 0) old = lds_or_rtn(lock_addr, bit);
        old = __builtin_amdgcn_readfirstlane(old);
        if ((old & bit) == 0u) need &= ~bit;
      }
      locked = need == 0u;
      if (!locked && lane == 0) lds_and(lock_addr, ~(want & ~need));  // give back what was taken
    }
    if (locked) {
      add_rows(srow + lane_e, srow + lane_o, Pb);
      asm volatile("" ::: "memory");
      release(want, want);
    } else if (lane == 0) {
      // The bounded wait ran out: queue the tile for the replay after the
      // walk (the queue holds every tile of the workgroup at most once).
      const uint32_t slot = __hip_atomic_fetch_add(dcount, 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_WORKGROUP);
      dq[slot] = (uint16_t)(((uint32_t)st << 4) | (uint32_t)t);
      atomicAdd(&g_lock_giveups, 1ull);
    }
  };
  // Up to two tiles of the current step set aside after a failed first try.
  int nset = 0;
  u32x4_t set0[2], set1[2];
  float* setrow0 = O;
  float* setrow1 = O;
  uint32_t setwant0 = 0u, setwant1 = 0u;
  int sett0 = 0, sett1 = 0;

  // EXT: the P^T operand of item ii's column -- the record of (query, head
  // gcol, list slot) -- read for every lane from a real record (padding
  // heads read head 0's) and zeroed after, so that no branch waits for it.
  // A chunk listed again later in the list (it_keep[ii]: the later slots)
  // adds those slots' records, summed in fp32 and rounded once.
  auto ext_rec = [&](int ii) {
    const int qq = it_q[ii];
    return a.ext_p +
           ((b * a.Lq + q0 + qq) * a.Hq + (int64_t)h * G + (gcol < G ? gcol : 0)) * K * 64 +
           16 * grp;
  };
  // the record of item ii's column (issued a tile ahead of its use)
  auto ext_load = [&](int ii, u32x4_t (&Pb)[2]) {
    const uint16_t* rec = ext_rec(ii) + it_slot[ii] * 64;
    Pb[0] = *reinterpret_cast<const u32x4_t*>(rec);
    Pb[1] = *reinterpret_cast<const u32x4_t*>(rec + 8);
  };
  // padding columns zeroed; the later duplicate slots' records added
  auto ext_finish = [&](int ii, bool cvalid, u32x4_t (&Pb)[2]) {
    const u32x4_t z = {0u, 0u, 0u, 0u};
    Pb[0] = cvalid ? Pb[0] : z;
    Pb[1] = cvalid ? Pb[1] : z;
    uint64_t dm = cvalid ? it_keep[ii] : 0ull;
    const uint16_t* rec0 = ext_rec(ii);
    if (dm) {
      float f[2][8];
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f[h2][2 * i] = bf16_lo(Pb[h2][i]);
          f[h2][2 * i + 1] = bf16_hi(Pb[h2][i]);
        }
      while (dm) {
        const int s2 = __builtin_ctzll(dm);
        dm &= dm - 1ull;
        const u32x4_t y0 = *reinterpret_cast<const u32x4_t*>(rec0 + s2 * 64);
        const u32x4_t y1 = *reinterpret_cast<const u32x4_t*>(rec0 + s2 * 64 + 8);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f[0][2 * i] += bf16_lo(y0[i]);
          f[0][2 * i + 1] += bf16_hi(y0[i]);
          f[1][2 * i] += bf16_lo(y1[i]);
          f[1][2 * i + 1] += bf16_hi(y1[i]);
        }
      }
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2)
#pragma unroll
        for (int i = 0; i < 4; ++i) Pb[h2][i] = pack_bf16x2(f[h2][2 * i], f[h2][2 * i + 1]);
    }
  };

  // One tile: columns 2 t + own of the step's owners.  The last tile of a
  // step (LAST) prefetches the next step's first Q and its K (after the QK
  // product) and V (after the PV product); other tiles prefetch the next
  // tile's Q.  Every path issues the same loads into the same registers (a
  // missing next step reloads the current chunk and reads Q as zeros), so
  // the waits before each product cover only what it consumes.
  auto do_tile = [&](int t, auto last_tag) {
    constexpr bool LAST = decltype(last_tag)::value;
    const int o = 2 * t + own;
    const bool cvalid = o < n && gcol < G;
    const int ii = i0 + (o < n ? o : n - 1);
    // The tile's two owners (wave-uniform, read a tile ahead); the next
    // tile's are read now and used after the QK product.
    const bool hb = 2 * t + 1 < n;
    const int qa = (int)(own2 & 0xffu);
    const int qb1 = (int)(own2 >> 8);
    uint32_t nx_a = 0u, nx_b = 0u;
    if constexpr (!LAST) {
      const int e2 = i0 + 2 * t + 2;
      nx_a = it_q[e2];
      nx_b = it_q[e2 + (2 * t + 3 < n ? 1 : 0)];
    }
    // The column's weight, read for every lane (ii is a real item of the
    // step) and consumed after the QK product, so that no branch waits for it.
    uint32_t wraw = TOKEN || EXT ? 0u : it_w[ii * 8 + gcol];
    // S^T = K . Q^T: lane (grp, j) gets keys 16 mt + 4 grp + r of column j.
    f32x4_t S[4];
    u32x4_t Pe[2];
    if constexpr (EXT) {
      Pe[0] = Pn[0];
      Pe[1] = Pn[1];
      ext_finish(ii, cvalid, Pe);
      // the next tile's records: the next tile of this step, or the first
      // tile of the next step (this one again when there is none)
      int in = ii;
      if constexpr (!LAST) in = i0 + min(2 * t + 2 + own, n - 1);
      else if (more) in = i0n + min(own, nn - 1);
      ext_load(in, Pn);
    } else {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        S[mt] = zero4();
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) S[mt] = mfma_bf16_16x16x32(kb[mt][ks], Qb[ks], S[mt]);
      }
    }
    uint32_t nown2;
    if constexpr (EXT) {
      if constexpr (!LAST) nown2 = (uint32_t)__builtin_amdgcn_readfirstlane(nx_a | (nx_b << 8));
      else nown2 = own2n;
    } else if constexpr (!LAST) {
      // read after the QK issue
      asm volatile("" : "+v"(nx_a), "+v"(nx_b), "+v"(wraw) : "v"(S[3][3]));
      nown2 = (uint32_t)__builtin_amdgcn_readfirstlane(nx_a | (nx_b << 8));
      load_q(Qb, qrs, qoff(nown2, o + 2 < n && gcol < G), qks);
    } else {
      asm volatile("" : "+v"(wraw) : "v"(S[3][3]));
      nown2 = own2n;
      load_q(Qb, qrs, qoff(nown2, more && own < nn && gcol < G), qks);
      load_k(kb, frs, flo, (uint32_t)cn * kFragBytes);
    }
    const uint64_t msh = msk >> (4 * grp);  // bit 16 mt + r: key 16 mt + 4 grp + r
    // First try for the owners' lock bits, issued now so that its LDS round
    // trip overlaps the softmax (the result is read after it).
    uint32_t want = (1u << qa) | (hb ? 1u << qb1 : 0u);
    // Every lane takes part (no divergent region, so the wait for the
    // result stays where it is used): lane 0 ORs the bits into the lock word,
    // the others OR 0 into words of their own.
    uint32_t first_try = 0u, tick_b = 0u;
    if constexpr (!TOKEN) {
      if (DET) {
        // the owners' tickets (read now, compared after the softmax)
        first_try = __hip_atomic_load(tick + qa, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        tick_b = __hip_atomic_load(tick + (hb ? qb1 : qa), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
      } else {
        first_try = __hip_atomic_fetch_or(lane == 0 ? lock : idle_or + lane,
                                          lane == 0 && a.spin_limit > 0 ? want : 0u,
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }

    if constexpr (TOKEN) {
      // max over the owner's head columns (lanes j, j ^ 1, j ^ 2, j ^ 4
      // share the owner), excluded keys -inf, times sm_scale.
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v = gcol < G ? S[mt][r] : neg_inf();
          v = fmaxf(v, __shfl_xor(v, 1, 64));
          v = fmaxf(v, __shfl_xor(v, 2, 64));
          v = fmaxf(v, __shfl_xor(v, 4, 64));
          S[mt][r] = v;
        }
      if (gcol == 0 && o < n) {
        const int qi = it_q[ii];
        const int slot = it_slot[ii];
        float* dst = a.tscores + (((b * a.Lq + q0 + qi) * a.Hkv + h) * K + slot) * 64 + 4 * grp;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          f32x4_t v;
#pragma unroll
          for (int r = 0; r < 4; ++r)
            v[r] = ((msh >> (16 * mt + r)) & 1ull) ? neg_inf() : S[mt][r] * a.sm_scale;
          *reinterpret_cast<f32x4_t*>(dst + 16 * mt) = v;
        }
      }
    } else {
      u32x4_t Pb[2];
      if constexpr (EXT) {
        Pb[0] = Pe[0];
        Pb[1] = Pe[1];
      } else {
        const float wv = cvalid ? bf16_to_f32(wraw) : 0.f;
        tile_P(S, msk, wv, KEEP && o < n ? it_keep[ii] : ~0ull, Pb);
      }
      // Add the tile into its owners' rows under the lock: the rows are read
      // into the accumulators and O^T_tile = V^T . P^T is added onto them
      // (lane (grp, j): column j, dims 16 nt + 4 grp + r).  A missing second
      // owner's columns go to the spare slot and padding heads to padding
      // rows, with P = 0.
      const int qb = hb ? qb1 : sinkq;
      float* const srow = O + (own ? qb : qa) * 1024;
      if constexpr (!EXT)
        asm volatile("" : "+v"(first_try), "+v"(tick_b) : "v"(Pb[1][3]));  // read after the softmax
      const uint32_t seen = __builtin_amdgcn_readfirstlane(first_try);
      // In the fixed-order mode `want` packs the owners and their ranks
      // (slot a | slot b << 6 | rank a << 12 | rank b << 18 | second owner << 24)
      // and the rows are free when both tickets equal the ranks.
      uint32_t dwant = 0u;
      bool free_now;
      if (DET) {
        const int ra = it_rank[i0 + 2 * t];
        const int rb = hb ? it_rank[i0 + 2 * t + 1] : 0;
        dwant = (uint32_t)qa | ((uint32_t)qb << 6) | ((uint32_t)ra << 12) | ((uint32_t)rb << 18) |
                ((uint32_t)hb << 24);
        const uint32_t sb = __builtin_amdgcn_readfirstlane(tick_b);
        free_now = seen == (uint32_t)ra && (!hb || sb == (uint32_t)rb);
      } else {
        free_now = (seen & want) == 0u;
      }
      // The lock word / tickets are read back with lgkmcnt(0): the row reads
      // of add_rows are issued after them.
      if (a.spin_limit > 0 && free_now) {
        add_rows(srow + lane_e, srow + lane_o, Pb);
        // The row writes are issued before the release and the LDS
        // completes one wave's operations in order.
        asm volatile("" ::: "memory");
        release(want, dwant);
      } else {
        // Some owner's rows are busy: give back the bits the try took and
        // set the tile aside (P kept in registers) while the step's other
        // tiles run; the last tile of the step adds it.  With both places
        // taken, wait for the rows now.
        const uint32_t took = want & ~seen;
        if (!DET && lane == 0 && a.spin_limit > 0 && took) lds_and(lock_addr, ~took);
        if (DET) want = dwant;
        if (nset == 0) {
          set0[0] = Pb[0];
          set0[1] = Pb[1];
          setrow0 = srow;
          setwant0 = want;
          sett0 = t;
          nset = 1;
        } else if (nset == 1) {
          set1[0] = Pb[0];
          set1[1] = Pb[1];
          setrow1 = srow;
          setwant1 = want;
          sett1 = t;
          nset = 2;
        } else {
          add_locked(srow, want, t, Pb);
        }
      }
      if constexpr (LAST) {
        // tiles set aside in this step (the chunk's V is still in vb)
        if (nset > 0) add_locked(setrow0, setwant0, sett0, set0);
        if (nset > 1) add_locked(setrow1, setwant1, sett1, set1);
        nset = 0;
        load_v(vb, frs, flo, (uint32_t)cn * kFragBytes);
      }
    }
    own2 = nown2;
  };

  // A deferred tile (queue entry step << 4 | tile), recomputed from its
  // chunk and added onto its owners' rows without the lock: it runs after
  // the walk's barrier, on wave 0 alone.
  auto replay_tile = [&](uint32_t entry) {
    const u32x4_t r = s_rec[entry >> 4];
    const int t = (int)(entry & 15u);
    const int64_t rc = (int64_t)__builtin_amdgcn_readfirstlane(r[0] & 0xffffffu);
    const int rn = __builtin_amdgcn_readfirstlane(r[0] >> 24);
    const int ri0 = __builtin_amdgcn_readfirstlane(r[1] & 0xffffu);
    const uint64_t rmsk = uniform64(((uint64_t)r[3] << 32) | r[2]);
    const int o = 2 * t + own;
    const bool hb = 2 * t + 1 < rn;
    const int qa = __builtin_amdgcn_readfirstlane(it_q[ri0 + 2 * t]);
    const int qb = hb ? __builtin_amdgcn_readfirstlane(it_q[ri0 + 2 * t + 1]) : sinkq;
    const int ii = ri0 + (o < rn ? o : rn - 1);
    const bool cvalid = o < rn && gcol < G;
    u32x4_t Pb[2];
    if constexpr (EXT) {
      load_v(vb, frs, flo, (uint32_t)rc * kFragBytes);
      ext_load(ii, Pb);
      ext_finish(ii, cvalid, Pb);
    } else {
      const float wv = cvalid ? bf16_to_f32(it_w[ii * 8 + gcol]) : 0.f;
      load_q(Qb, qrs, qoff((uint32_t)qa | ((uint32_t)(hb ? qb : 0) << 8), cvalid), qks);
      load_k(kb, frs, flo, (uint32_t)rc * kFragBytes);
      load_v(vb, frs, flo, (uint32_t)rc * kFragBytes);
      f32x4_t S[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        S[mt] = zero4();
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) S[mt] = mfma_bf16_16x16x32(kb[mt][ks], Qb[ks], S[mt]);
      }
      tile_P(S, rmsk, wv, KEEP && o < rn ? it_keep[ii] : ~0ull, Pb);
    }
    float* const srow = O + (own ? qb : qa) * 1024;
    add_rows(srow + lane_e, srow + lane_o, Pb);
  };

  if (st < st_hi) {
    {
      const u32x4_t r = s_rec[st];
      c = (int64_t)__builtin_amdgcn_readfirstlane(r[0] & 0xffffffu);
      n = __builtin_amdgcn_readfirstlane(r[0] >> 24);
      i0 = __builtin_amdgcn_readfirstlane(r[1] & 0xffffu);
      own2 = __builtin_amdgcn_readfirstlane(r[1] >> 16);
      msk = uniform64(((uint64_t)r[3] << 32) | r[2]);
    }
    more = nst < st_hi;
    u32x4_t rn = s_rec[more ? nst : st];
    // the order of the prefetches at a step's end: Q, K, then V
    if constexpr (!EXT) {
      load_q(Qb, qrs, qoff(own2, own < n && gcol < G), qks);
      load_k(kb, frs, flo, (uint32_t)c * kFragBytes);
    } else {
      ext_load(i0 + min(own, n - 1), Pn);
    }
    if constexpr (!TOKEN) load_v(vb, frs, flo, (uint32_t)c * kFragBytes);
    while (true) {
      // Claim the step after the next one (steps after the first 2 kWaves go
      // to whichever wave asks first); the claim's round trip overlaps this
      // step.  Lane 0 adds 1 to the counter, the other lanes add 0 to words
      // of their own (no divergent region).
      const uint32_t tk = __hip_atomic_fetch_add(lane == 0 ? claim : idle_or + lane,
                                                 lane == 0 ? 1u : 0u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_WORKGROUP);
      const int T = (n + 1) >> 1;
      for (int t = 0; t + 1 < T; ++t) do_tile(t, std::false_type{});
      // the next step's record, read a step ago (the current chunk when
      // there is none: the prefetches then reload it and read Q as zeros)
      {
        u32x4_t r = rn;
        r[0] = __builtin_amdgcn_readfirstlane(r[0]);
        r[1] = __builtin_amdgcn_readfirstlane(r[1]);
        r[2] = __builtin_amdgcn_readfirstlane(r[2]);
        r[3] = __builtin_amdgcn_readfirstlane(r[3]);
        decode_next(r);
        if (!more) cn = c;
      }
      do_tile(T - 1, std::true_type{});
      if (!more) break;
      st = nst;
      c = cn;
      i0 = i0n;
      n = nn;
      msk = mskn;
      nst = st_lo + 2 * kWaves + (int)__builtin_amdgcn_readfirstlane(tk);
      more = nst < st_hi;
      rn = s_rec[more ? nst : st];
    }
  }

  // ---- epilogue -----------------------------------------------------------
  if constexpr (!TOKEN) {
    __syncthreads();
    // Deferred tiles, replayed while no wave is inside a row (every other
    // wave waits at the barrier below).
    const uint32_t nd = *dcount;
    if (nd > 0u) {
      if (wave == 0) {
        if (DET && nd > 1u) {
          // Fixed order: a query's deferred items are the tail of its walk
          // order (a later item waits for the ticket of an earlier one), so
          // replaying the queue in step order keeps each row's order.
          if (lane == 0)
            for (uint32_t i = 1; i < nd; ++i) {
              const uint16_t x = dq[i];
              uint32_t j = i;
              for (; j > 0 && dq[j - 1] > x; --j) dq[j] = dq[j - 1];
              dq[j] = x;
            }
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
        for (uint32_t e = 0; e < nd; ++e) replay_tile(dq[e]);
      }
      __syncthreads();
    }
    // Work item e: output row rho = e / 16 (query rho / G, head rho % G),
    // dims 8 u .. 8 u + 7 (u = e % 16), LDS blocks 2 u and 2 u + 1 stored at
    // block ^ g.  A thread has at most kEpi items; with the output fusion
    // their local-branch rows are all loaded before the first store.
    constexpr int kEpi = kMaxTQ * 8 * 16 / kThreads;
    const int rows = nq * G;
    auto item_row = [&](int e, int& u, int& qq, int& g) {
      const int rho = e >> 4;
      u = e & 15;
      qq = rho / G;
      g = rho - qq * G;
      return (b * a.Lq + q0 + qq) * a.Hq + h * G + g;
    };
    auto lds_rows = [&](int qq, int g, int u, f32x4_t& x0, f32x4_t& x1) {
      const float* src = O + (qq * 8 + g) * 128;
      x0 = *reinterpret_cast<const f32x4_t*>(src + 4 * ((2 * u) ^ g));
      x1 = *reinterpret_cast<const f32x4_t*>(src + 4 * ((2 * u + 1) ^ g));
    };
    if constexpr (EXT) {
      // the rows added into ext_out (each row belongs to this workgroup alone)
      for (int e = tid; e < rows * 16; e += kThreads) {
        int u, qq, g;
        const int64_t row = item_row(e, u, qq, g);
        f32x4_t x0, x1;
        lds_rows(qq, g, u, x0, x1);
        f32x4_t* dst = reinterpret_cast<f32x4_t*>(a.ext_out + row * 128 + 8 * u);
        f32x4_t y0 = dst[0], y1 = dst[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          y0[i] += x0[i];
          y1[i] += x1[i];
        }
        dst[0] = y0;
        dst[1] = y1;
      }
    } else if (a.parts > 1) {
      for (int e = tid; e < rows * 16; e += kThreads) {
        int u, qq, g;
        const int64_t row = item_row(e, u, qq, g);
        f32x4_t x0, x1;
        lds_rows(qq, g, u, x0, x1);
        float* prow = a.partial + ((int64_t)part * a.B * a.Lq * a.Hq + row) * 128 + 8 * u;
        reinterpret_cast<f32x4_t*>(prow)[0] = x0;
        reinterpret_cast<f32x4_t*>(prow)[1] = x1;
      }
    } else {
      u32x4_t lrow[kEpi];
      float wl[kEpi];
      if (a.fuse_local) {
#pragma unroll
        for (int k = 0; k < kEpi; ++k) {
          const int e = tid + k * kThreads;
          if (e < rows * 16) {
            int u, qq, g;
            const int64_t row = item_row(e, u, qq, g);
            wl[k] = bf16_to_f32(a.fuse_w[row]);
            lrow[k] = *reinterpret_cast<const u32x4_t*>(a.fuse_local + row * 128 + 8 * u);
          }
        }
      }
#pragma unroll
      for (int k = 0; k < kEpi; ++k) {
        const int e = tid + k * kThreads;
        if (e >= rows * 16) break;
        int u, qq, g;
        const int64_t row = item_row(e, u, qq, g);
        f32x4_t x0, x1;
        lds_rows(qq, g, u, x0, x1);
        const float x[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
        u32x4_t o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
        if (a.fuse_local) {
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = fuse_bf16x2(o[i], lrow[k][i], wl[k]);
        }
        *reinterpret_cast<u32x4_t*>(a.out + row * 128 + 8 * u) = o;
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

// Lock tries before a tile is deferred (mrsa_set_routed_lock_spin_limit).
int g_spin_limit = kDefaultSpinLimit;

// Largest tile (<= 32 queries, <= 1024 items) whose LDS layout fits, 0 if none.
int pick_tile(int G, int K, int64_t Ck, bool token, bool keep, bool det) {
  for (int tq = std::min(kMaxTQ, kMaxItems / K); tq >= 4; tq -= 4) {
    const RaLayout l = ra_layout(tq, G, K, Ck, token, keep, det);
    if (l.total <= kLdsBytes && l.cap <= 65535) return tq;
  }
  return 0;
}

template <bool TOKEN, bool KEEP, bool ALIBI = false, bool EXT = false>
int launch_routed(RaArgs& a, hipStream_t s) {
  if (TOKEN && a.det) return MRSA_ERR_UNSUPPORTED;  // token scoring has no fixed-order walk
  const int tq = pick_tile(a.G, a.K, a.Ck, TOKEN, KEEP || EXT, a.det != 0);
  if (tq == 0) return MRSA_ERR_UNSUPPORTED;
  a.tq = tq;
  a.ntiles = (a.Lq + tq - 1) / tq;
  a.units = a.B * a.Hkv * a.parts * a.ntiles;
  const int64_t grid = (a.units + 7) / 8 * 8;
  if (grid > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  const RaLayout l = ra_layout(tq, a.G, a.K, a.Ck, TOKEN, KEEP || EXT, a.det != 0);
  a.spin_limit = g_spin_limit;
  // the fixed-order walk is its own instance, so the lock path carries none of its branches
  auto kern = a.det ? routed_attn_kernel<TOKEN, KEEP, !TOKEN && !EXT, ALIBI, EXT>
                     : routed_attn_kernel<TOKEN, KEEP, false, ALIBI, EXT>;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)l.total) != hipSuccess)
    return MRSA_ERR_LAUNCH;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kThreads), l.total, s, a);
  return mrsa_launch_status();
}

int check_common(const void* q, const void* kv_frags, const int32_t* indices, int64_t batch,
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
  // a KV head's fragments are addressed with 32-bit byte offsets
  if (kv_len / 64 >= 131072 || q_heads > 65535) return MRSA_ERR_UNSUPPORTED;
  if (batch > 0 && q_len > 0 && (!q || !kv_frags || !indices)) return MRSA_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)q | (uintptr_t)kv_frags) % 16 != 0) return MRSA_ERR_INVALID_ARGUMENT;
  return MRSA_OK;
}

RaArgs base_args(const void* q, const void* kv_frags, const void* weights,
                 const int32_t* indices, const uint8_t* key_valid, int64_t batch, int64_t q_len,
                 int64_t kv_len, int64_t q_heads, int64_t kv_heads, int64_t topk,
                 int mask_last_token, float sm_scale) {
  RaArgs a;
  a.q = (const uint16_t*)q;
  a.qf = nullptr;
  a.kvf = (const uint16_t*)kv_frags;
  a.w = (const uint16_t*)weights;
  a.idx = indices;
  a.key_valid = key_valid;
  a.keep = nullptr;
  a.B = batch;
  a.Lq = q_len;
  a.Lk = kv_len;
  a.Hq = (int)q_heads;
  a.Hkv = (int)kv_heads;
  a.G = (int)(q_heads / kv_heads);
  a.K = (int)topk;
  a.Ck = kv_len / 64;
  a.mask_last = mask_last_token;
  a.scale_log2 = sm_scale * kLog2e;
  a.sm_scale = sm_scale;
  a.out = nullptr;
  a.tscores = nullptr;
  a.parts = 1;
  a.partial = nullptr;
  a.fuse_local = nullptr;
  a.fuse_w = nullptr;
  a.tq = 0;
  a.ntiles = 0;
  a.units = 0;
  a.spin_limit = kDefaultSpinLimit;
  a.det = 0;
  a.slope = nullptr;
  a.ext_p = nullptr;
  a.ext_out = nullptr;
  return a;
}

// Routed attention with an optional walk split (parts > 1: fp32 partials in
// `partial`, summed into `out`), an optional token keep mask and an optional
// output fusion.
int selected_forward(const void* q, const void* kv_frags, const void* weights,
                     const int32_t* indices, const uint8_t* key_valid, const int8_t* keep,
                     int64_t batch, int64_t q_len, int64_t kv_len, int64_t q_heads,
                     int64_t kv_heads, int64_t head_dim, int64_t topk, int64_t chunk_size,
                     int mask_last_token, float sm_scale, int64_t parts, float* partial,
                     const void* fuse_local, const void* fuse_w, void* out, void* stream,
                     const void* q_frags = nullptr, int flags = 0, const float* slope = nullptr) {
  int st = check_common(q, kv_frags, indices, batch, q_len, kv_len, q_heads, kv_heads, head_dim,
                        topk, chunk_size, sm_scale);
  if (st != MRSA_OK) return st;
  if (parts < 1 || parts > kMaxParts) return MRSA_ERR_INVALID_ARGUMENT;
  if (batch * parts > 65535) return MRSA_ERR_UNSUPPORTED;
  if (batch == 0 || q_len == 0) return MRSA_OK;
  if (!weights || !out || (uintptr_t)out % 16 != 0) return MRSA_ERR_INVALID_ARGUMENT;
  if (parts > 1 && (!partial || (uintptr_t)partial % 16 != 0)) return MRSA_ERR_INVALID_ARGUMENT;
  if ((fuse_local == nullptr) != (fuse_w == nullptr)) return MRSA_ERR_INVALID_ARGUMENT;
  if (fuse_local && (uintptr_t)fuse_local % 16 != 0) return MRSA_ERR_INVALID_ARGUMENT;
  if (q_frags && (uintptr_t)q_frags % 16 != 0) return MRSA_ERR_INVALID_ARGUMENT;
  // Q fragments hold 2 KB per (query, KV head): 8 head columns of 128 dims
  if (q_frags && q_heads / kv_heads > 8) return MRSA_ERR_UNSUPPORTED;
  RaArgs a = base_args(q, kv_frags, weights, indices, key_valid, batch, q_len, kv_len, q_heads,
                       kv_heads, topk, mask_last_token, sm_scale);
  a.out = parts > 1 ? nullptr : (uint16_t*)out;
  a.parts = (int)parts;
  a.partial = parts > 1 ? partial : nullptr;
  a.keep = keep;
  a.fuse_local = parts > 1 ? nullptr : (const uint16_t*)fuse_local;
  a.fuse_w = parts > 1 ? nullptr : (const uint16_t*)fuse_w;
  a.qf = (const uint16_t*)q_frags;
  a.det = flags & MRSA_ROUTED_FIXED_ORDER;
  a.slope = slope;
  hipStream_t s = (hipStream_t)stream;
  if (slope)
    st = keep ? launch_routed<false, true, true>(a, s) : launch_routed<false, false, true>(a, s);
  else
    st = keep ? launch_routed<false, true>(a, s) : launch_routed<false, false>(a, s);
  if (st != MRSA_OK || parts == 1) return st;
  const int64_t n4 = batch * q_len * q_heads * 128 / 4;
  const int64_t blocks = std::min<int64_t>((n4 + 255) / 256, 4096);
  hipLaunchKernelGGL(sum_parts_kernel, dim3((unsigned)blocks), dim3(256), 0, s, partial,
                     (int)parts, n4, (uint16_t*)out, (const uint16_t*)fuse_local,
                     (const uint16_t*)fuse_w);
  return mrsa_launch_status();
}

}  // namespace

// The routed backward's dQ walk (EXT instance): dq += sum over each query's
// listed chunks (first occurrences) of dS . K, with the dS tiles read from
// the records the chunk-major backward kernel wrote; kv_frags_bwd =
// mrsa_kv_fragments(v, k), whose second half holds K^T.
int mrsa::routed_dq_walk(const void* kv_frags_bwd, const void* ds_records,
                         const int32_t* indices, const uint8_t* key_valid, int64_t batch,
                         int64_t q_len, int64_t kv_len, int64_t q_heads, int64_t kv_heads,
                         int64_t topk, float* grad_q, void* stream) {
  RaArgs a = base_args(ds_records, kv_frags_bwd, ds_records, indices, key_valid, batch, q_len,
                       kv_len, q_heads, kv_heads, topk, 1, 1.f);
  a.ext_p = (const uint16_t*)ds_records;
  a.ext_out = grad_q;
  return launch_routed<false, false, false, true>(a, (hipStream_t)stream);
}

extern "C" int mrsa_selected_attention_fwd(const void* q, const void* kv_frags,
                                           const void* weights, const int32_t* indices,
                                           const uint8_t* key_valid, int64_t batch,
                                           int64_t q_len, int64_t kv_len, int64_t q_heads,
                                           int64_t kv_heads, int64_t head_dim, int64_t topk,
                                           int64_t chunk_size, int mask_last_token,
                                           float sm_scale, void* out, void* stream) {
  return selected_forward(q, kv_frags, weights, indices, key_valid, nullptr, batch, q_len,
                          kv_len, q_heads, kv_heads, head_dim, topk, chunk_size, mask_last_token,
                          sm_scale, 1, nullptr, nullptr, nullptr, out, stream);
}

extern "C" int mrsa_candidate_token_scores_fwd(const void* q, const void* kv_frags,
                                               const int32_t* indices, const uint8_t* key_valid,
                                               int64_t batch, int64_t q_len, int64_t kv_len,
                                               int64_t q_heads, int64_t kv_heads,
                                               int64_t head_dim, int64_t topk,
                                               int64_t chunk_size, float sm_scale,
                                               float* scores, void* stream) {
  int st = check_common(q, kv_frags, indices, batch, q_len, kv_len, q_heads, kv_heads, head_dim,
                        topk, chunk_size, sm_scale);
  if (st != MRSA_OK) return st;
  if (batch == 0 || q_len == 0) return MRSA_OK;
  if (!scores || (uintptr_t)scores % 16 != 0) return MRSA_ERR_INVALID_ARGUMENT;
  hipStream_t s = (hipStream_t)stream;
  const int64_t n = batch * q_len * kv_heads * topk * chunk_size;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 8192);
  hipLaunchKernelGGL(fill_neg_inf, dim3((unsigned)blocks), dim3(256), 0, s, scores, n);
  st = mrsa_launch_status();
  if (st != MRSA_OK) return st;
  RaArgs a = base_args(q, kv_frags, nullptr, indices, key_valid, batch, q_len, kv_len, q_heads,
                       kv_heads, topk, 1, sm_scale);
  a.tscores = scores;
  return launch_routed<true, false>(a, s);
}

extern "C" int mrsa_selected_attention_split_fwd(
    const void* q, const void* kv_frags, const void* weights,
    const int32_t* indices, const uint8_t* key_valid, int64_t batch, int64_t q_len,
    int64_t kv_len, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t topk,
    int64_t chunk_size, int mask_last_token, float sm_scale, int64_t parts, float* partial,
    void* out, void* stream) {
  return selected_forward(q, kv_frags, weights, indices, key_valid, nullptr, batch, q_len,
                          kv_len, q_heads, kv_heads, head_dim, topk, chunk_size, mask_last_token,
                          sm_scale, parts, partial, nullptr, nullptr, out, stream);
}

extern "C" int mrsa_selected_attention_keep_fwd(
    const void* q, const void* kv_frags, const void* weights,
    const int32_t* indices, const uint8_t* key_valid, const int8_t* token_keep, int64_t batch,
    int64_t q_len, int64_t kv_len, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
    int64_t topk, int64_t chunk_size, int mask_last_token, float sm_scale, int64_t parts,
    float* partial, void* out, void* stream) {
  if (batch > 0 && q_len > 0 && !token_keep) return MRSA_ERR_INVALID_ARGUMENT;
  return selected_forward(q, kv_frags, weights, indices, key_valid, token_keep, batch, q_len,
                          kv_len, q_heads, kv_heads, head_dim, topk, chunk_size, mask_last_token,
                          sm_scale, parts, partial, nullptr, nullptr, out, stream);
}

extern "C" int mrsa_selected_attention_fused_fwd(
    const void* q, const void* kv_frags, const void* weights,
    const int32_t* indices, const uint8_t* key_valid, const int8_t* token_keep,
    const void* local_output, const void* local_weight, int64_t batch, int64_t q_len,
    int64_t kv_len, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t topk,
    int64_t chunk_size, int mask_last_token, float sm_scale, int64_t parts, float* partial,
    void* out, void* stream) {
  if (batch > 0 && q_len > 0 && (!local_output || !local_weight))
    return MRSA_ERR_INVALID_ARGUMENT;
  return selected_forward(q, kv_frags, weights, indices, key_valid, token_keep, batch, q_len,
                          kv_len, q_heads, kv_heads, head_dim, topk, chunk_size, mask_last_token,
                          sm_scale, parts, partial, local_output, local_weight, out, stream);
}

extern "C" int mrsa_set_routed_lock_spin_limit(int limit) {
  g_spin_limit = limit > 0 ? limit : 0;
  return MRSA_OK;
}

extern "C" int mrsa_selected_attention_fused_qf_fwd(
    const void* q, const void* q_frags, const void* kv_frags, const void* weights,
    const int32_t* indices, const uint8_t* key_valid, const int8_t* token_keep,
    const void* local_output, const void* local_weight, int64_t batch, int64_t q_len,
    int64_t kv_len, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t topk,
    int64_t chunk_size, int mask_last_token, float sm_scale, int64_t parts, float* partial,
    void* out, void* stream) {
  if (batch > 0 && q_len > 0 && (!local_output || !local_weight || !q_frags))
    return MRSA_ERR_INVALID_ARGUMENT;
  return selected_forward(q, kv_frags, weights, indices, key_valid, token_keep, batch, q_len,
                          kv_len, q_heads, kv_heads, head_dim, topk, chunk_size, mask_last_token,
                          sm_scale, parts, partial, local_output, local_weight, out, stream,
                          q_frags);
}

extern "C" int mrsa_selected_attention_ex_fwd(
    const void* q, const void* q_frags, const void* kv_frags, const void* weights,
    const int32_t* indices, const uint8_t* key_valid, const int8_t* token_keep,
    const void* local_output, const void* local_weight, int64_t batch, int64_t q_len,
    int64_t kv_len, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t topk,
    int64_t chunk_size, int mask_last_token, float sm_scale, int64_t parts, float* partial,
    int flags, void* out, void* stream) {
  if (flags & ~MRSA_ROUTED_FIXED_ORDER) return MRSA_ERR_INVALID_ARGUMENT;
  if (q_frags && batch > 0 && q_len > 0 && !local_output) return MRSA_ERR_INVALID_ARGUMENT;
  return selected_forward(q, kv_frags, weights, indices, key_valid, token_keep, batch, q_len,
                          kv_len, q_heads, kv_heads, head_dim, topk, chunk_size, mask_last_token,
                          sm_scale, parts, partial, local_output, local_weight, out, stream,
                          q_frags, flags);
}

extern "C" int mrsa_selected_attention_alibi_fwd(
    const void* q, const void* q_frags, const void* kv_frags, const void* weights,
    const int32_t* indices, const uint8_t* key_valid, const int8_t* token_keep,
    const void* local_output, const void* local_weight, const float* slope, int64_t batch,
    int64_t q_len, int64_t kv_len, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
    int64_t topk, int64_t chunk_size, int mask_last_token, float sm_scale, int64_t parts,
    float* partial, int flags, void* out, void* stream) {
  if (flags & ~MRSA_ROUTED_FIXED_ORDER) return MRSA_ERR_INVALID_ARGUMENT;
  if (batch > 0 && q_len > 0 && !slope) return MRSA_ERR_INVALID_ARGUMENT;
  if (q_frags && batch > 0 && q_len > 0 && !local_output) return MRSA_ERR_INVALID_ARGUMENT;
  return selected_forward(q, kv_frags, weights, indices, key_valid, token_keep, batch, q_len,
                          kv_len, q_heads, kv_heads, head_dim, topk, chunk_size, mask_last_token,
                          sm_scale, parts, partial, local_output, local_weight, out, stream,
                          q_frags, flags, slope);
}

// Reads the current device's count of routed-attention tiles whose bounded
// lock wait ran out (waits for the device's queued work first) and clears
// it when `reset` is nonzero.
extern "C" int mrsa_routed_lock_giveups(uint64_t* count, int reset) {
  if (!count) return MRSA_ERR_INVALID_ARGUMENT;
  if (hipDeviceSynchronize() != hipSuccess) return MRSA_ERR_LAUNCH;
  unsigned long long v = 0;
  if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_lock_giveups), sizeof(v), 0,
                          hipMemcpyDeviceToHost) != hipSuccess)
    return MRSA_ERR_LAUNCH;
  *count = (uint64_t)v;
  if (reset) {
    const unsigned long long z = 0;
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_lock_giveups), &z, sizeof(z), 0,
                          hipMemcpyHostToDevice) != hipSuccess)
      return MRSA_ERR_LAUNCH;
  }
  return MRSA_OK;
}
