// Bidirectional sliding-window GQA attention (flash-attn window semantics).
//
// Work split: one workgroup of 8 waves per (batch, KV head, block of QB
// queries).  Each wave owns one column tile of 16 (query, head) columns: for
// G = 1, 2, 4, 8 that is 16 / G queries x G heads (QB = 8 (16 / G)); other
// group sizes pack the workgroup's 128 columns as (query c / G, head c % G),
// QB = floor(128 / G): 18 queries for G = 7, 2 padding columns instead of
// the 16 a power-of-two head count would leave.
// Q^T operands and O^T accumulators stay in registers.  A workgroup needs
// 128 VGPRs per lane and ~69 KB of LDS, so two workgroups share a CU and
// their barriers fall at different times.
//
// Key tiles of 64 arrive by buffer->LDS DMA in a ring of kRing 32 KB slots
// holding the tile's K / V fragments (mrsa_kv_fragments: the 32 matrix-core
// operand images of 1 KB, lane l's 16 bytes at 16 l), so every operand read
// is one 16-byte LDS read at the lane's slot address plus an immediate
// offset, free of bank conflicts; every wave issues 4 of a tile's 32 DMA
// instructions, with wave-uniform offsets.  One barrier per key tile,
// with no memory fence: each wave waits (vmcnt) for its own share of tile t,
// the barrier publishes the whole tile and frees the slot of tile t - 1,
// which then receives tile t + kRing - 1.  The inert-key words of all the
// block's key tiles are built once, before the first DMA.
//
// Matrix-core formulation (per 64-key tile and column tile):
//   S^T[key][col] = K_tile (A: 64 x 128) . Q^T (B: 128 x 16)   -> 16 MFMAs
//   softmax down each column, in the exp2 domain
//   O^T[d][col]  += V^T (A: 128 x 64) . P^T (B: 64 x 16)      -> 16 MFMAs
// P^T is fed to the second product straight from the accumulator registers
// of the first: lane l holds keys 16t + 4(l/16) + i of its column, and the
// fragments' V images number the reduction slots to match (the tiled order).
//
// Softmax with an anchored stabiliser.  On gfx950 ordinary VALU work does not
// overlap the matrix products of the same SIMD, so the per-tile VALU count
// sets the speed.  A column's stabiliser m (log2 units) is the exact max of
// its first tile with a visible key; later tiles take p = 2^(s c - m)
// directly -- no per-tile max, no rescale -- and each lane keeps a running
// sum of its own p (summed across the column's four lanes once, at the end).
// p is at most 2^kSumCap: a tile whose lane sum leaves [0, 2^kSumCap] (a logit
// far above m, or NaN) is recomputed on the exact path, which moves m to the
// tile's max and rescales the accumulators.  The sum never underflows: the
// anchor key itself contributes p = 1.  Mathematically this is the same
// softmax; the fp32 values differ from a per-tile running max only in
// rounding.
//
// Semantics (dream_dllm_hils/local_attention.py:35-107):
//   * key j is visible to a query at position p iff |p - j| <= window;
//   * inert keys (failed key_valid, or landmark slots when inert_chunk > 0)
//     carry zero K and V: logit exactly 0, no contribution to the output;
//   * P is rounded to bf16 before the PV product, the row sum uses fp32 P
//     (flash-attn's convention); out = O / l in bf16; lse = ln(sum exp(s)).
#include "chunk_tile.h"
#include "mrsa_device.h"

using namespace mrsa;

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kRing = 2;               // key-tile slots
constexpr int kBlocksPerCU = 2;        // 128 VGPRs, 2 x 69 KB LDS
constexpr int kDepth = 8;              // LDS operand reads in flight
constexpr int kSlotBytes = 32768;
constexpr float kSumCap = 64.f;        // log2 of the largest lane sum of p on the fast path
constexpr int kMaskTiles = 512;        // inert-key words kept in LDS per block

struct LocalArgs {
  const uint16_t* q;
  const uint16_t* kvf;        // [B, Hkv, NTk, 16384] K / V fragments
  const uint8_t* key_valid;
  const int64_t* qpos;
  int64_t B, Lq, Lk;
  int Hq, Hkv, G;
  int64_t W;
  int64_t inert_chunk;
  float scale_log2;
  int64_t NTk;
  uint16_t* out;
  float* lse;
  // Key split: `parts` workgroups share each query block, each taking an
  // equal share of its key tiles and writing unnormalised fp32 partials
  // part_o [parts][B][Lq][Hq][128] and (m, l) pairs part_ml [parts][B][Lq][Hq][2]
  // (m in log2 units) that local_merge_kernel combines.
  int parts;
  float* part_o;
  float* part_ml;
  // Optional by-product: the Q operand images of the routed attention,
  // [B, Hkv, Lq, 1024] bf16 (mrsa_q_fragments), written from the Q^T
  // registers every wave loads anyway.
  uint16_t* qf;
};

// Inert-key bits (bit s = key 64 kt + s carries zero K / V) of one key tile:
// keys in range that fail key_valid, and the landmark slots (positions j with
// (j + 1) % inert_chunk == 0) when inert_chunk > 0.  The key_valid bytes are
// read by the whole wave; the landmark slots come from one wave-uniform
// remainder per tile.
__device__ __forceinline__ uint64_t tile_inert_bits(const LocalArgs& a, int64_t b, int64_t kt) {
  const int lane = threadIdx.x & 63;
  const int64_t j0 = kt * 64;
  const int64_t j = j0 + lane;
  const bool bad = j < a.Lk && a.key_valid && a.key_valid[b * a.Lk + j] == 0;
  uint64_t m = __builtin_amdgcn_ballot_w64(bad);
  if (a.inert_chunk > 0) {
    const int64_t r = (j0 + 1) % a.inert_chunk;
    for (int64_t s = r == 0 ? 0 : a.inert_chunk - r; s < 64 && j0 + s < a.Lk; s += a.inert_chunk)
      m |= 1ull << s;
  }
  return m;
}

// Column layout.  GP = G = 1, 2, 4 or 8: each wave's 16 columns are 16 / G
// queries x G heads.  GP == 0 (packed, G = 3, 5, 6 or 7): the workgroup's
// 16 kWaves columns are numbered c = 16 wave + col and hold (query c / G,
// head c % G) of floor(16 kWaves / G) queries, so at most 16 kWaves mod G
// columns are padding (2 of 128 for G = 7, where 8 head columns per query
// would pad 16).
__host__ __device__ constexpr int queries_per_block(int GP, int G) {
  return GP > 0 ? kWaves * (16 / GP) : (16 * kWaves) / G;
}

template <int GP>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2 * kBlocksPerCU, 2 * kBlocksPerCU)))
local_attn_kernel(LocalArgs a) {
  constexpr bool kPacked = GP == 0;
  const int QB = queries_per_block(GP, a.G);  // queries per workgroup
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* ring = smem;                                              // kRing slots
  uint64_t* valid_tab = reinterpret_cast<uint64_t*>(smem + kRing * kSlotBytes);  // [kMaskTiles]
  int64_t* pos_range = reinterpret_cast<int64_t*>(valid_tab + kMaskTiles);      // [2]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  // XCD-aware order: workgroups are dealt to the 8 XCDs round-robin by
  // linear id; renumber so that each XCD runs a contiguous range of query
  // blocks of one head, whose key windows overlap in that XCD's L2.  With
  // total = 8 q + r workgroups, XCD x holds q + (x < r) of them and takes
  // the range starting at x q + min(x, r).
  const int64_t nx = gridDim.x, nyz = (int64_t)gridDim.y * gridDim.z;
  const int64_t total = nx * nyz;
  int64_t lin = blockIdx.x + nx * (blockIdx.y + (int64_t)gridDim.y * blockIdx.z);
  {
    const int64_t x = lin % 8, q8 = total / 8, r8 = total % 8;
    lin = x * q8 + min(x, r8) + lin / 8;
  }
  const int64_t qblock = lin % nx;
  const int h = (int)((lin / nx) % gridDim.y);
  const int64_t z = lin / (nx * gridDim.y);
  const int64_t b = z % a.B;
  const int part = (int)(z / a.B);
  const int64_t qb = qblock * QB;
  const int G = a.G;
  const int cw = 16 * wave + col;  // the column's number in the workgroup (packed layout)
  constexpr int GPd = kPacked ? 1 : GP;
  const int gg = kPacked ? cw % G : col % GPd;

  // Position range of the block's queries.
  if (wave == 0) {
    int64_t lo = INT64_MAX, hi = INT64_MIN;
    for (int i = lane; i < QB; i += 64) {
      if (qb + i < a.Lq) {
        const int64_t p = a.qpos ? a.qpos[qb + i] : qb + i;
        lo = min(lo, p);
        hi = max(hi, p);
      }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      lo = min(lo, (int64_t)__shfl_xor(lo, o, 64));
      hi = max(hi, (int64_t)__shfl_xor(hi, o, 64));
    }
    if (lane == 0) {
      pos_range[0] = lo;
      pos_range[1] = hi;
    }
  }

  // Q^T operands and position of this lane's column.
  u32x4_t Qb[4];
  const int64_t qi = kPacked ? qb + cw / G : qb + wave * (16 / GPd) + col / GPd;
  const bool colok = kPacked ? cw < QB * G : gg < G;  // not a padding column
  const bool qok = qi < a.Lq && colok;
  const int qp = qi < a.Lq ? (int)(a.qpos ? a.qpos[qi] : qi) : 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    u32x4_t z = {0u, 0u, 0u, 0u};
    Qb[j] = z;
    if (qok)
      Qb[j] = *reinterpret_cast<const u32x4_t*>(
          a.q + ((b * a.Lq + qi) * a.Hq + h * G + gg) * 128 + 32 * j + 8 * grp);
  }
  // Q fragments: lane (grp, col)'s k-step j image bytes of its column --
  // query qi, head gg -- sit at 512 j + 128 grp + 16 gg of the query's 2 KB
  // image; the query's columns also write zeros into head slots G..7.
  if (a.qf && part == 0 && qok) {
    uint16_t* dst = a.qf + ((b * a.Hkv + h) * a.Lq + qi) * 1024 + 64 * grp;
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4_t*>(dst + 8 * gg + 256 * j) = Qb[j];
    const u32x4_t zq = {0u, 0u, 0u, 0u};
    for (int zs = G + gg; zs < 8; zs += G)
#pragma unroll
      for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4_t*>(dst + 8 * zs + 256 * j) = zq;
  }
  __syncthreads();
  const int64_t plo = pos_range[0], phi = pos_range[1];
  int64_t kt0 = max(plo - a.W, (int64_t)0) / 64;
  int64_t kt1 = min(phi + a.W, a.Lk - 1) / 64;
  if (a.parts > 1) {
    const int64_t n = kt1 - kt0 + 1;
    const int64_t s0 = kt0 + n * part / a.parts;
    kt1 = kt0 + n * (part + 1) / a.parts - 1;
    kt0 = s0;
  }
  const int ntiles = (int)max(kt1 - kt0 + 1, (int64_t)0);
  const bool tab = ntiles <= kMaskTiles;

  // DMA of key tile kt into ring slot `slot`: this wave's 4 of the tile's
  // 32 operand images (image i at slot + 1024 i; lane l's 16 bytes at 16 l).
  // Tiles past kv_len hold zeros.
  const __amdgpu_buffer_rsrc_t frs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.kvf + (b * a.Hkv + h) * a.NTk * (int64_t)16384), (short)0,
      (int)(uint32_t)(a.NTk * 32768), 0x00020000);
  const uint32_t dma_lane = 16u * lane;
  auto issue_tile = [&](int64_t kt, int slot) {
    unsigned char* dst = ring + slot * kSlotBytes + (4 * wave) * 1024;
    const uint32_t src = (uint32_t)kt * 32768u + (uint32_t)(4 * wave) * 1024u;
    // (the immediate offset of a buffer->LDS load moves the LDS address too,
    // so the image offset goes into the scalar offset)
#pragma unroll
    for (int u = 0; u < 4; ++u)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(frs, (lds_void_t*)(dst + u * 1024), 16, dma_lane,
                                               src + 1024u * u, 0, 0);
  };
  // Inert-key words of the block's key tiles (when they fit the table),
  // before the first DMA: waiting for these loads must not wait for it.
  if (tab)
    for (int t = wave; t < ntiles; t += kWaves) {
      const uint64_t bits = tile_inert_bits(a, b, kt0 + t);
      if (lane == 0) lds_write_u64(lds_addr(&valid_tab[t]), bits);
    }
  // Q^T operands and the position complete here, before any DMA is in
  // flight: otherwise the compiler, tracking their loads into the loop,
  // waits for every outstanding load (the DMA prefetch included) at each
  // first use.
#pragma unroll
  for (int j = 0; j < 4; ++j) asm volatile("" : "+v"(Qb[j]));
  int qpv = qp;
  asm volatile("" : "+v"(qpv));
  for (int t = 0; t < kRing - 1 && t < ntiles; ++t) issue_tile(kt0 + t, t);

  f32x4_t acc[8];
#pragma unroll
  for (int td = 0; td < 8; ++td) acc[td] = zero4();
  // Stabiliser (log2 units) and this lane's running sum of p.  Absent
  // columns start anchored at 0: their logits are 0 or masked.
  float m_run = qok ? neg_inf() : 0.f;
  float l_lane = 0.f;
  bool anchored = __all(m_run != neg_inf());
  const float c = a.scale_log2;
  const float sum_cap = __builtin_ldexpf(1.f, (int)kSumCap);
  const int W32 = (int)min(a.W, (int64_t)1 << 30);  // |positions| < 2^30 (host check)
  const uint64_t kLast = 1ull << 63;

  for (int t = 0; t < ntiles; ++t) {
    // This wave's DMA of tile t has landed once at most the tiles issued
    // after it (up to kRing - 2 of them, 4 instructions each) are pending.
    const int later = max(0, min(kRing - 2, ntiles - 1 - t));
    if (later >= 2) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else if (later == 1) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // (first pass: the inert table)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (t + kRing - 1 < ntiles) issue_tile(kt0 + t + kRing - 1, (t + kRing - 1) % kRing);

    const int64_t kt = kt0 + t;
    const int64_t j0 = kt * 64;
    const uint32_t sbase = lds_addr(ring + (t % kRing) * kSlotBytes);
    // Keys of the tile before kv_len (kin) and inert keys (ibits: failed
    // key_valid or a landmark slot).
    const int64_t left = a.Lk - j0;
    const int kin = left >= 64 ? 64 : (int)left;
    const uint64_t ibits =
        uniform_u64(tab ? lds_read_u64(lds_addr(&valid_tab[t])) : tile_inert_bits(a, b, kt));
    // Tiles entirely inside every query's window need no position mask.
    const bool full = kin == 64 && (j0 >= phi - a.W) && (j0 + 63 <= plo + a.W);
    const uint32_t laddr = sbase + 16u * lane;  // this lane's 16 bytes of every image

    // Inert keys: lanes of group g hold keys 16 tt + 4 g + i.  The landmark
    // slot (key 63, lanes 48..63) is the usual only one; other inert keys
    // (failed key_valid) take the per-element path.  Values are patched in
    // place (no register copies at the joins).
    const uint64_t last_lanes = (ibits >> 63) ? 0xFFFF000000000000ull : 0ull;
    const bool other_inert = (ibits & ~kLast) != 0ull;
    auto inert_lanes = [&](int tt, int i) {
      uint64_t m = 0ull;
#pragma unroll
      for (int g = 0; g < 4; ++g)
        m |= ((ibits >> (16 * tt + 4 * g + i)) & 1ull) ? (0xFFFFull << (16 * g)) : 0ull;
      return m;
    };
    const float zero_v = 0.f;
    auto zero_inert = [&](f32x4_t (&X)[4]) {
      X[3][3] = set_where(X[3][3], last_lanes, zero_v);
      if (other_inert) {
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) X[tt][i] = set_where(X[tt][i], inert_lanes(tt, i), zero_v);
      }
    };
    // S^T of the column tile from the slot, inert keys 0 and invisible keys
    // -inf: keys outside the window, past kv_len or of an absent column.
    auto logits = [&](f32x4_t (&X)[4]) {
      qk_frag<kDepth>(laddr, Qb, X);
      zero_inert(X);
      if (!full) {
        // This lane's key 16 tt + i of its group (position j0 + 4 grp + 16 tt
        // + i) is visible iff 16 tt + i lies in [klo, khi]: inside the window
        // and before kv_len.  One unsigned compare per element: k - klo > span.
        const int rel = (int)j0 + 4 * grp - qpv;
        int klo = -W32 - rel;
        const int khi = min(W32 - rel, kin - 4 * grp - 1);
        if (!qok || khi < klo) klo = 64;  // nothing visible
        const uint32_t span = klo == 64 ? 0u : (uint32_t)(khi - klo);
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if ((uint32_t)(16 * tt + i - klo) > span) X[tt][i] = neg_inf();
      }
    };
    auto lane_sum = [&](const f32x4_t (&X)[4]) {
      return ((X[0][0] + X[0][1]) + (X[0][2] + X[0][3])) + ((X[1][0] + X[1][1]) + (X[1][2] + X[1][3])) +
             (((X[2][0] + X[2][1]) + (X[2][2] + X[2][3])) + ((X[3][0] + X[3][1]) + (X[3][2] + X[3][3])));
    };

    f32x4_t S[4];
    logits(S);
    bool exact = !anchored;
    if (anchored) {
      // fast path: p = 2^(s c - m), the lane sum checked against the cap
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) S[tt][i] = exp2_hw(__builtin_fmaf(S[tt][i], c, -m_run));
      const float ps = lane_sum(S);
      exact = !__all(ps <= sum_cap);
      if (!exact) l_lane += ps;
    }
    if (exact) {
      // exact path: the column max as the new stabiliser, accumulators and
      // sums rescaled (after a fast-path overflow, the tile's logits again)
      if (anchored) logits(S);
      const float mx = across4_max(max16_raw(S)) * c;
      const float m_new = fmaxf(m_run, mx);
      // A column with no visible key yet keeps m = -inf; exponentiate against
      // 0 there so that every term (and alpha) is exp2(-inf) = 0.
      const float m_use = m_new == neg_inf() ? 0.f : m_new;
      const float alpha = exp2_hw(m_run - m_use);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) S[tt][i] = exp2_hw(__builtin_fmaf(S[tt][i], c, -m_use));
      l_lane = l_lane * alpha + lane_sum(S);
      m_run = m_new;
      if (!__all(alpha == 1.f)) {
#pragma unroll
        for (int td = 0; td < 8; ++td) acc[td] *= alpha;
      }
      anchored = __all(m_run != neg_inf());
    }
    // Inert keys count in the denominator but carry zero V.
    zero_inert(S);
    u32x4_t Pb[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      Pb[jj][0] = pack_bf16x2(S[2 * jj][0], S[2 * jj][1]);
      Pb[jj][1] = pack_bf16x2(S[2 * jj][2], S[2 * jj][3]);
      Pb[jj][2] = pack_bf16x2(S[2 * jj + 1][0], S[2 * jj + 1][1]);
      Pb[jj][3] = pack_bf16x2(S[2 * jj + 1][2], S[2 * jj + 1][3]);
    }
    // O^T += V^T . P^T, kDepth reads in flight.  Product o (d rows
    // 16 (o & 7).., keys 32 (o >> 3)..) reads V image 2 (o & 7) + (o >> 3).
    // (The reads are issued on one path only: a value read by asm and
    // waited for later must not meet a second definition at a join, where
    // the compiler may copy its register before the data has landed.)
    u32x4_t vb[16];
    static_for<kDepth>([&](auto oc) {
      constexpr int o = decltype(oc)::value;
      vb[o] = lds_read_b128<16384 + (2 * (o & 7) + (o >> 3)) * 1024>(laddr);
    });
    static_for<16>([&](auto oc) {
      constexpr int o = decltype(oc)::value;
      lds_wait<(15 - o < kDepth - 1 ? 15 - o : kDepth - 1)>(vb[o]);
      acc[o & 7] = mfma_bf16_16x16x32(vb[o], Pb[o >> 3], acc[o & 7]);
      if constexpr (o + kDepth < 16)
        vb[o + kDepth] =
            lds_read_b128<16384 + (2 * ((o + kDepth) & 7) + ((o + kDepth) >> 3)) * 1024>(laddr);
      __builtin_amdgcn_sched_barrier(0);
    });
  }

  // The column's sum: its four lanes' running sums.
  const float l_run = across4_sum(l_lane);
  if (!qok) return;
  if (a.parts > 1) {
    const int64_t row = ((int64_t)part * a.B * a.Lq + b * a.Lq + qi) * a.Hq + h * G + gg;
    float* prow = a.part_o + row * 128;
#pragma unroll
    for (int td = 0; td < 8; ++td)
      *reinterpret_cast<f32x4_t*>(prow + 16 * td + 4 * grp) = acc[td];
    if (grp == 0) {
      a.part_ml[2 * row] = m_run;
      a.part_ml[2 * row + 1] = l_run;
    }
    return;
  }
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  uint16_t* orow = a.out + ((b * a.Lq + qi) * a.Hq + h * G + gg) * 128;
#pragma unroll
  for (int td = 0; td < 8; ++td) {
    u32x2_t o;
    o[0] = pack_bf16x2(acc[td][0] * inv, acc[td][1] * inv);
    o[1] = pack_bf16x2(acc[td][2] * inv, acc[td][3] * inv);
    *reinterpret_cast<u32x2_t*>(orow + 16 * td + 4 * grp) = o;
  }
  if (grp == 0)
    a.lse[(b * a.Lq + qi) * a.Hq + h * G + gg] =
        l_run > 0.f ? (m_run + log2f(l_run)) * kLn2 : neg_inf();
}

// Combines the key-split partials of one (query, head) row: with
// M = max_p m_p, O = sum_p o_p 2^(m_p - M) / sum_p l_p 2^(m_p - M), as the
// single-pass online softmax would have; lse = (M + log2 l) ln 2.
__global__ void __launch_bounds__(256) local_merge_kernel(LocalArgs a, int64_t rows) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // (row, 4-dim group)
  if (e >= rows * 32) return;
  const int64_t row = e >> 5;
  const int d4 = (int)(e & 31);
  float M = neg_inf();
  for (int p = 0; p < a.parts; ++p) M = fmaxf(M, a.part_ml[2 * (p * rows + row)]);
  const float Mu = M == neg_inf() ? 0.f : M;
  float l = 0.f;
  f32x4_t o = zero4();
  for (int p = 0; p < a.parts; ++p) {
    const int64_t pr = p * rows + row;
    const float w = exp2_hw(a.part_ml[2 * pr] - Mu);
    l += a.part_ml[2 * pr + 1] * w;
    const f32x4_t x = reinterpret_cast<const f32x4_t*>(a.part_o + pr * 128)[d4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] += x[i] * w;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  u32x2_t ob;
  ob[0] = pack_bf16x2(o[0] * inv, o[1] * inv);
  ob[1] = pack_bf16x2(o[2] * inv, o[3] * inv);
  reinterpret_cast<u32x2_t*>(a.out + row * 128)[d4] = ob;
  if (d4 == 0) a.lse[row] = l > 0.f ? (M + log2f(l)) * kLn2 : neg_inf();
}

template <int GP>
int launch_local(const LocalArgs& a, hipStream_t s) {
  const int QB = queries_per_block(GP, a.G);
  const size_t smem = (size_t)kRing * kSlotBytes + kMaskTiles * 8 + 16;
  auto kern = local_attn_kernel<GP>;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess)
    return MRSA_ERR_LAUNCH;
  dim3 grid((unsigned)((a.Lq + QB - 1) / QB), (unsigned)a.Hkv, (unsigned)(a.B * a.parts));
  hipLaunchKernelGGL(kern, grid, dim3(kThreads), smem, s, a);
  int st = mrsa_launch_status();
  if (st != MRSA_OK || a.parts == 1) return st;
  const int64_t rows = a.B * a.Lq * a.Hq;
  hipLaunchKernelGGL(local_merge_kernel, dim3((unsigned)((rows * 32 + 255) / 256)), dim3(256), 0,
                     s, a, rows);
  return mrsa_launch_status();
}

}  // namespace

namespace {

int local_attention(const void* q, const void* kv_frags, const uint8_t* key_valid,
                    const int64_t* query_positions, int64_t batch, int64_t q_len, int64_t kv_len,
                    int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t window,
                    int64_t inert_chunk, float sm_scale, int64_t parts, void* workspace,
                    void* out, float* lse, void* stream, void* q_frags = nullptr) {
  if (batch < 0 || q_len < 0 || kv_len < 0 || q_heads <= 0 || kv_heads <= 0 ||
      q_heads % kv_heads != 0 || head_dim <= 0 || window < 0 || inert_chunk < 0 ||
      !(sm_scale > 0.f) || sm_scale == __builtin_inff())
    return MRSA_ERR_INVALID_ARGUMENT;
  if (batch == 0 || q_len == 0) return MRSA_OK;
  if (kv_len == 0 || !q || !kv_frags || !out || !lse) return MRSA_ERR_INVALID_ARGUMENT;
  if (head_dim != 128) return MRSA_ERR_UNSUPPORTED;
  if (((uintptr_t)q | (uintptr_t)kv_frags | (uintptr_t)q_frags) % 16 != 0 ||
      (uintptr_t)out % 8 != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  // a KV head's fragments are addressed with 32-bit byte offsets
  if ((kv_len + 63) / 64 >= 131072) return MRSA_ERR_UNSUPPORTED;
  const int64_t G = q_heads / kv_heads;
  if (kv_heads > 65535 || batch > 65535) return MRSA_ERR_UNSUPPORTED;
  LocalArgs a;
  a.q = (const uint16_t*)q;
  a.kvf = (const uint16_t*)kv_frags;
  a.key_valid = key_valid;
  a.qpos = query_positions;
  a.B = batch;
  a.Lq = q_len;
  a.Lk = kv_len;
  a.Hq = (int)q_heads;
  a.Hkv = (int)kv_heads;
  a.G = (int)G;
  a.W = window;
  a.inert_chunk = inert_chunk;
  a.scale_log2 = sm_scale * kLog2e;
  a.NTk = (kv_len + 63) / 64;
  a.out = (uint16_t*)out;
  a.lse = lse;
  a.parts = (int)parts;
  a.part_o = (float*)workspace;
  a.part_ml = parts > 1 ? (float*)workspace + parts * batch * q_len * q_heads * 128 : nullptr;
  a.qf = (uint16_t*)q_frags;
  if (q_frags && G > 8) return MRSA_ERR_UNSUPPORTED;
  hipStream_t s = (hipStream_t)stream;
  switch (G) {
    case 1: return launch_local<1>(a, s);
    case 2: return launch_local<2>(a, s);
    case 4: return launch_local<4>(a, s);
    case 8: return launch_local<8>(a, s);
    case 3:
    case 5:
    case 6:
    case 7: return launch_local<0>(a, s);
    default: return MRSA_ERR_UNSUPPORTED;
  }
}

}  // namespace

extern "C" int mrsa_local_attention_fwd(const void* q, const void* kv_frags,
                                        const uint8_t* key_valid, const int64_t* query_positions,
                                        int64_t batch, int64_t q_len, int64_t kv_len,
                                        int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                        int64_t window, int64_t inert_chunk, float sm_scale,
                                        void* out, float* lse, void* stream) {
  return local_attention(q, kv_frags, key_valid, query_positions, batch, q_len, kv_len,
                         q_heads, kv_heads, head_dim, window, inert_chunk, sm_scale, 1, nullptr,
                         out, lse, stream);
}

extern "C" int64_t mrsa_local_attention_workspace_bytes(int64_t batch, int64_t q_len,
                                                        int64_t q_heads, int64_t parts) {
  if (batch < 0 || q_len < 0 || q_heads < 0 || parts < 1) return -1;
  return parts > 1 ? parts * batch * q_len * q_heads * 130 * 4 : 0;
}

extern "C" int mrsa_local_attention_split_fwd(const void* q, const void* kv_frags,
                                              const uint8_t* key_valid,
                                              const int64_t* query_positions, int64_t batch,
                                              int64_t q_len, int64_t kv_len, int64_t q_heads,
                                              int64_t kv_heads, int64_t head_dim, int64_t window,
                                              int64_t inert_chunk, float sm_scale, int64_t parts,
                                              void* workspace, int64_t workspace_bytes, void* out,
                                              float* lse, void* stream) {
  if (parts < 1 || parts > 64) return MRSA_ERR_INVALID_ARGUMENT;
  if (parts > 1) {
    if (!workspace || (uintptr_t)workspace % 16 != 0 ||
        workspace_bytes < mrsa_local_attention_workspace_bytes(batch, q_len, q_heads, parts))
      return MRSA_ERR_INVALID_ARGUMENT;
    if (batch * parts > 65535) return MRSA_ERR_UNSUPPORTED;
  }
  return local_attention(q, kv_frags, key_valid, query_positions, batch, q_len, kv_len,
                         q_heads, kv_heads, head_dim, window, inert_chunk, sm_scale, parts,
                         parts > 1 ? workspace : nullptr, out, lse, stream);
}

extern "C" int mrsa_local_attention_qf_fwd(const void* q, const void* kv_frags,
                                           const uint8_t* key_valid,
                                           const int64_t* query_positions, int64_t batch,
                                           int64_t q_len, int64_t kv_len, int64_t q_heads,
                                           int64_t kv_heads, int64_t head_dim, int64_t window,
                                           int64_t inert_chunk, float sm_scale, void* q_frags,
                                           void* out, float* lse, void* stream) {
  if (batch > 0 && q_len > 0 && !q_frags) return MRSA_ERR_INVALID_ARGUMENT;
  return local_attention(q, kv_frags, key_valid, query_positions, batch, q_len, kv_len,
                         q_heads, kv_heads, head_dim, window, inert_chunk, sm_scale, 1, nullptr,
                         out, lse, stream, q_frags);
}
