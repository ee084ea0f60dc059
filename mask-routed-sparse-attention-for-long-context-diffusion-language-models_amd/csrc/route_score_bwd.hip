// Backward of the route scores.
//
// Forward (ops/topk_head_softmax.py:1055-1061, the recompute kernel): for
// query row l, KV head h, group head g and list slot k whose chunk
// c = idx[l, h, k] lies in [0, C):
//   score[l, h, g, k] = scale * q[l, h, g] . lmk[c, hl]
// with hl = h * G + g for per-head landmarks and hl = h for landmarks shared
// by the group.  The reference backward (:1074-1122) scatters the incoming
// gradient, multiplied by scale in the gradient's dtype, into a dense
// [L, C] matrix D per (h, g) and runs two batched products:
//   grad_q[l, h, g] = sum_c D[l, c] lmk[c, hl]
//   grad_lmk[c, hl] = sum_l D[l, c] q[l, h, g]   (also summed over g when
//                                                 the landmarks are shared)
// Slots whose chunk lies outside [0, C) contribute nothing.  A chunk listed
// twice in one list keeps one of its two gradients, as the reference's
// scatter_ does (the forward never lists a chunk twice).
//
// The dense matrix never reaches HBM.  A workgroup owns one landmark head
// (all group heads when the landmarks are shared) and a range of 32-row
// query tiles.  Per tile and group head it builds D (rows x chunks) and D^T
// in LDS from the tile's list slots, for a block of 256 chunks, and runs
// both products on the matrix cores:
//   grad_q^T   (dims x rows)   = lmk^T . D^T   (lmk^T of the block held in
//                                               registers, wave w: dims 16 w..)
//   grad_lmk^T (dims x chunks) += Q^T . D      (the tile's rows transposed
//                                               into LDS, wave w: chunks 32 w..)
// grad_lmk accumulates in registers over the workgroup's rows and is written
// as one fp32 part; route_score_bwd_finish sums the parts in a fixed order
// (the result does not depend on timing) and rounds to bf16.  Landmark rows
// beyond 256 chunks are handled block by block; grad_q then accumulates in
// an fp32 workspace that the finishing kernel rounds.
#include "mrsa_device.h"

using namespace mrsa;

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kTileQ = 32;
constexpr int kBlockC = 256;
constexpr int kDim = 128;
constexpr int kTargetUnits = 512;  // two rounds of the 256 CUs
constexpr int kPf = 4;             // prefetched list slots per thread (topk <= 64)

struct ScoreBwdArgs {
  const uint16_t* q;    // [B, L, Hkv, G, 128] bf16
  const uint16_t* lmk;  // [B, C, NL, 128] bf16, NL = Hkv * G (per head) or Hkv
  const int32_t* idx;   // [B, L, Hkv, K]
  const void* gs;       // [B, L, Hkv, G, K] bf16 or fp32
  int gs_fp32;
  int64_t B, L, C;
  int Hkv, G, K, NL, per_head;
  int parts, tiles_per_part, nblk;
  float scale;
  uint16_t* gq;         // [B, L, Hkv, G, 128] bf16 (one chunk block)
  float* gq32;          // same shape, fp32 (several chunk blocks)
  float* ws;            // [parts, B, NL, C, 128] fp32 parts of grad_lmk
};

// LDS (46 KB), all bf16:
//   D    [32 rows][256 chunks]: row l 512 B, 16-byte block b at b ^ (l & 15)
//   D^T  [256 chunks][32 rows]: row c 80 B (64 used)
//   Q^T  [128 dims][32 rows]:   row d 80 B (64 used)
// The swizzle and the 80-byte strides put the 16 rows of one matrix-operand
// read in 16 different 4-bank groups; Q^T is written two rows per 32-bit
// store, also without bank conflicts.
constexpr uint32_t kRow80 = 80;
constexpr uint32_t kDOff = 0;
constexpr uint32_t kDtOff = kTileQ * kBlockC * 2;
constexpr uint32_t kQtOff = kDtOff + kBlockC * kRow80;
constexpr uint32_t kSmemBytes = kQtOff + kDim * kRow80;

__device__ __forceinline__ uint32_t d_off(int l, int c) {
  return kDOff + l * 512 + ((((c >> 3) ^ (l & 15))) << 4) + (c & 7) * 2;
}
__device__ __forceinline__ uint32_t t80_off(uint32_t base, int r, int l) {
  return base + r * kRow80 + l * 2;
}

__global__ __launch_bounds__(kThreads, 1) void route_score_bwd_kernel(ScoreBwdArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[kSmemBytes];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int j = lane & 15;
  const int kg = lane >> 4;
  int64_t unit = blockIdx.x;
  const int part = (int)(unit % a.parts);
  unit /= a.parts;
  const int hl = (int)(unit % a.NL);
  const int64_t b = unit / a.NL;
  const int h = a.per_head ? hl / a.G : hl;
  const int g_lo = a.per_head ? hl % a.G : 0;
  const int g_hi = a.per_head ? g_lo + 1 : a.G;
  const int64_t ntiles = (a.L + kTileQ - 1) / kTileQ;
  const int64_t t0 = (int64_t)part * a.tiles_per_part;
  const int64_t t1 = t0 + a.tiles_per_part < ntiles ? t0 + a.tiles_per_part : ntiles;
  const int K = a.K;
  // This thread's list slots p = tid + kThreads * i of a tile: row sl, slot sk
  // (sl = kTileQ for none).
  int sl[kPf], sk[kPf];
#pragma unroll
  for (int i = 0; i < kPf; ++i) {
    const int p = tid + kThreads * i;
    sl[i] = p < kTileQ * K ? p / K : kTileQ;
    sk[i] = p < kTileQ * K ? p - (p / K) * K : 0;
  }

  for (int blk = 0; blk < a.nblk; ++blk) {
    const int64_t c0 = (int64_t)blk * kBlockC;
    // lmk^T operands of dims 16 w.. (A: rows = dims, reduction = chunks):
    // la[s] lane (j, kg) holds lmk[c0 + 32 s + 8 kg + e][hl][16 w + j].  The
    // block's landmark rows pass through LDS (natural [chunk][dim] order,
    // 128 chunks at a time, in the D / D^T region) with 16-byte loads.
    u32x4_t la[8];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      __syncthreads();  // the region is free (previous products / reads done)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int idx = tid + kThreads * i;
        const int r = idx >> 4;
        const int seg = idx & 15;
        const int64_t c = c0 + 128 * half + r;
        u32x4_t v = {0, 0, 0, 0};
        if (c < a.C)
          v = *reinterpret_cast<const u32x4_t*>(a.lmk + ((b * a.C + c) * a.NL + hl) * kDim +
                                                8 * seg);
        *reinterpret_cast<u32x4_t*>(smem + kDOff + r * 256 + seg * 16) = v;
      }
      __syncthreads();
#pragma unroll
      for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          const int c = 32 * s + 8 * kg + 2 * e2;
          const uint32_t lo = *reinterpret_cast<const uint16_t*>(smem + kDOff + c * 256 +
                                                                 (16 * w + j) * 2);
          const uint32_t hi = *reinterpret_cast<const uint16_t*>(smem + kDOff + (c + 1) * 256 +
                                                                 (16 * w + j) * 2);
          la[4 * half + s][e2] = lo | (hi << 16);
        }
      }
    }
    // The staging region becomes the D / D^T tiles: all zero to start.
    __syncthreads();
    for (uint32_t o = 16 * tid; o < kQtOff; o += 16 * kThreads)
      *reinterpret_cast<u32x4_t*>(smem + o) = u32x4_t{0, 0, 0, 0};
    f32x4_t acc[2][8];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[ct][dt] = zero4();

    // Items (tile, group head) in order; the next item's Q row segment and
    // list slots are loaded into registers while this item's products run.
    const int ng = g_hi - g_lo;
    const int64_t nitems = (t1 - t0) * ng;
    // Q rows of a tile: thread (rows 2 p, 2 p + 1, dims 4 m .. 4 m + 3) with
    // p = tid & 15, m = tid >> 4.
    u32x2_t qv0 = {0u, 0u}, qv1 = {0u, 0u};
    int32_t pc[kPf], pcp[kPf];
    float pg[kPf];
#pragma unroll
    for (int i = 0; i < kPf; ++i) pcp[i] = -1;
    auto fetch = [&](int64_t it) {
      const int64_t l0 = (t0 + it / ng) * kTileQ;
      const int g = g_lo + (int)(it % ng);
      const int64_t row = l0 + 2 * (tid & 15);
      const int64_t qoff = (((b * a.L + row) * a.Hkv + h) * a.G + g) * kDim + 4 * (tid >> 4);
      const int64_t qstep = (int64_t)a.Hkv * a.G * kDim;  // one row further
      qv0 = u32x2_t{0u, 0u};
      qv1 = u32x2_t{0u, 0u};
      if (row < a.L) qv0 = *reinterpret_cast<const u32x2_t*>(a.q + qoff);
      if (row + 1 < a.L) qv1 = *reinterpret_cast<const u32x2_t*>(a.q + qoff + qstep);
#pragma unroll
      for (int i = 0; i < kPf; ++i) {
        pc[i] = -1;
        pg[i] = 0.f;
        const int64_t r = l0 + sl[i];
        if (sl[i] < kTileQ && r < a.L) {
          pc[i] = a.idx[((b * a.L + r) * a.Hkv + h) * K + sk[i]];
          const int64_t gi = (((b * a.L + r) * a.Hkv + h) * a.G + g) * K + sk[i];
          pg[i] = a.gs_fp32 ? static_cast<const float*>(a.gs)[gi]
                            : bf16_to_f32(static_cast<const uint16_t*>(a.gs)[gi]);
        }
      }
    };
    if (nitems > 0) fetch(0);
    for (int64_t it = 0; it < nitems; ++it) {
      const int64_t l0 = (t0 + it / ng) * kTileQ;
      const int g = g_lo + (int)(it % ng);
      {
        __syncthreads();  // the previous products are done with the LDS tiles
        if (K <= kPf * kThreads / kTileQ) {
          // clear the previous item's entries (the tiles start at zero)
#pragma unroll
          for (int i = 0; i < kPf; ++i) {
            if (pcp[i] < 0) continue;
            *reinterpret_cast<uint16_t*>(smem + d_off(sl[i], pcp[i])) = 0;
            *reinterpret_cast<uint16_t*>(smem + t80_off(kDtOff, pcp[i], sl[i])) = 0;
          }
        } else {
          for (uint32_t o = 16 * tid; o < kQtOff; o += 16 * kThreads)
            *reinterpret_cast<u32x4_t*>(smem + o) = u32x4_t{0, 0, 0, 0};
        }
        {
          // Q^T: dims 4 m + e, rows 2 p and 2 p + 1 in one 32-bit store
          const int p2 = 2 * (tid & 15);
          const int m4 = 4 * (tid >> 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t lo = (qv0[e >> 1] >> (16 * (e & 1))) & 0xffffu;
            const uint32_t hi = (qv1[e >> 1] >> (16 * (e & 1))) & 0xffffu;
            *reinterpret_cast<uint32_t*>(smem + t80_off(kQtOff, m4 + e, p2)) = lo | (hi << 16);
          }
        }
        __syncthreads();  // zeros written before the scatter
        auto put = [&](int l, int64_t c, float gv) {
          if (c < c0 || c >= c0 + kBlockC || c >= a.C) return false;
          const uint16_t val = (uint16_t)f32_to_bf16(gv * a.scale);
          const int cr = (int)(c - c0);
          *reinterpret_cast<uint16_t*>(smem + d_off(l, cr)) = val;
          *reinterpret_cast<uint16_t*>(smem + t80_off(kDtOff, cr, l)) = val;
          return true;
        };
#pragma unroll
        for (int i = 0; i < kPf; ++i) {
          pcp[i] = -1;  // block-relative chunk written by this slot, for the clear
          if (pc[i] >= 0 && put(sl[i], pc[i], pg[i])) pcp[i] = (int)(pc[i] - c0);
        }
        // Lists longer than kPf * kThreads / kTileQ slots: the rest directly.
        for (int p = tid + kPf * kThreads; p < kTileQ * K; p += kThreads) {
          const int l = p / K;
          const int k = p - l * K;
          const int64_t row = l0 + l;
          if (row >= a.L) continue;
          const int64_t c = a.idx[((b * a.L + row) * a.Hkv + h) * K + k];
          const int64_t gi = (((b * a.L + row) * a.Hkv + h) * a.G + g) * K + k;
          put(l, c, a.gs_fp32 ? static_cast<const float*>(a.gs)[gi]
                              : bf16_to_f32(static_cast<const uint16_t*>(a.gs)[gi]));
        }
        __syncthreads();  // D, D^T and Q^T complete
        if (it + 1 < nitems) fetch(it + 1);

        // grad_q^T (dims 16 w.. x rows 16 lt..) = lmk^T . D^T; B operand lane
        // (j, kg) of step s: D[16 lt + j][32 s + 8 kg ..].
        f32x4_t gq[2] = {zero4(), zero4()};
#pragma unroll
        for (int s = 0; s < 8; ++s) {
#pragma unroll
          for (int lt = 0; lt < 2; ++lt) {
            const u32x4_t bo = *reinterpret_cast<const u32x4_t*>(
                smem + kDOff + (16 * lt + j) * 512 + (((4 * s + kg) ^ j) << 4));
            gq[lt] = mfma_bf16_16x16x32(la[s], bo, gq[lt]);
          }
          if (s % 2 == 1) __builtin_amdgcn_sched_barrier(0);
        }
        // grad_lmk^T (dims 16 dt.. x chunks 32 w + 16 ct..) += Q^T . D; A lane
        // (j, kg): Q^T[16 dt + j][8 kg ..], B lane (j, kg): D^T[c][8 kg ..].
        u32x4_t bo[2];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
          const int c = 32 * w + 16 * ct + j;
          bo[ct] = *reinterpret_cast<const u32x4_t*>(smem + kDtOff + c * kRow80 + 16 * kg);
        }
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const int d = 16 * dt + j;
          const u32x4_t qa = *reinterpret_cast<const u32x4_t*>(smem + kQtOff + d * kRow80 + 16 * kg);
          acc[0][dt] = mfma_bf16_16x16x32(qa, bo[0], acc[0][dt]);
          acc[1][dt] = mfma_bf16_16x16x32(qa, bo[1], acc[1][dt]);
          if (dt % 4 == 3) __builtin_amdgcn_sched_barrier(0);
        }
        // grad_q rows: lane (j, kg) holds dims 16 w + 4 kg .. +3 of row 16 lt + j.
#pragma unroll
        for (int lt = 0; lt < 2; ++lt) {
          const int64_t row = l0 + 16 * lt + j;
          if (row >= a.L) continue;
          const int64_t o = (((b * a.L + row) * a.Hkv + h) * a.G + g) * kDim + 16 * w + 4 * kg;
          if (a.nblk == 1) {
            u32x2_t pk;
            pk[0] = pack_bf16x2(gq[lt][0], gq[lt][1]);
            pk[1] = pack_bf16x2(gq[lt][2], gq[lt][3]);
            *reinterpret_cast<u32x2_t*>(a.gq + o) = pk;
          } else {
            f32x4_t* dst = reinterpret_cast<f32x4_t*>(a.gq32 + o);
            *dst = blk == 0 ? gq[lt] : *dst + gq[lt];
          }
        }
      }
    }
    // This part's grad_lmk rows: lane (j, kg) of tile (ct, dt) holds dims
    // 16 dt + 4 kg .. +3 of chunk c0 + 32 w + 16 ct + j.
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int64_t c = c0 + 32 * w + 16 * ct + j;
      if (c >= a.C) continue;
      float* dst = a.ws + ((((int64_t)part * a.B + b) * a.NL + hl) * a.C + c) * kDim + 4 * kg;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) *reinterpret_cast<f32x4_t*>(dst + 16 * dt) = acc[ct][dt];
    }
  }
}

// grad_lmk[b, c, hl, :] = bf16(sum over parts in order; zero for no parts) and, with several
// chunk blocks, grad_q = bf16(grad_q fp32).  One thread per 4 values.
__global__ __launch_bounds__(256) void route_score_bwd_finish(const float* ws, int parts,
                                                              int64_t B, int64_t C, int NL,
                                                              uint16_t* glmk, const float* gq32,
                                                              uint16_t* gq, int64_t nq4) {
  const int64_t nl4 = B * C * NL * (kDim / 4);
  const int64_t part_stride = B * NL * C * kDim;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nl4 + nq4;
       i += (int64_t)gridDim.x * blockDim.x) {
    f32x4_t v;
    uint16_t* dst;
    if (i < nl4) {
      const int d4 = (int)(i % (kDim / 4));
      int64_t r = i / (kDim / 4);
      const int hl = (int)(r % NL);
      r /= NL;
      const int64_t c = r % C;
      const int64_t b = r / C;
      const float* src = ws + ((b * NL + hl) * C + c) * kDim + 4 * d4;
      v = zero4();
      for (int p = 0; p < parts; ++p) v += *reinterpret_cast<const f32x4_t*>(src + p * part_stride);
      dst = glmk + 4 * i;
    } else {
      const int64_t k = i - nl4;
      v = *reinterpret_cast<const f32x4_t*>(gq32 + 4 * k);
      dst = gq + 4 * k;
    }
    u32x2_t pk;
    pk[0] = pack_bf16x2(v[0], v[1]);
    pk[1] = pack_bf16x2(v[2], v[3]);
    *reinterpret_cast<u32x2_t*>(dst) = pk;
  }
}

struct Plan {
  int parts, tiles_per_part, nblk;
  int64_t ws_lmk, ws_q;  // bytes
};

Plan make_plan(int64_t B, int64_t L, int64_t C, int64_t Hkv, int64_t G, int per_head) {
  Plan p;
  const int64_t NL = per_head ? Hkv * G : Hkv;
  const int64_t ntiles = (L + kTileQ - 1) / kTileQ;
  // One workgroup per CU: at most kTargetUnits so that a last, partly
  // filled round of workgroups does not cost a whole round.
  int64_t parts = kTargetUnits / (B * NL);
  if (parts > ntiles) parts = ntiles;
  if (parts < 1) parts = 1;
  const int64_t tpp = (ntiles + parts - 1) / parts;
  parts = (ntiles + tpp - 1) / tpp;
  p.parts = (int)parts;
  p.tiles_per_part = (int)tpp;
  p.nblk = (int)((C + kBlockC - 1) / kBlockC);
  p.ws_lmk = parts * B * NL * C * kDim * 4;
  p.ws_q = p.nblk > 1 ? B * L * Hkv * G * kDim * 4 : 0;
  return p;
}

bool shapes_ok(int64_t B, int64_t L, int64_t C, int64_t Hkv, int64_t G, int64_t D,
               int64_t K) {
  return B >= 0 && L >= 0 && C > 0 && Hkv > 0 && G > 0 && D > 0 && K > 0;
}

}  // namespace

extern "C" int64_t mrsa_route_score_bwd_workspace_bytes(int64_t batch, int64_t q_len,
                                                        int64_t num_chunks, int64_t kv_heads,
                                                        int64_t groups, int per_head_landmarks) {
  if (!shapes_ok(batch, q_len, num_chunks, kv_heads, groups, 1, 1)) return -1;
  if (batch == 0 || q_len == 0) return 0;
  const Plan p = make_plan(batch, q_len, num_chunks, kv_heads, groups, per_head_landmarks);
  return p.ws_lmk + p.ws_q;
}

extern "C" int mrsa_route_score_bwd(const void* q, const void* landmarks, const int32_t* indices,
                                    const void* grad_scores, int grad_scores_fp32, int64_t batch,
                                    int64_t q_len, int64_t num_chunks, int64_t kv_heads,
                                    int64_t groups, int64_t head_dim, int64_t topk,
                                    int per_head_landmarks, float sm_scale, void* grad_q,
                                    void* grad_landmarks, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
  if (!shapes_ok(batch, q_len, num_chunks, kv_heads, groups, head_dim, topk) ||
      !(sm_scale == sm_scale) || sm_scale == __builtin_inff() || sm_scale == -__builtin_inff())
    return MRSA_ERR_INVALID_ARGUMENT;
  if (head_dim != kDim) return MRSA_ERR_UNSUPPORTED;
  const int64_t NL = per_head_landmarks ? kv_heads * groups : kv_heads;
  if (topk > 4096 || NL > 0x7fffffff / 2 || num_chunks > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  if (!grad_landmarks) return MRSA_ERR_INVALID_ARGUMENT;
  if (batch == 0) return MRSA_OK;
  if (q_len == 0) {
    // No rows: the finishing kernel writes a zero landmark gradient.
    const int64_t total = batch * num_chunks * NL * (kDim / 4);
    int64_t blocks = (total + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(route_score_bwd_finish, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, (const float*)nullptr, 0, batch, num_chunks,
                       (int)NL, (uint16_t*)grad_landmarks, (const float*)nullptr,
                       (uint16_t*)nullptr, (int64_t)0);
    return mrsa_launch_status();
  }
  const Plan p = make_plan(batch, q_len, num_chunks, kv_heads, groups, per_head_landmarks);
  if (!q || !landmarks || !indices || !grad_scores || !grad_q || !workspace)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (workspace_bytes < p.ws_lmk + p.ws_q) return MRSA_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)q | (uintptr_t)grad_q | (uintptr_t)grad_landmarks | (uintptr_t)workspace) %
          16 != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  ScoreBwdArgs a;
  a.q = (const uint16_t*)q;
  a.lmk = (const uint16_t*)landmarks;
  a.idx = indices;
  a.gs = grad_scores;
  a.gs_fp32 = grad_scores_fp32 ? 1 : 0;
  a.B = batch;
  a.L = q_len;
  a.C = num_chunks;
  a.Hkv = (int)kv_heads;
  a.G = (int)groups;
  a.K = (int)topk;
  a.NL = (int)NL;
  a.per_head = per_head_landmarks ? 1 : 0;
  a.parts = p.parts;
  a.tiles_per_part = p.tiles_per_part;
  a.nblk = p.nblk;
  a.scale = sm_scale;
  a.gq = (uint16_t*)grad_q;
  a.ws = (float*)workspace;
  a.gq32 = p.ws_q ? (float*)((char*)workspace + p.ws_lmk) : nullptr;
  const int64_t units = batch * NL * p.parts;
  if (units > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(route_score_bwd_kernel, dim3((unsigned)units), dim3(kThreads), 0,
                     (hipStream_t)stream, a);
  int st = mrsa_launch_status();
  if (st != MRSA_OK) return st;
  const int64_t nq4 = p.ws_q ? batch * q_len * kv_heads * groups * (kDim / 4) : 0;
  const int64_t total = batch * num_chunks * NL * (kDim / 4) + nq4;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(route_score_bwd_finish, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, (const float*)workspace, p.parts, batch, num_chunks,
                     (int)NL, (uint16_t*)grad_landmarks, a.gq32, (uint16_t*)grad_q, nq4);
  return mrsa_launch_status();
}
