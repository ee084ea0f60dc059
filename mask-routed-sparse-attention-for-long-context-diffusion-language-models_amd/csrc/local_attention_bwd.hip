// Backward of the bidirectional window attention (the gradient flash-attn's
// flash_attn_func gives dream_dllm_hils/local_attention.py:67-107; the
// forward is local_attention.hip).
//
// With k' = k m, v' = v m (m = 0 for inert keys: failed key_valid, landmark
// slots), s = q . k' * scale over the window |i - j| <= W, P = exp(s - lse)
// (lse saved by the forward) and D_i = sum_d dO_i O_i:
//   dV'_j = sum_i P_ij dO_i,  dP_ij = dO_i . v'_j,  dS_ij = P_ij (dP_ij - D_i),
//   dQ_i = scale sum_j dS_ij k'_j,  dK'_j = scale sum_i dS_ij q_i,
// and dk = dK' m, dv = dV' m.  The LSE output carries no gradient (flash-attn's
// autograd drops it).  Rounding points as flash-attn's: P and dS are rounded
// to bf16 as matrix operands, every sum is fp32.
//
// Both passes are one kernel template with the forward's structure: 16
// matrix columns per wave in registers, 64-row tiles of fragment images
// streamed through a 2-slot LDS ring by buffer->LDS DMA, one barrier per tile.
// A slot holds two fragment tiles (mrsa_kv_fragments layout, 32 KB each):
//   [A: rows x dims images | A': dims x rows images (tiled order)]
//   [B: rows x dims images | B': dims x rows images (tiled order)]
//   per tile:  S^T  = A . X1^T,  dP^T = B . X2^T          (32 products)
//              acc4 += B' . dS^T  (and acc3 += A' . P^T)  (16 or 32 products)
//  dQ pass   (columns: (query, head); rows: keys):
//     A = K, B = V, B' = K^T, X1 = Q, X2 = dO  ->  acc4 = dQ / scale
//  dK/dV pass (columns: keys; rows: (query, head) pairs, row = query G + head):
//     A = Q, A' = dO^T, B = dO, B' = Q^T, X1 = K, X2 = V
//     ->  acc3 = dV, acc4 = dK / scale
// The dQ pass also writes each (query, head) row's lse (log2 units) and D in
// row order for the dK/dV pass.  The row images of Q and dO come from
// row_fragments_kernel, which lays out any [B, L, Hkv * G, 128] tensor as a
// [B, Hkv, L * G] row sequence in the kv_fragments format.
#include "chunk_tile.h"
#include "mrsa_device.h"

#include <algorithm>

using namespace mrsa;

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kRing = 2;
constexpr int kSlotBytes = 65536;     // two fragment tiles
constexpr int kTileBytes = 32768;
constexpr int kFragElems = 16384;
constexpr int kFragPitch = 136;       // LDS row pitch of the layout kernel (elements)
constexpr int kMaskTiles = 512;       // inert-key words of the dQ pass kept in LDS

// Row r of tile c of (b, h): element ((b L + r / G) Hq + h G + r % G) 128 of
// x / y (G = 1, Hq = Hkv for key rows); rows >= nrows are zero.  Output as
// mrsa_kv_fragments: x's rows x dims images, then y's dims x rows images.
__global__ void __launch_bounds__(256)
    row_fragments_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ y,
                         int64_t L, int Hq, int Hkv, int G, int64_t NT,
                         uint16_t* __restrict__ frags) {
  __shared__ __align__(16) uint16_t xs[64 * kFragPitch];
  __shared__ __align__(16) uint16_t ys[64 * kFragPitch];
  const int64_t c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int64_t nrows = L * G;
  for (int p = tid; p < 1024; p += 256) {
    const int r = p >> 4, u = p & 15;
    const int64_t s = c * 64 + r;
    u32x4_t xv = {0u, 0u, 0u, 0u}, yv = {0u, 0u, 0u, 0u};
    if (s < nrows) {
      const int64_t i = s / G, g = s - i * G;
      const int64_t off = ((b * L + i) * Hq + h * G + g) * 128 + 8 * u;
      xv = *reinterpret_cast<const u32x4_t*>(x + off);
      yv = *reinterpret_cast<const u32x4_t*>(y + off);
    }
    *reinterpret_cast<u32x4_t*>(xs + r * kFragPitch + 8 * u) = xv;
    *reinterpret_cast<u32x4_t*>(ys + r * kFragPitch + 8 * u) = yv;
  }
  __syncthreads();
  uint16_t* dst = frags + ((b * Hkv + h) * NT + c) * (int64_t)kFragElems;
  for (int p = tid; p < 1024; p += 256) {
    const int i = p >> 6, l = p & 63, j = l & 15, grp = l >> 4;
    const int mt = i >> 2, kq = i & 3;
    *reinterpret_cast<u32x4_t*>(dst + 8 * p) =
        *reinterpret_cast<const u32x4_t*>(xs + (16 * mt + j) * kFragPitch + 32 * kq + 8 * grp);
    const int nt = i >> 1, kv = i & 1, d = 16 * nt + j;
    u32x4_t yv;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int r0 = 32 * kv + 16 * (w >> 1) + 4 * grp + 2 * (w & 1);
      yv[w] = (uint32_t)ys[r0 * kFragPitch + d] | ((uint32_t)ys[(r0 + 1) * kFragPitch + d] << 16);
    }
    *reinterpret_cast<u32x4_t*>(dst + 8192 + 8 * p) = yv;
  }
}

struct BwdArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* out;
  const uint16_t* dout;
  const float* lse;           // [B, L, Hq] natural log
  const uint8_t* key_valid;
  const uint16_t* fa;         // per pass: the A | A' fragment sequence
  const uint16_t* fb;         // per pass: the B | B' fragment sequence
  int64_t B, L;
  int Hq, Hkv, G;
  int64_t W;
  int64_t inert_chunk;
  float scale, scale_log2;
  float* lse_rows;            // [B, Hkv, L G] log2 units (written by the dQ pass)
  float* d_rows;              // [B, Hkv, L G]
  float* dq;                  // [B, L, Hq, 128] fp32
  float* dk;                  // [B, L, Hkv, 128] fp32
  float* dv;
};

// Inert-key bits of key tile kt (bit s = key 64 kt + s): failed key_valid and
// the landmark slots ((j + 1) % inert_chunk == 0).
__device__ __forceinline__ uint64_t inert_bits(const BwdArgs& a, int64_t b, int64_t kt) {
  const int lane = threadIdx.x & 63;
  const int64_t j0 = kt * 64;
  const int64_t j = j0 + lane;
  const bool bad = j < a.L && a.key_valid && a.key_valid[b * a.L + j] == 0;
  uint64_t m = __builtin_amdgcn_ballot_w64(bad);
  if (a.inert_chunk > 0) {
    const int64_t r = (j0 + 1) % a.inert_chunk;
    for (int64_t s = r == 0 ? 0 : a.inert_chunk - r; s < 64 && j0 + s < a.L; s += a.inert_chunk)
      m |= 1ull << s;
  }
  return m;
}

__device__ __forceinline__ bool key_inert(const BwdArgs& a, int64_t b, int64_t j) {
  if (a.key_valid && a.key_valid[b * a.L + j] == 0) return true;
  return a.inert_chunk > 0 && (j + 1) % a.inert_chunk == 0;
}

// The 16 S^T accumulator values of a lane packed as the B operand of a
// dims x rows product (reduction index 8 grp + e of step ks = row 32 ks + 16
// (e >> 2) + 4 grp + (e & 3), the tiled order of the fragments).
__device__ __forceinline__ void pack_rows(const f32x4_t (&X)[4], u32x4_t (&Xb)[2]) {
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    Xb[jj][0] = pack_bf16x2(X[2 * jj][0], X[2 * jj][1]);
    Xb[jj][1] = pack_bf16x2(X[2 * jj][2], X[2 * jj][3]);
    Xb[jj][2] = pack_bf16x2(X[2 * jj + 1][0], X[2 * jj + 1][1]);
    Xb[jj][3] = pack_bf16x2(X[2 * jj + 1][2], X[2 * jj + 1][3]);
  }
}

// acc += (dims x rows images at laddr + OFF) . Xb
template <int OFF>
__device__ __forceinline__ void dims_rows_product(uint32_t laddr, const u32x4_t (&Xb)[2],
                                                  f32x4_t (&acc)[8]) {
  constexpr int kD = 8;
  u32x4_t vb[16];
  static_for<kD>([&](auto oc) {
    constexpr int o = decltype(oc)::value;
    vb[o] = lds_read_b128<OFF + (2 * (o & 7) + (o >> 3)) * 1024>(laddr);
  });
  static_for<16>([&](auto oc) {
    constexpr int o = decltype(oc)::value;
    lds_wait<(15 - o < kD - 1 ? 15 - o : kD - 1)>(vb[o]);
    acc[o & 7] = mfma_bf16_16x16x32(vb[o], Xb[o >> 3], acc[o & 7]);
    if constexpr (o + kD < 16)
      vb[o + kD] = lds_read_b128<OFF + (2 * ((o + kD) & 7) + ((o + kD) >> 3)) * 1024>(laddr);
    __builtin_amdgcn_sched_barrier(0);
  });
}

template <bool DKV>
__global__ void __launch_bounds__(kThreads, 1) local_bwd_kernel(BwdArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* ring = smem;
  uint64_t* inert_tab = reinterpret_cast<uint64_t*>(smem + kRing * kSlotBytes);  // [kMaskTiles]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  // XCD-aware order (as the forward): XCD x takes a contiguous range.
  const int64_t nx = gridDim.x, nyz = (int64_t)gridDim.y * gridDim.z;
  const int64_t total = nx * nyz;
  int64_t lin = blockIdx.x + nx * (blockIdx.y + (int64_t)gridDim.y * blockIdx.z);
  {
    const int64_t x = lin % 8, q8 = total / 8, r8 = total % 8;
    lin = x * q8 + min(x, r8) + lin / 8;
  }
  const int64_t blk = lin % nx;
  const int h = (int)((lin / nx) % gridDim.y);
  const int64_t b = lin / (nx * gridDim.y);
  const int G = a.G, Hq = a.Hq;
  const int64_t L = a.L, W = a.W;
  const int cw = 16 * wave + col;

  // ---- this lane's column: operands, per-column values, visible row range
  u32x4_t X1[4], X2[4];
  bool cok;
  int64_t rlo, rhi;           // visible rows [rlo, rhi] (tile-row units)
  float lse2_c = 0.f, d_c = 0.f;
  int64_t nrows;              // rows of the streamed sequence
  int64_t cq = 0, cj = 0;
  int cg = 0;
  if constexpr (!DKV) {
    const int QB = 128 / G;
    cq = blk * QB + cw / G;
    cg = cw % G;
    cok = cw < QB * G && cq < L;
    nrows = L;
    rlo = max(cq - W, (int64_t)0);
    rhi = min(cq + W, L - 1);
    const int64_t row = ((b * L + cq) * Hq + (int64_t)h * G + cg) * 128;
    float dsum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4_t z = {0u, 0u, 0u, 0u};
      X1[j] = z;
      X2[j] = z;
      u32x4_t o = z;
      if (cok) {
        X1[j] = *reinterpret_cast<const u32x4_t*>(a.q + row + 32 * j + 8 * grp);
        X2[j] = *reinterpret_cast<const u32x4_t*>(a.dout + row + 32 * j + 8 * grp);
        o = *reinterpret_cast<const u32x4_t*>(a.out + row + 32 * j + 8 * grp);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
        dsum += bf16_lo(X2[j][e]) * bf16_lo(o[e]) + bf16_hi(X2[j][e]) * bf16_hi(o[e]);
    }
    d_c = across4_sum(dsum);
    const float lse = cok ? a.lse[(b * L + cq) * Hq + (int64_t)h * G + cg] : 0.f;
    lse2_c = lse * kLog2e;
    if (cok && grp == 0) {
      const int64_t ridx = (b * a.Hkv + h) * (L * G) + cq * G + cg;
      a.lse_rows[ridx] = lse2_c;
      a.d_rows[ridx] = d_c;
    }
  } else {
    cj = blk * 128 + cw;
    cok = cj < L;
    nrows = L * G;
    rlo = G * max(cj - W, (int64_t)0);
    rhi = G * min(cj + W, L - 1) + G - 1;
    const int64_t row = ((b * L + (cok ? cj : 0)) * a.Hkv + h) * 128;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4_t z = {0u, 0u, 0u, 0u};
      X1[j] = z;
      X2[j] = z;
      if (cok) {
        X1[j] = *reinterpret_cast<const u32x4_t*>(a.k + row + 32 * j + 8 * grp);
        X2[j] = *reinterpret_cast<const u32x4_t*>(a.v + row + 32 * j + 8 * grp);
      }
    }
  }
  if (!cok) {
    rlo = 1;  // nothing visible
    rhi = 0;
  }

  // ---- the workgroup's row tiles: the union of its columns' windows
  int64_t lo_all, hi_all;
  if constexpr (!DKV) {
    const int QB = 128 / G;
    const int64_t q0 = blk * QB, q1 = min(q0 + QB, L) - 1;
    lo_all = max(q0 - W, (int64_t)0);
    hi_all = min(q1 + W, L - 1);
  } else {
    const int64_t j0 = blk * 128, j1 = min(j0 + 128, L) - 1;
    lo_all = G * max(j0 - W, (int64_t)0);
    hi_all = G * min(j1 + W, L - 1) + G - 1;
  }
  const int64_t t0 = lo_all / 64, t1 = hi_all / 64;
  const int ntiles = (int)max(t1 - t0 + 1, (int64_t)0);
  const int64_t NT = (nrows + 63) / 64;
  const bool tab = !DKV && ntiles <= kMaskTiles;

  const __amdgpu_buffer_rsrc_t ras = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.fa + (b * a.Hkv + h) * NT * (int64_t)kFragElems), (short)0,
      (int)(uint32_t)(NT * kTileBytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t rbs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.fb + (b * a.Hkv + h) * NT * (int64_t)kFragElems), (short)0,
      (int)(uint32_t)(NT * kTileBytes), 0x00020000);
  const uint32_t dma_lane = 16u * lane;
  // Tile t into slot s: each wave 4 images of A|A' and 4 of B|B' (the dQ
  // pass reads no A', the images of waves 4..7).
  auto issue_tile = [&](int64_t t, int s) {
    unsigned char* da = ring + s * kSlotBytes + (4 * wave) * 1024;
    unsigned char* db = da + kTileBytes;
    const uint32_t src = (uint32_t)t * (uint32_t)kTileBytes + (uint32_t)(4 * wave) * 1024u;
    if (DKV || wave < 4) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ras, (lds_void_t*)(da + u * 1024), 16, dma_lane,
                                                 src + 1024u * u, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rbs, (lds_void_t*)(db + u * 1024), 16, dma_lane,
                                               src + 1024u * u, 0, 0);
  };
  if constexpr (!DKV) {
    if (tab)
      for (int t = wave; t < ntiles; t += kWaves) {
        const uint64_t bits = inert_bits(a, b, t0 + t);
        if (lane == 0) lds_write_u64(lds_addr(&inert_tab[t]), bits);
      }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    asm volatile("" : "+v"(X1[j]));
    asm volatile("" : "+v"(X2[j]));
  }
  if (ntiles > 0) issue_tile(t0, 0);

  f32x4_t acc3[8], acc4[8];
#pragma unroll
  for (int td = 0; td < 8; ++td) {
    acc3[td] = zero4();
    acc4[td] = zero4();
  }
  const float c = a.scale_log2;

  for (int t = 0; t < ntiles; ++t) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const int64_t r0 = (t0 + t) * 64;
    // per-row values of the dK/dV pass (row-ordered lse and D, clamped
    // rows), issued before the next tile's DMA so that their wait does not
    // wait for it
    float lse2_r[4][4], d_r[4][4];
    if constexpr (DKV) {
      const int64_t rb = (b * a.Hkv + h) * nrows;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t rr = min(r0 + 16 * mt + 4 * grp + r, nrows - 1);
          lse2_r[mt][r] = a.lse_rows[rb + rr];
          d_r[mt][r] = a.d_rows[rb + rr];
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (t + 1 < ntiles) issue_tile(t0 + t + 1, (t + 1) % kRing);
    const uint32_t sbase = lds_addr(ring + (t % kRing) * kSlotBytes);
    const uint32_t laddr = sbase + 16u * lane;
    uint64_t inert = 0ull;
    if constexpr (!DKV) inert = uniform_u64(tab ? lds_read_u64(lds_addr(&inert_tab[t]))
                                                : inert_bits(a, b, t0 + t));

    f32x4_t S[4], dP[4];
    qk_frag<8>(laddr, X1, S);
    qk_frag<8>(laddr + kTileBytes, X2, dP);

    // P and dS of the visible rows: row r0 + 16 mt + 4 grp + r lies in
    // [rlo, rhi] (one unsigned compare); the dQ pass drops inert key rows
    // from dS (their k' = 0 adds nothing to dQ).
    const int64_t rel = r0 + 4 * grp - rlo;
    const uint64_t span = (uint64_t)(rhi - rlo);
    const uint64_t msh = inert >> (4 * grp);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool vis = rhi >= rlo && (uint64_t)(rel + 16 * mt + r) <= span;
        const float l2 = DKV ? lse2_r[mt][r] : lse2_c;
        const float dd = DKV ? d_r[mt][r] : d_c;
        const float p = vis ? exp2_hw(__builtin_fmaf(S[mt][r], c, -l2)) : 0.f;
        const bool ds_ok = vis && (DKV || !((msh >> (16 * mt + r)) & 1ull));
        S[mt][r] = p;
        dP[mt][r] = ds_ok ? p * (dP[mt][r] - dd) : 0.f;
      }
    u32x4_t Sb[2];
    pack_rows(dP, Sb);
    dims_rows_product<kTileBytes + 16384>(laddr, Sb, acc4);
    if constexpr (DKV) {
      u32x4_t Pb[2];
      pack_rows(S, Pb);
      dims_rows_product<16384>(laddr, Pb, acc3);
    }
  }

  // ---- outputs (fp32): the lane holds dims 16 td + 4 grp .. + 3 of its column
  if (!cok) return;
  if constexpr (!DKV) {
    float* dst = a.dq + ((b * L + cq) * Hq + (int64_t)h * G + cg) * 128;
#pragma unroll
    for (int td = 0; td < 8; ++td) {
      f32x4_t o = acc4[td];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] *= a.scale;
      *reinterpret_cast<f32x4_t*>(dst + 16 * td + 4 * grp) = o;
    }
  } else {
    const bool dead = key_inert(a, b, cj);  // dk = dK' m, dv = dV' m
    float* dk = a.dk + ((b * L + cj) * a.Hkv + h) * 128;
    float* dv = a.dv + ((b * L + cj) * a.Hkv + h) * 128;
#pragma unroll
    for (int td = 0; td < 8; ++td) {
      f32x4_t ok = acc4[td], ov = acc3[td];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        ok[e] = dead ? 0.f : ok[e] * a.scale;
        ov[e] = dead ? 0.f : ov[e];
      }
      *reinterpret_cast<f32x4_t*>(dk + 16 * td + 4 * grp) = ok;
      *reinterpret_cast<f32x4_t*>(dv + 16 * td + 4 * grp) = ov;
    }
  }
}

struct BwdPlan {
  int64_t ntk, ntr;               // key tiles, row tiles per (batch, KV head)
  size_t kv, vk, qd, dq, lse, d;  // workspace offsets
  size_t total;
};

BwdPlan bwd_plan(int64_t B, int64_t L, int64_t Hkv, int64_t G) {
  BwdPlan p;
  p.ntk = (L + 63) / 64;
  p.ntr = (L * G + 63) / 64;
  size_t o = 0;
  auto take = [&](size_t n) {
    const size_t at = o;
    o += (n + 255) & ~(size_t)255;
    return at;
  };
  const size_t kf = (size_t)(B * Hkv * p.ntk) * kTileBytes;
  const size_t rf = (size_t)(B * Hkv * p.ntr) * kTileBytes;
  p.kv = take(kf);
  p.vk = take(kf);
  p.qd = take(rf);
  p.dq = take(rf);
  p.lse = take((size_t)(B * Hkv * L * G) * 4);
  p.d = take((size_t)(B * Hkv * L * G) * 4);
  p.total = o;
  return p;
}

}  // namespace

extern "C" int64_t mrsa_local_attention_bwd_workspace_bytes(int64_t batch, int64_t seq_len,
                                                            int64_t q_heads, int64_t kv_heads) {
  if (batch < 0 || seq_len < 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0)
    return -1;
  return (int64_t)bwd_plan(batch, seq_len, kv_heads, q_heads / kv_heads).total;
}

extern "C" int mrsa_local_attention_bwd(const void* q, const void* k, const void* v,
                                        const uint8_t* key_valid, const void* out,
                                        const float* lse, const void* grad_out, int64_t batch,
                                        int64_t seq_len, int64_t q_heads, int64_t kv_heads,
                                        int64_t head_dim, int64_t window, int64_t inert_chunk,
                                        float sm_scale, float* grad_q, float* grad_k,
                                        float* grad_v, void* workspace, int64_t workspace_bytes,
                                        void* stream) {
  if (batch < 0 || seq_len < 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0 ||
      head_dim <= 0 || window < 0 || inert_chunk < 0 || !(sm_scale > 0.f) ||
      sm_scale == __builtin_inff())
    return MRSA_ERR_INVALID_ARGUMENT;
  if (batch == 0 || seq_len == 0) return MRSA_OK;
  if (head_dim != 128) return MRSA_ERR_UNSUPPORTED;
  const int64_t G = q_heads / kv_heads;
  if (G > 128 || kv_heads > 65535 || batch > 65535) return MRSA_ERR_UNSUPPORTED;
  // fragment sequences are addressed with 32-bit byte offsets
  if ((seq_len * G + 63) / 64 >= 131072) return MRSA_ERR_UNSUPPORTED;
  if (!q || !k || !v || !out || !lse || !grad_out || !grad_q || !grad_k || !grad_v || !workspace)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out | (uintptr_t)grad_out |
       (uintptr_t)grad_q | (uintptr_t)grad_k | (uintptr_t)grad_v) % 16 != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  const BwdPlan p = bwd_plan(batch, seq_len, kv_heads, G);
  if (workspace_bytes < (int64_t)p.total || (uintptr_t)workspace % 256 != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  char* ws = (char*)workspace;
  uint16_t* f_kv = (uint16_t*)(ws + p.kv);
  uint16_t* f_vk = (uint16_t*)(ws + p.vk);
  uint16_t* f_qd = (uint16_t*)(ws + p.qd);
  uint16_t* f_dq = (uint16_t*)(ws + p.dq);
  hipStream_t s = (hipStream_t)stream;
  const uint16_t *q16 = (const uint16_t*)q, *k16 = (const uint16_t*)k, *v16 = (const uint16_t*)v,
                 *o16 = (const uint16_t*)out, *do16 = (const uint16_t*)grad_out;
  const dim3 kgrid((unsigned)p.ntk, (unsigned)kv_heads, (unsigned)batch);
  const dim3 rgrid((unsigned)p.ntr, (unsigned)kv_heads, (unsigned)batch);
  hipLaunchKernelGGL(row_fragments_kernel, kgrid, dim3(256), 0, s, k16, v16, seq_len,
                     (int)kv_heads, (int)kv_heads, 1, p.ntk, f_kv);
  hipLaunchKernelGGL(row_fragments_kernel, kgrid, dim3(256), 0, s, v16, k16, seq_len,
                     (int)kv_heads, (int)kv_heads, 1, p.ntk, f_vk);
  hipLaunchKernelGGL(row_fragments_kernel, rgrid, dim3(256), 0, s, q16, do16, seq_len,
                     (int)q_heads, (int)kv_heads, (int)G, p.ntr, f_qd);
  hipLaunchKernelGGL(row_fragments_kernel, rgrid, dim3(256), 0, s, do16, q16, seq_len,
                     (int)q_heads, (int)kv_heads, (int)G, p.ntr, f_dq);
  int st = mrsa_launch_status();
  if (st != MRSA_OK) return st;

  BwdArgs a;
  a.q = q16;
  a.k = k16;
  a.v = v16;
  a.out = o16;
  a.dout = do16;
  a.lse = lse;
  a.key_valid = key_valid;
  a.B = batch;
  a.L = seq_len;
  a.Hq = (int)q_heads;
  a.Hkv = (int)kv_heads;
  a.G = (int)G;
  a.W = window;
  a.inert_chunk = inert_chunk;
  a.scale = sm_scale;
  a.scale_log2 = sm_scale * kLog2e;
  a.lse_rows = (float*)(ws + p.lse);
  a.d_rows = (float*)(ws + p.d);
  a.dq = grad_q;
  a.dk = grad_k;
  a.dv = grad_v;
  const size_t smem = (size_t)kRing * kSlotBytes + kMaskTiles * 8;
  // dQ pass: columns (query, head), rows = keys: A = K, B = V, B' = K^T
  a.fa = f_kv;
  a.fb = f_vk;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(local_bwd_kernel<false>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess)
    return MRSA_ERR_LAUNCH;
  const int64_t QB = 128 / G;
  hipLaunchKernelGGL(local_bwd_kernel<false>,
                     dim3((unsigned)((seq_len + QB - 1) / QB), (unsigned)kv_heads, (unsigned)batch),
                     dim3(kThreads), smem, s, a);
  st = mrsa_launch_status();
  if (st != MRSA_OK) return st;
  // dK/dV pass: columns = keys, rows = (query, head): A = Q, A' = dO^T, B = dO, B' = Q^T
  a.fa = f_qd;
  a.fb = f_dq;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(local_bwd_kernel<true>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) != hipSuccess)
    return MRSA_ERR_LAUNCH;
  hipLaunchKernelGGL(local_bwd_kernel<true>,
                     dim3((unsigned)((seq_len + 127) / 128), (unsigned)kv_heads, (unsigned)batch),
                     dim3(kThreads), smem, s, a);
  return mrsa_launch_status();
}
