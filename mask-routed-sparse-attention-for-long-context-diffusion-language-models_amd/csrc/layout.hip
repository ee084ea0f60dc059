// Layout helpers: the remote-route drop mask and the K / V fragments both
// attention kernels read.
#include "mrsa_device.h"
#include "pool_wave.h"

#include <algorithm>

using namespace mrsa;

namespace {

// drop[b, i, c] = chunk c overlaps the chunk-aligned window of query i, or
// chunk c has no valid real key (or the packed-sequence mask forbids it).
// kernel_utils.py:75-99 (bounds) and :102-161 (mask).
constexpr int kDropRows = 8;  // output rows per workgroup (x 256 chunks)

__global__ void __launch_bounds__(256)
    drop_mask_kernel(const uint8_t* __restrict__ valid, const uint8_t* __restrict__ allowed,
                     const int64_t* __restrict__ qpos, int64_t rows_total, int64_t L, int64_t W,
                     int64_t S, int32_t* __restrict__ out) {
  const int64_t b = blockIdx.z;
  const int64_t C = L / S;
  const int64_t c = (int64_t)blockIdx.y * 256 + threadIdx.x;
  if (c >= C) return;
  // Chunk c has a valid real key (the last slot is its landmark).
  const uint8_t* vc = valid + b * L + c * S;
  bool any = false;
  if (S % 16 == 0 && ((uintptr_t)vc & 15) == 0) {
    u32x4_t acc = {0u, 0u, 0u, 0u};
    for (int64_t s = 0; s < S - 16; s += 16) {
      const u32x4_t x = *reinterpret_cast<const u32x4_t*>(vc + s);
      acc[0] |= x[0]; acc[1] |= x[1]; acc[2] |= x[2]; acc[3] |= x[3];
    }
    const u32x4_t t = *reinterpret_cast<const u32x4_t*>(vc + S - 16);  // all but the last byte
    any = (acc[0] | acc[1] | acc[2] | acc[3] | t[0] | t[1] | t[2] | (t[3] & 0x00ffffffu)) != 0u;
  } else {
    for (int64_t s = 0; s < S - 1; ++s) any |= vc[s] != 0;
  }
  const int64_t i0 = (int64_t)blockIdx.x * kDropRows;
  const int64_t i1 = min(rows_total, i0 + kDropRows);
  for (int64_t i = i0; i < i1; ++i) {
    const int64_t p = qpos ? qpos[i] : i;  // cache position of output row i
    const int64_t lc = max(p - W, (int64_t)0) / S;
    const int64_t rc = min(p + W, L - 1) / S;
    bool drop = (c >= lc && c <= rc) || !any;
    if (allowed) drop = drop || allowed[(b * L + p) * L + c * S + S - 1] == 0;
    out[(b * rows_total + i) * C + c] = drop ? 1 : 0;
  }
}

// K and V fragments of one 64-key chunk: the register images of the matrix
// operands the routed and window attention feed to 16x16x32 bf16 matrix
// products (lane l = 16 grp + j holds 8 consecutive elements e of one
// instruction):
//   K part (operand of S^T = K . Q^T), instruction i = 4 mt + ks:
//     f[512 i + 8 l + e]        = K[key 16 mt + j][dim 32 ks + 8 grp + e]
//   V part (operand of O = P . V, or of O^T = V^T . P^T), instruction i = 2 nt + ks:
//     f[8192 + 512 i + 8 l + e] = V[key 32 ks + 16 (e >> 2) + 4 grp + (e & 3)][dim 16 nt + j]
// (key 32a + 16b + 4c + e sits at reduction slot 32a + 8c + 4b + e: the eight
// keys a lane feeds to one 32-deep reduction are the ones the S^T
// accumulator of the first product hands it).  Every operand load of a chunk
// is one contiguous 1 KB read.  Keys past the sequence end are zero, and the
// whole V part without a V input (the token scores read only K).
constexpr int kFragElems = 16384;  // bf16 per (batch, KV head, chunk)
constexpr int kFragPitch = 136;    // LDS row pitch (elements): 16-byte aligned rows

__device__ __forceinline__ int frag_k_index(int r, int d) {
  return 512 * (4 * (r >> 4) + (d >> 5)) + 8 * (16 * ((d >> 3) & 3) + (r & 15)) + (d & 7);
}
__device__ __forceinline__ int frag_v_index(int r, int d) {
  const int e = 4 * ((r >> 4) & 1) + (r & 3);
  return 8192 + 512 * (2 * (d >> 4) + (r >> 5)) + 8 * (16 * ((r >> 2) & 3) + (d & 15)) + e;
}

__global__ void __launch_bounds__(256)
    kv_fragments_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                        int64_t L, int64_t H, int64_t NT, uint16_t* __restrict__ frags) {
  __shared__ __align__(16) uint16_t ks_[64 * kFragPitch];
  __shared__ __align__(16) uint16_t vs_[64 * kFragPitch];
  const int64_t c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  // 64 rows x 16 pieces of 16 bytes for each of K and V
  for (int p = tid; p < 1024; p += 256) {
    const int r = p >> 4, u = p & 15;
    const int64_t s = c * 64 + r;
    u32x4_t xk = {0u, 0u, 0u, 0u}, xv = {0u, 0u, 0u, 0u};
    if (s < L) {
      const int64_t off = ((b * L + s) * H + h) * 128 + 8 * u;
      xk = *reinterpret_cast<const u32x4_t*>(k + off);
      if (v) xv = *reinterpret_cast<const u32x4_t*>(v + off);
    }
    *reinterpret_cast<u32x4_t*>(ks_ + r * kFragPitch + 8 * u) = xk;
    *reinterpret_cast<u32x4_t*>(vs_ + r * kFragPitch + 8 * u) = xv;
  }
  __syncthreads();
  uint16_t* dst = frags + ((b * H + h) * NT + c) * (int64_t)kFragElems;
  for (int p = tid; p < 1024; p += 256) {
    const int i = p >> 6, l = p & 63, j = l & 15, grp = l >> 4;
    // K: 8 consecutive dims of one key row
    const int mt = i >> 2, kq = i & 3;
    const u32x4_t xk =
        *reinterpret_cast<const u32x4_t*>(ks_ + (16 * mt + j) * kFragPitch + 32 * kq + 8 * grp);
    *reinterpret_cast<u32x4_t*>(dst + 8 * p) = xk;
    // V: one dim of 8 keys in the tiled order
    const int nt = i >> 1, kv = i & 1, d = 16 * nt + j;
    u32x4_t xv;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int r0 = 32 * kv + 16 * (w >> 1) + 4 * grp + 2 * (w & 1);
      xv[w] = (uint32_t)vs_[r0 * kFragPitch + d] | ((uint32_t)vs_[(r0 + 1) * kFragPitch + d] << 16);
    }
    *reinterpret_cast<u32x4_t*>(dst + 8192 + 8 * p) = xv;
  }
}

// Rewrites the fragment entries of the listed rows only; positions outside
// [0, L) are ignored.  One thread per dim: its K and V elements.
__global__ void __launch_bounds__(128)
    kv_fragments_rows_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                             int64_t L, int64_t H, int64_t NT,
                             const int64_t* __restrict__ positions,
                             uint16_t* __restrict__ frags) {
  const int64_t p = positions[blockIdx.x];
  const int64_t h = blockIdx.y, b = blockIdx.z;
  if (p < 0 || p >= L) return;
  const int r = (int)(p & 63), d = threadIdx.x;
  uint16_t* dst = frags + ((b * H + h) * NT + p / 64) * (int64_t)kFragElems;
  const int64_t src = ((b * L + p) * H + h) * 128 + d;
  dst[frag_k_index(r, d)] = k[src];
  dst[frag_v_index(r, d)] = v[src];
}

// The K/V rows of a cache update written in one pass: row i of k_rows /
// v_rows ([B, count, H, 128]) goes to cache position positions[i] of key /
// value ([B, L, H, 128]) and, when frags is given, into that position's
// fragment entries.  One thread per dim; positions outside [0, L) are
// ignored.
__global__ void __launch_bounds__(128)
    kv_replace_rows_kernel(const uint16_t* __restrict__ k_rows, const uint16_t* __restrict__ v_rows,
                           int64_t count, const int64_t* __restrict__ positions, int64_t L,
                           int64_t H, int64_t NT, uint16_t* __restrict__ key,
                           uint16_t* __restrict__ value, uint16_t* __restrict__ frags) {
  const int64_t i = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int64_t p = positions[i];
  if (p < 0 || p >= L) return;
  const int d = threadIdx.x;
  const uint16_t kx = k_rows[((b * count + i) * H + h) * 128 + d];
  const uint16_t vx = v_rows[((b * count + i) * H + h) * 128 + d];
  const int64_t dst = ((b * L + p) * H + h) * 128 + d;
  key[dst] = kx;
  value[dst] = vx;
  if (frags) {
    uint16_t* fr = frags + ((b * H + h) * NT + p / 64) * (int64_t)kFragElems;
    const int r = (int)(p & 63);
    fr[frag_k_index(r, d)] = kx;
    fr[frag_v_index(r, d)] = vx;
  }
}

// Q fragments: per (batch, KV head, query) the 2 KB register image of the
// routed attention's Q^T operand for the query's G head columns --
//   qf[((b Hkv + h) L + i) 1024 + 256 ks + 64 grp + 8 g + e]
//     = q[b, i, h G + g, 32 ks + 8 grp + e]   (g < G; zeros for g in [G, 8))
// -- so the lanes of one lane group (grp) read the 8 head columns of a query
// as one 128-byte line.  One thread per 16-byte block, stores coalesced.
__global__ void __launch_bounds__(256)
    q_fragments_kernel(const uint16_t* __restrict__ q, int64_t L, int Hq, int Hkv, int G,
                       int64_t nblocks, uint16_t* __restrict__ qf) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < nblocks; e += stride) {
    const int u = (int)(e & 127);
    const int64_t img = e >> 7;
    const int64_t i = img % L;
    const int64_t bh = img / L;
    const int h = (int)(bh % Hkv);
    const int64_t b = bh / Hkv;
    const int ks = u >> 5, grp = (u >> 3) & 3, g = u & 7;
    u32x4_t x = {0u, 0u, 0u, 0u};
    if (g < G)
      x = *reinterpret_cast<const u32x4_t*>(q + ((b * L + i) * Hq + (int64_t)h * G + g) * 128 +
                                            32 * ks + 8 * grp);
    *reinterpret_cast<u32x4_t*>(qf + e * 8) = x;
  }
}

// K/V fragments and the landmark pool of the same chunks in one pass
// (kv_fragments_kernel + the matrix-core pool): a workgroup per (chunk, KV
// head, batch) stages the chunk's K and V rows in LDS once, writes the
// fragments and pools K against the chunk's landmark-slot query rows.  The
// pool is split over the four waves -- wave w takes keys 16 w .. 16 w + 15
// and landmark dims 32 w .. 32 w + 31 -- with the column max, sum and
// entropy partials and the P blocks exchanged through LDS (pool_wave.h
// fixes the summation order, so the bits equal the one-wave pool's).  The
// fragment stores are issued between the exchanges.  Needs whole chunks (L a
// multiple of 64).
struct PitchRows {
  const uint16_t* ks;
  __device__ u32x4_t row16(int key, int blk) const {
    return *reinterpret_cast<const u32x4_t*>(ks + key * kFragPitch + 8 * blk);
  }
  __device__ uint32_t elem(int key, int dim) const { return ks[key * kFragPitch + dim]; }
};

__global__ void __launch_bounds__(256)
    kv_fragments_pool_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                             int64_t L, int64_t H, int64_t NT, uint16_t* __restrict__ frags,
                             const uint16_t* __restrict__ mu_q, int64_t mu_stride,
                             const uint8_t* __restrict__ key_valid, int G, float sm_scale,
                             const float* __restrict__ bias_scale, uint16_t* __restrict__ lmk,
                             float* __restrict__ entropy, float* __restrict__ prior) {
  __shared__ __align__(16) uint16_t ks_[64 * kFragPitch];
  __shared__ __align__(16) uint16_t vs_[64 * kFragPitch];
  __shared__ float red[3][4][16];       // column max, sum, sum p ln p of each key block
  __shared__ __align__(16) u32x2_t pbl[4][64];  // bf16 P of each key block, per lane
  const int64_t c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int j = lane & 15, grp = lane >> 4;
  const int64_t bc = b * NT + c;
  for (int p = tid; p < 1024; p += 256) {
    const int r = p >> 4, u = p & 15;
    const int64_t off = ((b * L + c * 64 + r) * H + h) * 128 + 8 * u;
    *reinterpret_cast<u32x4_t*>(ks_ + r * kFragPitch + 8 * u) =
        *reinterpret_cast<const u32x4_t*>(k + off);
    *reinterpret_cast<u32x4_t*>(vs_ + r * kFragPitch + 8 * u) =
        *reinterpret_cast<const u32x4_t*>(v + off);
  }
  u32x4_t Qb[4];
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    Qb[q4] = u32x4_t{0u, 0u, 0u, 0u};
    if (j < G)
      Qb[q4] = *reinterpret_cast<const u32x4_t*>(mu_q + bc * mu_stride +
                                                 (int64_t)(h * G + j) * 128 + 32 * q4 + 8 * grp);
  }
  const uint64_t real = __builtin_amdgcn_ballot_w64(key_valid[bc * 64 + lane] != 0) & ~(1ull << 63);
  const bool chunk_valid = real != 0ull;
  __syncthreads();
  const PitchRows rows{ks_};
  uint16_t* dst = frags + ((b * H + h) * NT + c) * (int64_t)kFragElems;
  // fragment pieces p = tid + 256 i: K 16 bytes of one key row, V one dim of
  // 8 keys in the tiled order
  auto frag_piece = [&](int p) {
    const int i = p >> 6, l = p & 63, jj = l & 15, gg = l >> 4;
    const int mt = i >> 2, kq = i & 3;
    *reinterpret_cast<u32x4_t*>(dst + 8 * p) =
        *reinterpret_cast<const u32x4_t*>(ks_ + (16 * mt + jj) * kFragPitch + 32 * kq + 8 * gg);
    const int nt = i >> 1, kv = i & 1, d = 16 * nt + jj;
    u32x4_t xv;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r0 = 32 * kv + 16 * (e >> 1) + 4 * gg + 2 * (e & 1);
      xv[e] = (uint32_t)vs_[r0 * kFragPitch + d] | ((uint32_t)vs_[(r0 + 1) * kFragPitch + d] << 16);
    }
    *reinterpret_cast<u32x4_t*>(dst + 8192 + 8 * p) = xv;
  };
  f32x4_t S = pool_logits(rows, Qb, real, sm_scale, w, lane);
  const float bmax = across4_max(pool_max4(S));
  if (grp == 0) red[0][w][j] = bmax;
  frag_piece(tid);
  frag_piece(tid + 256);
  __syncthreads();
  const float mx = fmaxf(fmaxf(red[0][0][j], red[0][1][j]), fmaxf(red[0][2][j], red[0][3][j]));
  const float bsum = pool_exp(S, mx);
  if (grp == 0) red[1][w][j] = bsum;
  frag_piece(tid + 512);
  frag_piece(tid + 768);
  __syncthreads();
  const float sum = ((red[1][0][j] + red[1][1][j]) + red[1][2][j]) + red[1][3][j];
  const float bt = pool_prob(S, sum);
  if (grp == 0) red[2][w][j] = bt;
  pbl[w][lane] = u32x2_t{pack_bf16x2(S[0], S[1]), pack_bf16x2(S[2], S[3])};
  __syncthreads();
  if (w == 0)
    pool_stats(((red[2][0][j] + red[2][1][j]) + red[2][2][j]) + red[2][3][j], chunk_valid, G,
               (bc * H + h) * G, bias_scale, (int)h * G, entropy, prior, lane);
  u32x4_t Pb[2];
#pragma unroll
  for (int k2 = 0; k2 < 2; ++k2) {
    const u32x2_t lo = pbl[2 * k2][lane], hi = pbl[2 * k2 + 1][lane];
    Pb[k2] = u32x4_t{lo[0], lo[1], hi[0], hi[1]};
  }
  uint16_t* lrow = lmk + (bc * H + h) * G * 128;
  pool_lmk(rows, Pb, 2 * w, chunk_valid, G, lrow, lane);
  pool_lmk(rows, Pb, 2 * w + 1, chunk_valid, G, lrow, lane);
}

// Device-side argument checks of the cached block step in one launch (one
// workgroup): flags[0] query positions not strictly ascending, flags[1] a
// position outside [0, L), flags[2] an affected chunk outside [0, C),
// flags[3] an affected chunk whose landmark position (c S + S - 1) is not a
// query position (lower-bound search; meaningful once flags[0] is clear).
__global__ void __launch_bounds__(256)
    cached_step_checks_kernel(const int64_t* __restrict__ qp, int64_t lq,
                              const int64_t* __restrict__ aff, int64_t n, int64_t L, int64_t C,
                              int64_t S, int32_t* __restrict__ flags) {
  __shared__ int f[4];
  const int tid = threadIdx.x;
  if (tid < 4) f[tid] = 0;
  __syncthreads();
  int a0 = 0, a1 = 0, a2 = 0, a3 = 0;
  for (int64_t i = tid; i < lq; i += blockDim.x) {
    const int64_t p = qp[i];
    if (i + 1 < lq && qp[i + 1] <= p) a0 = 1;
    if (p < 0 || p >= L) a1 = 1;
  }
  for (int64_t j = tid; j < n; j += blockDim.x) {
    const int64_t c = aff[j];
    if (c < 0 || c >= C) a2 = 1;
    const int64_t lp = c * S + S - 1;
    int64_t lo = 0, hi = lq;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (qp[mid] < lp) lo = mid + 1;
      else hi = mid;
    }
    if (lo >= lq || qp[lo] != lp) a3 = 1;
  }
  if (a0) atomicOr(&f[0], 1);
  if (a1) atomicOr(&f[1], 1);
  if (a2) atomicOr(&f[2], 1);
  if (a3) atomicOr(&f[3], 1);
  __syncthreads();
  if (tid < 4) flags[tid] = f[tid];
}

// Up to kMaxCopies buffer copies in one launch: buffer i is `units[i]` units
// of 16 bytes (wide[i]) or 8 bytes; start[i] is the first unit of buffer i in
// the flattened unit range [0, start[count]).
constexpr int kMaxCopies = 8;
struct CopyList {
  const void* src[kMaxCopies];
  void* dst[kMaxCopies];
  int64_t start[kMaxCopies + 1];
  int32_t wide[kMaxCopies];
  int32_t count;
};

__global__ void __launch_bounds__(256) copy_list_kernel(CopyList l) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < l.start[l.count];
       u += stride) {
    // the buffer holding unit u (static indices only: the list stays in
    // kernel-argument registers)
    const void* s = l.src[0];
    void* d = l.dst[0];
    int64_t base = l.start[0];
    int32_t w = l.wide[0];
#pragma unroll
    for (int k = 1; k < kMaxCopies; ++k)
      if (k < l.count && u >= l.start[k]) {
        s = l.src[k];
        d = l.dst[k];
        base = l.start[k];
        w = l.wide[k];
      }
    const int64_t e = u - base;
    if (w)
      reinterpret_cast<u32x4_t*>(d)[e] = reinterpret_cast<const u32x4_t*>(s)[e];
    else
      reinterpret_cast<u32x2_t*>(d)[e] = reinterpret_cast<const u32x2_t*>(s)[e];
  }
}

}  // namespace

extern "C" int mrsa_remote_drop_mask(const uint8_t* valid_mask, const uint8_t* allowed_mask,
                                     int64_t batch, int64_t seq_len, int64_t window,
                                     int64_t chunk_size, int32_t* drop_mask, void* stream) {
  if (batch < 0 || seq_len <= 0 || window < 0 || chunk_size <= 0 || seq_len % chunk_size != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (batch == 0) return MRSA_OK;
  if (!valid_mask || !drop_mask) return MRSA_ERR_INVALID_ARGUMENT;
  const int64_t C = seq_len / chunk_size;
  if (C > 65535 * 256 || batch > 65535 || seq_len > ((int64_t)1 << 33))
    return MRSA_ERR_UNSUPPORTED;
  if (C == 0) return MRSA_OK;
  dim3 grid((unsigned)((seq_len + kDropRows - 1) / kDropRows), (unsigned)((C + 255) / 256),
            (unsigned)batch);
  hipLaunchKernelGGL(drop_mask_kernel, grid, dim3(256), 0, (hipStream_t)stream, valid_mask,
                     allowed_mask, nullptr, seq_len, seq_len, window, chunk_size, drop_mask);
  return mrsa_launch_status();
}

extern "C" int mrsa_remote_drop_mask_rows(const uint8_t* valid_mask,
                                          const int64_t* query_positions, int64_t batch,
                                          int64_t seq_len, int64_t rows, int64_t window,
                                          int64_t chunk_size, int32_t* drop_mask, void* stream) {
  if (batch < 0 || seq_len <= 0 || rows < 0 || window < 0 || chunk_size <= 0 ||
      seq_len % chunk_size != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (batch == 0 || rows == 0) return MRSA_OK;
  if (!valid_mask || !query_positions || !drop_mask) return MRSA_ERR_INVALID_ARGUMENT;
  const int64_t C = seq_len / chunk_size;
  if (C > 65535 * 256 || batch > 65535 || rows > ((int64_t)1 << 33)) return MRSA_ERR_UNSUPPORTED;
  dim3 grid((unsigned)((rows + kDropRows - 1) / kDropRows), (unsigned)((C + 255) / 256),
            (unsigned)batch);
  hipLaunchKernelGGL(drop_mask_kernel, grid, dim3(256), 0, (hipStream_t)stream, valid_mask,
                     nullptr, query_positions, rows, seq_len, window, chunk_size, drop_mask);
  return mrsa_launch_status();
}

extern "C" int64_t mrsa_kv_fragments_bytes(int64_t batch, int64_t seq_len, int64_t kv_heads,
                                           int64_t head_dim) {
  if (batch < 0 || seq_len < 0 || kv_heads < 0 || head_dim != 128) return -1;
  return batch * kv_heads * ((seq_len + 63) / 64) * (int64_t)kFragElems * 2;
}

extern "C" int mrsa_kv_fragments(const void* k, const void* v, int64_t batch, int64_t seq_len,
                                 int64_t kv_heads, int64_t head_dim, void* kv_frags,
                                 void* stream) {
  if (batch < 0 || seq_len < 0 || kv_heads <= 0 || head_dim <= 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (head_dim != 128) return MRSA_ERR_UNSUPPORTED;
  if (batch == 0 || seq_len == 0) return MRSA_OK;
  if (!k || !kv_frags || ((uintptr_t)k | (uintptr_t)v | (uintptr_t)kv_frags) % 16 != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  const int64_t NT = (seq_len + 63) / 64;
  if (kv_heads > 65535 || batch > 65535 || NT > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(kv_fragments_kernel, dim3((unsigned)NT, (unsigned)kv_heads, (unsigned)batch),
                     dim3(256), 0, (hipStream_t)stream, (const uint16_t*)k, (const uint16_t*)v,
                     seq_len, kv_heads, NT, (uint16_t*)kv_frags);
  return mrsa_launch_status();
}

extern "C" int mrsa_kv_fragments_pool_fwd(const void* k, const void* v, const void* mu_q,
                                          int64_t mu_row_stride, const uint8_t* key_valid,
                                          int64_t batch, int64_t seq_len, int64_t kv_heads,
                                          int64_t groups, int64_t head_dim, float sm_scale,
                                          const float* bias_scale, void* kv_frags,
                                          void* landmark_keys, float* entropy,
                                          float* prior_bias, void* stream) {
  if (batch < 0 || seq_len < 0 || kv_heads <= 0 || groups <= 0 || head_dim <= 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  if ((prior_bias != nullptr) != (bias_scale != nullptr)) return MRSA_ERR_INVALID_ARGUMENT;
  if (mu_row_stride < kv_heads * groups * head_dim) return MRSA_ERR_INVALID_ARGUMENT;
  // groups == 1 takes the reference's dense torch twin, which this kernel
  // does not restate (mrsa_chunk_attn_pool_gqa_fwd does)
  if (head_dim != 128 || groups < 2 || groups > 16 || seq_len % 64 != 0)
    return MRSA_ERR_UNSUPPORTED;
  if (batch == 0 || seq_len == 0) return MRSA_OK;
  if (!k || !v || !mu_q || !key_valid || !kv_frags || !landmark_keys || !entropy)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)k | (uintptr_t)v | (uintptr_t)kv_frags | (uintptr_t)mu_q |
       (uintptr_t)landmark_keys) % 16 != 0 || mu_row_stride % 8 != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  const int64_t NT = seq_len / 64;
  if (kv_heads > 65535 || batch > 65535 || NT > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(kv_fragments_pool_kernel,
                     dim3((unsigned)NT, (unsigned)kv_heads, (unsigned)batch), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)k, (const uint16_t*)v, seq_len,
                     kv_heads, NT, (uint16_t*)kv_frags, (const uint16_t*)mu_q, mu_row_stride,
                     key_valid, (int)groups, sm_scale, bias_scale, (uint16_t*)landmark_keys,
                     entropy, prior_bias);
  return mrsa_launch_status();
}

extern "C" int mrsa_cached_step_checks(const int64_t* query_positions, int64_t count,
                                       const int64_t* affected_chunks, int64_t affected_count,
                                       int64_t cache_len, int64_t chunk_size, int32_t* flags,
                                       void* stream) {
  if (count < 0 || affected_count < 0 || cache_len < 0 || chunk_size <= 0 || !flags)
    return MRSA_ERR_INVALID_ARGUMENT;
  if ((count > 0 && !query_positions) || (affected_count > 0 && !affected_chunks))
    return MRSA_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(cached_step_checks_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream,
                     query_positions, count, affected_chunks, affected_count, cache_len,
                     cache_len / chunk_size, chunk_size, flags);
  return mrsa_launch_status();
}

extern "C" int mrsa_copy_buffers(int32_t count, const void* const* src, void* const* dst,
                                 const int64_t* bytes, void* stream) {
  if (count < 0 || count > kMaxCopies) return MRSA_ERR_INVALID_ARGUMENT;
  if (count > 0 && (!src || !dst || !bytes)) return MRSA_ERR_INVALID_ARGUMENT;
  CopyList l{};
  l.count = 0;
  int64_t total = 0;
  for (int i = 0; i < count; ++i) {
    if (bytes[i] < 0) return MRSA_ERR_INVALID_ARGUMENT;
    if (bytes[i] == 0) continue;
    if (!src[i] || !dst[i]) return MRSA_ERR_INVALID_ARGUMENT;
    const uintptr_t a = (uintptr_t)src[i] | (uintptr_t)dst[i] | (uintptr_t)bytes[i];
    if (a % 8 != 0) return MRSA_ERR_UNSUPPORTED;
    const int k = l.count++;
    l.src[k] = src[i];
    l.dst[k] = dst[i];
    l.wide[k] = a % 16 == 0;
    l.start[k] = total;
    total += bytes[i] / (l.wide[k] ? 16 : 8);
  }
  l.start[l.count] = total;
  if (total == 0) return MRSA_OK;
  const int64_t grid = std::min<int64_t>((total + 255) / 256, 1024);
  hipLaunchKernelGGL(copy_list_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                     l);
  return mrsa_launch_status();
}

extern "C" int mrsa_kv_replace_rows(const void* k_rows, const void* v_rows,
                                    const int64_t* positions, int64_t count, int64_t batch,
                                    int64_t seq_len, int64_t kv_heads, int64_t head_dim, void* key,
                                    void* value, void* kv_frags, void* stream) {
  if (batch < 0 || seq_len < 0 || kv_heads <= 0 || head_dim <= 0 || count < 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (head_dim != 128) return MRSA_ERR_UNSUPPORTED;
  if (batch == 0 || seq_len == 0 || count == 0) return MRSA_OK;
  if (!k_rows || !v_rows || !positions || !key || !value) return MRSA_ERR_INVALID_ARGUMENT;
  if (kv_heads > 65535 || batch > 65535 || count > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(kv_replace_rows_kernel,
                     dim3((unsigned)count, (unsigned)kv_heads, (unsigned)batch), dim3(128), 0,
                     (hipStream_t)stream, (const uint16_t*)k_rows, (const uint16_t*)v_rows, count,
                     positions, seq_len, kv_heads, (seq_len + 63) / 64, (uint16_t*)key,
                     (uint16_t*)value, (uint16_t*)kv_frags);
  return mrsa_launch_status();
}

extern "C" int mrsa_kv_fragments_rows(const void* k, const void* v, int64_t batch,
                                      int64_t seq_len, int64_t kv_heads, int64_t head_dim,
                                      const int64_t* positions, int64_t count, void* kv_frags,
                                      void* stream) {
  if (batch < 0 || seq_len < 0 || kv_heads <= 0 || head_dim <= 0 || count < 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (head_dim != 128) return MRSA_ERR_UNSUPPORTED;
  if (batch == 0 || seq_len == 0 || count == 0) return MRSA_OK;
  if (!k || !v || !kv_frags || !positions) return MRSA_ERR_INVALID_ARGUMENT;
  if (kv_heads > 65535 || batch > 65535 || count > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  const int64_t NT = (seq_len + 63) / 64;
  hipLaunchKernelGGL(kv_fragments_rows_kernel,
                     dim3((unsigned)count, (unsigned)kv_heads, (unsigned)batch), dim3(128), 0,
                     (hipStream_t)stream, (const uint16_t*)k, (const uint16_t*)v, seq_len,
                     kv_heads, NT, positions, (uint16_t*)kv_frags);
  return mrsa_launch_status();
}

extern "C" int64_t mrsa_q_fragments_bytes(int64_t batch, int64_t seq_len, int64_t kv_heads,
                                          int64_t head_dim) {
  if (batch < 0 || seq_len < 0 || kv_heads < 0 || head_dim != 128) return -1;
  return batch * kv_heads * seq_len * 2048;
}

extern "C" int mrsa_q_fragments(const void* q, int64_t batch, int64_t seq_len, int64_t q_heads,
                                int64_t kv_heads, int64_t head_dim, void* q_frags,
                                void* stream) {
  if (batch < 0 || seq_len < 0 || q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 ||
      q_heads % kv_heads != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (head_dim != 128 || q_heads / kv_heads > 8) return MRSA_ERR_UNSUPPORTED;
  if (batch == 0 || seq_len == 0) return MRSA_OK;
  if (!q || !q_frags || ((uintptr_t)q | (uintptr_t)q_frags) % 16 != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (q_heads > 65535) return MRSA_ERR_UNSUPPORTED;
  const int64_t nblocks = batch * kv_heads * seq_len * 128;
  const int64_t grid = std::min<int64_t>((nblocks + 255) / 256, 8192);
  hipLaunchKernelGGL(q_fragments_kernel, dim3((unsigned)grid), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)q, seq_len, (int)q_heads,
                     (int)kv_heads, (int)(q_heads / kv_heads), nblocks, (uint16_t*)q_frags);
  return mrsa_launch_status();
}
