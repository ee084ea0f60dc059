// Bidirectional sliding-window GQA attention (flash-attn window semantics).
//
// Work split: one workgroup per (batch, KV head, block of 32 queries) with one
// wave per query head of the group, so the K / V tiles of the KV head are
// staged in LDS once and shared by all G query heads.  Each wave owns two
// 16-query column tiles of its head.
//
// Matrix-core formulation (per 64-key tile):
//   S^T[key][query] = K_tile (A: 64 x 128) . Q^T (B: 128 x 16)   -> 4 x 4 MFMAs
//   online softmax down each column (query), in the exp2 domain
//   O^T[d][query]  += V^T (A: 128 x 64) . P^T (B: 64 x 16)      -> 8 x 2 MFMAs
// P^T is fed to the second product straight from the accumulator registers of
// the first: lane l holds keys 16t + 4(l/16) + i of its query column, and the
// reduction slots of the second product are numbered so that slot e of lane
// group g is key 32j + 16(e/4) + 4g + e%4.  V^T is read from the tiled,
// transposed V layout with the same numbering.
//
// Semantics (dream_dllm_hils/local_attention.py:35-107):
//   * key j is visible to a query at position p iff |p - j| <= window;
//   * inert keys (failed key_valid, or landmark slots when inert_chunk > 0)
//     carry zero K and V: logit exactly 0, no contribution to the output;
//   * P is rounded to bf16 before the PV product, the row sum uses fp32 P
//     (flash-attn's convention); out = O / l in bf16; lse = ln(sum exp(s)).
#include "mrsa_device.h"

using namespace mrsa;

namespace {

constexpr int kQB = 32;        // queries per workgroup
constexpr int kKPitch = 136;   // bf16 per staged K row   (272 B)
constexpr int kVPitch = 72;    // bf16 per staged V^T row (144 B)
constexpr int kStageVecs = 2048;  // 16-byte vectors per staged tile (K + V^T)

struct LocalArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* vt;
  const uint8_t* key_valid;
  const int64_t* qpos;
  int64_t B, Lq, Lk;
  int Hq, Hkv;
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
};

template <int G>
__global__ void __launch_bounds__(64 * G) local_attn_kernel(LocalArgs a) {
  constexpr int NTHR = 64 * G;
  constexpr int PER = (kStageVecs + NTHR - 1) / NTHR;
  __shared__ __align__(16) uint16_t Ks[64 * kKPitch + 128 * kVPitch];
  uint16_t* const Vs = Ks + 64 * kKPitch;
  __shared__ uint64_t inert_bits, range_bits;
  __shared__ int64_t pos_lo, pos_hi;

  const int tid = threadIdx.x;
  const int lane = tid & 63, g = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, grp = lane >> 4;
  const int64_t b = blockIdx.z % a.B;
  const int part = (int)(blockIdx.z / a.B);
  const int h = blockIdx.y;
  const int64_t qb = (int64_t)blockIdx.x * kQB;
  const int hq = h * G + g;

  // Position range of this block's queries.
  if (g == 0) {
    int64_t lo = INT64_MAX, hi = INT64_MIN;
    if (lane < kQB && qb + lane < a.Lq) {
      const int64_t p = a.qpos ? a.qpos[qb + lane] : qb + lane;
      lo = p;
      hi = p;
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      lo = min(lo, (int64_t)__shfl_xor(lo, o, 64));
      hi = max(hi, (int64_t)__shfl_xor(hi, o, 64));
    }
    if (lane == 0) {
      pos_lo = lo;
      pos_hi = hi;
    }
  }

  // Q^T operands and query positions for this lane's two columns.
  u32x4_t Qb[2][4];
  int qp[2];
  bool qok[2];
  int rel[2];  // (tile start) - (query position), refreshed per key tile
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int64_t qi = qb + 16 * nt + col;
    qok[nt] = qi < a.Lq;
    qp[nt] = qok[nt] ? (int)(a.qpos ? a.qpos[qi] : qi) : 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4_t z = {0u, 0u, 0u, 0u};
      Qb[nt][j] = z;
      if (qok[nt])
        Qb[nt][j] = *reinterpret_cast<const u32x4_t*>(
            a.q + ((b * a.Lq + qi) * a.Hq + hq) * 128 + 32 * j + 8 * grp);
    }
  }
  __syncthreads();
  const int64_t plo = pos_lo, phi = pos_hi;
  const int64_t klo = max(plo - a.W, (int64_t)0);
  const int64_t khi = min(phi + a.W, a.Lk - 1);
  int64_t kt0 = klo / 64, kt1 = khi / 64;
  if (a.parts > 1) {
    const int64_t n = kt1 - kt0 + 1;
    const int64_t s0 = kt0 + n * part / a.parts;
    kt1 = kt0 + n * (part + 1) / a.parts - 1;
    kt0 = s0;
  }

  f32x4_t acc[2][8];
  float m_run[2], l_run[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    m_run[nt] = neg_inf();
    l_run[nt] = 0.f;
#pragma unroll
    for (int td = 0; td < 8; ++td) acc[nt][td] = zero4();
  }

  // Uniform (scalar) tile bases plus 32-bit per-lane offsets keep the
  // staging addresses out of the vector registers.
  const uint16_t* kbase = a.k + (b * a.Lk) * (int64_t)a.Hkv * 128 + (int64_t)h * 128;
  const uint16_t* vbase = a.vt + ((b * a.Hkv + h) * a.NTk) * (int64_t)(128 * 64);
  const int kstride = a.Hkv * 128;
  uint32_t goff[PER], loff[PER];
  int krow[PER];
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const int v = tid + p * NTHR;
    if (v < 1024) {
      const int s = v >> 4, part = v & 15;
      goff[p] = (uint32_t)(s * kstride + part * 8);
      loff[p] = (uint32_t)(s * kKPitch + part * 8);
      krow[p] = s;
    } else {
      const int d = (v - 1024) >> 3, part = (v - 1024) & 7;
      goff[p] = (uint32_t)((v - 1024) * 8);
      loff[p] = (uint32_t)(64 * kKPitch + d * kVPitch + part * 8);
      krow[p] = -1;
    }
  }

  u32x4_t pre[PER];
  auto prefetch = [&](int64_t kt) {
    const uint16_t* kt_base = kbase + kt * 64 * (int64_t)kstride;
    const uint16_t* vt_base = vbase + kt * (128 * 64);
    const int rows_left = (int)min((int64_t)64, a.Lk - kt * 64);
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int v = tid + p * NTHR;
      u32x4_t val = {0u, 0u, 0u, 0u};
      if (v < 1024) {
        if (krow[p] < rows_left) val = *reinterpret_cast<const u32x4_t*>(kt_base + goff[p]);
      } else if (v < kStageVecs) {
        val = *reinterpret_cast<const u32x4_t*>(vt_base + goff[p]);
      }
      pre[p] = val;
    }
  };
  auto commit = [&]() {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int v = tid + p * NTHR;
      if (v < kStageVecs) *reinterpret_cast<u32x4_t*>(Ks + loff[p]) = pre[p];
    }
  };

  if (kt0 <= kt1) prefetch(kt0);
  for (int64_t kt = kt0; kt <= kt1; ++kt) {
    __syncthreads();
    commit();
    if (g == 0) {
      const int64_t j = kt * 64 + lane;
      bool inert = false;
      if (j < a.Lk) {
        if (a.key_valid && a.key_valid[b * a.Lk + j] == 0) inert = true;
        if (a.inert_chunk > 0 && (j + 1) % a.inert_chunk == 0) inert = true;
      }
      const uint64_t ib = __ballot(inert);
      const uint64_t rb = __ballot(j < a.Lk);
      if (lane == 0) {
        inert_bits = ib;
        range_bits = rb;
      }
    }
    __syncthreads();
    if (kt < kt1) prefetch(kt + 1);

    const uint64_t ibits = inert_bits, rbits = range_bits;
    const int64_t j0 = kt * 64;
    rel[0] = (int)j0 - qp[0];
    rel[1] = (int)j0 - qp[1];
    const int W32 = (int)a.W;
    // Tiles entirely inside every query's window need no position mask.
    const bool full = (rbits == ~0ull) && (j0 >= phi - a.W) && (j0 + 63 <= plo + a.W);

    f32x4_t S[2][4];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int t = 0; t < 4; ++t) S[nt][t] = zero4();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4_t Ka[4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        Ka[t] = *reinterpret_cast<const u32x4_t*>(Ks + (16 * t + col) * kKPitch + 32 * j + 8 * grp);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int t = 0; t < 4; ++t) S[nt][t] = mfma_bf16_16x16x32(Ka[t], Qb[nt][j], S[nt][t]);
      __builtin_amdgcn_sched_barrier(0);
    }

    // Logits in units of log2: s * scale_log2.  Keys outside the window (or
    // past kv_len, or of an absent query) are -inf; inert keys inside it are
    // exactly 0.  The scale is folded into one FMA before the exponential
    // (scale_log2 > 0, so the maximum of the raw products is the maximum of
    // the logits).
    const float c = a.scale_log2;
    const uint64_t kLast = 1ull << 63;
    u32x4_t Pb[2][2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      if (!full) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int s = 16 * t + 4 * grp + i;
            const int dd = rel[nt] + s;
            if (!((rbits >> s) & 1ull) || dd > W32 || dd < -W32 || !qok[nt])
              S[nt][t][i] = neg_inf();
          }
      }
      if (ibits == kLast) {
        // Only the tile's last slot is inert (the landmark of a 64-key chunk).
        if (grp == 3 && S[nt][3][3] != neg_inf()) S[nt][3][3] = 0.f;
      } else if (ibits != 0ull) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int s = 16 * t + 4 * grp + i;
            if (((ibits >> s) & 1ull) && S[nt][t][i] != neg_inf()) S[nt][t][i] = 0.f;
          }
      }
      const float mx = across4_max(max16_raw(S[nt]));
      const float m_new = fmaxf(m_run[nt], mx * c);
      // A column with no visible key yet keeps m = -inf; exponentiate against 0
      // there so that every term (and alpha) is exp2(-inf) = 0.
      const float m_use = m_new == neg_inf() ? 0.f : m_new;
      const float alpha = exp2_hw(m_run[nt] - m_use);
      float pv[4][4];
      float part[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) pv[t][i] = exp2_hw(__builtin_fmaf(S[nt][t][i], c, -m_use));
        part[t] = (pv[t][0] + pv[t][1]) + (pv[t][2] + pv[t][3]);
      }
      const float rsum = across4_sum((part[0] + part[1]) + (part[2] + part[3]));
      // Inert keys count in the denominator but carry zero V.
      if (ibits == kLast) {
        if (grp == 3) pv[3][3] = 0.f;
      } else if (ibits != 0ull) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if ((ibits >> (16 * t + 4 * grp + i)) & 1ull) pv[t][i] = 0.f;
      }
      l_run[nt] = l_run[nt] * alpha + rsum;
      m_run[nt] = m_new;
      if (!__all(alpha == 1.f)) {
#pragma unroll
        for (int td = 0; td < 8; ++td) acc[nt][td] *= alpha;
      }
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        u32x4_t pb;
        pb[0] = pack_bf16x2(pv[2 * jj][0], pv[2 * jj][1]);
        pb[1] = pack_bf16x2(pv[2 * jj][2], pv[2 * jj][3]);
        pb[2] = pack_bf16x2(pv[2 * jj + 1][0], pv[2 * jj + 1][1]);
        pb[3] = pack_bf16x2(pv[2 * jj + 1][2], pv[2 * jj + 1][3]);
        Pb[nt][jj] = pb;
      }
    }

    // V^T rows hold each lane's eight reduction keys contiguously (tiled V
    // layout), so one 16-byte read per operand.
#pragma unroll
    for (int td = 0; td < 8; ++td) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const u32x4_t Va =
            *reinterpret_cast<const u32x4_t*>(Vs + (16 * td + col) * kVPitch + 32 * jj + 8 * grp);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[nt][td] = mfma_bf16_16x16x32(Va, Pb[nt][jj], acc[nt][td]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  if (a.parts > 1) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      if (!qok[nt]) continue;
      const int64_t row = ((int64_t)part * a.B * a.Lq + b * a.Lq + qb + 16 * nt + col) * a.Hq + hq;
      float* prow = a.part_o + row * 128;
#pragma unroll
      for (int td = 0; td < 8; ++td)
        *reinterpret_cast<f32x4_t*>(prow + 16 * td + 4 * grp) = acc[nt][td];
      if (grp == 0) {
        a.part_ml[2 * row] = m_run[nt];
        a.part_ml[2 * row + 1] = l_run[nt];
      }
    }
    return;
  }
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    if (!qok[nt]) continue;
    const int64_t qi = qb + 16 * nt + col;
    const float inv = l_run[nt] > 0.f ? 1.f / l_run[nt] : 0.f;
    uint16_t* orow = a.out + ((b * a.Lq + qi) * a.Hq + hq) * 128;
#pragma unroll
    for (int td = 0; td < 8; ++td) {
      u32x2_t o;
      o[0] = pack_bf16x2(acc[nt][td][0] * inv, acc[nt][td][1] * inv);
      o[1] = pack_bf16x2(acc[nt][td][2] * inv, acc[nt][td][3] * inv);
      *reinterpret_cast<u32x2_t*>(orow + 16 * td + 4 * grp) = o;
    }
    if (grp == 0)
      a.lse[(b * a.Lq + qi) * a.Hq + hq] =
          l_run[nt] > 0.f ? (m_run[nt] + log2f(l_run[nt])) * kLn2 : neg_inf();
  }
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

template <int G>
int launch_local(const LocalArgs& a, hipStream_t s) {
  dim3 grid((unsigned)((a.Lq + kQB - 1) / kQB), (unsigned)a.Hkv, (unsigned)(a.B * a.parts));
  hipLaunchKernelGGL(local_attn_kernel<G>, grid, dim3(64 * G), 0, s, a);
  int st = mrsa_launch_status();
  if (st != MRSA_OK || a.parts == 1) return st;
  const int64_t rows = a.B * a.Lq * a.Hq;
  hipLaunchKernelGGL(local_merge_kernel, dim3((unsigned)((rows * 32 + 255) / 256)), dim3(256), 0,
                     s, a, rows);
  return mrsa_launch_status();
}

}  // namespace

namespace {

int local_attention(const void* q, const void* k, const void* v_tiles, const uint8_t* key_valid,
                    const int64_t* query_positions, int64_t batch, int64_t q_len, int64_t kv_len,
                    int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t window,
                    int64_t inert_chunk, float sm_scale, int64_t parts, void* workspace,
                    void* out, float* lse, void* stream) {
  if (batch < 0 || q_len < 0 || kv_len < 0 || q_heads <= 0 || kv_heads <= 0 ||
      q_heads % kv_heads != 0 || head_dim <= 0 || window < 0 || inert_chunk < 0 ||
      !(sm_scale > 0.f) || sm_scale == __builtin_inff())
    return MRSA_ERR_INVALID_ARGUMENT;
  if (batch == 0 || q_len == 0) return MRSA_OK;
  if (kv_len == 0 || !q || !k || !v_tiles || !out || !lse) return MRSA_ERR_INVALID_ARGUMENT;
  if (head_dim != 128) return MRSA_ERR_UNSUPPORTED;
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v_tiles) % 16 != 0 || (uintptr_t)out % 8 != 0)
    return MRSA_ERR_INVALID_ARGUMENT;
  const int64_t G = q_heads / kv_heads;
  if (kv_heads > 65535 || batch > 65535) return MRSA_ERR_UNSUPPORTED;
  LocalArgs a;
  a.q = (const uint16_t*)q;
  a.k = (const uint16_t*)k;
  a.vt = (const uint16_t*)v_tiles;
  a.key_valid = key_valid;
  a.qpos = query_positions;
  a.B = batch;
  a.Lq = q_len;
  a.Lk = kv_len;
  a.Hq = (int)q_heads;
  a.Hkv = (int)kv_heads;
  a.W = window;
  a.inert_chunk = inert_chunk;
  a.scale_log2 = sm_scale * kLog2e;
  a.NTk = (kv_len + 63) / 64;
  a.out = (uint16_t*)out;
  a.lse = lse;
  a.parts = (int)parts;
  a.part_o = (float*)workspace;
  a.part_ml = parts > 1 ? (float*)workspace + parts * batch * q_len * q_heads * 128 : nullptr;
  hipStream_t s = (hipStream_t)stream;
  switch (G) {
    case 1: return launch_local<1>(a, s);
    case 2: return launch_local<2>(a, s);
    case 4: return launch_local<4>(a, s);
    case 7: return launch_local<7>(a, s);
    case 8: return launch_local<8>(a, s);
    default: return MRSA_ERR_UNSUPPORTED;
  }
}

}  // namespace

extern "C" int mrsa_local_attention_fwd(const void* q, const void* k, const void* v_tiles,
                                        const uint8_t* key_valid, const int64_t* query_positions,
                                        int64_t batch, int64_t q_len, int64_t kv_len,
                                        int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                        int64_t window, int64_t inert_chunk, float sm_scale,
                                        void* out, float* lse, void* stream) {
  return local_attention(q, k, v_tiles, key_valid, query_positions, batch, q_len, kv_len,
                         q_heads, kv_heads, head_dim, window, inert_chunk, sm_scale, 1, nullptr,
                         out, lse, stream);
}

extern "C" int64_t mrsa_local_attention_workspace_bytes(int64_t batch, int64_t q_len,
                                                        int64_t q_heads, int64_t parts) {
  if (batch < 0 || q_len < 0 || q_heads < 0 || parts < 1) return -1;
  return parts > 1 ? parts * batch * q_len * q_heads * 130 * 4 : 0;
}

extern "C" int mrsa_local_attention_split_fwd(const void* q, const void* k, const void* v_tiles,
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
  return local_attention(q, k, v_tiles, key_valid, query_positions, batch, q_len, kv_len,
                         q_heads, kv_heads, head_dim, window, inert_chunk, sm_scale, parts,
                         parts > 1 ? workspace : nullptr, out, lse, stream);
}
