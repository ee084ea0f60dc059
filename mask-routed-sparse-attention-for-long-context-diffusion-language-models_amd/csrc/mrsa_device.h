// Device-side helpers shared by every MRSA kernel (gfx950 / CDNA4 only).
//
// Storage conventions used across the library:
//   * bf16 tensors are passed as raw uint16_t bit patterns; arithmetic is done
//     in fp32 after widening, and results are narrowed with round-to-nearest-
//     even (the rounding torch's .to(torch.bfloat16) uses).
//   * MFMA operands for v_mfma_f32_16x16x32_bf16 are 8 bf16 values (16 bytes)
//     per lane.  Lane l supplies row (l % 16) of A and column (l % 16) of B;
//     lane group (l / 16) supplies one quarter of the 32-deep reduction.  The
//     16x16 fp32 result lands as C[4 * (l / 16) + i][l % 16], i = 0..3.
//     Only the M/N placement and the C layout matter for correctness: any
//     assignment of reduction indices to (lane group, element) is fine as long
//     as A and B use the same one, which every kernel here guarantees.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "mrsa.h"

namespace mrsa {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// fp32 -> bf16, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
__device__ __forceinline__ uint32_t f32_to_bf16(float f) { return pack_bf16x2(f, 0.f) & 0xffffu; }
// Output fusion of two packed bf16 pairs: bf16(r + w * l) per element, the
// multiply and the add rounded separately (no FMA contraction), as
// ops/hils_bidir_output_fusion_tilelang.py:28-35 evaluates it in fp32.
__device__ __forceinline__ uint32_t fuse_bf16x2(uint32_t r, uint32_t l, float w) {
  const float lo = __fadd_rn(bf16_lo(r), __fmul_rn(w, bf16_lo(l)));
  const float hi = __fadd_rn(bf16_hi(r), __fmul_rn(w, bf16_hi(l)));
  return pack_bf16x2(lo, hi);
}

__device__ __forceinline__ f32x4_t mfma_bf16_16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x4_t zero4() {
  f32x4_t z = {0.f, 0.f, 0.f, 0.f};
  return z;
}

// Reductions inside groups of 16 lanes (lanes sharing l / 16) with DPP lane
// moves, no LDS round trip: swap neighbours, swap pairs (quad_perm), then
// mirror within 8 lanes (row_half_mirror) and within 16 (row_mirror).  After
// each step every lane holds the reduction of a twice larger lane set.  Every
// lane of the wave must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf,
                                                            0xf, false));
}
__device__ __forceinline__ float group16_max(float v) {
  v = fmaxf(v, dpp_mov<0xb1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_mov<0x4e>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_mov<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_mov<0x140>(v));  // row_mirror
  return v;
}
__device__ __forceinline__ float group16_sum(float v) {
  v += dpp_mov<0xb1>(v);
  v += dpp_mov<0x4e>(v);
  v += dpp_mov<0x141>(v);
  v += dpp_mov<0x140>(v);
  return v;
}
__device__ __forceinline__ int group16_sum_i(int v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// Integer reductions and prefix sums inside groups of 8 consecutive lanes
// (lanes sharing l / 8), with DPP lane moves instead of LDS permutes:
// quad_perm swaps, then row_half_mirror pairs the two quads of each 8-lane
// half-row.  Every lane of the wave must be active.
template <int CTRL>
__device__ __forceinline__ int dpp_mov_i(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ int group8_sum_i(int v) {
  v += dpp_mov_i<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov_i<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov_i<0x141>(v);  // row_half_mirror
  return v;
}
__device__ __forceinline__ uint32_t group8_min_u(uint32_t v) {
  v = min(v, (uint32_t)dpp_mov_i<0xb1>((int)v));
  v = min(v, (uint32_t)dpp_mov_i<0x4e>((int)v));
  v = min(v, (uint32_t)dpp_mov_i<0x141>((int)v));
  return v;
}
__device__ __forceinline__ uint32_t group8_max_u(uint32_t v) {
  v = max(v, (uint32_t)dpp_mov_i<0xb1>((int)v));
  v = max(v, (uint32_t)dpp_mov_i<0x4e>((int)v));
  v = max(v, (uint32_t)dpp_mov_i<0x141>((int)v));
  return v;
}
__device__ __forceinline__ float group8_max_f(float v) {
  v = fmaxf(v, __int_as_float(dpp_mov_i<0xb1>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_mov_i<0x4e>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_mov_i<0x141>(__float_as_int(v))));
  return v;
}
// Exclusive prefix sum over the 8 lanes of a group (sub = l % 8): row_shr:o
// brings lane l - o, which is in the same group when sub >= o.
__device__ __forceinline__ int group8_excl_scan_i(int v, int sub) {
  int incl = v, up;
  up = dpp_mov_i<0x111>(incl);  // row_shr:1
  if (sub >= 1) incl += up;
  up = dpp_mov_i<0x112>(incl);  // row_shr:2
  if (sub >= 2) incl += up;
  up = dpp_mov_i<0x114>(incl);  // row_shr:4
  if (sub >= 4) incl += up;
  return incl - v;
}

// Reductions across the four lane groups (lanes sharing l % 16), with the
// gfx950 row-swap instructions: v_permlane32_swap exchanges the upper half of
// one operand with the lower half of the other, so swapping a value with
// itself leaves lane l holding the values of lanes l and l ^ 32 in the two
// results (v_permlane16_swap likewise pairs lanes l and l ^ 16).  Pure VALU,
// no LDS round trip.
__device__ __forceinline__ void pair32(float v, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ void pair16(float v, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
  float d;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}
__device__ __forceinline__ float max_raw(float a, float b) {
  float d;
  asm("v_max_f32 %0, %1, %2" : "=v"(d) : "v"(a), "v"(b));
  return d;
}
// Max of the 16 accumulator values a lane holds for one 64-row tile.
__device__ __forceinline__ float across4_max(float v) {
  float a, b;
  pair32(v, a, b);
  pair16(max_raw(a, b), a, b);
  return max_raw(a, b);
}
__device__ __forceinline__ float across4_sum(float v) {
  float a, b;
  pair32(v, a, b);
  pair16(a + b, a, b);
  return a + b;
}

// 2^x with the hardware instruction (v_exp_f32): exact at 0, 2^-inf = 0;
// results below the normal range flush to zero, which no caller can observe
// after bf16 rounding of probabilities that are normalised to at most 1.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// 1/x with the hardware reciprocal (1 ulp).
__device__ __forceinline__ float rcp_hw(float x) { return __builtin_amdgcn_rcpf(x); }

// log2(x) with the hardware instruction (v_log_f32, ~1 ulp for normal x).
__device__ __forceinline__ float log2_hw(float x) { return __builtin_amdgcn_logf(x); }
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v = min(v, __shfl_xor(v, o, 64));
  return v;
}

// Max of the 16 accumulator values a lane holds for one 64-row tile.  Plain
// builtins (the compiler forms v_max3 and needs no input canonicalisation
// for matrix-core results): inline asm must not read matrix-core results,
// since the compiler cannot insert the wait states the hardware requires
// between an MFMA and an asm instruction that reads its result.
__device__ __forceinline__ float max16_raw(const f32x4_t (&S)[4]) {
  float m = __builtin_fmaxf(__builtin_fmaxf(S[0][0], S[0][1]), S[0][2]);
#pragma unroll
  for (int i = 3; i < 16; ++i) m = __builtin_fmaxf(m, S[i >> 2][i & 3]);
  return m;
}
// x = v in the lanes set in `lanes` (v_cndmask with the mask as condition).
__device__ __forceinline__ float set_where(float x, uint64_t lanes, float v) {
  return __builtin_amdgcn_inverse_ballot_w64(lanes) ? v : x;
}

// Order-preserving map from fp32 to uint32 (larger float -> larger key).
__device__ __forceinline__ uint32_t float_order_key(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// torch.logaddexp for fp32 scalars: both -inf -> -inf.
__device__ __forceinline__ float logaddexp_f(float a, float b) {
  float m = fmaxf(a, b);
  if (m == neg_inf()) return m;
  return m + log1pf(expf(-fabsf(a - b)));
}

// The routed backward's dQ walk (routed_attention.hip): grad_q += the dS . K
// terms of each query's listed chunks (first occurrences), from the dS
// records the chunk-major backward kernel wrote ([B, Lq, Hq, K] x 64 bf16).
int routed_dq_walk(const void* kv_frags_bwd, const void* ds_records, const int32_t* indices,
                   const uint8_t* key_valid, int64_t batch, int64_t q_len, int64_t kv_len,
                   int64_t q_heads, int64_t kv_heads, int64_t topk, float* grad_q,
                   void* stream);

}  // namespace mrsa

// Host helpers for launch-status mapping.
static inline int mrsa_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? MRSA_OK : MRSA_ERR_LAUNCH;
}
