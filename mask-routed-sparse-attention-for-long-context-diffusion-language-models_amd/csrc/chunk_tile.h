// Shared pieces of the window-attention kernel: asm LDS operand reads with
// explicit waits, and the S^T = K.Q^T product of one 16-column tile over a
// 64-key tile held in an LDS slot.
//
// Slot layout (32 KB): the tile's K / V fragments (mrsa_kv_fragments): 32
// operand images of 1 KB, lane l's 16 bytes at 16 l; K image 4 mt + ks holds
// keys 16 mt.. x dims 32 ks.., V image 2 nt + ks holds dims 16 nt.. x keys
// 32 ks.. (tiled order).
#pragma once

#include <utility>

#include "mrsa_device.h"

namespace mrsa {

typedef __attribute__((address_space(3))) void lds_void_t;

// Matrix-operand reads from LDS with explicit waits.  With global->LDS DMA in
// the same loop the compiler waits for every outstanding LDS read before each
// use (lgkmcnt(0)); issuing the reads as asm and waiting with lgkmcnt(n) on
// the value itself keeps eight reads in flight.  LDS reads complete in issue
// order, so lgkmcnt(n) after a read followed by >= n later LDS reads
// guarantees that read has landed (other LDS accesses only add to the count).
template <int OFF>
__device__ __forceinline__ u32x4_t lds_read_b128(uint32_t addr) {
  u32x4_t r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
template <int N>
__device__ __forceinline__ void lds_wait(u32x4_t& v) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(v) : "i"(N));
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

template <int N, class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}

// S^T = K . Q^T for one column tile: 16 K operand reads from a fragment slot
// (laddr = slot + 16 lane; product o = rows 16 (o & 3).., reduction step
// o >> 2 reads image 4 (o & 3) + (o >> 2)) and 16 products, read o + DEPTH
// issued after product o so DEPTH reads stay in flight.
template <int O>
constexpr int kimg_off() { return (4 * (O & 3) + (O >> 2)) * 1024; }

template <int DEPTH = 8>
__device__ __forceinline__ void qk_frag(uint32_t laddr, const u32x4_t (&Q)[4], f32x4_t (&S)[4]) {
#pragma unroll
  for (int t = 0; t < 4; ++t) S[t] = zero4();
  u32x4_t kb[16];
  static_for<16>([&](auto oc) {
    constexpr int o = decltype(oc)::value;
    if constexpr (o < DEPTH) kb[o] = lds_read_b128<kimg_off<o>()>(laddr);
  });
  static_for<16>([&](auto oc) {
    constexpr int o = decltype(oc)::value;
    lds_wait<(15 - o < DEPTH - 1 ? 15 - o : DEPTH - 1)>(kb[o]);
    S[o & 3] = mfma_bf16_16x16x32(kb[o], Q[o >> 2], S[o & 3]);
    if constexpr (o + DEPTH < 16) kb[o + DEPTH] = lds_read_b128<kimg_off<o + DEPTH>()>(laddr);
    __builtin_amdgcn_sched_barrier(0);
  });
}

// A wave-uniform 64-bit value in scalar registers.
__device__ __forceinline__ uint64_t uniform_u64(uint64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}

// 64-bit LDS word accesses as asm: the compiler would otherwise wait for all
// outstanding global->LDS DMA before touching LDS it cannot prove disjoint.
__device__ __forceinline__ uint64_t lds_read_u64(uint32_t addr) {
  uint64_t v;
  asm volatile("ds_read_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
  return v;
}
__device__ __forceinline__ void lds_write_u64(uint32_t addr, uint64_t v) {
  asm volatile("ds_write_b64 %0, %1" ::"v"(addr), "v"(v) : "memory");
}

}  // namespace mrsa
