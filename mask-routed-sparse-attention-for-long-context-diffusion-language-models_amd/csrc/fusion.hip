// Output fusion: out = bf16(remote + local_weight * local), one HBM stream.
// Semantics: ops/hils_bidir_output_fusion_tilelang.py:28-35 (fp32 math on
// widened bf16, one rounding to bf16 at the end).  The multiply and the add
// are rounded separately (no FMA contraction) so the result is bit-identical
// to the same expression evaluated in fp32 on the CPU.
#include "mrsa_device.h"

using namespace mrsa;

namespace {

__device__ __forceinline__ uint32_t fuse_pair(uint32_t r, uint32_t l, float w) {
  return fuse_bf16x2(r, l, w);
}

// Vector path: 8 bf16 (16 bytes) per lane-iteration; head_dim % 8 == 0.
__global__ void __launch_bounds__(256) fuse_vec_kernel(const u32x4_t* __restrict__ remote,
                                                       const u32x4_t* __restrict__ local,
                                                       const uint16_t* __restrict__ weight,
                                                       u32x4_t* __restrict__ out, int64_t nvec,
                                                       int64_t vec_per_row) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < nvec; v += stride) {
    const float w = bf16_to_f32(weight[v / vec_per_row]);
    const u32x4_t r = __builtin_nontemporal_load(&remote[v]);
    const u32x4_t l = __builtin_nontemporal_load(&local[v]);
    u32x4_t o;
    o[0] = fuse_pair(r[0], l[0], w);
    o[1] = fuse_pair(r[1], l[1], w);
    o[2] = fuse_pair(r[2], l[2], w);
    o[3] = fuse_pair(r[3], l[3], w);
    __builtin_nontemporal_store(o, &out[v]);
  }
}

__global__ void __launch_bounds__(256) fuse_scalar_kernel(const uint16_t* __restrict__ remote,
                                                          const uint16_t* __restrict__ local,
                                                          const uint16_t* __restrict__ weight,
                                                          uint16_t* __restrict__ out, int64_t n,
                                                          int64_t head_dim) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += stride) {
    const float w = bf16_to_f32(weight[e / head_dim]);
    const float v = __fadd_rn(bf16_to_f32(remote[e]), __fmul_rn(w, bf16_to_f32(local[e])));
    out[e] = (uint16_t)f32_to_bf16(v);
  }
}

}  // namespace

extern "C" int mrsa_fuse_hils_outputs_fwd(const void* remote_output, const void* local_output,
                                          const void* local_weight, void* output, int64_t rows,
                                          int64_t head_dim, void* stream) {
  if (rows < 0 || head_dim <= 0) return MRSA_ERR_INVALID_ARGUMENT;
  if (rows == 0) return MRSA_OK;
  if (!remote_output || !local_output || !local_weight || !output) return MRSA_ERR_INVALID_ARGUMENT;
  const bool aligned = ((uintptr_t)remote_output | (uintptr_t)local_output | (uintptr_t)output) % 16 == 0;
  hipStream_t s = (hipStream_t)stream;
  if (head_dim % 8 == 0 && aligned) {
    const int64_t nvec = rows * head_dim / 8;
    const int64_t blocks = std::min<int64_t>((nvec + 255) / 256, 256 * 32);
    hipLaunchKernelGGL(fuse_vec_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                       (const u32x4_t*)remote_output, (const u32x4_t*)local_output,
                       (const uint16_t*)local_weight, (u32x4_t*)output, nvec, head_dim / 8);
  } else {
    const int64_t n = rows * head_dim;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 256 * 32);
    hipLaunchKernelGGL(fuse_scalar_kernel, dim3((unsigned)blocks), dim3(256), 0, s,
                       (const uint16_t*)remote_output, (const uint16_t*)local_output,
                       (const uint16_t*)local_weight, (uint16_t*)output, n, head_dim);
  }
  return mrsa_launch_status();
}

namespace {

// Backward of the fusion (ops/hils_bidir_output_fusion_tilelang.py:40-77):
// d_remote = g, d_local = bf16(w g), d_weight = bf16(sum_d g l) with fp32
// products and sum.  Sixteen lanes per row, four rows per wave; a lane walks
// the row in 16-byte vectors (VEC: head_dim % 8 == 0, aligned rows) or in
// single elements, and the row sum closes with xor shuffles inside each
// 16-lane group.
template <bool VEC>
__global__ void __launch_bounds__(256) fuse_bwd_kernel(const uint16_t* __restrict__ local,
                                                       const uint16_t* __restrict__ weight,
                                                       const uint16_t* __restrict__ grad,
                                                       uint16_t* __restrict__ d_remote,
                                                       uint16_t* __restrict__ d_local,
                                                       uint16_t* __restrict__ d_weight,
                                                       int64_t rows, int D) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = t >> 4;
  const int sub = (int)(t & 15);
  const bool ok = row < rows;
  float part = 0.f;
  if (ok) {
    const float w = bf16_to_f32(weight[row]);
    const int64_t base = row * D;
    if (VEC) {
      for (int e = sub * 8; e < D; e += 128) {
        const u32x4_t g = *reinterpret_cast<const u32x4_t*>(grad + base + e);
        const u32x4_t l = *reinterpret_cast<const u32x4_t*>(local + base + e);
        *reinterpret_cast<u32x4_t*>(d_remote + base + e) = g;
        u32x4_t dl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float g0 = bf16_lo(g[i]), g1 = bf16_hi(g[i]);
          dl[i] = pack_bf16x2(g0 * w, g1 * w);
          part += g0 * bf16_lo(l[i]);
          part += g1 * bf16_hi(l[i]);
        }
        *reinterpret_cast<u32x4_t*>(d_local + base + e) = dl;
      }
    } else {
      for (int e = sub; e < D; e += 16) {
        const uint16_t gb = grad[base + e];
        const float g = bf16_to_f32(gb);
        d_remote[base + e] = gb;
        d_local[base + e] = (uint16_t)f32_to_bf16(g * w);
        part += g * bf16_to_f32(local[base + e]);
      }
    }
  }
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) part += __shfl_xor(part, o, 64);
  if (ok && sub == 0) d_weight[row] = (uint16_t)f32_to_bf16(part);
}

}  // namespace

extern "C" int mrsa_fuse_hils_outputs_bwd(const void* local_output, const void* local_weight,
                                          const void* grad_output, void* d_remote, void* d_local,
                                          void* d_weight, int64_t rows, int64_t head_dim,
                                          void* stream) {
  if (rows < 0 || head_dim <= 0) return MRSA_ERR_INVALID_ARGUMENT;
  if (rows == 0) return MRSA_OK;
  if (!local_output || !local_weight || !grad_output || !d_remote || !d_local || !d_weight)
    return MRSA_ERR_INVALID_ARGUMENT;
  if (head_dim > 0x7fffffff / 16) return MRSA_ERR_UNSUPPORTED;
  const bool vec = head_dim % 8 == 0 && ((uintptr_t)local_output | (uintptr_t)grad_output |
                                         (uintptr_t)d_remote | (uintptr_t)d_local) % 16 == 0;
  const int64_t blocks = (rows * 16 + 255) / 256;
  if (blocks > 0x7fffffff) return MRSA_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(vec ? fuse_bwd_kernel<true> : fuse_bwd_kernel<false>, dim3((unsigned)blocks),
                     dim3(256), 0, (hipStream_t)stream, (const uint16_t*)local_output,
                     (const uint16_t*)local_weight, (const uint16_t*)grad_output,
                     (uint16_t*)d_remote, (uint16_t*)d_local, (uint16_t*)d_weight, rows,
                     (int)head_dim);
  return mrsa_launch_status();
}
