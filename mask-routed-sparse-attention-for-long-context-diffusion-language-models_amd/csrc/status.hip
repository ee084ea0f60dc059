// Status strings, ABI version and the matrix-core layout self-test.
#include "mrsa_device.h"

using namespace mrsa;

extern "C" const char* mrsa_status_string(int status) {
  switch (status) {
    case MRSA_OK: return "ok";
    case MRSA_ERR_INVALID_ARGUMENT: return "invalid argument (shape, size or pointer)";
    case MRSA_ERR_UNSUPPORTED: return "unsupported configuration for the gfx950 kernels";
    case MRSA_ERR_LAUNCH: return "HIP kernel launch failed";
    case MRSA_ERR_SCRATCH:
      return "problem needs more workspace than the static scratch buffer of the "
             "no-allocation entry point";
    default: return "unknown status";
  }
}

extern "C" int mrsa_abi_version(void) { return 8; }

// One wave: lane l loads row (l % 16) of A and column (l % 16) of B, eight
// consecutive reduction elements starting at 8 * (l / 16), and stores the
// result assuming C[4 * (l / 16) + i][l % 16].
__global__ void __launch_bounds__(64) selftest_mfma_kernel(const uint16_t* a, const uint16_t* b,
                                                           float* c) {
  const int l = threadIdx.x;
  const int r = l & 15, g = l >> 4;
  uint32_t av[4], bv[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int k0 = 8 * g + 2 * e;
    av[e] = (uint32_t)a[r * 32 + k0] | ((uint32_t)a[r * 32 + k0 + 1] << 16);
    bv[e] = (uint32_t)b[k0 * 16 + r] | ((uint32_t)b[(k0 + 1) * 16 + r] << 16);
  }
  u32x4_t A = {av[0], av[1], av[2], av[3]};
  u32x4_t B = {bv[0], bv[1], bv[2], bv[3]};
  f32x4_t acc = mfma_bf16_16x16x32(A, B, zero4());
#pragma unroll
  for (int i = 0; i < 4; ++i) c[(4 * g + i) * 16 + r] = acc[i];
}

extern "C" int mrsa_selftest_mfma_layout(const void* a, const void* b, float* c, void* stream) {
  if (!a || !b || !c) return MRSA_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(selftest_mfma_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     (const uint16_t*)a, (const uint16_t*)b, c);
  return mrsa_launch_status();
}
