// Same-run ceiling for the int8 GEMM: a loop of nothing but v_mfma_i32_32x32x32_i8 on every SIMD, two
// waves per SIMD as in the GEMM, operands in registers.  Each wave holds 8 A and 8 B fragments of
// pseudo-random int8 codes and cycles through all 64 pairs, so consecutive MFMAs see different operands
// (the chip's power, and with it the clock, depends on how many operand bits toggle).  The number it gives
// is the int8 MFMA rate this board sustains in the current run, for comparison with the GEMM.
//
// A measurement aid of bench.py, built into its own library (libk2q_probe.so), not part of the product's
// C ABI (libk2q.so, include/k2q.h).  bench.py binds the two entry points with ctypes:
//   int64_t k2q_mfma_probe_i8_ops(int64_t iters, int64_t workgroups)   int8 operations of one launch
//   int k2q_mfma_probe_i8(int64_t iters, int64_t workgroups, int32_t* out, void* stream)
//     iters x 64 MFMAs per wave, 8 waves per workgroup; out holds workgroups * 512 int32 checksums.
#include "k2q_common.h"

namespace {

__device__ __forceinline__ uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return x;
}

__global__ __launch_bounds__(512, 1) void mfma_probe_i8_kernel(int64_t iters, int32_t* __restrict__ out) {
  const uint32_t seed = (uint32_t)(blockIdx.x * 512 + threadIdx.x) * 64u;
  v4i a[8], b[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a[j][e] = (int)mix32(seed + 8 * j + e);
      b[j][e] = (int)mix32(seed + 8 * j + e + 32);
    }
  v16i acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = v16i{0};
  for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i)   // 8 independent accumulators back to back
        acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[(i + j) & 7], b[j], acc[i], 0, 0, 0);
  }
  int s = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) s ^= acc[i][e];
  out[blockIdx.x * 512 + threadIdx.x] = s;
}

}  // namespace

extern "C" int64_t k2q_mfma_probe_i8_ops(int64_t iters, int64_t workgroups) {
  return workgroups * 8 * iters * 64 * (int64_t)(2 * 32 * 32 * 32);
}

extern "C" int k2q_mfma_probe_i8(int64_t iters, int64_t workgroups, int32_t* out, void* stream) {
  if (iters < 1 || workgroups < 1 || workgroups > 65535 || !out) return K2Q_EINVAL;
  hipLaunchKernelGGL(mfma_probe_i8_kernel, dim3((unsigned)workgroups), dim3(512), 0,
                     static_cast<hipStream_t>(stream), iters, out);
  return k2q_launch_status();
}
