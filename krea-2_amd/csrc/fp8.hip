// fp8-e4m3 weight-only base, the reference's own quantized Linear (Fp8Linear, quantize.py:23-51):
//   init     scale[n] = max(amax_k |W[n,k]|, 1e-8) / 448 (f32), q = e4m3(clamp(W / scale, +-448)) (round to
//            nearest even), scale stored as bf16
//   forward  w = bf16(float(q) * float(bf16 scale)) per element (the reference's `q.to(bf16) * scale`), then
//            a bf16 GEMM with f32 accumulation plus bias (F.linear)
// The e4m3 encode/decode is written out from the format (1 sign, 4 exponent bits with bias 7, 3 mantissa
// bits, no infinities, S.1111.111 = NaN, largest finite 448), so it does not depend on a conversion mode of
// the hardware.  Dequantization writes the bf16 weight (or its transpose, for dX) for the bf16 GEMMs of
// gemm.hip.
#include "k2q_common.h"

namespace {

// f32 (|v| <= 448 or NaN) -> e4m3fn code, round to nearest even.
__device__ __forceinline__ uint32_t e4m3_encode(float v) {
  const uint32_t bits = __float_as_uint(v);
  const uint32_t sign = (bits >> 24) & 0x80u;
  if (v != v) return sign | 0x7Fu;
  const float a = fabsf(v);
  uint32_t code;
  if (a < 0.015625f) {                       // below 2^-6: subnormal step 2^-9 (exact scaling, RNE)
    code = (uint32_t)__builtin_rintf(a * 512.f);   // 0..8; 8 is the smallest normal's code
  } else {
    const uint32_t ab = __float_as_uint(a);
    const uint32_t e = (ab >> 23) - 127 + 7;   // 1..8
    const uint32_t mant = ab & 0x7FFFFFu;
    uint32_t r = mant >> 20;
    const uint32_t rem = mant & 0xFFFFFu;
    r += (rem > 0x80000u || (rem == 0x80000u && (r & 1u))) ? 1u : 0u;
    code = (e << 3) + r;                     // a carry out of the mantissa moves into the exponent
  }
  return sign | code;
}

// e4m3fn code -> f32 (exact).
__device__ __forceinline__ float e4m3_decode(uint32_t b) {
  const uint32_t sign = (b & 0x80u) << 24;
  const uint32_t e = (b >> 3) & 15u, m = b & 7u;
  if ((b & 0x7Fu) == 0x7Fu) return __uint_as_float(sign | 0x7FC00000u);
  if (e == 0) return __uint_as_float(sign | __float_as_uint((float)m * 0.001953125f));   // m * 2^-9
  return __uint_as_float(sign | ((e + 120u) << 23) | (m << 20));
}

template <typename T>
__device__ __forceinline__ float load_f32(const T* p, int64_t i);
template <>
__device__ __forceinline__ float load_f32<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float load_f32<uint16_t>(const uint16_t* p, int64_t i) { return bf16_bits_to_f32(p[i]); }

// One row per 256-thread workgroup.
template <typename T>
__global__ __launch_bounds__(256) void quant_fp8_kernel(const T* __restrict__ w, int64_t K, uint8_t* __restrict__ q,
                                                        uint16_t* __restrict__ s) {
  __shared__ float red[4];
  const int64_t n = blockIdx.x;
  const T* row = w + n * K;
  float amax = 0.f;
  for (int64_t k = threadIdx.x; k < K; k += 256) amax = fmaxf(amax, fabsf(load_f32(row, k)));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float scale = __fdiv_rn(fmaxf(amax, 1e-8f), 448.f);
  for (int64_t k = threadIdx.x; k < K; k += 256) {
    float v = __fdiv_rn(load_f32(row, k), scale);
    if (v == v) v = fminf(fmaxf(v, -448.f), 448.f);
    q[n * K + k] = (uint8_t)e4m3_encode(v);
  }
  if (threadIdx.x == 0) s[n] = (uint16_t)f32_to_bf16_bits(scale);
}

// w[n][k] = bf16(decode(q[n][k]) * bf16 s[n]), 16 codes per thread.
__global__ __launch_bounds__(256) void dequant_fp8_kernel(const uint8_t* __restrict__ q, const uint16_t* __restrict__ s,
                                                          int64_t N, int64_t K, uint16_t* __restrict__ w) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 16;   // element index, K % 16 == 0
  if (i >= N * K) return;
  const float sc = bf16_bits_to_f32(s[i / K]);
  const v4u c = *reinterpret_cast<const v4u*>(q + i);
  v4u o[2];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t word = c[j >> 1], sh = 16 * (j & 1);
    const float a = e4m3_decode((word >> sh) & 0xFFu) * sc;
    const float b = e4m3_decode((word >> (sh + 8)) & 0xFFu) * sc;
    o[j >> 2][j & 3] = pack_bf16x2(a, b);
  }
  *reinterpret_cast<v4u*>(w + i) = o[0];
  *reinterpret_cast<v4u*>(w + i + 8) = o[1];
}

// wt[k][n] = the same values transposed (K x N), through a 64 x 64 LDS tile.
__global__ __launch_bounds__(256) void dequant_fp8_t_kernel(const uint8_t* __restrict__ q, const uint16_t* __restrict__ s,
                                                            int64_t N, int64_t K, uint16_t* __restrict__ wt) {
  __shared__ uint16_t tile[64][64 + 2];
  const int t = threadIdx.x;
  const int64_t n0 = (int64_t)blockIdx.x * 64, k0 = (int64_t)blockIdx.y * 64;
  {
    const int nl = t >> 2, kl = 16 * (t & 3);
    const int64_t n = n0 + nl;
    if (n < N) {
      const float sc = bf16_bits_to_f32(s[n]);
      const v4u c = *reinterpret_cast<const v4u*>(q + n * K + k0 + kl);
#pragma unroll
      for (int j = 0; j < 16; ++j)
        tile[kl + j][nl] = (uint16_t)f32_to_bf16_bits(e4m3_decode((c[j >> 2] >> (8 * (j & 3))) & 0xFFu) * sc);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) tile[kl + j][nl] = 0;
    }
  }
  __syncthreads();
  const int kl = t >> 2, nl = 16 * (t & 3);
  const int64_t k = k0 + kl;
  if (k >= K) return;
  uint16_t* dst = wt + k * N + n0 + nl;
  if (n0 + nl + 16 <= N) {
    uint32_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (uint32_t)tile[kl][nl + 2 * j] | ((uint32_t)tile[kl][nl + 2 * j + 1] << 16);
    *reinterpret_cast<v4u*>(dst) = v4u{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<v4u*>(dst + 8) = v4u{v[4], v[5], v[6], v[7]};
  } else {
    for (int j = 0; j < 16 && n0 + nl + j < N; ++j) dst[j] = tile[kl][nl + j];
  }
}

}  // namespace

extern "C" int k2q_quant_weight_fp8(const void* w, int w_dtype, int64_t N, int64_t K, uint8_t* q, uint16_t* s,
                                    void* stream) {
  if (!w || !q || !s || N < 1 || K < 1 || N > 0x7fffffff) return K2Q_EINVAL;
  if (w_dtype != K2Q_DTYPE_BF16 && w_dtype != K2Q_DTYPE_F32) return K2Q_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (w_dtype == K2Q_DTYPE_BF16)
    hipLaunchKernelGGL(quant_fp8_kernel<uint16_t>, dim3((unsigned)N), dim3(256), 0, st,
                       static_cast<const uint16_t*>(w), K, q, s);
  else
    hipLaunchKernelGGL(quant_fp8_kernel<float>, dim3((unsigned)N), dim3(256), 0, st, static_cast<const float*>(w),
                       K, q, s);
  return k2q_launch_status();
}

extern "C" int k2q_dequant_fp8(const uint8_t* q, const uint16_t* s, int64_t N, int64_t K, int transpose,
                               uint16_t* out, void* stream) {
  if (!q || !s || !out || N < 1 || K < 64 || K % 64) return K2Q_EINVAL;
  if (!k2q_aligned(q, 16) || !k2q_aligned(out, 16)) return K2Q_EINVAL;
  if (transpose && N % 8) return K2Q_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (transpose) {
    const dim3 grid((unsigned)((N + 63) / 64), (unsigned)(K / 64));
    hipLaunchKernelGGL(dequant_fp8_t_kernel, grid, dim3(256), 0, st, q, s, N, K, out);
  } else {
    const int64_t threads = N * K / 16;
    hipLaunchKernelGGL(dequant_fp8_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, q, s, N, K, out);
  }
  return k2q_launch_status();
}
