// Kernel (1): block Walsh-Hadamard rotation + per-row int8 quantization (and the int4 group-64 weight
// quantizer), one HBM pass.
//
// Spec (no reference code exists for it): BASELINE.json north_star kernel (1); the absmax floor mirrors
// reference quantize.py:36.  Arithmetic, fixed so the int8 codes are bit-exact:
//   * FWHT of every 128-wide block, float32, unnormalised, radix-2 butterfly with stage strides
//     1, 2, 4, ..., 64 in that order; the pair (i, i+s) becomes (a+b, a-b).
//   * absmax over the whole rotated row, floored at 1e-8; inv = 127/absmax and s = absmax/127, each one
//     correctly rounded float32 division; q = rint(v*inv) (round half to even), |q| <= 127.
//   * int4 groups: absmax of each 64-wide group, s = bf16_rne(absmax/7), q = clamp(rint(v/s), -7, 7).
//
// Layout in registers: a team of T = 64*WPR lanes owns one row.  Each lane holds 16 contiguous elements
// per chunk (two 16-byte loads for bf16).  Inside a 16-lane DPP row, lane bit 2 selects one of two
// Hadamard blocks and lane bits 0, 1, 3 are block bits 4, 5, 6, so the four in-lane stages are strides
// 1..8 and the three cross-lane stages are single DPP ops: quad_perm xor1, quad_perm xor2, row_ror:8.
// Cross-lane stages are one exact FMA per element: v <- partner * c + v with c = -1 on the lane holding
// the upper element, which leaves that lane holding the negated result.  The sign each lane ends with is
// (-1)^(lane bit0 + bit1 + bit3); it is folded into the quantizer's multiplier (sign flips are exact).
#include "k2q_common.h"

namespace {

constexpr int kMaxNCH = 4;  // chunks of 16 elements per lane (K <= 1024 * WPR * 4)

enum { MODE_ROW_I8 = 0, MODE_GROUP_I4 = 1 };

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

template <typename Tin>
__device__ __forceinline__ void load16(const Tin* p, bool ok, float (&v)[16]);

template <>
__device__ __forceinline__ void load16<__bf16>(const __bf16* p, bool ok, float (&v)[16]) {
  uint4 a = make_uint4(0, 0, 0, 0), b = make_uint4(0, 0, 0, 0);
  if (ok) {
    a = *reinterpret_cast<const uint4*>(p);
    b = *reinterpret_cast<const uint4*>(p + 8);
  }
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    v[2 * j] = __uint_as_float(w[j] << 16);
    v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
  }
}

template <>
__device__ __forceinline__ void load16<float>(const float* p, bool ok, float (&v)[16]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
    if (ok) a = reinterpret_cast<const float4*>(p)[j];
    v[4 * j] = a.x;
    v[4 * j + 1] = a.y;
    v[4 * j + 2] = a.z;
    v[4 * j + 3] = a.w;
  }
}

__device__ __forceinline__ float wave_max(float m) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  return m;
}

template <typename Tin, int WPR, int MODE, int kNCH>
__global__ __launch_bounds__(256) void rotquant_kernel(const Tin* __restrict__ x, int64_t M, int K,
                                                       int64_t ldx, int8_t* __restrict__ q,
                                                       float* __restrict__ s,
                                                       uint16_t* __restrict__ xrot,
                                                       uint8_t* __restrict__ q4,
                                                       uint16_t* __restrict__ s4) {
  constexpr int T = 64 * WPR;        // lanes per row
  constexpr int CW = T * 16;         // elements per chunk
  constexpr int ROWS = 4 / WPR;      // rows per workgroup
  __shared__ float smax[4];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * ROWS + wave / WPR;
  const int t = (wave % WPR) * 64 + lane;
  const int l = t & 15;
  const int blk = 2 * (t >> 4) + ((l >> 2) & 1);
  const int pos = 16 * ((l & 1) | (((l >> 1) & 1) << 1) | (((l >> 3) & 1) << 2));
  const int off = blk * K2Q_HADAMARD + pos;
  const bool row_ok = row < M;
  constexpr int nch = kNCH;

  const Tin* xr = x + (row_ok ? row : 0) * ldx;
  float v[kNCH][16];
#pragma unroll
  for (int c = 0; c < kNCH; ++c) {
    const int col = c * CW + off;
    load16<Tin>(xr + col, row_ok && c < nch && col < K, v[c]);
  }

  // Cross-lane stage multipliers: -1 on the lane holding the upper element of each pair.
  const float c1 = (l & 1) ? -1.f : 1.f;
  const float c2 = (l & 2) ? -1.f : 1.f;
  const float c8 = (l & 8) ? -1.f : 1.f;
  const float sigma = c1 * c2 * c8;  // sign each lane's stored values carry after the DPP stages

  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < kNCH; ++c) {
#pragma unroll
    for (int st = 1; st < 16; st <<= 1) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (i & st) continue;
        const float a = v[c][i], b = v[c][i + st];
        v[c][i] = a + b;
        v[c][i + st] = a - b;
      }
    }
    // One v_fmac_f32_dpp per element and stage: v += partner(v) * c.  The 16 registers are visited
    // round-robin, so a DPP read never follows the VALU write of its own source closer than 15
    // instructions; the s_nop before each stage covers the in-lane stage's last writes.
    asm volatile("s_nop 1" ::: "memory");
#pragma unroll
    for (int i = 0; i < 16; ++i)
      asm volatile("v_fmac_f32_dpp %0, %0, %1 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf" : "+v"(v[c][i]) : "v"(c1));
    asm volatile("s_nop 1" ::: "memory");
#pragma unroll
    for (int i = 0; i < 16; ++i)
      asm volatile("v_fmac_f32_dpp %0, %0, %1 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf" : "+v"(v[c][i]) : "v"(c2));
    asm volatile("s_nop 1" ::: "memory");
#pragma unroll
    for (int i = 0; i < 16; ++i)
      asm volatile("v_fmac_f32_dpp %0, %0, %1 row_ror:8 row_mask:0xf bank_mask:0xf" : "+v"(v[c][i]) : "v"(c8));
    if (MODE == MODE_ROW_I8) {
#pragma unroll
      for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[c][i]));
    }
  }

  if (MODE == MODE_ROW_I8) {
    amax = wave_max(amax);
    if (WPR > 1) {
      if (lane == 0) smax[wave] = amax;
      __syncthreads();
      const int w0 = (wave / WPR) * WPR;
#pragma unroll
      for (int w = 0; w < WPR; ++w) amax = fmaxf(amax, smax[w0 + w]);
    }
    amax = fmaxf(amax, 1e-8f);
    const float inv = __fdiv_rn(127.f, amax);
    if (!row_ok) return;
    if (t == 0) s[row] = __fdiv_rn(amax, 127.f);
    const float mul = inv * sigma;
    const float rs = 0.08838834764831845f * sigma;  // float32(1/sqrt(128)) with the lane's sign
    int8_t* qr = q + row * (int64_t)K;
#pragma unroll
    for (int c = 0; c < kNCH; ++c) {
      const int col = c * CW + off;
      if (c >= nch || col >= K) continue;
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t p = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int qi = (int)__builtin_rintf(v[c][4 * j + e] * mul);
          p |= ((uint32_t)qi & 0xffu) << (8 * e);
        }
        w[j] = p;
      }
      *reinterpret_cast<uint4*>(qr + col) = make_uint4(w[0], w[1], w[2], w[3]);
      if (xrot) {
        uint32_t h[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = pack_bf16x2(v[c][2 * j] * rs, v[c][2 * j + 1] * rs);
        uint16_t* xo = xrot + row * (int64_t)K + col;
        reinterpret_cast<uint4*>(xo)[0] = make_uint4(h[0], h[1], h[2], h[3]);
        reinterpret_cast<uint4*>(xo)[1] = make_uint4(h[4], h[5], h[6], h[7]);
      }
    }
  } else {
    // int4 groups of 64: a group is the 4 lanes of one DPP quad (lane bits 0, 1) x 16 elements.
    if (!row_ok) return;
#pragma unroll
    for (int c = 0; c < kNCH; ++c) {
      const int col = c * CW + off;
      float gm = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) gm = fmaxf(gm, fabsf(v[c][i]));
      gm = fmaxf(gm, dpp_f<0xB1>(gm));
      gm = fmaxf(gm, dpp_f<0x4E>(gm));
      if (c >= nch || col >= K) continue;
      gm = fmaxf(gm, 1e-8f);
      const uint32_t sb = f32_to_bf16_bits(__fdiv_rn(gm, 7.f));
      const float sv = bf16_bits_to_f32(sb);
      if ((l & 3) == 0) s4[(int64_t)(col / 64) * M + row] = (uint16_t)sb;  // group-major
      int qi[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float r = __builtin_rintf(__fdiv_rn(v[c][i] * sigma, sv));
        r = fminf(fmaxf(r, -7.f), 7.f);
        qi[i] = (int)r;
      }
      uint32_t w0 = 0, w1 = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        w0 |= (((uint32_t)qi[j] & 0xfu) | (((uint32_t)qi[j + 8] & 0xfu) << 4)) << (8 * j);
        w1 |= (((uint32_t)qi[j + 4] & 0xfu) | (((uint32_t)qi[j + 12] & 0xfu) << 4)) << (8 * j);
      }
      *reinterpret_cast<uint2*>(q4 + row * (int64_t)(K / 2) + col / 2) = make_uint2(w0, w1);
    }
  }
}

template <typename Tin, int WPR, int MODE>
void launch_wpr(const Tin* xp, int64_t M, int64_t K, int64_t ldx, int8_t* q, float* s, uint16_t* xrot, uint8_t* q4,
                uint16_t* s4, hipStream_t st) {
  const dim3 grid((unsigned)((M + (4 / WPR) - 1) / (4 / WPR)));
  const int nch = (int)((K + 1024 * WPR - 1) / (1024 * WPR));   // chunks of 16 elements per lane
  switch (nch) {
    case 1: hipLaunchKernelGGL((rotquant_kernel<Tin, WPR, MODE, 1>), grid, dim3(256), 0, st, xp, M, (int)K, ldx, q, s, xrot, q4, s4); break;
    case 2: hipLaunchKernelGGL((rotquant_kernel<Tin, WPR, MODE, 2>), grid, dim3(256), 0, st, xp, M, (int)K, ldx, q, s, xrot, q4, s4); break;
    case 3: hipLaunchKernelGGL((rotquant_kernel<Tin, WPR, MODE, 3>), grid, dim3(256), 0, st, xp, M, (int)K, ldx, q, s, xrot, q4, s4); break;
    default: hipLaunchKernelGGL((rotquant_kernel<Tin, WPR, MODE, 4>), grid, dim3(256), 0, st, xp, M, (int)K, ldx, q, s, xrot, q4, s4); break;
  }
}

template <typename Tin, int MODE>
int launch_rotquant(const void* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, float* s, uint16_t* xrot,
                    uint8_t* q4, uint16_t* s4, hipStream_t st) {
  const Tin* xp = static_cast<const Tin*>(x);
  if (K <= 4096) launch_wpr<Tin, 1, MODE>(xp, M, K, ldx, q, s, xrot, q4, s4, st);
  else if (K <= 8192) launch_wpr<Tin, 2, MODE>(xp, M, K, ldx, q, s, xrot, q4, s4, st);
  else if (K <= 16384) launch_wpr<Tin, 4, MODE>(xp, M, K, ldx, q, s, xrot, q4, s4, st);
  else return K2Q_EUNSUPPORTED;
  return k2q_launch_status();
}

int check_rotquant_args(const void* x, int dtype, int64_t M, int64_t K, int64_t ldx) {
  if (!x || M < 1 || K < K2Q_HADAMARD || K % K2Q_HADAMARD || ldx < K) return K2Q_EINVAL;
  if (dtype != K2Q_DTYPE_BF16 && dtype != K2Q_DTYPE_F32) return K2Q_EINVAL;
  if (!k2q_aligned(x, 16) || ldx % (dtype == K2Q_DTYPE_BF16 ? 8 : 4)) return K2Q_EINVAL;
  if (K > 16384) return K2Q_EUNSUPPORTED;
  return K2Q_OK;
}

}  // namespace

extern "C" int k2q_rotquant(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx, int8_t* q,
                            float* s, uint16_t* x_rot, void* stream) {
  int rc = check_rotquant_args(x, x_dtype, M, K, ldx);
  if (rc) return rc;
  if (!q || !s || !k2q_aligned(q, 16) || (x_rot && !k2q_aligned(x_rot, 16))) return K2Q_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (x_dtype == K2Q_DTYPE_BF16)
    return launch_rotquant<__bf16, MODE_ROW_I8>(x, M, K, ldx, q, s, x_rot, nullptr, nullptr, st);
  return launch_rotquant<float, MODE_ROW_I8>(x, M, K, ldx, q, s, x_rot, nullptr, nullptr, st);
}

extern "C" int k2q_quant_weight_i4(const void* w, int w_dtype, int64_t N, int64_t K, uint8_t* qw4,
                                   uint16_t* sw4, void* stream) {
  int rc = check_rotquant_args(w, w_dtype, N, K, K);
  if (rc) return rc;
  if (!qw4 || !sw4 || !k2q_aligned(qw4, 16) || !k2q_aligned(sw4, 4)) return K2Q_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (w_dtype == K2Q_DTYPE_BF16)
    return launch_rotquant<__bf16, MODE_GROUP_I4>(w, N, K, K, nullptr, nullptr, nullptr, qw4, sw4, st);
  return launch_rotquant<float, MODE_GROUP_I4>(w, N, K, K, nullptr, nullptr, nullptr, qw4, sw4, st);
}
