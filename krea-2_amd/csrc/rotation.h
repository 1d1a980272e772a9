// Register-resident pieces of the block Walsh-Hadamard rotation + per-row int8 quantization, shared by
// rotate/quant (rotquant.hip) and the producer-fused variants (producers.hip).
//
// Layout in registers: a team of T = 64*WPR lanes owns one row.  Each lane holds 16 contiguous elements
// per chunk (two 16-byte loads for bf16).  Inside a 16-lane DPP row, lane bit 2 selects one of two
// Hadamard blocks and lane bits 0, 1, 3 are block bits 4, 5, 6, so the four in-lane stages are strides
// 1..8 and the three cross-lane stages are single DPP ops: quad_perm xor1, quad_perm xor2, row_ror:8.
// Cross-lane stages are one exact FMA per element: v <- partner * c + v with c = -1 on the lane holding
// the upper element, which leaves that lane holding the negated result.  The sign each lane ends with is
// (-1)^(lane bit0 + bit1 + bit3); it is folded into the quantizer's multiplier (sign flips are exact).
#pragma once

#include "k2q_common.h"

namespace k2q_rot {

// Position of lane t's 16 elements inside a 1024*WPR-element chunk (t = lane index within the row team).
__device__ __forceinline__ int lane_offset(int t) {
  const int l = t & 15;
  const int blk = 2 * (t >> 4) + ((l >> 2) & 1);
  const int pos = 16 * ((l & 1) | (((l >> 1) & 1) << 1) | (((l >> 3) & 1) << 2));
  return blk * K2Q_HADAMARD + pos;
}

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

// 16 bf16 values (already representable in bf16) stored as two 16-byte vectors.
__device__ __forceinline__ void store16_bf16(uint16_t* p, const float (&v)[16]) {
  uint32_t h[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) h[j] = pack_bf16x2(v[2 * j], v[2 * j + 1]);
  reinterpret_cast<uint4*>(p)[0] = make_uint4(h[0], h[1], h[2], h[3]);
  reinterpret_cast<uint4*>(p)[1] = make_uint4(h[4], h[5], h[6], h[7]);
}

// Wave-wide reductions, result in every lane: DPP inside each 16-lane row (quad_perm xor1, xor2,
// row_half_mirror, row_mirror), then the four row results through readlane.  The operation order is
// fixed, so the sum is deterministic.
template <bool kMax>
__device__ __forceinline__ float wave_reduce(float m) {
  auto op = [](float a, float b) { return kMax ? fmaxf(a, b) : a + b; };
  m = op(m, dpp_f<0xB1>(m));
  m = op(m, dpp_f<0x4E>(m));
  m = op(m, dpp_f<0x141>(m));
  m = op(m, dpp_f<0x140>(m));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 48));
  return op(op(r0, r1), op(r2, r3));
}

__device__ __forceinline__ float wave_max(float m) { return wave_reduce<true>(m); }

__device__ __forceinline__ float wave_sum(float m) { return wave_reduce<false>(m); }

// The seven butterfly stages of one chunk: strides 1, 2, 4, 8 in-lane, then 16, 32, 64 across lanes.
// c1, c2, c8 are the cross-lane multipliers (-1 on the lane holding the upper element of each pair).
__device__ __forceinline__ void rotate16(float (&v)[16], float c1, float c2, float c8) {
#pragma unroll
  for (int st = 1; st < 16; st <<= 1) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (i & st) continue;
      const float a = v[i], b = v[i + st];
      v[i] = a + b;
      v[i + st] = a - b;
    }
  }
  // One v_fmac_f32_dpp per element and stage: v += partner(v) * c.  The 16 registers are visited
  // round-robin, so a DPP read never follows the VALU write of its own source closer than 15
  // instructions; the s_nop before each stage covers the in-lane stage's last writes.
  asm volatile("s_nop 1" ::: "memory");
#pragma unroll
  for (int i = 0; i < 16; ++i)
    asm volatile("v_fmac_f32_dpp %0, %0, %1 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf" : "+v"(v[i]) : "v"(c1));
  asm volatile("s_nop 1" ::: "memory");
#pragma unroll
  for (int i = 0; i < 16; ++i)
    asm volatile("v_fmac_f32_dpp %0, %0, %1 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf" : "+v"(v[i]) : "v"(c2));
  asm volatile("s_nop 1" ::: "memory");
#pragma unroll
  for (int i = 0; i < 16; ++i)
    asm volatile("v_fmac_f32_dpp %0, %0, %1 row_ror:8 row_mask:0xf bank_mask:0xf" : "+v"(v[i]) : "v"(c8));
}

// q = rint(v * mul) for 16 values, stored as one 16-byte vector (|v * mul| <= 127 by construction).  The
// product is rounded to f32 first (a multiply of its own: the build does not contract it into an FMA), then
// 1.5 * 2^23 is added: in [2^23, 2^24) floats are the integers, so the adder rounds t to rint(t) (to nearest,
// ties to even, like rintf; 2^23 * 1.5 is even) and the sum's bit pattern is 0x4B400000 + rint(t), whose low
// byte is the two's-complement code.  That replaces the round + convert of each value.
__device__ __forceinline__ uint4 pack_codes16(const float (&v)[16], float mul) {
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t b[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) b[e] = __float_as_uint(v[4 * j + e] * mul + 12582912.0f);
    // bytes 0 of b0, b1, b2, b3 (v_perm_b32 selects bytes of {S0, S1}: 0-3 from S1, 4-7 from S0, 0x0c = 0)
    w[j] = __builtin_amdgcn_perm(b[1], b[0], 0x0c0c0400u) | __builtin_amdgcn_perm(b[3], b[2], 0x04000c0cu);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ void store_codes16(int8_t* p, const float (&v)[16], float mul) {
  *reinterpret_cast<uint4*>(p) = pack_codes16(v, mul);
}

}  // namespace k2q_rot
