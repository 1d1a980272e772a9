// Shared definitions for the k2q gfx950 kernels (ConvRot QuantLinear + LoRA).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/k2q.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef unsigned short v8us __attribute__((ext_vector_type(8)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

#define K2Q_HADAMARD 128

// float -> bf16 bits, round to nearest even (NaN kept quiet); the rounding of torch's .to(bfloat16).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// Status helpers for the C ABI.
static inline int k2q_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? K2Q_OK : K2Q_ELAUNCH;
}

static inline int k2q_aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }
