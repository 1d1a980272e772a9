// Shared definitions for the k2q gfx950 kernels (ConvRot QuantLinear + LoRA).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

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

// float -> bf16, round to nearest even (NaN stays NaN): the rounding of torch's .to(bfloat16).  gfx950
// converts two floats per v_cvt_pk_bf16_f32.
typedef float k2q_v2f __attribute__((ext_vector_type(2)));
typedef __bf16 k2q_v2bf __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(k2q_v2f{lo, hi}, k2q_v2bf));
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) { return pack_bf16x2(f, 0.f) & 0xffffu; }

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// Raw byte buffer over [base, base + bytes) for the workgroup-uniform base and extent (bytes < 2^31); reads
// past the extent return zero.  LDS-DMA through it (buffer_load ... lds) is a MUBUF instruction, counted in
// vmcnt only, so the compiler keeps exact lgkmcnt waits for the LDS reads around it.  The pieces go
// through readfirstlane so the descriptor is built in SGPRs (a descriptor the compiler cannot prove
// uniform is used through a per-lane loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t k2q_rsrc(const void* base, int64_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  const int n = __builtin_amdgcn_readfirstlane((int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0, n,
                                          0x00020000);
}

// Compile-time loop: f(std::integral_constant<int, i>) for i = 0 .. N-1 (for scheduling hints and register
// arrays that need constant indices).
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Skinny-M forward (gemv.hip), used by k2q_gemm_w8a8 for 1 <= M <= K2Q_GEMV_MAX_M.
#define K2Q_GEMV_MAX_M 8
int k2q_launch_gemv_w8a8(const int8_t* qx, const float* sx, const int8_t* qw, const float* sw, const float* bias,
                         const float* u, const float* lora_b, int r, float lora_scale, int64_t M, int64_t N,
                         int64_t K, uint16_t* y, hipStream_t st);

// LoRA down-projection u = x (scale F)^T (lora.hip); F is r x K row-major (a_kstride = 1) or given as its
// K x r transpose (a_kstride = r).  k2q_lora_down is the a_kstride = 1, scale = 1 case.
int lora_down_impl(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const float* a, int64_t a_kstride,
                   float a_scale, int64_t r, void* ws, int64_t ws_bytes, float* u, hipStream_t st);

// The down-projection's K-slice partials without the reduce, for a consumer that adds them as it reads them
// (r <= 128; factor as for lora_down_impl): *parts slices of M x r, rows of stride ldo, M * ldo floats apart
// (one slice is u itself); with ldo = r, dst receives lora_down_parts_floats(M, K, r) floats.
int64_t lora_down_parts_floats(int64_t M, int64_t K, int64_t r);
int lora_down_parts(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const float* a, int64_t a_kstride,
                    float a_scale, int64_t r, float* dst, int64_t ldo, int* parts, hipStream_t st);

// k2q_gemm_w8a8 with the factors u given as u_parts K-slice partials u_pstride floats apart (added in slice
// order in the epilogue, exactly as the down-projection's reduce adds them) and a tile shape (-1: automatic).
int gemm_w8a8_impl(const int8_t* qx, const float* sx, const int8_t* qw, const float* sw, const float* bias,
                   const float* u, int u_parts, int64_t u_pstride, const float* lora_b, int64_t r, float lora_scale,
                   int64_t M, int64_t N, int64_t K, uint16_t* y, void* ws, int64_t ws_bytes, int tile,
                   hipStream_t st);

// Status helpers for the C ABI.
static inline int k2q_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? K2Q_OK : K2Q_ELAUNCH;
}

static inline int k2q_aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

// Compute units of the current device (launch planning only; 256 on MI355X).  Looked up once per device and
// cached (api.hip): the attribute query costs more host time than a kernel launch.
int k2q_cu_count();

// Raises kernel fn's dynamic-LDS limit to `bytes` once per device; `done` (one static per kernel instance, a
// bit per device) remembers it, so a launch pays for the attribute call only the first time on a device.
// Callers pass the most the instance can need, so a later launch never needs a higher limit.
template <class Fn>
int k2q_lds_limit_once(Fn* fn, int bytes, std::atomic<uint64_t>& done) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return K2Q_ELAUNCH;
  const uint64_t bit = dev >= 0 && dev < 64 ? (uint64_t(1) << dev) : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return K2Q_OK;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize, bytes) !=
      hipSuccess)
    return K2Q_ELAUNCH;
  done.fetch_or(bit, std::memory_order_acq_rel);
  return K2Q_OK;
}

// Rotate/quant with the LoRA down-projection from the same pass (rotquant.hip): the codes of k2q_rotquant and
// u = x A^T (A: r x K f32) for K <= 4096, K % 512 == 0, r in {16, 32, 48, 64} (k2q_rotquant_lora_fits).
int k2q_rotquant_lora_fits(int64_t K, int64_t r);
int rotquant_lora_impl(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, float* s, const float* a,
                       int64_t r, float* u, int64_t ldu, hipStream_t st);
