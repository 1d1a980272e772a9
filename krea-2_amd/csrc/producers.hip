// Producer-fused rotate/quant: the elementwise or row-normalising operation that makes a quantized
// linear's input, fused into the same register pass that rotates and quantizes it.
//
//   * SwiGLU (reference mmdit.py:177-178, `self.down(F.silu(self.gate(x)) * self.up(x))`):
//       h = bf16(bf16(silu(g)) * u),  silu(g) = g / (1 + exp(-g)) in float32,
//     the rounding order of the reference's eager bf16 ops (F.silu returns bf16, the product rounds again).
//   * Modulated RMSNorm (reference mmdit.py:314-317 with RMSNorm.forward at mmdit.py:156-161):
//       n = bf16((x * rsqrt(mean(x^2) + eps)) * (w + 1))   [float32, the whole row]
//       h = bf16(bf16(bf16(1 + p) * n) + b)               [p, b: the bf16 modulation scale / shift of the
//                                                          row's batch entry]
// Both write h (bf16, the tensor the next linear receives: its LoRA down-projection and the saved input of
// the backward read it) and the int8 codes + scales of rotate/quant applied to h, computed from the same
// registers, so the codes equal those of a separate rotate/quant call on h bit for bit.
//
// The backward of the SwiGLU product (dg, du from dh) is the elementwise swiglu_bwd_kernel:
//   s = bf16(silu(g)), du = bf16(dh * s), ds = bf16(dh * u),
//   dg = bf16((ds * sig) * (1 + g * (1 - sig))) with sig = 1 / (1 + exp(-g)),
// the derivative d/dg [g sig(g)] = sig(g) (1 + g (1 - sig(g))) applied with the reference autograd's
// bf16 roundings (each eager op rounds its result to bf16).
#include "rotation.h"

namespace {

using namespace k2q_rot;

enum { PROD_SWIGLU = 0, PROD_RMSMOD = 1 };

struct ProdArgs {
  const __bf16* x0;          // SwiGLU: gate output g;  RMSNorm: x
  const __bf16* x1;          // SwiGLU: up output u
  int64_t ld0, ld1;          // row strides of x0 / x1 (elements)
  const float* nw;           // RMSNorm scale parameter (K,), the norm weight is nw + 1
  const uint16_t* mscale;    // bf16 modulation scale, entry b = row / rpb at mscale + b * ldm
  const uint16_t* mshift;    // bf16 modulation shift, same indexing
  int64_t ldm, rpb;
  float eps;
  int64_t M;
  int K;
  uint16_t* h;               // M x K bf16 (row stride K)
  int8_t* q;                 // M x K int8 codes of h R
  float* s;                  // M per-row scales
};

__device__ __forceinline__ float bf16r(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// Two values rounded to bf16 by one v_cvt_pk_bf16_f32 (round to nearest even), unpacked in place.
__device__ __forceinline__ void bf16r2(float& a, float& b) {
  const uint32_t u = pack_bf16x2(a, b);
  a = __uint_as_float(u << 16);
  b = __uint_as_float(u & 0xffff0000u);
}

// sigmoid(g) = 1 / (1 + exp(-g)) with exp(-g) = 2^(-g log2 e) on v_exp_f32 and the reciprocal on v_rcp_f32:
// a few float32 ulp from the correctly rounded quotient, which the bf16 rounding of the result hides except
// in rare near-ties (the reference's own exp differs from the oracle's by as much).
__device__ __forceinline__ float sigmoid_f32(float g) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(g * -1.44269504088896341f));
}

__device__ __forceinline__ float silu_f32(float g) { return g * sigmoid_f32(g); }

template <int PROD, int WPR, int kNCH, bool kTail>
__global__ __launch_bounds__(256) void prodquant_kernel(ProdArgs a) {
  constexpr int T = 64 * WPR;
  constexpr int CW = T * 16;
  constexpr int ROWS = 4 / WPR;
  __shared__ float sred[2][4];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * ROWS + wave / WPR;
  const int t = (wave % WPR) * 64 + lane;
  const int l = t & 15;
  const int off = lane_offset(t);
  const bool row_ok = row < a.M;
  const int K = a.K;
  const int64_t rr = row_ok ? row : 0;

  // Loads are unconditional from clamped (always valid) addresses, which keeps the kernel free of branches
  // and lets each chunk's operands die before the next chunk's arrive; lanes past K hold zeros (their
  // Hadamard blocks enter the row absmax).
  float v[kNCH][16];
#pragma unroll
  for (int c = 0; c < kNCH; ++c) {
    const int col = c * CW + off;
    const bool ok = !kTail || col < K;
    load16<__bf16>(a.x0 + rr * a.ld0 + (ok ? col : 0), true, v[c]);
    if (kTail) {
#pragma unroll
      for (int i = 0; i < 16; ++i) v[c][i] = ok ? v[c][i] : 0.f;
    }
  }

  if (PROD == PROD_SWIGLU) {
#pragma unroll
    for (int c = 0; c < kNCH; ++c) {
      const int col = c * CW + off;
      float u[16];
      load16<__bf16>(a.x1 + rr * a.ld1 + (!kTail || col < K ? col : 0), true, u);
#pragma unroll
      for (int i = 0; i < 16; i += 2) {   // silu(0) * u = 0 past K
        float s0 = silu_f32(v[c][i]), s1 = silu_f32(v[c][i + 1]);
        bf16r2(s0, s1);
        float h0 = s0 * u[i], h1 = s1 * u[i + 1];
        bf16r2(h0, h1);
        v[c][i] = h0;
        v[c][i + 1] = h1;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < kNCH; ++c)
#pragma unroll
      for (int i = 0; i < 16; ++i) ss += v[c][i] * v[c][i];   // squares rounded, then summed (x.pow(2).mean())
    ss = wave_sum(ss);
    if (WPR > 1) {
      if (lane == 0) sred[0][wave] = ss;
      __syncthreads();
      const int w0 = (wave / WPR) * WPR;
      ss = 0.f;
#pragma unroll
      for (int w = 0; w < WPR; ++w) ss += sred[0][w0 + w];
    }
    const float rinv = __fdiv_rn(1.f, __fsqrt_rn(__fdiv_rn(ss, (float)K) + a.eps));
    const int64_t b = rr / a.rpb;
    const uint16_t* ms = a.mscale + b * a.ldm;
    const uint16_t* mb = a.mshift + b * a.ldm;
    // Per chunk: the norm weight (f32) and the two modulation vectors (bf16, kept packed) are loaded and
    // consumed before the next chunk's, so at most one chunk of them is live (occupancy).
#pragma unroll
    for (int c = 0; c < kNCH; ++c) {
      const int col = c * CW + off;
      const bool ok = !kTail || col < K;
      const int cc = ok ? col : 0;
      // unconditional loads from a clamped (always valid) address; lanes past K are zeroed below
      float w[16];
      load16<float>(a.nw + cc, true, w);
      const uint4 pv0 = reinterpret_cast<const uint4*>(ms + cc)[0], pv1 = reinterpret_cast<const uint4*>(ms + cc)[1];
      const uint4 bv0 = reinterpret_cast<const uint4*>(mb + cc)[0], bv1 = reinterpret_cast<const uint4*>(mb + cc)[1];
      const uint32_t pw[8] = {pv0.x, pv0.y, pv0.z, pv0.w, pv1.x, pv1.y, pv1.z, pv1.w};
      const uint32_t bw[8] = {bv0.x, bv0.y, bv0.z, bv0.w, bv1.x, bv1.y, bv1.z, bv1.w};
#pragma unroll
      for (int i = 0; i < 16; i += 2) {   // element pairs share each bf16 conversion
        float n0 = (v[c][i] * rinv) * (w[i] + 1.f), n1 = (v[c][i + 1] * rinv) * (w[i + 1] + 1.f);
        bf16r2(n0, n1);
        float p0 = 1.f + __uint_as_float(pw[i >> 1] << 16), p1 = 1.f + __uint_as_float(pw[i >> 1] & 0xffff0000u);
        bf16r2(p0, p1);
        float m0 = p0 * n0, m1 = p1 * n1;
        bf16r2(m0, m1);
        float h0 = m0 + __uint_as_float(bw[i >> 1] << 16), h1 = m1 + __uint_as_float(bw[i >> 1] & 0xffff0000u);
        bf16r2(h0, h1);
        v[c][i] = !kTail || ok ? h0 : 0.f;   // blocks past K must stay zero: they enter the row absmax
        v[c][i + 1] = !kTail || ok ? h1 : 0.f;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  if (row_ok) {
#pragma unroll
    for (int c = 0; c < kNCH; ++c) {
      const int col = c * CW + off;
      if (col < K) store16_bf16(a.h + row * (int64_t)K + col, v[c]);
    }
  }

  const float c1 = (l & 1) ? -1.f : 1.f;
  const float c2 = (l & 2) ? -1.f : 1.f;
  const float c8 = (l & 8) ? -1.f : 1.f;
  const float sigma = c1 * c2 * c8;
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < kNCH; ++c) {
    rotate16(v[c], c1, c2, c8);
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[c][i]));
  }
  amax = wave_max(amax);
  if (WPR > 1) {
    if (lane == 0) sred[1][wave] = amax;
    __syncthreads();
    const int w0 = (wave / WPR) * WPR;
#pragma unroll
    for (int w = 0; w < WPR; ++w) amax = fmaxf(amax, sred[1][w0 + w]);
  }
  amax = fmaxf(amax, 1e-8f);
  const float inv = __fdiv_rn(127.f, amax);
  if (!row_ok) return;
  if (t == 0) a.s[row] = __fdiv_rn(amax, 127.f);
  const float mul = inv * sigma;
#pragma unroll
  for (int c = 0; c < kNCH; ++c) {
    const int col = c * CW + off;
    if (col < K) store_codes16(a.q + row * (int64_t)K + col, v[c], mul);
  }
}

template <int PROD, int WPR, bool kTail>
void launch_prod_nch(const ProdArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)((a.M + (4 / WPR) - 1) / (4 / WPR)));
  const int nch = (a.K + 1024 * WPR - 1) / (1024 * WPR);
  switch (nch) {
    case 1: hipLaunchKernelGGL((prodquant_kernel<PROD, WPR, 1, kTail>), grid, dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL((prodquant_kernel<PROD, WPR, 2, kTail>), grid, dim3(256), 0, st, a); break;
    case 3: hipLaunchKernelGGL((prodquant_kernel<PROD, WPR, 3, kTail>), grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL((prodquant_kernel<PROD, WPR, 4, kTail>), grid, dim3(256), 0, st, a); break;
  }
}

// kTail: K is not a whole number of chunks, so some lanes' columns lie past K.
template <int PROD, int WPR>
void launch_prod_wpr(const ProdArgs& a, hipStream_t st) {
  if (a.K % (1024 * WPR)) launch_prod_nch<PROD, WPR, true>(a, st);
  else launch_prod_nch<PROD, WPR, false>(a, st);
}

template <int PROD>
int launch_prod(const ProdArgs& a, hipStream_t st) {
  if (a.K <= 4096) launch_prod_wpr<PROD, 1>(a, st);
  else if (a.K <= 8192) launch_prod_wpr<PROD, 2>(a, st);
  else launch_prod_wpr<PROD, 4>(a, st);
  return k2q_launch_status();
}

int check_prod_common(int64_t M, int64_t K, const uint16_t* h, const int8_t* q, const float* s) {
  if (M < 1 || K < K2Q_HADAMARD || K % K2Q_HADAMARD) return K2Q_EINVAL;
  if (K > 16384) return K2Q_EUNSUPPORTED;
  if (!h || !q || !s || !k2q_aligned(h, 16) || !k2q_aligned(q, 16) || !k2q_aligned(s, 4)) return K2Q_EINVAL;
  return K2Q_OK;
}

// 8 elements per lane per step: dh, g, u in; dg, du out (all bf16, contiguous, n elements, n % 8 == 0).
__global__ __launch_bounds__(256) void swiglu_bwd_kernel(const uint4* __restrict__ dh, const uint4* __restrict__ g,
                                                         const uint4* __restrict__ u, int64_t n8,
                                                         uint4* __restrict__ dg, uint4* __restrict__ du) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += (int64_t)gridDim.x * blockDim.x) {
    const uint4 a = dh[i], b = g[i], c = u[i];
    const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w}, cw[4] = {c.x, c.y, c.z, c.w};
    uint32_t og[4], ou[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float rg[2], ru[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float d = bf16_bits_to_f32((aw[j] >> (16 * e)) & 0xffffu);
        const float x = bf16_bits_to_f32((bw[j] >> (16 * e)) & 0xffffu);
        const float up = bf16_bits_to_f32((cw[j] >> (16 * e)) & 0xffffu);
        const float sig = sigmoid_f32(x);
        const float sl = bf16r(x * sig);   // the forward's silu_f32, bit for bit
        ru[e] = d * sl;
        const float ds = bf16r(d * up);
        rg[e] = (ds * sig) * (1.f + x * (1.f - sig));
      }
      og[j] = pack_bf16x2(rg[0], rg[1]);
      ou[j] = pack_bf16x2(ru[0], ru[1]);
    }
    dg[i] = make_uint4(og[0], og[1], og[2], og[3]);
    du[i] = make_uint4(ou[0], ou[1], ou[2], ou[3]);
  }
}

// Input gradient of the modulated RMSNorm (the autograd of the forward's eager ops for x alone):
//   dn = bf16(dh * bf16(1 + p)),  g = dn * (w + 1),  r = rsqrt(mean x^2 + eps),
//   dx = bf16(g r - x (r^3 / K) sum_k(g x)).
// A team of 64 * WPR lanes owns a row; lane t handles the 8-element chunks at 8 t + 8 T c, c < kNCH, held
// packed (bf16 pairs) between the two row reductions.
template <int WPR, int kNCH>
__global__ __launch_bounds__(256) void rmsmod_bwd_kernel(const uint16_t* __restrict__ dh, const uint16_t* __restrict__ x,
                                                         int64_t M, int K, const float* __restrict__ nw, float eps,
                                                         const uint16_t* __restrict__ mscale, int64_t ldm, int64_t rpb,
                                                         uint16_t* __restrict__ dx) {
  constexpr int T = 64 * WPR;
  constexpr int ROWS = 4 / WPR;
  __shared__ float sred[2][4];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * ROWS + wave / WPR;
  const int t = (wave % WPR) * 64 + lane;
  const bool row_ok = row < M;
  const int64_t rr = row_ok ? row : 0;
  const uint16_t* ms = mscale + (rr / rpb) * ldm;

  uint4 xv[kNCH], dv[kNCH];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kNCH; ++c) {
    const int col = 8 * t + 8 * T * c;
    const bool ok = col < K;
    xv[c] = ok ? *reinterpret_cast<const uint4*>(x + rr * K + col) : make_uint4(0, 0, 0, 0);
    dv[c] = ok ? *reinterpret_cast<const uint4*>(dh + rr * K + col) : make_uint4(0, 0, 0, 0);
    const uint32_t w[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = __uint_as_float(w[j] << 16), b = __uint_as_float(w[j] & 0xffff0000u);
      ss += a * a;
      ss += b * b;
    }
  }
  ss = wave_sum(ss);
  if (WPR > 1) {
    if (lane == 0) sred[0][wave] = ss;
    __syncthreads();
    const int w0 = (wave / WPR) * WPR;
    ss = 0.f;
#pragma unroll
    for (int w = 0; w < WPR; ++w) ss += sred[0][w0 + w];
  }
  const float r = __fdiv_rn(1.f, __fsqrt_rn(__fdiv_rn(ss, (float)K) + eps));

  // g = bf16(dh * p1) * (w + 1), kept in f32 (8 per chunk) for the final pass
  float gv[kNCH][8];
  float dot = 0.f;
#pragma unroll
  for (int c = 0; c < kNCH; ++c) {
    const int col = 8 * t + 8 * T * c;
    const int cc = col < K ? col : 0;
    float w[8];
    const float4 w0 = *reinterpret_cast<const float4*>(nw + cc), w1 = *reinterpret_cast<const float4*>(nw + cc + 4);
    w[0] = w0.x; w[1] = w0.y; w[2] = w0.z; w[3] = w0.w; w[4] = w1.x; w[5] = w1.y; w[6] = w1.z; w[7] = w1.w;
    const uint4 pv = *reinterpret_cast<const uint4*>(ms + cc);
    const uint32_t pw[4] = {pv.x, pv.y, pv.z, pv.w};
    const uint32_t dw[4] = {dv[c].x, dv[c].y, dv[c].z, dv[c].w};
    const uint32_t xw[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float p0 = 1.f + __uint_as_float(pw[j] << 16), p1 = 1.f + __uint_as_float(pw[j] & 0xffff0000u);
      bf16r2(p0, p1);
      float n0 = __uint_as_float(dw[j] << 16) * p0, n1 = __uint_as_float(dw[j] & 0xffff0000u) * p1;
      bf16r2(n0, n1);
      const float g0 = n0 * (w[2 * j] + 1.f), g1 = n1 * (w[2 * j + 1] + 1.f);
      gv[c][2 * j] = g0;
      gv[c][2 * j + 1] = g1;
      dot += g0 * __uint_as_float(xw[j] << 16);
      dot += g1 * __uint_as_float(xw[j] & 0xffff0000u);
    }
  }
  dot = wave_sum(dot);
  if (WPR > 1) {
    if (lane == 0) sred[1][wave] = dot;
    __syncthreads();
    const int w0 = (wave / WPR) * WPR;
    dot = 0.f;
#pragma unroll
    for (int w = 0; w < WPR; ++w) dot += sred[1][w0 + w];
  }
  if (!row_ok) return;
  const float c3 = __fdiv_rn(r * r * r * dot, (float)K);
#pragma unroll
  for (int c = 0; c < kNCH; ++c) {
    const int col = 8 * t + 8 * T * c;
    if (col >= K) continue;
    const uint32_t xw[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float d0 = gv[c][2 * j] * r - __uint_as_float(xw[j] << 16) * c3;
      const float d1 = gv[c][2 * j + 1] * r - __uint_as_float(xw[j] & 0xffff0000u) * c3;
      o[j] = pack_bf16x2(d0, d1);
    }
    *reinterpret_cast<uint4*>(dx + row * K + col) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

template <int WPR>
void launch_rmsmod_bwd(const uint16_t* dh, const uint16_t* x, int64_t M, int K, const float* nw, float eps,
                       const uint16_t* ms, int64_t ldm, int64_t rpb, uint16_t* dx, hipStream_t st) {
  const dim3 grid((unsigned)((M + (4 / WPR) - 1) / (4 / WPR)));
  const int nch = (K + 512 * WPR - 1) / (512 * WPR);
#define K2Q_RMB(N)                                                                                            \
  case N:                                                                                                     \
    hipLaunchKernelGGL((rmsmod_bwd_kernel<WPR, N>), grid, dim3(256), 0, st, dh, x, M, K, nw, eps, ms, ldm, rpb, dx); \
    break;
  switch (nch) {
    K2Q_RMB(1) K2Q_RMB(2) K2Q_RMB(3) K2Q_RMB(4) K2Q_RMB(5) K2Q_RMB(6) K2Q_RMB(7)
    default: hipLaunchKernelGGL((rmsmod_bwd_kernel<WPR, 8>), grid, dim3(256), 0, st, dh, x, M, K, nw, eps, ms, ldm,
                                rpb, dx); break;
  }
#undef K2Q_RMB
}

}  // namespace

extern "C" int k2q_rmsmod_bwd(const uint16_t* dh, const uint16_t* x, int64_t M, int64_t K, const float* norm_scale,
                              float eps, const uint16_t* mod_scale, int64_t ld_mod, int64_t rows_per_batch,
                              uint16_t* dx, void* stream) {
  if (M < 1 || K < 8 || K % 8) return K2Q_EINVAL;
  if (K > 16384) return K2Q_EUNSUPPORTED;
  if (!dh || !x || !norm_scale || !mod_scale || !dx || !k2q_aligned(dh, 16) || !k2q_aligned(x, 16) ||
      !k2q_aligned(norm_scale, 16) || !k2q_aligned(mod_scale, 16) || !k2q_aligned(dx, 16) || ld_mod < 0 ||
      ld_mod % 8 || rows_per_batch < 1 || !(eps >= 0.f))
    return K2Q_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (K <= 4096) launch_rmsmod_bwd<1>(dh, x, M, (int)K, norm_scale, eps, mod_scale, ld_mod, rows_per_batch, dx, st);
  else if (K <= 8192) launch_rmsmod_bwd<2>(dh, x, M, (int)K, norm_scale, eps, mod_scale, ld_mod, rows_per_batch, dx, st);
  else launch_rmsmod_bwd<4>(dh, x, M, (int)K, norm_scale, eps, mod_scale, ld_mod, rows_per_batch, dx, st);
  return k2q_launch_status();
}

extern "C" int k2q_swiglu_rotquant(const uint16_t* gate, int64_t ldg, const uint16_t* up, int64_t ldu, int64_t M,
                                   int64_t K, uint16_t* h, int8_t* q, float* s, void* stream) {
  int rc = check_prod_common(M, K, h, q, s);
  if (rc) return rc;
  if (!gate || !up || !k2q_aligned(gate, 16) || !k2q_aligned(up, 16) || ldg < K || ldu < K || ldg % 8 || ldu % 8)
    return K2Q_EINVAL;
  ProdArgs a{};
  a.x0 = reinterpret_cast<const __bf16*>(gate);
  a.x1 = reinterpret_cast<const __bf16*>(up);
  a.ld0 = ldg;
  a.ld1 = ldu;
  a.M = M;
  a.K = (int)K;
  a.h = h;
  a.q = q;
  a.s = s;
  return launch_prod<PROD_SWIGLU>(a, static_cast<hipStream_t>(stream));
}

extern "C" int k2q_rmsmod_rotquant(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const float* norm_scale,
                                   float eps, const uint16_t* mod_scale, const uint16_t* mod_shift, int64_t ld_mod,
                                   int64_t rows_per_batch, uint16_t* h, int8_t* q, float* s, void* stream) {
  int rc = check_prod_common(M, K, h, q, s);
  if (rc) return rc;
  if (!x || !norm_scale || !mod_scale || !mod_shift || !k2q_aligned(x, 16) || !k2q_aligned(norm_scale, 16) ||
      !k2q_aligned(mod_scale, 16) || !k2q_aligned(mod_shift, 16) || ldx < K || ldx % 8 || ld_mod < 0 ||
      ld_mod % 8 || rows_per_batch < 1 || !(eps >= 0.f))
    return K2Q_EINVAL;
  ProdArgs a{};
  a.x0 = reinterpret_cast<const __bf16*>(x);
  a.ld0 = ldx;
  a.nw = norm_scale;
  a.mscale = mod_scale;
  a.mshift = mod_shift;
  a.ldm = ld_mod;
  a.rpb = rows_per_batch;
  a.eps = eps;
  a.M = M;
  a.K = (int)K;
  a.h = h;
  a.q = q;
  a.s = s;
  return launch_prod<PROD_RMSMOD>(a, static_cast<hipStream_t>(stream));
}

extern "C" int k2q_swiglu_bwd(const uint16_t* dh, const uint16_t* gate, const uint16_t* up, int64_t n,
                              uint16_t* dgate, uint16_t* dup, void* stream) {
  if (n < 1 || n % 8 || !dh || !gate || !up || !dgate || !dup) return K2Q_EINVAL;
  if (!k2q_aligned(dh, 16) || !k2q_aligned(gate, 16) || !k2q_aligned(up, 16) || !k2q_aligned(dgate, 16) ||
      !k2q_aligned(dup, 16))
    return K2Q_EINVAL;
  const int64_t n8 = n / 8;
  const int64_t blocks = (n8 + 255) / 256;
  const unsigned grid = (unsigned)(blocks < 8192 ? blocks : 8192);
  hipLaunchKernelGGL(swiglu_bwd_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                     reinterpret_cast<const uint4*>(dh), reinterpret_cast<const uint4*>(gate),
                     reinterpret_cast<const uint4*>(up), n8, reinterpret_cast<uint4*>(dgate),
                     reinterpret_cast<uint4*>(dup));
  return k2q_launch_status();
}
