// LoRA down-projection u = x A^T (reference lora.py:47, first product) and the operand preparation of
// the input-gradient GEMM (transposed dequantized weight, transposed LoRA A).
//
// u: A (r x K, f32) is split once per call into bf16 hi + lo parts (A = hi + lo to ~2^-16 relative), and
// u = x hi^T + x lo^T runs on v_mfma_f32_16x16x32_bf16 with f32 accumulation; x is bf16 already, so the
// only roundings are A's split residue and the f32 accumulation.  HBM-bound on reading x once.
#include "k2q_common.h"

namespace {

typedef __bf16 v8bf_t __attribute__((ext_vector_type(8)));
typedef float v4f_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void split_bf16_kernel(const float* __restrict__ a, int64_t n,
                                                         uint16_t* __restrict__ hi,
                                                         uint16_t* __restrict__ lo) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float v = a[i];
  const uint32_t h = f32_to_bf16_bits(v);
  hi[i] = (uint16_t)h;
  lo[i] = (uint16_t)f32_to_bf16_bits(v - bf16_bits_to_f32(h));
}

// u = x A^T for 32 rows per workgroup: the 4 waves split K in quarters, each runs 2 row tiles x RT rank
// tiles of v_mfma_f32_16x16x32_bf16 (x hi and x lo), and the partial sums meet in LDS where wave 0..3
// are added in that fixed order (deterministic).  Fragments come straight from global memory in MFMA
// layout: lane l holds row l%16 (of x, or of A) and 8 contiguous k at 8*(l/16) of each 32-wide step.
template <int RT>
__global__ __launch_bounds__(256) void lora_down_kernel(const uint16_t* __restrict__ x, int64_t M, int K,
                                                        int64_t ldx, const uint16_t* __restrict__ hi,
                                                        const uint16_t* __restrict__ lo,
                                                        float* __restrict__ u) {
  constexpr int UNR = RT <= 2 ? 4 : (RT <= 4 ? 2 : 1);   // 32-wide k steps whose loads fly together
  __shared__ float part[4][2][RT][4][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t m0 = (int64_t)blockIdx.x * 32;
  const int kq = K / 4;                 // this wave's quarter of K (a multiple of 32)
  const int kbeg = wave * kq;
  const int kofs = 8 * (lane >> 4);
  const uint16_t* xp[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    int64_t mr = m0 + 16 * t + (lane & 15);
    mr = mr < M ? mr : M - 1;
    xp[t] = x + mr * ldx + kofs;
  }
  const int64_t arow = (int64_t)(lane & 15) * K + kofs;

  v4f acc[2][RT];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int j = 0; j < RT; ++j) acc[t][j] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int k0 = kbeg; k0 < kbeg + kq; k0 += 32 * UNR) {
    v4i fx[UNR][2], fh[UNR][RT], fl[UNR][RT];
#pragma unroll
    for (int q = 0; q < UNR; ++q) {
      const int k = k0 + 32 * q;
      const bool ok = k < kbeg + kq;
#pragma unroll
      for (int t = 0; t < 2; ++t) fx[q][t] = ok ? *reinterpret_cast<const v4i*>(xp[t] + k) : v4i{0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < RT; ++j) {
        const int64_t ao = (int64_t)16 * j * K + arow + (ok ? k : kbeg);
        fh[q][j] = *reinterpret_cast<const v4i*>(hi + ao);
        fl[q][j] = *reinterpret_cast<const v4i*>(lo + ao);
      }
    }
#pragma unroll
    for (int q = 0; q < UNR; ++q)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int j = 0; j < RT; ++j) {
          const v8bf xa = __builtin_bit_cast(v8bf, fx[q][t]);
          acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, __builtin_bit_cast(v8bf, fh[q][j]), acc[t][j], 0, 0, 0);
          acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, __builtin_bit_cast(v8bf, fl[q][j]), acc[t][j], 0, 0, 0);
        }
  }
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) part[wave][t][j][i][lane] = acc[t][j][i];
  __syncthreads();
  // C layout (16x16): lane l owns column l%16 and rows 4*(l/16) + i.  Thread = (t, j, lane) slot.
  for (int slot = threadIdx.x; slot < 2 * RT * 64; slot += 256) {
    const int ln = slot & 63, j = (slot >> 6) % RT, t = (slot >> 6) / RT;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = ((part[0][t][j][i][ln] + part[1][t][j][i][ln]) + part[2][t][j][i][ln]) + part[3][t][j][i][ln];
      const int64_t m = m0 + 16 * t + 4 * (ln >> 4) + i;
      if (m < M) u[m * (16 * RT) + 16 * j + (ln & 15)] = v;
    }
  }
}

// wt[k][n] = bf16(W_hat[n][k]) for a 64 x 64 tile; W_hat = s_w[n] q[n][k] (int8) or
// s_w4[k/64][n] q4[n][k] (int4, group-major scales).  Thread t reads 16 k of row n = t/4 and writes 16 n
// of row k = t/4 through an LDS transpose.
template <bool W4>
__global__ __launch_bounds__(256) void dequant_t_kernel(const int8_t* __restrict__ qw,
                                                        const float* __restrict__ sw,
                                                        const uint8_t* __restrict__ qw4,
                                                        const uint16_t* __restrict__ sw4, int64_t N,
                                                        int64_t K, uint16_t* __restrict__ wt) {
  __shared__ uint16_t tile[64][64 + 2];
  const int t = threadIdx.x;
  const int64_t n0 = (int64_t)blockIdx.x * 64, k0 = (int64_t)blockIdx.y * 64;
  {
    const int nl = t >> 2, kl = 16 * (t & 3);
    const int64_t n = n0 + nl;
    float v[16];
    if (n < N) {
      if (W4) {
        const uint2 p = *reinterpret_cast<const uint2*>(qw4 + n * (K / 2) + (k0 + kl) / 2);
        const float s = bf16_bits_to_f32(sw4[((k0 + kl) / 64) * N + n]);
        const uint32_t w[2] = {p.x, p.y};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t byte = (w[j >> 2] >> (8 * (j & 3))) & 0xffu;
          const int lo4 = (int)((byte & 0xfu) ^ 8u) - 8;
          const int hi4 = (int)((byte >> 4) ^ 8u) - 8;
          v[j] = (float)lo4 * s;
          v[j + 8] = (float)hi4 * s;
        }
      } else {
        const uint4 p = *reinterpret_cast<const uint4*>(qw + n * K + k0 + kl);
        const float s = sw[n];
        const uint32_t w[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = (float)(int8_t)((w[j >> 2] >> (8 * (j & 3))) & 0xffu) * s;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) tile[kl + j][nl] = (uint16_t)f32_to_bf16_bits(v[j]);
  }
  __syncthreads();
  {
    const int kl = t >> 2, nl = 16 * (t & 3);
    const int64_t k = k0 + kl;
    if (k >= K) return;
    uint32_t w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = (uint32_t)tile[kl][nl + 2 * j] | ((uint32_t)tile[kl][nl + 2 * j + 1] << 16);
    uint16_t* dst = wt + k * N + n0 + nl;
    if (n0 + nl + 16 <= N) {
      reinterpret_cast<uint4*>(dst)[0] = make_uint4(w[0], w[1], w[2], w[3]);
      reinterpret_cast<uint4*>(dst)[1] = make_uint4(w[4], w[5], w[6], w[7]);
    } else {
      for (int j = 0; j < 16 && n0 + nl + j < N; ++j) dst[j] = tile[kl][nl + j];
    }
  }
}

__global__ __launch_bounds__(256) void transpose_f32_kernel(const float* __restrict__ a, int64_t R,
                                                            int64_t C, float* __restrict__ at) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // index into at (C x R)
  if (i >= R * C) return;
  const int64_t c = i / R, r = i % R;
  at[i] = a[r * C + c];
}

}  // namespace

extern "C" int k2q_lora_down(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const float* lora_a,
                             int64_t r, uint16_t* ws, float* u, void* stream) {
  if (!x || !lora_a || !ws || !u || M < 1 || K < 128 || K % 128 || ldx < K || ldx % 8) return K2Q_EINVAL;
  if (r < 16 || r > 128 || r % 16) return K2Q_EINVAL;
  if (!k2q_aligned(x, 16) || !k2q_aligned(ws, 16) || !k2q_aligned(u, 16)) return K2Q_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t n = r * K;
  uint16_t* hi = ws;
  uint16_t* lo = ws + n;
  hipLaunchKernelGGL(split_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, lora_a, n, hi,
                     lo);
  const dim3 grid((unsigned)((M + 31) / 32));
  switch (r / 16) {
#define K2Q_LD_CASE(RT)                                                                                     \
  case RT:                                                                                                  \
    hipLaunchKernelGGL(lora_down_kernel<RT>, grid, dim3(256), 0, st, x, M, (int)K, ldx, hi, lo, u);        \
    break;
    K2Q_LD_CASE(1) K2Q_LD_CASE(2) K2Q_LD_CASE(3) K2Q_LD_CASE(4)
    K2Q_LD_CASE(5) K2Q_LD_CASE(6) K2Q_LD_CASE(7) K2Q_LD_CASE(8)
#undef K2Q_LD_CASE
    default:
      return K2Q_EINVAL;
  }
  return k2q_launch_status();
}

extern "C" int k2q_dx_prep(const int8_t* qw, const float* sw, const uint8_t* qw4, const uint16_t* sw4,
                           int64_t N, int64_t K, const float* lora_a, int64_t r, uint16_t* wt, float* at,
                           void* stream) {
  const bool w4 = qw4 != nullptr;
  if (N < 1 || K < 128 || K % 128 || !wt) return K2Q_EINVAL;
  if (w4 ? (!sw4 || !k2q_aligned(qw4, 16)) : (!qw || !sw || !k2q_aligned(qw, 16))) return K2Q_EINVAL;
  if (!k2q_aligned(wt, 16) || N % 8) return K2Q_EINVAL;
  if (lora_a && (!at || r < 1)) return K2Q_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((N + 63) / 64), (unsigned)(K / 64));
  if (w4)
    hipLaunchKernelGGL(dequant_t_kernel<true>, grid, dim3(256), 0, st, nullptr, nullptr, qw4, sw4, N, K, wt);
  else
    hipLaunchKernelGGL(dequant_t_kernel<false>, grid, dim3(256), 0, st, qw, sw, nullptr, nullptr, N, K, wt);
  if (lora_a) {
    const int64_t n = r * K;
    hipLaunchKernelGGL(transpose_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, lora_a, r,
                       K, at);
  }
  return k2q_launch_status();
}
