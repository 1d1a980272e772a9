// LoRA down-projection u = x A^T (reference lora.py:47, first product) and the operand preparation of
// the input-gradient GEMM (transposed dequantized weight, transposed LoRA A).
//
// u: every A fragment (f32) is split in registers into bf16 hi + lo (A = hi + lo to ~2^-16 relative) and
// u = x hi^T + x lo^T runs on v_mfma_f32_16x16x32_bf16 with f32 accumulation; x is bf16 already, so the
// only roundings are A's split residue and the f32 accumulation.  Bound by streaming x (once) and A (once
// per workgroup) into the CUs.
#include "k2q_common.h"

namespace {

// hi = bf16(v), lo = bf16(v - hi) for 8 consecutive k (element e of the vectors = k + e).
__device__ __forceinline__ void split8(v4f p, v4f q, v8bf& hi, v8bf& lo) {
  const v4u h = v4u{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(q[0], q[1]), pack_bf16x2(q[2], q[3])};
  const v4u l = v4u{pack_bf16x2(p[0] - __uint_as_float(h[0] << 16), p[1] - __uint_as_float(h[0] & 0xffff0000u)),
                    pack_bf16x2(p[2] - __uint_as_float(h[1] << 16), p[3] - __uint_as_float(h[1] & 0xffff0000u)),
                    pack_bf16x2(q[0] - __uint_as_float(h[2] << 16), q[1] - __uint_as_float(h[2] & 0xffff0000u)),
                    pack_bf16x2(q[2] - __uint_as_float(h[3] << 16), q[3] - __uint_as_float(h[3] & 0xffff0000u))};
  hi = __builtin_bit_cast(v8bf, h);
  lo = __builtin_bit_cast(v8bf, l);
}

// u (or one K-slice's partial of it) for 16*TT rows: workgroup (blockIdx.x, blockIdx.y) covers rows
// 16*TT*blockIdx.x .. and the K-slice blockIdx.y * kslice .. + kslice; its 4 waves take a quarter of the
// slice each and run TT row tiles x RT rank tiles of 16x16 MFMAs (x hi and x lo).  Fragments come straight
// from global memory in MFMA layout (lane l: row l%16 of x or of A, 8 contiguous k at 8*(l/16) of each
// 32-wide step), double-buffered so one batch of loads is in flight while the previous one is multiplied.
// The wave partials meet in LDS and are added in the fixed order wave 0 + 1 + 2 + 3 (deterministic).
// out: u (M rows of row stride ldo, columns 0 .. 16RT) when gridDim.y == 1, else the partial slices
// [gridDim.y][M][ldo].
template <int RT, int TT>
__global__ __launch_bounds__(256) void lora_down_kernel(const uint16_t* __restrict__ x, int64_t M, int64_t ldx,
                                                        const float* __restrict__ a, int64_t K, int kslice,
                                                        int64_t ldo, float* __restrict__ out) {
  constexpr int UNR = RT <= 2 ? 2 : 1;   // 32-wide k steps per load batch
  __shared__ float part[3][TT][RT][4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t m0 = (int64_t)blockIdx.x * 16 * TT;
  const int nst = kslice / 128;          // this wave's 32-wide steps
  const int64_t kb = (int64_t)blockIdx.y * kslice + (int64_t)wave * (kslice / 4) + 8 * (lane >> 4);
  const uint16_t* xp[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    int64_t mr = m0 + 16 * t + (lane & 15);
    mr = mr < M ? mr : M - 1;
    xp[t] = x + mr * ldx + kb;
  }
  const float* ap = a + (int64_t)(lane & 15) * K + kb;
  // Every workgroup reads all of A; starting each at its own step of the slice spreads those reads over
  // the L2 channels instead of having every CU request the same lines at the same time.
  const int rot = (int)(((int64_t)blockIdx.x * 7 + blockIdx.y) % nst);

  v4f acc[TT][RT];
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int j = 0; j < RT; ++j) acc[t][j] = v4f{0.f, 0.f, 0.f, 0.f};

  auto load = [&](v4i (&fx)[UNR][TT], v4f (&fa)[UNR][RT][2], int s0) {
#pragma unroll
    for (int q = 0; q < UNR; ++q) {
      int s = s0 + q < nst ? s0 + q : nst - 1;   // past the end: a harmless re-load
      s += rot;
      s -= s >= nst ? nst : 0;
#pragma unroll
      for (int t = 0; t < TT; ++t) fx[q][t] = *reinterpret_cast<const v4i*>(xp[t] + 32 * s);
#pragma unroll
      for (int j = 0; j < RT; ++j) {
        fa[q][j][0] = *reinterpret_cast<const v4f*>(ap + 16 * j * K + 32 * s);
        fa[q][j][1] = *reinterpret_cast<const v4f*>(ap + 16 * j * K + 32 * s + 4);
      }
    }
  };
  auto compute = [&](const v4i (&fx)[UNR][TT], const v4f (&fa)[UNR][RT][2], int s0) {
#pragma unroll
    for (int q = 0; q < UNR; ++q) {
      if (s0 + q >= nst) break;
      v8bf hi[RT], lo[RT];
#pragma unroll
      for (int j = 0; j < RT; ++j) split8(fa[q][j][0], fa[q][j][1], hi[j], lo[j]);
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        const v8bf xa = __builtin_bit_cast(v8bf, fx[q][t]);
#pragma unroll
        for (int j = 0; j < RT; ++j) {
          acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, hi[j], acc[t][j], 0, 0, 0);
          acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, lo[j], acc[t][j], 0, 0, 0);
        }
      }
    }
  };
  v4i fx0[UNR][TT], fx1[UNR][TT];
  v4f fa0[UNR][RT][2], fa1[UNR][RT][2];
  load(fx0, fa0, 0);
  for (int s = 0; s < nst; s += 2 * UNR) {
    load(fx1, fa1, s + UNR);
    compute(fx0, fa0, s);
    load(fx0, fa0, s + 2 * UNR);
    compute(fx1, fa1, s + UNR);
  }

  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int j = 0; j < RT; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) part[wave - 1][t][j][i][lane] = acc[t][j][i];
  }
  __syncthreads();
  if (wave != 0) return;
  float* o = out + (int64_t)blockIdx.y * M * ldo;
  // C layout (16x16): lane l owns column (rank) l%16 and rows 4*(l/16) + i.
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = ((acc[t][j][i] + part[0][t][j][i][lane]) + part[1][t][j][i][lane]) + part[2][t][j][i][lane];
        const int64_t m = m0 + 16 * t + 4 * (lane >> 4) + i;
        if (m < M) o[m * ldo + 16 * j + (lane & 15)] = v;
      }
}

// A-stationary down-projection: workgroup (blockIdx.x, blockIdx.y) = rows [rows_per_wg * blockIdx.x, +rows_per_wg)
// x K-slice blockIdx.y of LD_NW * 32 * NS columns; wave w keeps the split fragments of its 32*NS columns of A in
// registers for the whole row range (A is read once per workgroup) and walks the 16-row tiles, the next tile's
// x fragments in flight while the current one is multiplied.  Per tile the 8 wave partials meet in LDS and
// are added in wave order (deterministic); out gets u (one slice; rows of stride ldo) or the slice partial
// [slice][M][ldo].
constexpr int LD_NW = 8;   // waves per workgroup
template <int RT>
struct LdShape {
  static constexpr int NS = RT <= 4 ? 4 : 2;   // 32-wide k steps per wave
  static constexpr int SPAN = LD_NW * 32 * NS; // k columns per workgroup
};

template <int RT>
__global__ __launch_bounds__(64 * LD_NW) void lora_down_as_kernel(const uint16_t* __restrict__ x, int64_t M,
                                                                  int64_t ldx, const float* __restrict__ a, int64_t K,
                                                                  int64_t a_kstride, float a_scale,
                                                                  int64_t rows_per_wg, int64_t ldo,
                                                                  float* __restrict__ out) {
  constexpr int NS = LdShape<RT>::NS;
  __shared__ float red[2][LD_NW][RT][4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t k0 = (int64_t)blockIdx.y * LdShape<RT>::SPAN + (int64_t)w * 32 * NS;
  const bool kok = k0 < K;                        // waves past K (a short last slice) contribute 0
  const int64_t kb = (kok ? k0 : 0) + 8 * (lane >> 4);
  const int64_t m_beg = (int64_t)blockIdx.x * rows_per_wg;
  const int64_t m_end = M < m_beg + rows_per_wg ? M : m_beg + rows_per_wg;
  const int ntiles = (int)((m_end - m_beg + 15) / 16);

  v8bf ah[RT][NS], al[RT][NS];
  // The factor fragments, a rank tile at a time: all of a tile's loads are issued before the first of them is
  // waited for, and the next tile's are in flight while this one is split.
  v4f fl[2][NS][2];
  auto fetch = [&](auto ROWS) {
    constexpr bool kRows = decltype(ROWS)::value;
    auto load = [&](int jt, v4f (&f)[NS][2]) {
      const int64_t rank = 16 * jt + (lane & 15);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int64_t k = kb + 32 * s;
        if constexpr (kRows) {   // factor rows (r x K), as nn.Linear stores A
          const float* pa = a + rank * K + k;
          f[s][0] = *reinterpret_cast<const v4f*>(pa);
          f[s][1] = *reinterpret_cast<const v4f*>(pa + 4);
        } else {                 // factor columns (K x r, e.g. lora_B for g = s dY B), scaled below
          const float* pa = a + k * a_kstride + rank;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            f[s][0][e] = pa[e * a_kstride];
            f[s][1][e] = pa[(e + 4) * a_kstride];
          }
        }
      }
    };
    load(0, fl[0]);
#pragma unroll
    for (int jt = 0; jt < RT; ++jt) {
      if (jt + 1 < RT) load(jt + 1, fl[(jt + 1) & 1]);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        if constexpr (kRows) split8(fl[jt & 1][s][0], fl[jt & 1][s][1], ah[jt][s], al[jt][s]);
        else split8(fl[jt & 1][s][0] * a_scale, fl[jt & 1][s][1] * a_scale, ah[jt][s], al[jt][s]);
      }
    }
  };
  if (a_kstride == 1) fetch(std::true_type{});
  else fetch(std::false_type{});

  auto load_x = [&](v4i (&f)[NS], int t) {
    int64_t m = m_beg + 16 * (int64_t)t + (lane & 15);
    m = m < m_end ? m : m_end - 1;
    const uint16_t* px = x + m * ldx + kb;
#pragma unroll
    for (int s = 0; s < NS; ++s) f[s] = *reinterpret_cast<const v4i*>(px + 32 * s);
  };
  auto tile = [&](const v4i (&f)[NS], int t) {
    if (t >= ntiles) return;
    v4f acc[RT];
#pragma unroll
    for (int jt = 0; jt < RT; ++jt) acc[jt] = v4f{0.f, 0.f, 0.f, 0.f};
    if (kok) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const v8bf xa = __builtin_bit_cast(v8bf, f[s]);
#pragma unroll
        for (int jt = 0; jt < RT; ++jt) {
          acc[jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, ah[jt][s], acc[jt], 0, 0, 0);
          acc[jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, al[jt][s], acc[jt], 0, 0, 0);
        }
      }
    }
    const int buf = t & 1;
#pragma unroll
    for (int jt = 0; jt < RT; ++jt)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[buf][w][jt][i][lane] = acc[jt][i];
    __syncthreads();
    // C layout (16x16): lane l owns column (rank) l%16 and rows 4*(l/16) + i of rank tile jt.
    for (int idx = threadIdx.x; idx < 256 * RT; idx += 64 * LD_NW) {
      const int ln = idx & 63, i = (idx >> 6) & 3, jt = idx >> 8;
      float v = red[buf][0][jt][i][ln];
#pragma unroll
      for (int ww = 1; ww < LD_NW; ++ww) v += red[buf][ww][jt][i][ln];
      const int64_t m = m_beg + 16 * (int64_t)t + 4 * (ln >> 4) + i;
      if (m < m_end) out[((int64_t)blockIdx.y * M + m) * ldo + 16 * jt + (ln & 15)] = v;
    }
  };
  v4i x0[NS], x1[NS];
  load_x(x0, 0);
  for (int t = 0; t < ntiles; t += 2) {
    load_x(x1, t + 1);
    tile(x0, t);
    load_x(x0, t + 2);
    tile(x1, t + 1);
  }
}

// u = sum of the K-slice partials in slice order (deterministic).  part: [ks][M][4 r4] f32; u: M rows of
// ldu4 float4s, of which the first r4 are written.  KS > 0: ks == KS, unrolled, so all KS loads are in flight
// before the first add (a loop over a run-time count waits for each load in turn); KS == 0: any ks.
template <int KS>
__global__ __launch_bounds__(256) void lora_reduce_kernel(const v4f* __restrict__ part, int ks, int64_t M, int64_t r4,
                                                          int64_t ldu4, v4f* __restrict__ u) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t n4 = M * r4;
  if (i >= n4) return;
  v4f s;
  if constexpr (KS > 0) {
    v4f t[KS];
#pragma unroll
    for (int p = 0; p < KS; ++p) t[p] = part[p * n4 + i];
    s = t[0];
#pragma unroll
    for (int p = 1; p < KS; ++p) s += t[p];
  } else {
    s = part[i];
    for (int p = 1; p < ks; ++p) s += part[p * n4 + i];
  }
  const int64_t m = i / r4;
  u[m * ldu4 + (i - m * r4)] = s;
}

void launch_reduce(const float* part, int ks, int64_t M, int64_t r, int64_t ldu, float* u, hipStream_t st) {
  const int64_t n4 = M * r / 4;
  const dim3 grid((unsigned)((n4 + 255) / 256));
  const v4f* pp = reinterpret_cast<const v4f*>(part);
  v4f* uu = reinterpret_cast<v4f*>(u);
  switch (ks) {
#define K2Q_RED_CASE(N) \
  case N: hipLaunchKernelGGL(lora_reduce_kernel<N>, grid, dim3(256), 0, st, pp, ks, M, r / 4, ldu / 4, uu); break;
    K2Q_RED_CASE(2) K2Q_RED_CASE(3) K2Q_RED_CASE(4) K2Q_RED_CASE(6) K2Q_RED_CASE(8) K2Q_RED_CASE(12)
    K2Q_RED_CASE(16)
#undef K2Q_RED_CASE
    default:
      hipLaunchKernelGGL(lora_reduce_kernel<0>, grid, dim3(256), 0, st, pp, ks, M, r / 4, ldu / 4, uu);
  }
}

// Launch plan: TT row tiles per workgroup (fewer for tiny M), and K cut into ks slices (K % (128 ks) == 0,
// slices of at least 512) until the grid covers the CUs; ks > 1 needs ks*M*r floats of workspace.
struct LoraPlan {
  int tt, ks;
  int64_t row_blocks;
};

LoraPlan lora_plan(int64_t M, int64_t K, int64_t r) {
  LoraPlan p{};
  p.tt = r / 16 <= 4 ? 4 : 2;
  while (p.tt > 1 && 16 * (p.tt / 2) >= M) p.tt /= 2;
  p.row_blocks = (M + 16 * p.tt - 1) / (16 * p.tt);
  const int cus = k2q_cu_count();
  p.ks = 1;
  if (p.row_blocks < cus)
    for (int d = 2; d <= 16; ++d) {
      if (K % (128 * d) || K / d < 512) continue;
      p.ks = d;
      if (p.row_blocks * d >= cus) break;
    }
  return p;
}

template <int RT>
void launch_lora_down(int tt, dim3 grid, hipStream_t st, const uint16_t* x, int64_t M, int64_t ldx, const float* a,
                      int64_t K, int kslice, int64_t ldo, float* out) {
  if (tt == 4)
    hipLaunchKernelGGL((lora_down_kernel<RT, (RT <= 4 ? 4 : 2)>), grid, dim3(256), 0, st, x, M, ldx, a, K, kslice, ldo,
                       out);
  else if (tt == 2)
    hipLaunchKernelGGL((lora_down_kernel<RT, 2>), grid, dim3(256), 0, st, x, M, ldx, a, K, kslice, ldo, out);
  else
    hipLaunchKernelGGL((lora_down_kernel<RT, 1>), grid, dim3(256), 0, st, x, M, ldx, a, K, kslice, ldo, out);
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

// wt[k][n] = bf16(2^-7 (W_hat R)[n][k]) for a 64 (n) x 128 (k) tile: the effective weight of the
// straight-through forward (x -> 2^-7 s_x (x R) W_hat^T, R the unnormalised block Hadamard), transposed, so
// the input gradient is the plain product dy wt^T.  Thread t holds 32 k of row n = t/4 (k = 32 (t%4) +
// 0..31 of the 128-wide Hadamard block); the butterflies on k bits 0-4 run in registers, bits 5 and 6
// between the four threads of a quad (DPP).  Then an LDS transpose, as in dequant_t_kernel.
//   W8: the rotation runs on the integer codes, exactly, and the row scale (times 2^-7) is applied once
//   to the result: each output is the exact (c R)[k] rounded once to f32 and once to bf16.  The codes are
//   offset by 128 (unsigned bytes, unpacked two per 32-bit register with one byte permute) and the block's
//   first output corrected by 128 * 128 (the rotation of the constant 128 row); every partial sum lies in
//   [-32640, 32640], so the butterflies run as packed 16-bit integer adds, two elements per instruction.
//   Register i holds elements i and i + 16, so k bits 0-3 pair registers and bit 4 pairs the two halves.
//   W4: the two 64-wide groups of a block carry different scales, so the codes are scaled first and the
//   butterflies run in f32.
typedef short k2q_v2s __attribute__((ext_vector_type(2)));
template <bool W4>
__global__ __launch_bounds__(256) void rot_dequant_t_kernel(const int8_t* __restrict__ qw,
                                                            const float* __restrict__ sw,
                                                            const uint8_t* __restrict__ qw4,
                                                            const uint16_t* __restrict__ sw4, int64_t N,
                                                            int64_t K, uint16_t* __restrict__ wt) {
  __shared__ uint16_t tile[128][64 + 2];
  const int t = threadIdx.x;
  const int64_t n0 = (int64_t)blockIdx.x * 64, k0 = (int64_t)blockIdx.y * 128;
  {
    const int nl = t >> 2, kq = t & 3;
    const int64_t n = n0 + nl < N ? n0 + nl : N - 1;   // rows past N computed on row N-1, never written
    if constexpr (!W4) {
      const uint4 p0 = *reinterpret_cast<const uint4*>(qw + n * K + k0 + 32 * kq);
      const uint4 p1 = *reinterpret_cast<const uint4*>(qw + n * K + k0 + 32 * kq + 16);
      const uint32_t w[8] = {p0.x ^ 0x80808080u, p0.y ^ 0x80808080u, p0.z ^ 0x80808080u, p0.w ^ 0x80808080u,
                             p1.x ^ 0x80808080u, p1.y ^ 0x80808080u, p1.z ^ 0x80808080u, p1.w ^ 0x80808080u};
      k2q_v2s r[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {   // halves: code i and code i + 16 (both + 128), zero-extended
        const uint32_t b = (uint32_t)(i & 3);
        r[i] = __builtin_bit_cast(k2q_v2s, __builtin_amdgcn_perm(w[(i >> 2) + 4], w[i >> 2],
                                                                   0x0c000c00u | b | ((4u + b) << 16)));
      }
#pragma unroll
      for (int st = 1; st < 16; st <<= 1)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (!(i & st)) {
            const k2q_v2s a = r[i], c = r[i + st];
            r[i] = a + c;
            r[i + st] = a - c;
          }
#pragma unroll
      for (int i = 0; i < 16; ++i) {   // k bit 4: the halves of one register
        const k2q_v2s sw2 = __builtin_shufflevector(r[i], r[i], 1, 0);
        r[i] = r[i] * k2q_v2s{1, -1} + sw2;
      }
      const k2q_v2s sg1 = (kq & 1) ? k2q_v2s{-1, -1} : k2q_v2s{1, 1};
      const k2q_v2s sg2 = (kq & 2) ? k2q_v2s{-1, -1} : k2q_v2s{1, 1};
#pragma unroll
      for (int i = 0; i < 16; ++i) {   // k bit 5: partner t ^ 1 (quad_perm 1,0,3,2)
        const k2q_v2s o = __builtin_bit_cast(k2q_v2s, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, r[i]), 0xB1, 0xF, 0xF, false));
        r[i] = r[i] * sg1 + o;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {   // k bit 6: partner t ^ 2 (quad_perm 2,3,0,1)
        const k2q_v2s o = __builtin_bit_cast(k2q_v2s, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, r[i]), 0x4E, 0xF, 0xF, false));
        r[i] = r[i] * sg2 + o;
      }
      if (kq == 0) r[0][0] = (short)(r[0][0] - 16384);   // the block's first output: minus 128 * 128
      const float s = sw[n] * 0.0078125f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t pk = pack_bf16x2((float)r[i][0] * s, (float)r[i][1] * s);
        tile[32 * kq + i][nl] = (uint16_t)pk;
        tile[32 * kq + i + 16][nl] = (uint16_t)(pk >> 16);
      }
    } else {
      float v[32];
      const uint4 p = *reinterpret_cast<const uint4*>(qw4 + n * (K / 2) + (k0 + 32 * kq) / 2);
      const float s = bf16_bits_to_f32(sw4[((k0 + 32 * kq) / 64) * N + n]);
      const uint32_t w[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
      for (int c = 0; c < 2; ++c)        // two 16-wide chunks: byte j holds codes j and j + 8
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t byte = (w[2 * c + (j >> 2)] >> (8 * (j & 3))) & 0xffu;
          v[16 * c + j] = (float)((int)((byte & 0xfu) ^ 8u) - 8) * s;
          v[16 * c + j + 8] = (float)((int)((byte >> 4) ^ 8u) - 8) * s;
        }
#pragma unroll
      for (int st = 1; st < 32; st <<= 1)
#pragma unroll
        for (int j = 0; j < 32; ++j)
          if (!(j & st)) {
            const float a = v[j], b = v[j + st];
            v[j] = a + b;
            v[j + st] = a - b;
          }
#pragma unroll
      for (int j = 0; j < 32; ++j) {   // k bit 5: partner t ^ 1 (quad_perm 1,0,3,2)
        const float o = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v[j]), 0xB1, 0xF, 0xF, false));
        v[j] = (kq & 1) ? o - v[j] : v[j] + o;
      }
#pragma unroll
      for (int j = 0; j < 32; ++j) {   // k bit 6: partner t ^ 2 (quad_perm 2,3,0,1)
        const float o = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v[j]), 0x4E, 0xF, 0xF, false));
        v[j] = (kq & 2) ? o - v[j] : v[j] + o;
      }
#pragma unroll
      for (int j = 0; j < 32; ++j) tile[32 * kq + j][nl] = (uint16_t)f32_to_bf16_bits(v[j] * 0.0078125f);
    }
  }
  __syncthreads();
#pragma unroll
  for (int pass = 0; pass < 4; ++pass) {
    const int kl = 32 * pass + (t >> 3), nl = 8 * (t & 7);
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = (uint32_t)tile[kl][nl + 2 * j] | ((uint32_t)tile[kl][nl + 2 * j + 1] << 16);
    uint16_t* dst = wt + (k0 + kl) * N + n0 + nl;
    if (n0 + nl + 8 <= N) *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// A-stationary plan: K cut into workgroup spans (slices), rows split so that slices x row groups ~ CUs.
struct AsPlan {
  int64_t slices, groups, rows;
};

AsPlan as_plan(int64_t M, int64_t K, int64_t r) {
  AsPlan p{};
  const int64_t span = r / 16 <= 4 ? LdShape<1>::SPAN : LdShape<8>::SPAN;
  p.slices = (K + span - 1) / span;
  const int64_t cus = k2q_cu_count();
  int64_t g = cus / p.slices;
  g = g < 1 ? 1 : g;
  const int64_t tiles = (M + 15) / 16;
  g = g > tiles ? tiles : g;
  p.rows = (tiles + g - 1) / g * 16;
  p.groups = (M + p.rows - 1) / p.rows;
  return p;
}

template <int RT>
void launch_as(const AsPlan& p, hipStream_t st, const uint16_t* x, int64_t M, int64_t ldx, const float* a, int64_t K,
               int64_t a_kstride, float a_scale, int64_t ldo, float* out) {
  hipLaunchKernelGGL(lora_down_as_kernel<RT>, dim3((unsigned)p.groups, (unsigned)p.slices), dim3(64 * LD_NW), 0, st,
                     x, M, ldx, a, K, a_kstride, a_scale, p.rows, ldo, out);
}

// Ranks run in chunks of at most LORA_CHUNK (the kernels' largest rank tile); chunk c covers factor rows
// [c LORA_CHUNK, ..) and writes its columns of u.  The chunks run one after another on the stream and share
// one workspace, so the workspace holds the largest chunk's slice partials.
constexpr int64_t LORA_CHUNK = 128;
constexpr int64_t LORA_MAX_RANK = 4096;

bool rank_ok(int64_t r) { return r >= 16 && r <= LORA_MAX_RANK && r % 16 == 0; }

int64_t chunk_ws_bytes(int64_t M, int64_t K, int64_t rc) {
  const AsPlan p = as_plan(M, K, rc);
  return p.slices > 1 ? p.slices * M * rc * 4 : 0;
}

}  // namespace

extern "C" int64_t k2q_lora_down_ws_bytes(int64_t M, int64_t K, int64_t r) {
  if (M < 1 || K < 128 || K % 128 || !rank_ok(r)) return 0;
  int64_t b = 0;
  for (int64_t c0 = 0; c0 < r; c0 += LORA_CHUNK) {
    const int64_t rc = r - c0 < LORA_CHUNK ? r - c0 : LORA_CHUNK;
    const int64_t bc = chunk_ws_bytes(M, K, rc);
    b = bc > b ? bc : b;
  }
  return b;
}

extern "C" int k2q_lora_down(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const float* lora_a,
                             int64_t r, void* ws, int64_t ws_bytes, float* u, void* stream) {
  return lora_down_impl(x, M, K, ldx, lora_a, 1, 1.f, r, ws, ws_bytes, u, static_cast<hipStream_t>(stream));
}

namespace {

// One chunk of rc <= LORA_CHUNK ranks: factor a (rows at stride K, or columns at stride a_kstride), output
// columns of u at row stride ldu.  The transposed-factor form needs the A-stationary path (one K slice, or a
// workspace for the slices).
int lora_down_chunk(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const float* a, int64_t a_kstride,
                    float a_scale, int64_t rc, void* ws, int64_t ws_bytes, float* u, int64_t ldu, hipStream_t st) {
  const AsPlan q = as_plan(M, K, rc);
  if (q.slices == 1 || (ws && ws_bytes >= q.slices * M * rc * 4)) {
    if (q.groups > 0x7fffffff || q.slices > 0xffff) return K2Q_EUNSUPPORTED;
    float* out = q.slices > 1 ? static_cast<float*>(ws) : u;
    const int64_t ldo = q.slices > 1 ? rc : ldu;
    switch (rc / 16) {
#define K2Q_AS_CASE(RT) \
  case RT: launch_as<RT>(q, st, x, M, ldx, a, K, a_kstride, a_scale, ldo, out); break;
      K2Q_AS_CASE(1) K2Q_AS_CASE(2) K2Q_AS_CASE(3) K2Q_AS_CASE(4)
      K2Q_AS_CASE(5) K2Q_AS_CASE(6) K2Q_AS_CASE(7) K2Q_AS_CASE(8)
#undef K2Q_AS_CASE
      default:
        return K2Q_EINVAL;
    }
    if (q.slices > 1) launch_reduce(static_cast<const float*>(ws), (int)q.slices, M, rc, ldu, u, st);
    return k2q_launch_status();
  }
  // No room for the slice partials: the row-tiled kernel over the whole of K in one launch.
  if (a_kstride != 1) return K2Q_EINVAL;
  const LoraPlan p = lora_plan(M, K, rc);
  if (p.row_blocks > 0x7fffffff) return K2Q_EUNSUPPORTED;
  const dim3 grid((unsigned)p.row_blocks, 1u);
  switch (rc / 16) {
#define K2Q_LD_CASE(RT) \
  case RT: launch_lora_down<RT>(p.tt, grid, st, x, M, ldx, a, K, (int)K, ldu, u); break;
    K2Q_LD_CASE(1) K2Q_LD_CASE(2) K2Q_LD_CASE(3) K2Q_LD_CASE(4)
    K2Q_LD_CASE(5) K2Q_LD_CASE(6) K2Q_LD_CASE(7) K2Q_LD_CASE(8)
#undef K2Q_LD_CASE
    default:
      return K2Q_EINVAL;
  }
  return k2q_launch_status();
}

}  // namespace

int64_t lora_down_parts_floats(int64_t M, int64_t K, int64_t r) {
  if (M < 1 || K < 128 || K % 128 || !rank_ok(r) || r > LORA_CHUNK) return 0;
  return as_plan(M, K, r).slices * M * r;
}

int lora_down_parts(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const float* lora_a, int64_t a_kstride,
                    float a_scale, int64_t r, float* dst, int64_t ldo, int* parts, hipStream_t st) {
  if (!x || !lora_a || !dst || !parts || M < 1 || K < 128 || K % 128 || ldx < K || ldx % 8) return K2Q_EINVAL;
  if (!rank_ok(r) || r > LORA_CHUNK || a_kstride < 1 || ldo < r || ldo % 4) return K2Q_EINVAL;
  if (!k2q_aligned(x, 16) || !k2q_aligned(lora_a, 16) || !k2q_aligned(dst, 16)) return K2Q_EINVAL;
  const AsPlan q = as_plan(M, K, r);
  if (q.groups > 0x7fffffff || q.slices > 0xffff) return K2Q_EUNSUPPORTED;
  switch (r / 16) {
#define K2Q_AS_CASE(RT) \
  case RT: launch_as<RT>(q, st, x, M, ldx, lora_a, K, a_kstride, a_scale, ldo, dst); break;
    K2Q_AS_CASE(1) K2Q_AS_CASE(2) K2Q_AS_CASE(3) K2Q_AS_CASE(4)
    K2Q_AS_CASE(5) K2Q_AS_CASE(6) K2Q_AS_CASE(7) K2Q_AS_CASE(8)
#undef K2Q_AS_CASE
    default:
      return K2Q_EINVAL;
  }
  *parts = (int)q.slices;
  return k2q_launch_status();
}

// u (M x r, row stride r) = x (a_scale F)^T for any rank r that is a multiple of 16, as consecutive chunks of at
// most LORA_CHUNK ranks.
int lora_down_impl(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const float* lora_a, int64_t a_kstride,
                   float a_scale, int64_t r, void* ws, int64_t ws_bytes, float* u, hipStream_t st) {
  if (!x || !lora_a || !u || M < 1 || K < 128 || K % 128 || ldx < K || ldx % 8) return K2Q_EINVAL;
  if (!rank_ok(r)) return K2Q_EINVAL;
  if (!k2q_aligned(x, 16) || !k2q_aligned(lora_a, 16) || !k2q_aligned(u, 16) || (ws && !k2q_aligned(ws, 16)))
    return K2Q_EINVAL;
  for (int64_t c0 = 0; c0 < r; c0 += LORA_CHUNK) {
    const int64_t rc = r - c0 < LORA_CHUNK ? r - c0 : LORA_CHUNK;
    const float* a = a_kstride == 1 ? lora_a + c0 * K : lora_a + c0;
    const int rc_status = lora_down_chunk(x, M, K, ldx, a, a_kstride, a_scale, rc, ws, ws_bytes, u + c0, r, st);
    if (rc_status) return rc_status;
  }
  return K2Q_OK;
}

extern "C" int k2q_dx_prep_eff(const int8_t* qw, const float* sw, const uint8_t* qw4, const uint16_t* sw4,
                               int64_t N, int64_t K, uint16_t* wt, void* stream) {
  const bool w4 = qw4 != nullptr;
  if (N < 1 || K < 128 || K % 128 || !wt) return K2Q_EINVAL;
  if (w4 ? (!sw4 || !k2q_aligned(qw4, 16)) : (!qw || !sw || !k2q_aligned(qw, 16))) return K2Q_EINVAL;
  if (!k2q_aligned(wt, 16) || N % 8) return K2Q_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((N + 63) / 64), (unsigned)(K / 128));
  if (w4)
    hipLaunchKernelGGL(rot_dequant_t_kernel<true>, grid, dim3(256), 0, st, nullptr, nullptr, qw4, sw4, N, K, wt);
  else
    hipLaunchKernelGGL(rot_dequant_t_kernel<false>, grid, dim3(256), 0, st, qw, sw, nullptr, nullptr, N, K, wt);
  return k2q_launch_status();
}

extern "C" int k2q_dx_prep(const int8_t* qw, const float* sw, const uint8_t* qw4, const uint16_t* sw4,
                           int64_t N, int64_t K, uint16_t* wt, void* stream) {
  const bool w4 = qw4 != nullptr;
  if (N < 1 || K < 128 || K % 128 || !wt) return K2Q_EINVAL;
  if (w4 ? (!sw4 || !k2q_aligned(qw4, 16)) : (!qw || !sw || !k2q_aligned(qw, 16))) return K2Q_EINVAL;
  if (!k2q_aligned(wt, 16) || N % 8) return K2Q_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((N + 63) / 64), (unsigned)(K / 64));
  if (w4)
    hipLaunchKernelGGL(dequant_t_kernel<true>, grid, dim3(256), 0, st, nullptr, nullptr, qw4, sw4, N, K, wt);
  else
    hipLaunchKernelGGL(dequant_t_kernel<false>, grid, dim3(256), 0, st, qw, sw, nullptr, nullptr, N, K, wt);
  return k2q_launch_status();
}
