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
// The register layout and the butterfly are in rotation.h.
#include "rotation.h"

namespace {

enum { MODE_ROW_I8 = 0, MODE_GROUP_I4 = 1 };

using namespace k2q_rot;

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
  const int off = lane_offset(t);
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
    rotate16(v[c], c1, c2, c8);
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
      store_codes16(qr + col, v[c], mul);
      if (xrot) {
        float xo[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) xo[i] = v[c][i] * rs;
        store16_bf16(xrot + row * (int64_t)K + col, xo);
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

// ---------------------------------------------------------------------------------------------------------
// Rotate/quant with the LoRA down-projection u = x A^T from the same pass over x (reference lora.py:47, the
// first product; kernel (3)'s A.x term).  K <= 3072 (one row per wave), K % 512 == 0, r = 16 RT <= 64.
//
// A workgroup of 16 waves owns tiles of 16 rows (the row count of v_mfma_f32_16x16x32_bf16), one row per wave,
// and walks its tiles persistently with the next tile's row in flight.  Each wave copies its raw bf16 row into
// LDS (row stride K + 8: rows start 16 bytes apart in the banks), rotates and quantizes it in registers exactly
// as rotquant_kernel does (the same codes, bit for bit), then the 16 waves split K into 16 column ranges and
// multiply the tile's rows (from LDS) by A (f32 from L2, split in registers into bf16 hi + lo, as the
// standalone down-projection does: ~2^-16 relative) on bf16 MFMA with f32 accumulation.  The 16 wave
// partials meet in LDS and are added in wave order (deterministic).  A is read once per 16-row tile: 4 r K
// bytes from L2 per 32 K bytes of x.
// ---------------------------------------------------------------------------------------------------------
constexpr int RQL_WAVES = 16;

__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// hi = bf16(v), lo = bf16(v - hi) for 8 consecutive k.
__device__ __forceinline__ void split8_hilo(v4f p, v4f q, v8bf& hi, v8bf& lo) {
  const v4u h = v4u{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]), pack_bf16x2(q[0], q[1]), pack_bf16x2(q[2], q[3])};
  const v4u l = v4u{pack_bf16x2(p[0] - __uint_as_float(h[0] << 16), p[1] - __uint_as_float(h[0] & 0xffff0000u)),
                    pack_bf16x2(p[2] - __uint_as_float(h[1] << 16), p[3] - __uint_as_float(h[1] & 0xffff0000u)),
                    pack_bf16x2(q[0] - __uint_as_float(h[2] << 16), q[1] - __uint_as_float(h[2] & 0xffff0000u)),
                    pack_bf16x2(q[2] - __uint_as_float(h[3] << 16), q[3] - __uint_as_float(h[3] & 0xffff0000u))};
  hi = __builtin_bit_cast(v8bf, h);
  lo = __builtin_bit_cast(v8bf, l);
}

template <int kNCH, int RT>
__global__ __launch_bounds__(64 * RQL_WAVES) void rotquant_lora_kernel(const __bf16* __restrict__ x, int64_t M, int K,
                                                                      int64_t ldx, int8_t* __restrict__ q,
                                                                      float* __restrict__ s,
                                                                      const float* __restrict__ a, int64_t ldu,
                                                                      float* __restrict__ u, int nwg) {
  // Loads complete in issue order as far as the wave's vmcnt wait knows, so the next tile's row (HBM) is issued
  // only after this tile's A fragments (L2): waiting for a fragment then never waits for the row.
  constexpr int NB = RT == 1 ? 4 : RT == 2 ? 2 : 1;   // 32-wide steps per A batch (<= 32 VGPRs of fragments)
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];   // [16][K + 8] bf16 rows; the u partials
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int l = lane & 15;
  const int off = lane_offset(lane);
  const int ldl = K + 8;
  const int64_t ntiles = (M + RQL_WAVES - 1) / RQL_WAVES;
  const int kw = K / RQL_WAVES;        // this wave's columns of the u product (a multiple of 32)
  const int nks = kw / 32;
  const float c1 = (l & 1) ? -1.f : 1.f;
  const float c2 = (l & 2) ? -1.f : 1.f;
  const float c8 = (l & 8) ? -1.f : 1.f;
  const float sigma = c1 * c2 * c8;
  const int kb = w * kw + 8 * (lane >> 4);
  const uint16_t* xl = xs + (lane & 15) * ldl + kb;
  const float* al = a + (int64_t)(lane & 15) * K + kb;

  uint4 raw[kNCH][2];
  auto load_row = [&](int64_t tile) {
    const int64_t row = tile * RQL_WAVES + w;
    const bool ok = tile < ntiles && row < M;
    const __bf16* xr = x + (ok ? row : 0) * ldx;
#pragma unroll
    for (int c = 0; c < kNCH; ++c) {
      const int col = c * 1024 + off;
      raw[c][0] = raw[c][1] = make_uint4(0, 0, 0, 0);
      if (ok && col < K) {
        raw[c][0] = *reinterpret_cast<const uint4*>(xr + col);
        raw[c][1] = *reinterpret_cast<const uint4*>(xr + col + 8);
      }
    }
  };

  v4f fa[NB][RT][2];
  // one batch of NB 32-wide steps of A from step k0 (steps past the wave's range repeat its last one, unused)
  auto load_a = [&](int k0) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int ks = k0 + b < nks ? k0 + b : nks - 1;
#pragma unroll
      for (int jt = 0; jt < RT; ++jt) {
        const float* p = al + (int64_t)16 * jt * K + 32 * ks;
        fa[b][jt][0] = *reinterpret_cast<const v4f*>(p);
        fa[b][jt][1] = *reinterpret_cast<const v4f*>(p + 4);
      }
    }
  };

  load_row(blockIdx.x);
  // nwg: the grid size, passed so that the kernel reads no hidden launch arguments (smaller launches)
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += nwg) {
    const int64_t row = tile * RQL_WAVES + w;
    const bool row_ok = row < M;
    // the raw row into LDS (rows past M are zeros: their u is never stored), then to f32 registers
    float v[kNCH][16];
#pragma unroll
    for (int c = 0; c < kNCH; ++c) {
      const int col = c * 1024 + off;
      if (col < K) {
        *reinterpret_cast<uint4*>(xs + w * ldl + col) = raw[c][0];
        *reinterpret_cast<uint4*>(xs + w * ldl + col + 8) = raw[c][1];
      }
      const uint32_t wd[8] = {raw[c][0].x, raw[c][0].y, raw[c][0].z, raw[c][0].w,
                              raw[c][1].x, raw[c][1].y, raw[c][1].z, raw[c][1].w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v[c][2 * j] = __uint_as_float(wd[j] << 16);
        v[c][2 * j + 1] = __uint_as_float(wd[j] & 0xffff0000u);
      }
    }
    // rotate + per-row int8 quantization: rotquant_kernel's arithmetic for one row per wave
    float amax = 0.f;
#pragma unroll
    for (int c = 0; c < kNCH; ++c) {
      rotate16(v[c], c1, c2, c8);
#pragma unroll
      for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[c][i]));
    }
    amax = fmaxf(wave_max(amax), 1e-8f);
    const float mul = __fdiv_rn(127.f, amax) * sigma;
    uint4 codes[kNCH];
#pragma unroll
    for (int c = 0; c < kNCH; ++c) {
      codes[c] = pack_codes16(v[c], mul);
      // the codes are formed here, before A's loads are issued (the rotated row's registers are then free)
      asm volatile("" ::"v"(codes[c].x), "v"(codes[c].y), "v"(codes[c].z), "v"(codes[c].w) : "memory");
    }
    // A's first batch is issued before the code stores, so waiting for it never waits for a store's completion
    // (loads and stores retire in issue order for vmcnt); with a single batch the next tile's row follows it.
    load_a(0);
    if (NB >= nks) load_row(tile + nwg);
    if (row_ok) {
      if (lane == 0) s[row] = __fdiv_rn(amax, 127.f);
      int8_t* qr = q + row * (int64_t)K;
#pragma unroll
      for (int c = 0; c < kNCH; ++c) {
        const int col = c * 1024 + off;
        if (col < K) *reinterpret_cast<uint4*>(qr + col) = codes[c];
      }
    }
    lds_sync();   // the tile's 16 rows are in LDS

    // u partial over columns [w kw, (w + 1) kw): lane l multiplies row l % 16 (8 k at 8 (l / 16) of each 32-wide
    // step) by rank l % 16 of each 16-rank tile.  Later batches of A are issued as the previous one is used up;
    // the next tile's row is issued right after the last batch's loads.
    v4f acc[RT];
#pragma unroll
    for (int jt = 0; jt < RT; ++jt) acc[jt] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < nks; k0 += NB) {
      if (k0 > 0) {
        load_a(k0);
        if (k0 + NB >= nks) load_row(tile + nwg);
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (k0 + b >= nks) break;
        const v8bf xa = __builtin_bit_cast(v8bf, *reinterpret_cast<const v4i*>(xl + 32 * (k0 + b)));
#pragma unroll
        for (int jt = 0; jt < RT; ++jt) {
          v8bf hi, lo;
          split8_hilo(fa[b][jt][0], fa[b][jt][1], hi, lo);
          acc[jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, hi, acc[jt], 0, 0, 0);
          acc[jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa, lo, acc[jt], 0, 0, 0);
        }
      }
    }
    lds_sync();   // every wave is done reading the rows
    float* part = reinterpret_cast<float*>(xs);   // [16 waves][RT][4][64]
#pragma unroll
    for (int jt = 0; jt < RT; ++jt)
#pragma unroll
      for (int i = 0; i < 4; ++i) part[((w * RT + jt) * 4 + i) * 64 + lane] = acc[jt][i];
    lds_sync();
    // C layout (16x16): lane ln owns rank 16 jt + ln % 16 and rows 4 (ln / 16) + i of the tile
    if (threadIdx.x < 256 * RT) {
      const int ln = threadIdx.x & 63, i = (threadIdx.x >> 6) & 3, jt = threadIdx.x >> 8;
      float sum = part[(jt * 4 + i) * 64 + ln];
#pragma unroll
      for (int ww = 1; ww < RQL_WAVES; ++ww) sum += part[((ww * RT + jt) * 4 + i) * 64 + ln];
      const int64_t m = tile * RQL_WAVES + 4 * (ln >> 4) + i;
      if (m < M) u[m * ldu + 16 * jt + (ln & 15)] = sum;
    }
    lds_sync();   // the partials are read before the next tile's rows overwrite them
  }
}

template <int kNCH, int RT>
int launch_rql(const __bf16* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, float* s, const float* a, int64_t ldu,
               float* u, hipStream_t st) {
  const int lds = RQL_WAVES * (int)(K + 8) * 2;
  static std::atomic<uint64_t> lds_set{0};   // the limit is set once, for the instance's largest K
  if (k2q_lds_limit_once(rotquant_lora_kernel<kNCH, RT>, RQL_WAVES * (1024 * kNCH + 8) * 2, lds_set))
    return K2Q_ELAUNCH;
  const int64_t tiles = (M + RQL_WAVES - 1) / RQL_WAVES;
  const int64_t cus = k2q_cu_count();
  const unsigned grid = (unsigned)(tiles < cus ? tiles : cus);
  hipLaunchKernelGGL((rotquant_lora_kernel<kNCH, RT>), dim3(grid), dim3(64 * RQL_WAVES), lds, st, x, M, (int)K, ldx,
                     q, s, a, ldu, u, (int)grid);
  return k2q_launch_status();
}

template <int RT>
int launch_rql_r(const __bf16* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, float* s, const float* a,
                 int64_t ldu, float* u, hipStream_t st) {
  switch ((K + 1023) / 1024) {
    case 1: return launch_rql<1, RT>(x, M, K, ldx, q, s, a, ldu, u, st);
    case 2: return launch_rql<2, RT>(x, M, K, ldx, q, s, a, ldu, u, st);
    default: return launch_rql<3, RT>(x, M, K, ldx, q, s, a, ldu, u, st);
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

// Shapes rotquant_lora_kernel takes: one row per wave in at most 3 chunks of 1024 (K <= 3072: 4 chunks leave
// no registers for the A fragments without spilling), 16 column ranges of whole 32-wide steps (K % 512 == 0),
// and the 16 wave partials of r ranks fitting where the rows sat in LDS.
int k2q_rotquant_lora_fits(int64_t K, int64_t r) {
  if (K < 512 || K > 3072 || K % 512 || r < 16 || r % 16 || r > 64) return 0;
  return (int64_t)RQL_WAVES * (r / 16) * 4 * 64 * 4 <= (int64_t)RQL_WAVES * (K + 8) * 2;
}

int rotquant_lora_impl(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, float* s, const float* a,
                       int64_t r, float* u, int64_t ldu, hipStream_t st) {
  if (!k2q_rotquant_lora_fits(K, r)) return K2Q_EUNSUPPORTED;
  const __bf16* xp = reinterpret_cast<const __bf16*>(x);
  switch (r / 16) {
    case 1: return launch_rql_r<1>(xp, M, K, ldx, q, s, a, ldu, u, st);
    case 2: return launch_rql_r<2>(xp, M, K, ldx, q, s, a, ldu, u, st);
    case 3: return launch_rql_r<3>(xp, M, K, ldx, q, s, a, ldu, u, st);
    default: return launch_rql_r<4>(xp, M, K, ldx, q, s, a, ldu, u, st);
  }
}

extern "C" int k2q_rotquant_lora(const void* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, float* s,
                                 const float* lora_a, int64_t r, float* u, int64_t ldu, void* stream) {
  int rc = check_rotquant_args(x, K2Q_DTYPE_BF16, M, K, ldx);
  if (rc) return rc;
  if (!q || !s || !lora_a || !u || !k2q_aligned(q, 16) || !k2q_aligned(lora_a, 16) || ldu < r || r % 16 != 0 || r < 16)
    return K2Q_EINVAL;
  if (!k2q_rotquant_lora_fits(K, r)) return K2Q_EUNSUPPORTED;
  return rotquant_lora_impl(static_cast<const uint16_t*>(x), M, K, ldx, q, s, lora_a, r, u, ldu,
                            static_cast<hipStream_t>(stream));
}
