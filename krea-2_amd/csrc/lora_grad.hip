// LoRA gradients through the frozen base: the autograd of lora.py:47-48 (out + scale * (x A^T) B^T)
//   g  = scale * dY B            (M x r)   also feeds the input gradient (dX += g A)
//   dA = g^T x                    (r x K)
//   dB = scale * dY^T u           (N x r)   u = x A^T from the forward
// in f32 accuracy from bf16 operands: x and dY are bf16 already (exact), the f32 factors (B, g, u) are
// split into bf16 hi + lo (to ~2^-16 relative) and every product runs on v_mfma_f32_16x16x32_bf16 with
// f32 accumulation.
//
// g is the LoRA down-projection kernel applied to dY with the rank-major factor scale * B^T.  dA and dB
// reduce over the M tokens: "wgrad" = P^T Q with a small f32 factor P (M x R) and a large bf16 Q (M x C,
// row-major).  The MFMA needs 8 consecutive m per lane for each column of Q, so Q tiles pass through LDS:
// stored row-major as loaded (coalesced 512-byte row segments) and gathered column-wise by 16-bit LDS
// reads.  P goes through a transposing split first (R x M rows of hi and lo).  Each workgroup owns 256
// columns and one slice of M; the slices' partials are added in slice order by a second kernel
// (deterministic).
#include "k2q_common.h"

namespace {

// out = transposed in (rows x cols f32, row-major): f32 out[c][r] = scale * in[r][c] (row stride ldo), or
// (SPLIT) bf16 hi/lo rows out_hi[c][r], out_lo[c][r]; columns r in [rows, ldo) of the output are zeroed.
template <bool SPLIT>
__global__ __launch_bounds__(256) void transpose_kernel(const float* __restrict__ in, int64_t rows, int64_t cols,
                                                        int64_t ldo, float scale, float* __restrict__ out,
                                                        uint16_t* __restrict__ out_hi, uint16_t* __restrict__ out_lo) {
  __shared__ float tile[32][33];
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 32 x 8
  const int64_t r0 = (int64_t)blockIdx.x * 32, c0 = (int64_t)blockIdx.y * 32;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t r = r0 + ty + 8 * i, c = c0 + tx;
    tile[ty + 8 * i][tx] = (r < rows && c < cols) ? in[r * cols + c] : 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t c = c0 + ty + 8 * i, r = r0 + tx;
    if (c >= cols || r >= ldo) continue;
    const float v = tile[tx][ty + 8 * i];
    if constexpr (SPLIT) {
      const uint32_t h = f32_to_bf16_bits(v);
      out_hi[c * ldo + r] = (uint16_t)h;
      out_lo[c * ldo + r] = (uint16_t)f32_to_bf16_bits(v - bf16_bits_to_f32(h));
    } else {
      out[c * ldo + r] = scale * v;
    }
  }
}

constexpr int WG_KB = 256;              // Q columns per workgroup (64 per wave)
constexpr int WG_MS = 32;               // m rows per step
constexpr int QROW = 2 * WG_KB + 8;     // LDS row stride (bytes): the 4 lane groups' 8-row bands sit 16 banks apart

// out (+ slice offset) = scale * P^T Q over the rows [mchunk*blockIdx.y, +mchunk) of M.
//   pth/ptl: R x Mp bf16 (P^T hi and lo, zero past M); q: M x C bf16, row stride ldq.
//   trans == 0: out[j][c] (R x C); trans == 1: out[c][j] (C x R).  With gridDim.y > 1 the partial of slice
//   blockIdx.y goes to out + blockIdx.y * R * C in the [j][c] layout, unscaled (wgrad_reduce finishes it).
template <int RT>
__global__ __launch_bounds__(256) void wgrad_kernel(const uint16_t* __restrict__ pth, const uint16_t* __restrict__ ptl,
                                                    int64_t M, int64_t Mp, const uint16_t* __restrict__ q, int64_t C,
                                                    int64_t ldq, int64_t mchunk, float scale, int trans,
                                                    float* __restrict__ out) {
  constexpr int R = 16 * RT;
  __shared__ __attribute__((aligned(16))) uint8_t qs[2][WG_MS * QROW];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t kb = (int64_t)blockIdx.x * WG_KB;
  const int64_t mb = (int64_t)blockIdx.y * mchunk;
  const int64_t me = M < mb + mchunk ? M : mb + mchunk;
  const int nsteps = (int)((me - mb + WG_MS - 1) / WG_MS);

  // Q tile: thread t holds rows (t/32) + 8i of the step, columns 8(t%32) .. +8 of the workgroup's 256.
  const int qc = 8 * (t & 31);
  const bool col_ok = kb + qc < C;
  const int64_t qcol = col_ok ? kb + qc : C - 8;
  v4i qr[4];
  auto load_q = [&](int s) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t m = mb + WG_MS * s + (t >> 5) + 8 * i;
      const v4i v = *reinterpret_cast<const v4i*>(q + (m < me ? m : me - 1) * ldq + qcol);
      qr[i] = (m < me && col_ok) ? v : v4i{0, 0, 0, 0};   // rows of other slices / past M contribute 0
    }
  };
  auto store_q = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint8_t* d = qs[buf] + ((t >> 5) + 8 * i) * QROW + 2 * qc;
      *reinterpret_cast<v2u*>(d) = v2u{(uint32_t)qr[i][0], (uint32_t)qr[i][1]};
      *reinterpret_cast<v2u*>(d + 8) = v2u{(uint32_t)qr[i][2], (uint32_t)qr[i][3]};
    }
  };
  // P^T fragments: lane l holds row 16 jt + l%16 and m = step base + 8 (l/16) .. +8.
  v4i ph[RT], pl[RT];
  auto load_p = [&](int s) {
    int64_t m = mb + WG_MS * s + 8 * (lane >> 4);
    m = m < Mp - 8 ? m : Mp - 8;
#pragma unroll
    for (int jt = 0; jt < RT; ++jt) {
      const int64_t o = (int64_t)(16 * jt + (lane & 15)) * Mp + m;
      ph[jt] = *reinterpret_cast<const v4i*>(pth + o);
      pl[jt] = *reinterpret_cast<const v4i*>(ptl + o);
    }
  };

  v4f acc[RT][4];
#pragma unroll
  for (int jt = 0; jt < RT; ++jt)
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) acc[jt][kt] = v4f{0.f, 0.f, 0.f, 0.f};

  load_q(0);
  store_q(0);
  load_p(0);
  __syncthreads();
  for (int s = 0; s < nsteps; ++s) {
    const int buf = s & 1;
    v4i ch[RT], cl[RT];
#pragma unroll
    for (int jt = 0; jt < RT; ++jt) {
      ch[jt] = ph[jt];
      cl[jt] = pl[jt];
    }
    if (s + 1 < nsteps) {
      load_q(s + 1);
      load_p(s + 1);
    }
    const uint8_t* base = qs[buf] + 8 * (lane >> 4) * QROW;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const int c = 64 * w + 16 * kt + (lane & 15);
      uint32_t e[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) e[i] = *reinterpret_cast<const uint16_t*>(base + i * QROW + 2 * c);
      const v8bf qf = __builtin_bit_cast(v8bf, v4u{e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16),
                                                   e[6] | (e[7] << 16)});
#pragma unroll
      for (int jt = 0; jt < RT; ++jt) {
        acc[jt][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, ch[jt]), qf, acc[jt][kt], 0, 0, 0);
        acc[jt][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, cl[jt]), qf, acc[jt][kt], 0, 0, 0);
      }
    }
    if (s + 1 < nsteps) store_q(buf ^ 1);   // the other buffer: every wave left it at the last barrier
    __syncthreads();
  }

  // C layout (16x16): lane l holds rows j = 4 (l/16) + i and column c = l%16 of tile (jt, kt).
  const bool partial = gridDim.y > 1;
  float* o = partial ? out + (int64_t)blockIdx.y * R * C : out;
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    const int64_t c = kb + 64 * w + 16 * kt + (lane & 15);
    if (c >= C) continue;
#pragma unroll
    for (int jt = 0; jt < RT; ++jt) {
      const int j = 16 * jt + 4 * (lane >> 4);
      if (partial || !trans) {
        const float f = partial ? 1.f : scale;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[(int64_t)(j + i) * C + c] = f * acc[jt][kt][i];
      } else {
        *reinterpret_cast<v4f*>(o + c * R + j) = scale * acc[jt][kt];
      }
    }
  }
}

// out = scale * sum over slices (slice order) of part[s][j][c]; layout [j][c] or (trans) [c][j].
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(const float* __restrict__ part, int S, int64_t R, int64_t C,
                                                           float scale, int trans, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;   // index into [j][c]
  if (i >= R * C) return;
  float v = part[i];
  for (int s = 1; s < S; ++s) v += part[s * R * C + i];
  v *= scale;
  if (trans) {
    const int64_t j = i / C, c = i % C;
    out[c * R + j] = v;
  } else {
    out[i] = v;
  }
}

struct WgradPlan {
  int64_t kblocks, slices, mchunk;
};

WgradPlan wgrad_plan(int64_t M, int64_t C) {
  WgradPlan p{};
  p.kblocks = (C + WG_KB - 1) / WG_KB;
  const int cus = k2q_cu_count();
  int64_t s = cus / p.kblocks;
  s = s < 1 ? 1 : s;
  p.mchunk = ((M + s - 1) / s + WG_MS - 1) / WG_MS * WG_MS;
  p.slices = (M + p.mchunk - 1) / p.mchunk;
  return p;
}

int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }

struct GradLayout {
  int64_t bt, ld, pt, part_a, part_b, total;   // byte offsets into the workspace
  int64_t mp;
  WgradPlan pa, pb;
};

GradLayout grad_layout(int64_t M, int64_t N, int64_t K, int64_t r) {
  GradLayout L{};
  L.mp = (M + 7) / 8 * 8;
  L.pa = wgrad_plan(M, K);
  L.pb = wgrad_plan(M, N);
  int64_t off = 0;
  L.bt = off;     off += align256(r * N * 4);
  L.ld = off;     off += align256(k2q_lora_down_ws_bytes(M, N, r));
  L.pt = off;     off += 4 * align256(r * L.mp * 2);
  L.part_a = off; off += L.pa.slices > 1 ? align256(L.pa.slices * r * K * 4) : 0;
  L.part_b = off; off += L.pb.slices > 1 ? align256(L.pb.slices * r * N * 4) : 0;
  L.total = off;
  return L;
}

template <int RT>
void launch_wgrad(const WgradPlan& p, hipStream_t st, const uint16_t* pth, const uint16_t* ptl, int64_t M, int64_t Mp,
                  const uint16_t* q, int64_t C, float scale, int trans, float* part, float* out) {
  const dim3 grid((unsigned)p.kblocks, (unsigned)p.slices);
  float* o = p.slices > 1 ? part : out;
  hipLaunchKernelGGL(wgrad_kernel<RT>, grid, dim3(256), 0, st, pth, ptl, M, Mp, q, C, C, p.mchunk, scale, trans, o);
  if (p.slices > 1) {
    const int64_t n = (int64_t)16 * RT * C;
    hipLaunchKernelGGL(wgrad_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, part,
                       (int)p.slices, (int64_t)16 * RT, C, scale, trans, out);
  }
}

void wgrad(int rt, const WgradPlan& p, hipStream_t st, const uint16_t* pth, const uint16_t* ptl, int64_t M,
           int64_t Mp, const uint16_t* q, int64_t C, float scale, int trans, float* part, float* out) {
  switch (rt) {
#define K2Q_WG_CASE(RT) \
  case RT: launch_wgrad<RT>(p, st, pth, ptl, M, Mp, q, C, scale, trans, part, out); break;
    K2Q_WG_CASE(1) K2Q_WG_CASE(2) K2Q_WG_CASE(3) K2Q_WG_CASE(4)
    K2Q_WG_CASE(5) K2Q_WG_CASE(6) K2Q_WG_CASE(7) K2Q_WG_CASE(8)
#undef K2Q_WG_CASE
    default: break;
  }
}

// P (M x r f32) -> hi/lo rows of P^T (r x Mp bf16).
void split_t(hipStream_t st, const float* P, int64_t M, int64_t r, int64_t Mp, uint16_t* hi, uint16_t* lo) {
  const dim3 grid((unsigned)((Mp + 31) / 32), (unsigned)((r + 31) / 32));
  hipLaunchKernelGGL(transpose_kernel<true>, grid, dim3(256), 0, st, P, M, r, Mp, 1.f, nullptr, hi, lo);
}

}  // namespace

extern "C" int64_t k2q_lora_grads_ws_bytes(int64_t M, int64_t N, int64_t K, int64_t r) {
  if (M < 1 || N < 128 || N % 128 || K < 128 || K % 128 || r < 16 || r > 128 || r % 16) return 0;
  return grad_layout(M, N, K, r).total;
}

extern "C" int k2q_lora_grads(const uint16_t* dy, const uint16_t* x, const float* u, const float* lora_b, int64_t r,
                              float scale, int64_t M, int64_t N, int64_t K, float* g, float* dA, float* dB, void* ws,
                              int64_t ws_bytes, void* stream) {
  if (M < 1 || N < 128 || N % 128 || K < 128 || K % 128 || r < 16 || r > 128 || r % 16) return K2Q_EINVAL;
  if (!dy || !lora_b || !g || !ws || (dA && !x) || (dB && !u)) return K2Q_EINVAL;
  if (!k2q_aligned(dy, 16) || !k2q_aligned(lora_b, 16) || !k2q_aligned(g, 16) || !k2q_aligned(ws, 256) ||
      (x && !k2q_aligned(x, 16)) || (u && !k2q_aligned(u, 16)) || (dA && !k2q_aligned(dA, 16)) ||
      (dB && !k2q_aligned(dB, 16)))
    return K2Q_EINVAL;
  const GradLayout L = grad_layout(M, N, K, r);
  if (ws_bytes < L.total) return K2Q_EINVAL;
  if (L.pa.kblocks > 0xffff || L.pa.slices > 0xffff || L.pb.slices > 0xffff) return K2Q_EUNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint8_t* w = static_cast<uint8_t*>(ws);
  float* bt = reinterpret_cast<float*>(w + L.bt);
  const int64_t pt_bytes = align256(r * L.mp * 2);
  uint16_t* pt[4];
  for (int i = 0; i < 4; ++i) pt[i] = reinterpret_cast<uint16_t*>(w + L.pt + i * pt_bytes);

  // g = dY (scale B^T)^T: the down-projection kernel with dY as the activation and scale * B^T as the factor.
  {
    const dim3 grid((unsigned)((N + 31) / 32), (unsigned)((r + 31) / 32));
    hipLaunchKernelGGL(transpose_kernel<false>, grid, dim3(256), 0, st, lora_b, N, r, N, scale, bt, nullptr, nullptr);
  }
  const int64_t ld_bytes = k2q_lora_down_ws_bytes(M, N, r);
  int rc = k2q_lora_down(dy, M, N, N, bt, r, ld_bytes ? w + L.ld : nullptr, ld_bytes, g, stream);
  if (rc) return rc;
  const int rt = (int)(r / 16);
  if (dA) {
    split_t(st, g, M, r, L.mp, pt[0], pt[1]);
    wgrad(rt, L.pa, st, pt[0], pt[1], M, L.mp, x, K, 1.f, 0, reinterpret_cast<float*>(w + L.part_a), dA);
  }
  if (dB) {
    split_t(st, u, M, r, L.mp, pt[2], pt[3]);
    wgrad(rt, L.pb, st, pt[2], pt[3], M, L.mp, dy, N, scale, 1, reinterpret_cast<float*>(w + L.part_b), dB);
  }
  return k2q_launch_status();
}
