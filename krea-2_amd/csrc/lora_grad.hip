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
// copied row-major by LDS-DMA (512-byte row segments) and gathered column-wise by 16-bit LDS reads.  P goes
// through a transposing split first (R x M rows of hi and lo) and reaches LDS the same way.  Each workgroup
// owns 256 columns and one slice of M; the slices' partials are added in slice order by a second kernel
// (deterministic).
#include <mutex>

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
constexpr int WG_MS = 32;               // m rows per stage
constexpr int WG_NST = 4;               // LDS ring depth (stages in flight: WG_NST - 1)
constexpr int WG_QBYTES = WG_MS * 2 * WG_KB;   // 16 KB of Q per stage: 32 rows of 512 B
constexpr int WG_QG = WG_QBYTES / 1024 / 4;    // Q DMA instructions per wave per stage

// Per stage, P^T arrives as 2 RT blocks of 16 rows x 32 m (1 KB: hi blocks 0 .. RT-1, lo blocks RT ..), one DMA
// instruction each, dealt PI per wave (padding instructions re-load block 0 into spare blocks).
template <int RT>
struct WgShape {
  static constexpr int PI = (2 * RT + 3) / 4;              // P DMA instructions per wave per stage
  static constexpr int G = WG_QG + PI;                     // all DMA instructions per wave per stage
  static constexpr int STAGE = WG_QBYTES + 4 * PI * 1024;  // bytes per ring slot
};

// Q: the 16-byte chunk c of row r sits at chunk c ^ wg_swz(r), so the four lane groups of a fragment
// gather (rows 8g + i) hit four different 64-byte bank windows.  P: chunk c of block row jr sits at
// c ^ ((jr >> 2) & 3), so the 16 rows of a fragment read cover all 64 banks.
__device__ __forceinline__ int wg_swz(int r) { return ((r >> 3) & 3) << 2; }

template <int N>
__device__ __forceinline__ void wg_wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// out (+ slice offset) = scale * P^T Q over the rows [mchunk*blockIdx.y, +mchunk) of M.
//   pth/ptl: R x Mp bf16 (P^T hi and lo, zero past M, Mp a multiple of 32); q: M x C bf16, row stride ldq.
//   trans == 0: out[j][c] (R x C); trans == 1: out[c][j] (C rows of stride ldt).  With gridDim.y > 1 the partial of slice
//   blockIdx.y goes to out + blockIdx.y * R * C in the [j][c] layout, unscaled (wgrad_reduce finishes it).
// Both operands arrive by LDS-DMA (global_load_lds_dwordx4) through a WG_NST-slot ring, one s_waitcnt and
// one s_barrier per stage (no __syncthreads: its fence would drain the prefetches).  Q rows past M are read
// clamped (finite values) and meet the zero padding of P^T, so they add nothing.
template <int RT>
__global__ __launch_bounds__(256) void wgrad_kernel(const uint16_t* __restrict__ pth, const uint16_t* __restrict__ ptl,
                                                    int64_t M, int64_t Mp, const uint16_t* __restrict__ q, int64_t C,
                                                    int64_t ldq, int64_t mchunk, float scale, int trans,
                                                    int64_t ldt, float* __restrict__ out) {
  using S = WgShape<RT>;
  constexpr int R = 16 * RT;
  __shared__ __attribute__((aligned(16))) uint8_t ring[WG_NST * S::STAGE];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t kb = (int64_t)blockIdx.x * WG_KB;
  const int64_t mb = (int64_t)blockIdx.y * mchunk;
  const int64_t me = M < mb + mchunk ? M : mb + mchunk;
  const int nsteps = (int)((me - mb + WG_MS - 1) / WG_MS);

  // Q sources: wave w's instruction i fills stage rows 2(WG_QG w + i) + lane/32, LDS chunk lane%32, which
  // holds the row's logical chunk (lane%32) ^ wg_swz(row).  Columns past C read the last valid chunk.
  uint32_t qrow[WG_QG];
  int64_t qcol[WG_QG];
#pragma unroll
  for (int i = 0; i < WG_QG; ++i) {
    const int row = 2 * (WG_QG * w + i) + (lane >> 5);
    qrow[i] = (uint32_t)row;
    const int64_t c = kb + 8 * ((lane & 31) ^ wg_swz(row));
    qcol[i] = c + 8 <= C ? c : C - 8;
  }
  // P sources: instruction PI w + i loads block b = PI w + i (block 0 again when b >= 2 RT): lane L -> block
  // row L/4, LDS chunk L%4, holding logical chunk (L%4) ^ ((row >> 2) & 3) of that row's 32 m.
  const uint16_t* prow[S::PI];
#pragma unroll
  for (int i = 0; i < S::PI; ++i) {
    const int b = S::PI * w + i < 2 * RT ? S::PI * w + i : 0;
    const int jr = lane >> 2;
    const uint16_t* base = b < RT ? pth : ptl;
    prow[i] = base + (int64_t)(16 * (b % RT) + jr) * Mp + 8 * ((lane & 3) ^ ((jr >> 2) & 3));
  }
  auto issue = [&](int st, int slot) {
    uint8_t* dst = ring + slot * S::STAGE;
#pragma unroll
    for (int i = 0; i < WG_QG; ++i) {
      int64_t m = mb + (int64_t)WG_MS * st + qrow[i];
      m = m < M ? m : M - 1;
      __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)(q + m * ldq + qcol[i]),
                                       (__attribute__((address_space(3))) void*)(dst + 1024 * (WG_QG * w + i)), 16,
                                       0, 0);
    }
    const int64_t m0 = mb + (int64_t)WG_MS * st;   // < Mp: stages never pass the 32-padded end of P^T
#pragma unroll
    for (int i = 0; i < S::PI; ++i)
      __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)(prow[i] + m0),
                                       (__attribute__((address_space(3))) void*)(dst + WG_QBYTES + 1024 * (S::PI * w + i)),
                                       16, 0, 0);
  };

  v4f acc[RT][4];
#pragma unroll
  for (int jt = 0; jt < RT; ++jt)
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) acc[jt][kt] = v4f{0.f, 0.f, 0.f, 0.f};

  // Past the last stage the DMA re-loads stage nsteps-1 into the freed slot (never one in use), which keeps
  // the count of outstanding instructions at the wait fixed.
#pragma unroll
  for (int st = 0; st < WG_NST - 1; ++st) issue(st < nsteps ? st : nsteps - 1, st);
  const int jr = lane & 15, g = lane >> 4;
  for (int s = 0; s < nsteps; ++s) {
    wg_wait_vmcnt<(WG_NST - 2) * S::G>();
    asm volatile("s_barrier" ::: "memory");   // stage s landed for every wave; stage s-1's slot is free
    const int nx = s + WG_NST - 1;
    issue(nx < nsteps ? nx : nsteps - 1, nx % WG_NST);
    const uint8_t* stg = ring + (s % WG_NST) * S::STAGE;
    v8bf ph[RT], pl[RT];
#pragma unroll
    for (int jt = 0; jt < RT; ++jt) {
      const int off = jr * 64 + 16 * (g ^ ((jr >> 2) & 3));
      ph[jt] = *reinterpret_cast<const v8bf*>(stg + WG_QBYTES + 1024 * jt + off);
      pl[jt] = *reinterpret_cast<const v8bf*>(stg + WG_QBYTES + 1024 * (RT + jt) + off);
    }
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const int c = 64 * w + 16 * kt + (lane & 15);
      uint32_t e[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = 8 * g + i;
        e[i] = *reinterpret_cast<const uint16_t*>(stg + r * (2 * WG_KB) + 16 * ((c >> 3) ^ wg_swz(r)) + 2 * (c & 7));
      }
      const v8bf qf = __builtin_bit_cast(v8bf, v4u{e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16),
                                                   e[6] | (e[7] << 16)});
#pragma unroll
      for (int jt = 0; jt < RT; ++jt) {
        acc[jt][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph[jt], qf, acc[jt][kt], 0, 0, 0);
        acc[jt][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pl[jt], qf, acc[jt][kt], 0, 0, 0);
      }
    }
  }
  wg_wait_vmcnt<0>();   // no LDS-DMA in flight when the workgroup ends

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
        *reinterpret_cast<v4f*>(o + c * ldt + j) = scale * acc[jt][kt];
      }
    }
  }
}

// out = scale * sum over slices (slice order) of part[s][j][c]; layout [j][c] or (trans) [c][j] with row stride ldt.
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(const float* __restrict__ part, int S, int64_t R, int64_t C,
                                                           float scale, int trans, int64_t ldt, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;   // index into [j][c]
  if (i >= R * C) return;
  float v = part[i];
  for (int s = 1; s < S; ++s) v += part[s * R * C + i];
  v *= scale;
  if (trans) {
    const int64_t j = i / C, c = i % C;
    out[c * ldt + j] = v;
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

// Ranks run in chunks of at most GRAD_CHUNK (the wgrad kernel's largest rank tile), one after another on the
// stream; dA's chunk c is rows [c GRAD_CHUNK, ..) of dA, dB's chunk c columns [c GRAD_CHUNK, ..) of dB.
constexpr int64_t GRAD_CHUNK = 128;
constexpr int64_t GRAD_MAX_RANK = 4096;

bool grad_shape_ok(int64_t M, int64_t N, int64_t K, int64_t r) {
  return M >= 1 && N >= 128 && N % 128 == 0 && K >= 128 && K % 128 == 0 && r >= 16 && r <= GRAD_MAX_RANK &&
         r % 16 == 0;
}

struct GradLayout {
  int64_t ld, pt, part_a, part_b, total;   // byte offsets into the workspace
  int64_t mp;
  WgradPlan pa, pb;
};

GradLayout grad_layout(int64_t M, int64_t N, int64_t K, int64_t r) {
  GradLayout L{};
  L.mp = (M + 31) / 32 * 32;
  L.pa = wgrad_plan(M, K);
  L.pb = wgrad_plan(M, N);
  int64_t off = 0;
  const int64_t rc = r < GRAD_CHUNK ? r : GRAD_CHUNK;   // ranks of the largest chunk (chunks share the partials)
  L.ld = off;     off += align256(k2q_lora_down_ws_bytes(M, N, r));
  L.pt = off;     off += 4 * align256(r * L.mp * 2);
  L.part_a = off; off += L.pa.slices > 1 ? align256(L.pa.slices * rc * K * 4) : 0;
  L.part_b = off; off += L.pb.slices > 1 ? align256(L.pb.slices * rc * N * 4) : 0;
  L.total = off;
  return L;
}

template <int RT>
void launch_wgrad(const WgradPlan& p, hipStream_t st, const uint16_t* pth, const uint16_t* ptl, int64_t M, int64_t Mp,
                  const uint16_t* q, int64_t C, float scale, int trans, int64_t ldt, float* part, float* out) {
  const dim3 grid((unsigned)p.kblocks, (unsigned)p.slices);
  float* o = p.slices > 1 ? part : out;
  hipLaunchKernelGGL(wgrad_kernel<RT>, grid, dim3(256), 0, st, pth, ptl, M, Mp, q, C, C, p.mchunk, scale, trans, ldt,
                     o);
  if (p.slices > 1) {
    const int64_t n = (int64_t)16 * RT * C;
    hipLaunchKernelGGL(wgrad_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, part,
                       (int)p.slices, (int64_t)16 * RT, C, scale, trans, ldt, out);
  }
}

void wgrad(int rt, const WgradPlan& p, hipStream_t st, const uint16_t* pth, const uint16_t* ptl, int64_t M,
           int64_t Mp, const uint16_t* q, int64_t C, float scale, int trans, int64_t ldt, float* part, float* out) {
  switch (rt) {
#define K2Q_WG_CASE(RT) \
  case RT: launch_wgrad<RT>(p, st, pth, ptl, M, Mp, q, C, scale, trans, ldt, part, out); break;
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
  if (!grad_shape_ok(M, N, K, r)) return 0;
  return grad_layout(M, N, K, r).total;
}

extern "C" int k2q_lora_grads(const uint16_t* dy, const uint16_t* x, const float* u, const float* lora_b, int64_t r,
                              float scale, int64_t M, int64_t N, int64_t K, float* g, float* dA, float* dB, void* ws,
                              int64_t ws_bytes, void* stream) {
  if (!grad_shape_ok(M, N, K, r)) return K2Q_EINVAL;
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
  const int64_t pt_bytes = align256(r * L.mp * 2);
  uint16_t* pt[4];
  for (int i = 0; i < 4; ++i) pt[i] = reinterpret_cast<uint16_t*>(w + L.pt + i * pt_bytes);

  // g = dY (scale B^T)^T: the down-projection kernel with dY as the activation and scale * B^T as the factor,
  // read from B (N x r) directly.
  const int64_t ld_bytes = k2q_lora_down_ws_bytes(M, N, r);
  int rc = lora_down_impl(dy, M, N, N, lora_b, r, scale, r, ld_bytes ? w + L.ld : nullptr, ld_bytes, g, st);
  if (rc) return rc;
  if (dA) split_t(st, g, M, r, L.mp, pt[0], pt[1]);
  if (dB) split_t(st, u, M, r, L.mp, pt[2], pt[3]);
  for (int64_t c0 = 0; c0 < r; c0 += GRAD_CHUNK) {
    const int rt = (int)((r - c0 < GRAD_CHUNK ? r - c0 : GRAD_CHUNK) / 16);
    if (dA)
      wgrad(rt, L.pa, st, pt[0] + c0 * L.mp, pt[1] + c0 * L.mp, M, L.mp, x, K, 1.f, 0, 0,
            reinterpret_cast<float*>(w + L.part_a), dA + c0 * K);
    if (dB)
      wgrad(rt, L.pb, st, pt[2] + c0 * L.mp, pt[3] + c0 * L.mp, M, L.mp, dy, N, scale, 1, r,
            reinterpret_cast<float*>(w + L.part_b), dB + c0);
  }
  return k2q_launch_status();
}

// ---------------------------------------------------------------------------------------------------------
// k2q_lora_grads_noalloc: the same gradients with the workspace taken from the library's own device scratch,
// for callers that cannot allocate.  The scratch is a file-scope device array (one copy per GPU, resident until
// the process ends); host code reaches it only through the per-device address hipGetSymbolAddress returns.
// Nothing in it needs to start at zero (the transposes zero their own padding, every partial is written before
// it is read).  All calls on one GPU share it: calls that overlap on one GPU race.
static __device__ __align__(256) uint8_t scratch[K2Q_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex scratch_mu;
void* scratch_ptr[MAX_DEVICES];

// The current device's address of `scratch`, looked up once per device (with that device current).
void* scratch_for_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return nullptr;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    scratch_ptr[dev] = ptr;
  }
  return scratch_ptr[dev];
}

}  // namespace

extern "C" int k2q_lora_grads_noalloc(const uint16_t* dy, const uint16_t* x, const float* u, const float* lora_b,
                                      int64_t r, float scale, int64_t M, int64_t N, int64_t K, float* g, float* dA,
                                      float* dB, void* stream) {
  if (!grad_shape_ok(M, N, K, r)) return K2Q_EINVAL;
  const int64_t need = grad_layout(M, N, K, r).total;
  if (need > K2Q_SCRATCH_BYTES) return K2Q_ESCRATCH;
  void* ws = scratch_for_current_device();
  if (!ws) return K2Q_ELAUNCH;
  return k2q_lora_grads(dy, x, u, lora_b, r, scale, M, N, K, g, dA, dB, ws, need, stream);
}
