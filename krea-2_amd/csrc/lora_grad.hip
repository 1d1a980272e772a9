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
//
// Launches per rank chunk (at most 128 ranks): the down-projection of dY (its K-slice partials), one prep
// kernel (the partials' sum g, and the hi/lo rows of g^T and u^T), one wgrad launch holding both dA and dB,
// and one reduce for both when M is sliced.
#include <algorithm>
#include <mutex>

#include "k2q_common.h"

namespace {

// The wgrad operands of one rank chunk (rc ranks, a multiple of 16), in one launch; blockIdx.z picks the factor:
//   z == 0: g = the sum of the down-projection's ns K-slice partials gp (rows of stride ldp, slice s at
//           gp + s M ldp; added in slice order, as the down-projection's own reduce adds them) -> g (row stride
//           ldg; null when gp is g itself) and, when gh is set, the bf16 hi/lo rows gh/gl of g^T (rc x Mp);
//   z == 1: the hi/lo rows uh/ul of u^T, from u (row stride ldu).
// Tiles of 32 m x 32 ranks pass through LDS (read as float4s along the ranks, written as 32 m per rank row);
// columns m in [M, Mp) of the transposes are zero.
__global__ __launch_bounds__(256) void grad_prep_kernel(const float* __restrict__ gp, int64_t ldp, int ns,
                                                        const float* __restrict__ u, int64_t ldu, int64_t M,
                                                        int64_t rc, int64_t Mp, float* __restrict__ g, int64_t ldg,
                                                        uint16_t* __restrict__ gh, uint16_t* __restrict__ gl,
                                                        uint16_t* __restrict__ uh, uint16_t* __restrict__ ul) {
  __shared__ float tile[32][33];
  const int64_t m0 = (int64_t)blockIdx.x * 32, j0 = (int64_t)blockIdx.y * 32;
  const bool isg = blockIdx.z == 0;
  {
    const int lm = threadIdx.x >> 3, lj = 4 * (threadIdx.x & 7);   // 32 rows x 8 float4s
    const int64_t m = m0 + lm, j = j0 + lj;
    v4f v = {0.f, 0.f, 0.f, 0.f};
    if (m < M && j < rc) {   // rc, ldp, ldu, ldg multiples of 4: the float4 lies inside the chunk, aligned
      if (isg) {
        const v4f* p = reinterpret_cast<const v4f*>(gp + m * ldp + j);
        const int64_t step = M * ldp / 4;
        v = p[0];
#pragma unroll 4
        for (int s = 1; s < ns; ++s) v += p[s * step];
        if (g) *reinterpret_cast<v4f*>(g + m * ldg + j) = v;
      } else {
        v = *reinterpret_cast<const v4f*>(u + m * ldu + j);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[lm][lj + e] = v[e];
  }
  uint16_t* hi = isg ? gh : uh;
  uint16_t* lo = isg ? gl : ul;
  if (!hi) return;   // the same for the whole workgroup
  __syncthreads();
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 32 m x 8 rank rows
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t jj = j0 + ty + 8 * i, m = m0 + tx;
    if (jj >= rc || m >= Mp) continue;
    const float v = tile[tx][ty + 8 * i];
    const uint32_t h = f32_to_bf16_bits(v);
    hi[jj * Mp + m] = (uint16_t)h;
    lo[jj * Mp + m] = (uint16_t)f32_to_bf16_bits(v - bf16_bits_to_f32(h));
  }
}

constexpr int WG_KB = 256;              // Q columns per workgroup (64 per wave)
constexpr int WG_MS = 32;               // m rows per stage
constexpr int WG_QBYTES = WG_MS * 2 * WG_KB;   // 16 KB of Q per stage: 32 rows of 512 B
constexpr int WG_QG = WG_QBYTES / 1024 / 4;    // Q DMA instructions per wave per stage

// Per stage, P^T arrives as 2 RT blocks of 16 rows x 32 m (1 KB: hi blocks 0 .. RT-1, lo blocks RT ..), one DMA
// instruction each, dealt PI per wave (padding instructions re-load block 0 into spare blocks).  Two workgroups
// share a CU where two rings of at least 3 slots fit its 160 KB of LDS (RT <= 4): a workgroup streams at the
// pace of its per-stage work (LDS gathers, MFMAs, one barrier), not of the memory latency (measured: 5 stages
// in flight run no faster than 3), so a second workgroup adds more than deeper rings do.
template <int RT>
struct WgShape {
  static constexpr int PI = (2 * RT + 3) / 4;              // P DMA instructions per wave per stage
  static constexpr int G = WG_QG + PI;                     // all DMA instructions per wave per stage
  static constexpr int STAGE = WG_QBYTES + 4 * PI * 1024;  // bytes per ring slot
  static constexpr int WPC = 2 * 3 * STAGE <= 160 * 1024 ? 2 : 1;   // workgroups per CU
  static constexpr int NST = 160 * 1024 / (WPC * STAGE);            // ring depth
  static_assert(NST >= 3 && (NST - 2) * G <= 63, "vmcnt counts at most 63 outstanding loads");
};

// Q: the 16-byte chunk c of row r sits at chunk c ^ wg_swz(r), so the four lane groups of a fragment
// gather (rows 8g + i) hit four different 64-byte bank windows.  P: chunk c of block row jr sits at
// c ^ ((jr >> 2) & 3), so the 16 rows of a fragment read cover all 64 banks.
__device__ __forceinline__ int wg_swz(int r) { return ((r >> 3) & 3) << 2; }

template <int N>
__device__ __forceinline__ void wg_wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One product out = scale * P^T Q of the LoRA gradients (dA: P = g, Q = x; dB: P = u, Q = dY, transposed out).
//   pth/ptl: R x Mp bf16 (P^T hi and lo, zero past M, Mp a multiple of 32); q: M x C bf16, row stride ldq.
//   The product runs as kblocks x slices workgroups: 256 columns each, over the rows [mchunk s, +mchunk) of M.
//   slices == 1: out[j][c] (trans == 0, row stride C) or out[c][j] (trans == 1, row stride ldt), scaled.
//   slices > 1: slice s's unscaled partial at out + s R C, [j][c] (row stride C) or [c][j] (row stride R);
//   wgrad_reduce_kernel finishes it.
struct WgJob {
  const uint16_t* pth;
  const uint16_t* ptl;
  const uint16_t* q;
  float* out;
  int64_t C, ldq, ldt, kblocks, slices, mchunk, blocks;   // blocks = kblocks * slices (0: no product)
  float scale;
  int trans;
};

// Up to WG_MAXJ products of one rank tile count in one launch, their workgroups laid out product after product.
constexpr int WG_MAXJ = 8;
struct WgJobs {
  WgJob j[WG_MAXJ];
  int n;
};

// The product workgroup b belongs to, and b's index inside it.  Constant-index copies keep the selected
// product's fields in scalar registers.
__device__ __forceinline__ WgJob pick_job(const WgJobs& js, int64_t b, int64_t& wi) {
  int sel = 0;
  wi = b;
#pragma unroll
  for (int i = 0; i < WG_MAXJ - 1; ++i)
    if (sel == i && i + 1 < js.n && wi >= js.j[i].blocks) {
      wi -= js.j[i].blocks;
      sel = i + 1;
    }
  WgJob job = js.j[0];
#pragma unroll
  for (int i = 1; i < WG_MAXJ; ++i)
    if (sel == i) job = js.j[i];
  return job;
}

// Both operands arrive by LDS-DMA (buffer_load ... lds through buffer resources, so the compiler's waits for the
// LDS reads stay exact) through an NST-slot ring, one s_waitcnt and one s_barrier per stage (no __syncthreads:
// its fence would drain the prefetches).  Q rows past M lie past the resource's range and read as zero; they
// meet the zero padding of P^T.
template <int RT>
__global__ __launch_bounds__(256) void wgrad_kernel(WgJobs jobs, int64_t M, int64_t Mp) {
  using S = WgShape<RT>;
  constexpr int R = 16 * RT;
  constexpr int NST = S::NST;
  __shared__ __attribute__((aligned(16))) uint8_t ring[NST * S::STAGE];
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);
  int64_t wi;
  const WgJob job = pick_job(jobs, (int64_t)blockIdx.x, wi);
  const uint16_t* pth = job.pth;
  const uint16_t* ptl = job.ptl;
  const uint16_t* q = job.q;
  float* out = job.out;
  const int64_t C = job.C, ldq = job.ldq, ldt = job.ldt, kblocks = job.kblocks, slices = job.slices;
  const int64_t mchunk = job.mchunk;
  const float scale = job.scale;
  const int trans = job.trans;
  const int64_t slice = wi / kblocks;
  const int64_t kb = (wi - slice * kblocks) * WG_KB;
  const int64_t mb = slice * mchunk;
  const int64_t me = M < mb + mchunk ? M : mb + mchunk;
  const int nsteps = (int)((me - mb + WG_MS - 1) / WG_MS);

  // Q sources: wave w's instruction i fills stage rows 2(WG_QG w + i) + lane/32, LDS chunk lane%32, which
  // holds the row's logical chunk (lane%32) ^ wg_swz(row).  Columns past C read the last valid chunk.  Each
  // stage reads through a resource over its own rows (at most WG_MS, up to this workgroup's last row me - 1;
  // mchunk is a multiple of WG_MS), so the per-lane offsets stay small whatever M and the row stride.
  uint32_t qoff[WG_QG];
#pragma unroll
  for (int i = 0; i < WG_QG; ++i) {
    const int row = 2 * (WG_QG * w + i) + (lane >> 5);
    const int64_t c = kb + 8 * ((lane & 31) ^ wg_swz(row));
    qoff[i] = (uint32_t)((row * ldq + (c + 8 <= C ? c : C - 8)) * 2);
  }
  // P sources: instruction PI w + i loads block b = PI w + i (block 0 again when b >= 2 RT): lane L -> block
  // row L/4, LDS chunk L%4, holding logical chunk (L%4) ^ ((row >> 2) & 3) of that row's 32 m.
  const __amdgpu_buffer_rsrc_t rph = k2q_rsrc(pth, (int64_t)R * Mp * 2);
  const __amdgpu_buffer_rsrc_t rpl = k2q_rsrc(ptl, (int64_t)R * Mp * 2);
  uint32_t poff[S::PI];
#pragma unroll
  for (int i = 0; i < S::PI; ++i) {
    const int b = S::PI * w + i < 2 * RT ? S::PI * w + i : 0;
    const int jr = lane >> 2;
    poff[i] = (uint32_t)(((int64_t)(16 * (b % RT) + jr) * Mp + 8 * ((lane & 3) ^ ((jr >> 2) & 3))) * 2);
  }
  auto issue = [&](int st, int slot) {
    uint8_t* dst = ring + slot * S::STAGE;
    const int64_t r0 = mb + (int64_t)WG_MS * st;
    const __amdgpu_buffer_rsrc_t rq = k2q_rsrc(q + r0 * ldq, (me - r0 < WG_MS ? me - r0 : WG_MS) * ldq * 2);
#pragma unroll
    for (int i = 0; i < WG_QG; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (__attribute__((address_space(3))) void*)(dst + 1024 * (WG_QG * w + i)),
                                               16, (int)qoff[i], 0, 0, 0);
    const int m0 = (int)((mb + (int64_t)WG_MS * st) * 2);   // < 2 Mp: stages never pass the 32-padded end of P^T
#pragma unroll
    for (int i = 0; i < S::PI; ++i) {
      const int b = S::PI * w + i < 2 * RT ? S::PI * w + i : 0;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(b < RT ? rph : rpl,
                                               (__attribute__((address_space(3))) void*)(dst + WG_QBYTES + 1024 * (S::PI * w + i)),
                                               16, (int)poff[i], m0, 0, 0);
    }
  };

  v4f acc[RT][4];
#pragma unroll
  for (int jt = 0; jt < RT; ++jt)
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) acc[jt][kt] = v4f{0.f, 0.f, 0.f, 0.f};

  // Past the last stage the DMA re-loads stage nsteps-1 into the freed slot (never one in use), which keeps
  // the count of outstanding instructions at the wait fixed.
#pragma unroll
  for (int st = 0; st < NST - 1; ++st) issue(st < nsteps ? st : nsteps - 1, st);
  const int jr = lane & 15, g = lane >> 4;
  for (int s = 0; s < nsteps; ++s) {
    wg_wait_vmcnt<(NST - 2) * S::G>();
    asm volatile("s_barrier" ::: "memory");   // stage s landed for every wave; stage s-1's slot is free
    const int nx = s + NST - 1;
    issue(nx < nsteps ? nx : nsteps - 1, nx % NST);
    const uint8_t* stg = ring + (s % NST) * S::STAGE;
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
  const bool partial = slices > 1;
  float* o = partial ? out + slice * R * C : out;
  const float f = partial ? 1.f : scale;
  const int64_t ldc = partial ? R : ldt;   // row stride of the [c][j] layout
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    const int64_t c = kb + 64 * w + 16 * kt + (lane & 15);
    if (c >= C) continue;
#pragma unroll
    for (int jt = 0; jt < RT; ++jt) {
      const int j = 16 * jt + 4 * (lane >> 4);
      if (trans) {
        *reinterpret_cast<v4f*>(o + c * ldc + j) = f * acc[jt][kt];
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) o[(int64_t)(j + i) * C + c] = f * acc[jt][kt][i];
      }
    }
  }
}

// The slice sum of one product: out[row][col] = scale * sum over slices (slice order) of part[s][row][col]
// (rows x cols, row stride cols, n4 = rows cols / 4 float4s per slice) with out rows of stride ldo.
struct RedJob {
  const float* part;
  float* out;
  int64_t cols, ldo, n4, blocks;   // blocks of 256 float4s (0: nothing to add)
  int slices;
  float scale;
};

struct RedJobs {
  RedJob j[WG_MAXJ];
  int n;
};

// The slice sums of a launch's products: workgroups laid out product after product (those without slices
// have none).
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(RedJobs reds) {
  int sel = 0;
  int64_t wi = blockIdx.x;
#pragma unroll
  for (int k = 0; k < WG_MAXJ - 1; ++k)
    if (sel == k && k + 1 < reds.n && wi >= reds.j[k].blocks) {
      wi -= reds.j[k].blocks;
      sel = k + 1;
    }
  RedJob rj = reds.j[0];
#pragma unroll
  for (int k = 1; k < WG_MAXJ; ++k)
    if (sel == k) rj = reds.j[k];
  const v4f* part = reinterpret_cast<const v4f*>(rj.part);
  const int64_t i = wi * 256 + threadIdx.x;
  if (i >= rj.n4) return;
  // Slices in groups of 8 whose loads are all issued before the adds (indices past the last slice re-read it;
  // their terms are not added), so the sum keeps slice order: ((p0 + p1) + p2) ...
  v4f v = part[i];
  for (int s0 = 1; s0 < rj.slices; s0 += 8) {
    v4f t[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int s = s0 + q < rj.slices ? s0 + q : rj.slices - 1;
      t[q] = part[s * rj.n4 + i];
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const v4f w = v + t[q];
      v = s0 + q < rj.slices ? w : v;
    }
  }
  v *= rj.scale;
  const int64_t e = 4 * i, row = e / rj.cols;
  *reinterpret_cast<v4f*>(rj.out + row * rj.ldo + (e - row * rj.cols)) = v;
}

// Slices of M shared by the products of one wgrad launch (kbs: their 256-column blocks in total) for RT rank
// tiles: one round of workgroups that fills every workgroup slot (WPC per CU), with at least 384 rows per
// workgroup (a workgroup's pipeline fill is ~3 stages of 32 rows) -- down to 128 rows when that leaves fewer
// than half the CUs busy.  Measured on MI355X (M = 4096-4608, columns 3072-16384, ranks 16-64, slice counts
// 1-16): the rule's count is within 3% of the fastest.
struct GradPlan {
  int64_t slices, mchunk;
};

int64_t col_blocks(int64_t C) { return (C + WG_KB - 1) / WG_KB; }

GradPlan grad_plan(int64_t M, int64_t kbs, int rt) {
  const int64_t cus = k2q_cu_count();
  const int64_t wpc = rt <= 2 ? WgShape<2>::WPC : rt <= 4 ? WgShape<4>::WPC : WgShape<8>::WPC;
  const int64_t fill = std::max<int64_t>(1, wpc * cus / std::max<int64_t>(kbs, 1));
  int64_t s = std::min(fill, std::max<int64_t>(1, M / 384));
  if (kbs * s < cus / 2) s = std::min(fill, std::max<int64_t>(1, M / 128));
  const int64_t mchunk = ((M + s - 1) / s + WG_MS - 1) / WG_MS * WG_MS;
  return GradPlan{(M + mchunk - 1) / mchunk, mchunk};
}

int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }

// Bytes of a product's slice partials (0 without slices).
int64_t part_bytes(const GradPlan& p, int64_t rc, int64_t C) {
  return p.slices > 1 ? align256(p.slices * rc * C * 4) : 0;
}

template <int RT>
void launch_wgrad(const WgJobs& jobs, int64_t blocks, int64_t M, int64_t Mp, hipStream_t st) {
  hipLaunchKernelGGL(wgrad_kernel<RT>, dim3((unsigned)blocks), dim3(256), 0, st, jobs, M, Mp);
}

// The products collected for one wgrad launch (one rank tile count) and the reduce that finishes the sliced ones.
struct ProductSet {
  WgJobs jobs{};
  RedJobs reds{};
  int64_t blocks = 0, red_blocks = 0;

  bool full = false;   // a product past WG_MAXJ, or too large to address, was refused (run() then fails)

  // Adds out = scale * P^T Q (P^T rows pth/ptl of R ranks; Q: M x C, row stride ldq; trans: out[c][j] with
  // row stride ldt) under plan p, its slice partials (when p slices M) at part.
  void add(const GradPlan& p, const uint16_t* pth, const uint16_t* ptl, const uint16_t* q, int64_t C, int64_t ldq,
           int64_t R, float scale, int trans, int64_t ldt, float* part, float* out) {
    // the kernel addresses P^T (R rows of the padded M) through one buffer resource: 31-bit byte offsets
    if (jobs.n == WG_MAXJ || R * (p.slices * p.mchunk + WG_MS) * 2 >= 0x7fffffffLL) {
      full = true;
      return;
    }
    WgJob& job = jobs.j[jobs.n++];
    job = WgJob{};
    job.pth = pth;
    job.ptl = ptl;
    job.q = q;
    job.C = C;
    job.ldq = ldq;
    job.ldt = ldt;
    job.kblocks = col_blocks(C);
    job.slices = p.slices;
    job.mchunk = p.mchunk;
    job.blocks = job.kblocks * p.slices;
    job.scale = scale;
    job.trans = trans;
    job.out = p.slices > 1 ? part : out;
    blocks += job.blocks;
    if (p.slices > 1) {
      RedJob& red = reds.j[reds.n++];
      red = RedJob{};
      red.part = part;
      red.out = out;
      red.cols = trans ? R : C;
      red.ldo = trans ? ldt : C;
      red.n4 = R * C / 4;
      red.blocks = (red.n4 + 255) / 256;
      red.slices = (int)p.slices;
      red.scale = scale;
      red_blocks += red.blocks;
    }
  }

  int run(int rt, int64_t M, int64_t Mp, hipStream_t st) const {
    if (full) return K2Q_EUNSUPPORTED;
    if (jobs.n == 0) return K2Q_OK;
    if (blocks > 0x7fffffff || red_blocks > 0x7fffffff) return K2Q_EUNSUPPORTED;
    switch (rt) {
#define K2Q_WG_CASE(RT) \
  case RT: launch_wgrad<RT>(jobs, blocks, M, Mp, st); break;
      K2Q_WG_CASE(1) K2Q_WG_CASE(2) K2Q_WG_CASE(3) K2Q_WG_CASE(4)
      K2Q_WG_CASE(5) K2Q_WG_CASE(6) K2Q_WG_CASE(7) K2Q_WG_CASE(8)
#undef K2Q_WG_CASE
      default: return K2Q_EINVAL;
    }
    if (red_blocks > 0)
      hipLaunchKernelGGL(wgrad_reduce_kernel, dim3((unsigned)red_blocks), dim3(256), 0, st, reds);
    return K2Q_OK;
  }
};

// The wgrad operands of one rank chunk: g from dY (the down-projection with the factor s B^T read from B's
// columns, its K-slice partials at gp with rows of stride ldp, or written straight into g when it has one
// slice and direct is set) and grad_prep_kernel's g (row stride ldg), g^T hi/lo rows (gh/gl) and u^T hi/lo rows
// (uh/ul, from u with row stride ldu); null outputs are skipped.
int prep_chunk(const uint16_t* dy, int64_t ldy, int64_t M, int64_t N, const float* b, int64_t ldb, float scale,
               int64_t rc, int64_t Mp, bool direct, float* gp, const float* u, int64_t ldu, float* g, int64_t ldg,
               uint16_t* gh, uint16_t* gl, uint16_t* uh, uint16_t* ul, hipStream_t st) {
  direct = direct && lora_down_parts_floats(M, N, rc) == M * rc;
  float* dst = direct ? g : gp;
  const int64_t ldp = direct ? ldg : rc;
  int ns = 0;
  const int rcode = lora_down_parts(dy, M, N, ldy, b, ldb, scale, rc, dst, ldp, &ns, st);
  if (rcode) return rcode;
  if (direct && !gh && !uh) return K2Q_OK;
  const dim3 grid((unsigned)(Mp / 32), (unsigned)((rc + 31) / 32), uh ? 2u : 1u);
  hipLaunchKernelGGL(grad_prep_kernel, grid, dim3(256), 0, st, dst, ldp, ns, u, ldu, M, rc, Mp,
                     direct ? nullptr : g, ldg, gh, gl, uh, ul);
  return K2Q_OK;
}

// Ranks run in chunks of at most GRAD_CHUNK (the wgrad kernel's largest rank tile), one after another on the
// stream; dA's chunk c is rows [c GRAD_CHUNK, ..) of dA, dB's chunk c columns [c GRAD_CHUNK, ..) of dB.
constexpr int64_t GRAD_CHUNK = 128;
constexpr int64_t GRAD_MAX_RANK = 4096;

bool grad_shape_ok(int64_t M, int64_t N, int64_t K, int64_t r) {
  return M >= 1 && N >= 128 && N % 128 == 0 && K >= 128 && K % 128 == 0 && r >= 16 && r <= GRAD_MAX_RANK &&
         r % 16 == 0;
}

int64_t chunk_ranks(int64_t r, int64_t c0) { return r - c0 < GRAD_CHUNK ? r - c0 : GRAD_CHUNK; }

// Workspace: the hi/lo rows of g^T and u^T (all ranks), then one region that holds, in turn, the
// down-projection's slice partials of g (read by grad_prep_kernel) and the products' slice partials (dA's,
// then dB's; written after the prep has run), sized for the largest chunk and any subset of {dA, dB}.
struct GradLayout {
  int64_t pt, parts, total;   // byte offsets into the workspace
  int64_t mp;
};

GradLayout grad_layout(int64_t M, int64_t N, int64_t K, int64_t r) {
  GradLayout L{};
  L.mp = (M + 31) / 32 * 32;
  int64_t parts = 0;
  for (int64_t c0 = 0; c0 < r; c0 += GRAD_CHUNK) {
    const int64_t rc = chunk_ranks(r, c0);
    const int rt = (int)(rc / 16);
    parts = std::max(parts, align256(lora_down_parts_floats(M, N, rc) * 4));
    const GradPlan both = grad_plan(M, col_blocks(K) + col_blocks(N), rt), a = grad_plan(M, col_blocks(K), rt),
                   b = grad_plan(M, col_blocks(N), rt);
    parts = std::max({parts, part_bytes(both, rc, K) + part_bytes(both, rc, N), part_bytes(a, rc, K),
                      part_bytes(b, rc, N)});
  }
  L.pt = 0;
  L.parts = 4 * align256(r * L.mp * 2);
  L.total = L.parts + parts;
  return L;
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
  if ((L.mp / 32) > 0x7fffffff) return K2Q_EUNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint8_t* w = static_cast<uint8_t*>(ws);
  const int64_t pt_bytes = align256(r * L.mp * 2);
  uint16_t* pt[4];
  for (int i = 0; i < 4; ++i) pt[i] = reinterpret_cast<uint16_t*>(w + L.pt + i * pt_bytes);
  float* parts = reinterpret_cast<float*>(w + L.parts);

  for (int64_t c0 = 0; c0 < r; c0 += GRAD_CHUNK) {
    const int64_t rc = chunk_ranks(r, c0);
    const int rt = (int)(rc / 16);
    int rcode = prep_chunk(dy, N, M, N, lora_b + c0, r, scale, rc, L.mp, r <= GRAD_CHUNK, parts, dB ? u + c0 : nullptr,
                           r, g + c0, r, dA ? pt[0] + c0 * L.mp : nullptr, dA ? pt[1] + c0 * L.mp : nullptr,
                           dB ? pt[2] + c0 * L.mp : nullptr, dB ? pt[3] + c0 * L.mp : nullptr, st);
    if (rcode) return rcode;
    if (!dA && !dB) continue;
    // dA and dB in one launch, sharing the slice count; their partials follow one another in the region
    const GradPlan p = grad_plan(M, (dA ? col_blocks(K) : 0) + (dB ? col_blocks(N) : 0), rt);
    ProductSet set;
    if (dA) set.add(p, pt[0] + c0 * L.mp, pt[1] + c0 * L.mp, x, K, K, rc, 1.f, 0, 0, parts, dA + c0 * K);
    if (dB)
      set.add(p, pt[2] + c0 * L.mp, pt[3] + c0 * L.mp, dy, N, N, rc, scale, 1, r,
              reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(parts) + (dA ? part_bytes(p, rc, K) : 0)),
              dB + c0);
    rcode = set.run(rt, M, L.mp, st);
    if (rcode) return rcode;
  }
  return k2q_launch_status();
}

// ---------------------------------------------------------------------------------------------------------
// k2q_lora_grads_grouped: the LoRA gradients of n linears that read one input (a grouped node's backward).
// Member i's g goes straight into columns [i r, (i+1) r) of the stacked g, which the grouped input gradient
// reads; dA of every member comes from one wgrad pass over x per 128 stacked ranks (rows of the stacked dA);
// the members' dB products share one launch.  Per member: the down-projection of dY_i and one prep launch.
namespace {

constexpr int64_t GROUP_MAX = WG_MAXJ;

bool group_ok(const k2q_lora_member* m, int64_t n, int64_t M, int64_t K, int64_t r) {
  if (!m || n < 1 || n > GROUP_MAX || M < 1 || K < 128 || K % 128 || r < 16 || r > GRAD_CHUNK || r % 16) return false;
  for (int64_t i = 0; i < n; ++i)
    if (m[i].N < 128 || m[i].N % 128 || m[i].ldy < m[i].N || m[i].ldy % 8) return false;
  return true;
}

struct GroupLayout {
  int64_t pt, parts, total;
  int64_t mp;
};

// The stacked ranks' dA launches: full 128-rank chunks share one launch, a shorter last chunk has its own.
int64_t group_da_chunks(int64_t R) { return (R + GRAD_CHUNK - 1) / GRAD_CHUNK; }

GroupLayout group_layout(const k2q_lora_member* m, int64_t n, int64_t M, int64_t K, int64_t r) {
  GroupLayout L{};
  L.mp = (M + 31) / 32 * 32;
  const int64_t R = n * r;
  int64_t parts = 0, nb = 0;
  for (int64_t i = 0; i < n; ++i) {
    parts = std::max(parts, align256(lora_down_parts_floats(M, m[i].N, r) * 4));
    nb += col_blocks(m[i].N);
  }
  // dA: the full chunks' launch, then the tail's
  const int64_t full = R / GRAD_CHUNK, tail = R % GRAD_CHUNK;
  if (full > 0) {
    const GradPlan p = grad_plan(M, full * col_blocks(K), 8);
    parts = std::max(parts, full * part_bytes(p, GRAD_CHUNK, K));
  }
  if (tail > 0) parts = std::max(parts, part_bytes(grad_plan(M, col_blocks(K), (int)(tail / 16)), tail, K));
  // dB: every member in one launch (any subset fits: fewer members plan more slices, but never more bytes than
  // the whole set at its own plan is guaranteed, so size for each subset size's worst case)
  for (int64_t kbs = 1; kbs <= nb; ++kbs) {
    const GradPlan p = grad_plan(M, kbs, (int)(r / 16));
    int64_t b = 0;
    for (int64_t i = 0; i < n; ++i) b += part_bytes(p, r, m[i].N);
    parts = std::max(parts, b);
  }
  L.pt = 0;
  L.parts = 4 * align256(R * L.mp * 2);
  L.total = L.parts + parts;
  return L;
}

}  // namespace

extern "C" int64_t k2q_lora_grads_grouped_ws_bytes(const k2q_lora_member* m, int64_t n, int64_t M, int64_t K,
                                                   int64_t r) {
  if (!group_ok(m, n, M, K, r)) return 0;
  return group_layout(m, n, M, K, r).total;
}

extern "C" int k2q_lora_grads_grouped(const k2q_lora_member* m, int64_t n, const uint16_t* x, const float* u,
                                      int64_t r, int64_t M, int64_t K, float* g, float* dA, void* ws,
                                      int64_t ws_bytes, void* stream) {
  if (!group_ok(m, n, M, K, r)) return K2Q_EINVAL;
  bool any_db = false;
  for (int64_t i = 0; i < n; ++i) {
    if (!m[i].dy || !m[i].lora_b || !k2q_aligned(m[i].dy, 16) || !k2q_aligned(m[i].lora_b, 16) ||
        (m[i].dB && !k2q_aligned(m[i].dB, 16)))
      return K2Q_EINVAL;
    any_db = any_db || m[i].dB;
  }
  if (!g || !ws || !k2q_aligned(g, 16) || !k2q_aligned(ws, 256) || (dA && (!x || !k2q_aligned(x, 16) ||
      !k2q_aligned(dA, 16))) || (any_db && (!u || !k2q_aligned(u, 16))))
    return K2Q_EINVAL;
  const GroupLayout L = group_layout(m, n, M, K, r);
  if (ws_bytes < L.total) return K2Q_EINVAL;
  if ((L.mp / 32) > 0x7fffffff) return K2Q_EUNSUPPORTED;
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint8_t* w = static_cast<uint8_t*>(ws);
  const int64_t R = n * r;
  const int64_t pt_bytes = align256(R * L.mp * 2);
  uint16_t* pt[4];
  for (int i = 0; i < 4; ++i) pt[i] = reinterpret_cast<uint16_t*>(w + L.pt + i * pt_bytes);
  float* parts = reinterpret_cast<float*>(w + L.parts);

  for (int64_t i = 0; i < n; ++i) {
    const k2q_lora_member& mi = m[i];
    const int64_t c0 = i * r;
    const int rcode = prep_chunk(mi.dy, mi.ldy, M, mi.N, mi.lora_b, r, mi.scale, r, L.mp, true, parts,
                                 mi.dB ? u + c0 : nullptr, R, g + c0, R, dA ? pt[0] + c0 * L.mp : nullptr,
                                 dA ? pt[1] + c0 * L.mp : nullptr, mi.dB ? pt[2] + c0 * L.mp : nullptr,
                                 mi.dB ? pt[3] + c0 * L.mp : nullptr, st);
    if (rcode) return rcode;
  }
  if (dA) {
    // the full 128-rank chunks of the stacked g in one launch, the tail in another
    const int64_t full = R / GRAD_CHUNK, tail = R % GRAD_CHUNK;
    if (full > 0) {
      const GradPlan p = grad_plan(M, full * col_blocks(K), 8);
      ProductSet set;
      for (int64_t c = 0; c < full; ++c)
        set.add(p, pt[0] + c * GRAD_CHUNK * L.mp, pt[1] + c * GRAD_CHUNK * L.mp, x, K, K, GRAD_CHUNK, 1.f, 0, 0,
                reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(parts) + c * part_bytes(p, GRAD_CHUNK, K)),
                dA + c * GRAD_CHUNK * K);
      const int rcode = set.run(8, M, L.mp, st);
      if (rcode) return rcode;
    }
    if (tail > 0) {
      const int64_t c0 = full * GRAD_CHUNK;
      const GradPlan p = grad_plan(M, col_blocks(K), (int)(tail / 16));
      ProductSet set;
      set.add(p, pt[0] + c0 * L.mp, pt[1] + c0 * L.mp, x, K, K, tail, 1.f, 0, 0, parts, dA + c0 * K);
      const int rcode = set.run((int)(tail / 16), M, L.mp, st);
      if (rcode) return rcode;
    }
  }
  if (any_db) {
    int64_t kbs = 0;
    for (int64_t i = 0; i < n; ++i)
      if (m[i].dB) kbs += col_blocks(m[i].N);
    const GradPlan p = grad_plan(M, kbs, (int)(r / 16));
    ProductSet set;
    int64_t off = 0;
    for (int64_t i = 0; i < n; ++i) {
      if (!m[i].dB) continue;
      const int64_t c0 = i * r;
      set.add(p, pt[2] + c0 * L.mp, pt[3] + c0 * L.mp, m[i].dy, m[i].N, m[i].ldy, r, m[i].scale, 1, r,
              reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(parts) + off), m[i].dB);
      off += part_bytes(p, r, m[i].N);
    }
    const int rcode = set.run((int)(r / 16), M, L.mp, st);
    if (rcode) return rcode;
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
