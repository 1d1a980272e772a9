// Kernels (2)-(4): LDS-tiled MFMA GEMMs with fused epilogues for gfx950.
//
// All three GEMMs of the path have both operands contiguous along the reduction axis ("NT"):
//   forward  acc[m,n] = sum_k qx[m,k] qw[n,k]          int8 x int8 -> int32 (v_mfma_i32_32x32x32_i8)
//   dX       t[m,k]   = sum_n dy[m,n] wt[k,n]          bf16 x bf16 -> f32   (v_mfma_f32_32x32x16_bf16)
// so one skeleton serves both: operand "A" supplies the rows of the MFMA output (n, or k for dX),
// operand "B" its columns (m); out[b_row][a_row] is row-major over (m, n|k).
//
// Tiling: 256 x 256 output tile per 512-thread workgroup (8 waves, 2 per SIMD; wave w owns 128 A-rows x
// 64 B-rows as 4 x 2 MFMA 32x32 blocks), 128 bytes of reduction per stage (128 int8 or 64 bf16), LDS
// double-buffered (2 x 64 KB) and filled by LDS-DMA.  LDS rows are 128 B; the 16-byte chunk c of row r
// lives at chunk c ^ f(r) with f(r) = (r & 7) ^ ((r >> 3) & 1), which keeps the 16-byte MFMA fragment
// reads free of bank conflicts.  Workgroup ids are remapped so that consecutive tiles land on the same
// XCD (ids are dealt round-robin over the 8 XCDs), then grouped GB B-tiles at a time (8 for launches of
// several rounds; 8, 4 or 2 by operand footprint for one-round launches) so concurrently running tiles share
// operand strips in that XCD's L2.
//
// Epilogues (in registers, MFMA C layout: lane l owns output column l%32 and rows 8j+4(l/32)+i):
//   EPI_W8   y = bf16(2^-7 s_x[m] s_w[n] acc + bias[n] + LoRA), LoRA = one bf16 MFMA per 16 of rank
//            accumulating lora_scale*u[m,:] . lora_b[n,:] onto the dequantized f32 value.
//   EPI_ACC  raw int32 acc (debug entry for bit-exact checks).
//   EPI_DX   inverse rotation: FWHT over each 128-block of k (a wave's 128 A-rows are one block),
//            times 2^-7, plus the LoRA term g[m,:] . A[:,k], stored bf16.
//   EPI_LIN  bf16 x bf16 linear (the fp8 weight-only base, quantize.py:48-51): y = bf16(acc + bias[n] + LoRA).
//   EPI_DXLIN its input gradient: dx = bf16(acc + LoRA), no rotation.
// Every bf16 output is rounded once, after the LoRA term is added in f32.
#include "k2q_common.h"

#include <type_traits>

namespace {

enum { EPI_W8 = 0, EPI_ACC = 1, EPI_DX = 2, EPI_LIN = 3, EPI_DXLIN = 4 };

typedef short k2q_v4s __attribute__((ext_vector_type(4)));   // 4 bf16 as the 16x16x16 bf16 MFMA's operand


constexpr int BKB = 128;    // reduction bytes per stage

// One segment of a grouped forward (EPI_W8): linears that read the same input, their weight rows stacked
// along A.  Each segment starts on a 256-row tile boundary, so a tile lies in one segment and takes its
// operands, output and LoRA factors from it.
constexpr int MAX_SEG = 4;
struct GemmSeg {
  const uint8_t* a;        // the segment's weight codes, rows x kbytes
  const float* sw;         // its per-row scales
  const float* bias;       // nullable
  const float* lora_ra;    // its lora_b (rows x r f32); nullable: no adapter on this segment
  void* out;               // its output, row stride ldo
  int64_t start, rows, ldo;   // first A-row of the segment in the stacked numbering, rows, output stride
  int64_t rb_off;          // column of its factors in lora_rb
  float lora_scale;
};

// One segment of a segmented reduction (EPI_DXLIN): stages end_prev .. end-1 of the reduction read A from a and
// B from b with their own row strides.
struct KSeg {
  const uint8_t* a;
  const uint8_t* b;
  int64_t lda_b, ldb_b;
  int end;                 // first stage (WBK reduction bytes) past this segment
};

struct GemmBase {
  const uint8_t* a;   // A operand, rows_a x kbytes, row stride lda_b bytes
  const uint8_t* b;   // B operand, rows_b x kbytes
  int64_t rows_a, rows_b, kbytes, lda_b, ldb_b;
  void* out;          // out[b_row][a_row], row stride ldo elements
  int64_t ldo;
  const float* sx;    // EPI_W8: per-B-row scale (already multiplied by nothing; 2^-7 applied here)
  const float* sw;    // EPI_W8: per-A-row scale
  const float* bias;  // EPI_W8: per-A-row bias (nullable)
  const float* lora_rb;  // per-B-row LoRA factor rows (u or g), rows_b x r f32 (nullable)
  const float* lora_ra;  // per-A-row LoRA factors: lora_b (rows_a x r f32) for the forward epilogues, the
                         // LoRA A itself (r x rows_a f32, so column a holds row a's factors) for EPI_DX/DXLIN
  int r;
  int ldr;            // row stride of lora_rb in elements (r unless the factors of several segments share rows)
  int rb_parts;       // > 1: lora_rb holds that many K-slice partials of the factors, rb_pstride elements apart,
  int64_t rb_pstride; //      added in slice order as they are read (the down-projection's reduce, folded in)
  float lora_scale;
  int nseg;           // 0: one linear; else rows_a stacks nseg segments (EPI_W8)
  int nks;            // 0: one reduction operand pair; else the reduction runs over nks segments (EPI_DXLIN)
  int nwg;            // workgroups of a full-K tile launch (the grid size, passed so that the kernel reads no
                      // hidden launch arguments and its launches write ~256 bytes less)
  // Split schedule for the last, partly filled round of tiles: tiles 0 .. dp_tiles-1 run over the full
  // reduction; each of the sk_rem remainder tiles dp_tiles + i is cut into sk_s pieces (piece q covers
  // reduction slice q / sk_rem) whose accumulators go to part, and a fixup launch adds them.
  int64_t dp_tiles;
  int sk_rem, sk_s;
  int32_t* part;
  int gb;             // B-tiles per group of the tile order (group_coords), set by launch_gemm
};

// The kernel arguments: the base fields, plus the segment tables (seg for nseg, ks for nks) in the kernels of
// grouped launches only.  The tables are most of the struct's bytes, and a launch's arguments are written out
// per launch: ~180 bytes instead of ~660 measured ~2 us less host time per launch while the GPU is busy.
template <int NS>
struct GemmArgsN : GemmBase {
  GemmSeg seg[NS];
  KSeg ks[NS];
};
template <>
struct GemmArgsN<0> : GemmBase {};
using GemmArgs = GemmArgsN<MAX_SEG>;   // what the host fills; a launch without segments passes its base

__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }
// The 16 x 16 fragment reads (lane l: row l%16 of a 16-row block, chunk 4 w + l/16) take this one instead:
// measured with the same reads over an LDS-resident buffer, swz conflicts on them (1.3e9 bank-conflict cycles
// where row & 7 has none, and is the faster of the two), while the 32 x 32 reads are conflict-free under swz.
__device__ __forceinline__ int swz16(int row) { return row & 7; }

// Workgroup ids are dealt round-robin over the 8 XCDs; renumber them so that consecutive ids share an XCD.
__device__ __forceinline__ int xcd_remap(int bid, int nwg) {
  const int xcd = bid & 7, idx = bid >> 3;
  const int per = (nwg + 7) >> 3, rem = nwg & 7;
  return (rem == 0 || xcd < rem) ? xcd * per + idx : rem * per + (xcd - rem) * (per - 1) + idx;
}

// Linear tile id -> (A tile, B tile), GB B-tiles per group so tiles running together share operand strips
// (GB chosen per launch by the host: group_width).
__host__ __device__ __forceinline__ void group_coords(int64_t lid, int64_t tiles_a, int64_t tiles_b, int GB,
                                                      int64_t& ta, int64_t& tb) {
  const int64_t in_group = (int64_t)GB * tiles_a;
  const int64_t g = lid / in_group;
  const int64_t first_b = g * GB;
  const int64_t gsize = (tiles_b - first_b) < GB ? (tiles_b - first_b) : GB;
  const int64_t r = lid % in_group;
  tb = first_b + r % gsize;
  ta = r / gsize;
}

// The same in 32-bit arithmetic, for the W4 kernel's one tile per workgroup (tile counts < 2^31).
__device__ __forceinline__ void tile_coords(uint32_t tiles_a, uint32_t tiles_b, uint32_t& ta, uint32_t& tb) {
  const uint32_t lid = (uint32_t)xcd_remap(blockIdx.x, tiles_a * tiles_b);   // the grid is one workgroup per tile
  constexpr uint32_t GB = 8;
  const uint32_t in_group = GB * tiles_a;
  const uint32_t g = lid / in_group;
  const uint32_t first_b = g * GB;
  const uint32_t gsize = (tiles_b - first_b) < GB ? (tiles_b - first_b) : GB;
  const uint32_t r = lid - g * in_group;
  tb = first_b + r % gsize;
  ta = r / gsize;
}

__device__ __forceinline__ v4i frag(const uint8_t* s, int row, int chunk) {
  return *reinterpret_cast<const v4i*>(s + row * BKB + 16 * (chunk ^ swz(row)));
}

template <bool BF16, class AccT>
__device__ __forceinline__ void mma(v4i a, v4i b, AccT& c) {
  if constexpr (std::is_same_v<AccT, v4i>) {   // int8, 16 x 16 blocks
    c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
  } else if constexpr (BF16) {
    v16f cf = __builtin_bit_cast(v16f, c);
    cf = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b),
                                                cf, 0, 0, 0);
    c = __builtin_bit_cast(v16i, cf);
  } else {
    c = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
}

// 8 consecutive f32 -> 8 bf16 (times s), as an MFMA fragment.
__device__ __forceinline__ v8bf f32x8_to_bf16(const float* p, float s) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  v4i w;
  w[0] = (int)pack_bf16x2(a.x * s, a.y * s);
  w[1] = (int)pack_bf16x2(a.z * s, a.w * s);
  w[2] = (int)pack_bf16x2(b.x * s, b.y * s);
  w[3] = (int)pack_bf16x2(b.z * s, b.w * s);
  return __builtin_bit_cast(v8bf, w);
}

// LoRA term of one 32 x 32 output block, accumulated onto its f32 values with bf16 MFMAs (r/16 of them):
// f[a_row][b_col] += lora_ra[a_row, :] . (scale * lora_rb[b_col, :]).
__device__ __forceinline__ v16f lora_block(const float* lora_ra, const float* lora_rb, int r, float scale,
                                           int64_t rows_a, int64_t rows_b, int64_t arow0, int64_t bcol0,
                                           int lane, v16f f) {
  const int h = lane >> 5, c = lane & 31;
  int64_t ra = arow0 + c, rb = bcol0 + c;
  ra = ra < rows_a ? ra : rows_a - 1;
  rb = rb < rows_b ? rb : rows_b - 1;
  for (int ks = 0; ks < r; ks += 16) {
    const v8bf fa = f32x8_to_bf16(lora_ra + ra * r + ks + 8 * h, 1.f);
    const v8bf fb = f32x8_to_bf16(lora_rb + rb * r + ks + 8 * h, scale);
    f = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa, fb, f, 0, 0, 0);
  }
  return f;
}

// Inverse rotation of one column slice: FWHT over the wave's 128 A-rows (one Hadamard block), times
// 2^-7.  Row-index bits: i -> 0-1 (register e bits 0-1), h -> 2 (partner lane l^32), j -> 3-4 (e bits
// 2-3), ia -> 5-6.  The order of the stages is free here: the result is held to a tolerance.
__device__ __forceinline__ void fwht128_rows(v16f (&f)[4], int h) {
#pragma unroll
  for (int st = 1; st <= 8; st <<= 1)
#pragma unroll
    for (int ia = 0; ia < 4; ++ia)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        if (e & st) continue;
        const float a = f[ia][e], b = f[ia][e + st];
        f[ia][e] = a + b;
        f[ia][e + st] = a - b;
      }
#pragma unroll
  for (int st = 1; st <= 2; st <<= 1)
#pragma unroll
    for (int ia = 0; ia < 4; ++ia) {
      if (ia & st) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float a = f[ia][e], b = f[ia + st][e];
        f[ia][e] = a + b;
        f[ia + st][e] = a - b;
      }
    }
#pragma unroll
  for (int ia = 0; ia < 4; ++ia)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float pv = __shfl_xor(f[ia][e], 32, 64);
      f[ia][e] = (h ? (pv - f[ia][e]) : (f[ia][e] + pv)) * 0.0078125f;
    }
}

// ---------------------------------------------------------------------------------------------------------
// Main-loop data movement: global -> LDS by the gfx950 LDS-DMA path (buffer_load_dwordx4 ... lds), no VGPR
// staging.  The FLAT form (global_load_lds_dwordx4) measured 4-6 % slower on every GEMM shape: the compiler
// counts a FLAT LDS write against lgkmcnt too, so each wait for a fragment read became lgkmcnt(0).  A stage is 128 bytes of the reduction axis for the tile's TA A-rows and TB B-rows (the
// frag()/swz() layout above); two stages alternate in LDS.  One DMA wave instruction fills 8 consecutive LDS
// rows (1 KB: lane l -> row l/8, physical chunk l%8) and each lane fetches the logical chunk (l%8) ^ swz(row)
// of its row, so every instruction reads 8 whole 128-byte lines.  Measured on MI355X (same box, random data)
// against 64-byte stages fetched as paired half lines through a 5-slot ring: cfg2 GEMM 643.6 -> 626.6 us,
// cfg3 input-gradient GEMM 331.5 -> 323.1 us; in a copy-only loop with the same waits and barriers, half
// lines, paired half lines and whole lines move 24, 31 and 35 B/clk/CU.  A stage is consumed after every
// wave's `s_waitcnt vmcnt` for it plus one lds_barrier() (the wave's LDS operations, then s_barrier; not
// __syncthreads, whose full memory fence would drain the prefetches).
constexpr int SBK = 64;                   // unit of reduction lengths in the split plan (half a stage)
constexpr int K2Q_DMA_CPOL = 1;           // cache policy bits of the main-loop copies: sc0
constexpr int WBK = 128;                  // reduction bytes per stage

#define K2Q_LPTR(p) ((__attribute__((address_space(3))) void*)(p))

constexpr int GW = 8;                     // waves per workgroup (two per SIMD)
constexpr int GT = 64 * GW;               // threads per workgroup
constexpr int LROW = 48;                  // epilogue LoRA staging row (bytes; see TileCfg)

// Output tile shapes.  A workgroup computes TA A-rows x TB B-rows with its 8 waves laid out WVA along A by
// 8/WVA along B; each wave owns NA x NB blocks of 32 x 32 (v_mfma 32x32 accumulators).  Per stage a wave
// issues DA + DB DMA instructions (8 rows each).  The epilogue stages the bf16 tile in LDS CROWS B-rows at a
// time (rows of CROW bytes: TA values plus 16 bytes of padding, which spreads a lane group's 8-byte writes
// over all banks), then 3 sets of scales, then the LoRA factor rows of one 16-rank chunk as bf16 (A-side rows,
// then B-side rows, LROW bytes each: 48, so the 16 rows read by a lane group start 12 words apart and cover
// all 64 banks).
//   T256 256 x 256: the general tile (4 x 2 blocks per wave, 128 accumulator registers).
//   T320 256 x 320: 2 x 5 blocks per wave; 10 % fewer global->LDS bytes per MAC, and M = 16896 (2048^2)
//        splits into 52.8 tiles of 320 where 256-row tiles leave 12.4 rounds of the GPU: 10 rounds instead
//        of 13.  Its epilogue stages 160 B-rows at a time.
//   T192 192 x 256 and T128 128 x 128 (two workgroups per CU): for grids that leave most of a round idle.
template <int TA_, int TB_, int WVA_, int WPC_>
struct TileCfg {
  static constexpr int TA = TA_, TB = TB_, WVA = WVA_, WVB = GW / WVA_, WPC = WPC_;   // WPC: workgroups per CU
  static constexpr int NA = TA / (32 * WVA), NB = TB / (32 * WVB);
  static constexpr int ARW = 32 * NA, BRW = 32 * NB;
  static constexpr int DA = TA / 8 / GW, DB = TB / 8 / GW;
  static constexpr int STAGE = (TA + TB) * WBK;
  static constexpr int CROW = 2 * TA + 16;
  static constexpr int CROWS = TB <= 256 ? TB : TB / 2;
  static constexpr int SCALE_OFF = CROWS * CROW;
  static constexpr int LORA_OFF = SCALE_OFF + (TB + 2 * TA) * 4;
  static constexpr int EPI_BYTES = LORA_OFF + (TA + TB) * LROW;
  static constexpr int LDS = 2 * STAGE > EPI_BYTES ? 2 * STAGE : EPI_BYTES;
  static constexpr int NBR = (TB + GT / 2 - 1) / (GT / 2);   // LoRA B-side rows staged per thread
  static_assert(NA * 32 * WVA == TA && NB * 32 * WVB == TB, "waves tile the output");
  static_assert(DA * 8 * GW == TA && DB * 8 * GW == TB, "DMA rows cover the stage");
  static_assert(TA <= GT / 2 && CROWS % BRW == 0 && TB % CROWS == 0, "epilogue staging");
  static_assert(LDS * WPC <= 160 * 1024, "gfx950 LDS is 160 KB per CU");
};
using T256 = TileCfg<256, 256, 2, 1>;
using T320 = TileCfg<256, 320, 4, 1>;
using T192 = TileCfg<192, 256, 2, 1>;
using T128 = TileCfg<128, 128, 2, 2>;
enum { TILE_AUTO = -1, TILE_256 = 0, TILE_320 = 1, TILE_192 = 2, TILE_128 = 3, TILE_COUNT = 4 };
static_assert(TILE_AUTO == K2Q_TILE_AUTO && TILE_256 == K2Q_TILE_256x256 && TILE_320 == K2Q_TILE_256x320 &&
                  TILE_192 == K2Q_TILE_192x256 && TILE_128 == K2Q_TILE_128x128 && TILE_COUNT == K2Q_TILE_GEMV,
              "tile ids of the C ABI");

// One 32 x 32 block of f32 (MFMA C layout) into the LDS tile as bf16: lane l owns tile row mrow0 + l%32
// and columns ncol0 + 8j + 4(l/32) .. +3.
template <int CROW>
__device__ __forceinline__ void ctile_put(uint8_t* ct, int mrow0, int ncol0, int lane, const v16f& f) {
  uint8_t* row = ct + (mrow0 + (lane & 31)) * CROW + 2 * (ncol0 + 4 * (lane >> 5));
#pragma unroll
  for (int j = 0; j < 4; ++j)
    *reinterpret_cast<v2u*>(row + 16 * j) = v2u{pack_bf16x2(f[4 * j], f[4 * j + 1]), pack_bf16x2(f[4 * j + 2], f[4 * j + 3])};
}

// One 16 x 16 block (MFMA C layout) into the LDS tile as bf16: lane l owns tile row mrow0 + l%16 and columns
// ncol0 + 4(l/16) .. +3.
template <int CROW>
__device__ __forceinline__ void ctile_put16(uint8_t* ct, int mrow0, int ncol0, int lane, const v4f& f) {
  uint8_t* row = ct + (mrow0 + (lane & 15)) * CROW + 2 * (ncol0 + 4 * (lane >> 4));
  *reinterpret_cast<v2u*>(row) = v2u{pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3])};
}

__device__ __forceinline__ v8bf f32x8_to_bf16v(v4f a, v4f b, float s) {
  const v4u w = v4u{pack_bf16x2(a[0] * s, a[1] * s), pack_bf16x2(a[2] * s, a[3] * s), pack_bf16x2(b[0] * s, b[1] * s),
                    pack_bf16x2(b[2] * s, b[3] * s)};
  return __builtin_bit_cast(v8bf, w);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier for LDS hand-offs: the wave's own LDS operations complete first (s_barrier alone does
// not wait for them, and a ds_write still queued when another wave passes the barrier is not yet visible
// to it); outstanding global loads, the LDS-DMA prefetches among them, are not waited for.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

enum { MODE_TILE = 0, MODE_PIECE = 1, MODE_FIXUP = 2, MODE_KSEG = 3 };

// MODE_TILE: full-K tiles 0 .. dp_tiles-1 with their epilogues; workgroup b takes tiles r * nwg + b'
// (b' its XCD-remapped id) for rounds r = 0, 1, ... while they exist, so the launch can use fewer
// workgroups than CUs and give each the same number of tiles.  MODE_PIECE: one piece of a remainder tile,
// accumulators parked in part.  MODE_FIXUP: the pieces of remainder tile dp_tiles + blockIdx.x added in
// slice order, then the epilogue.  MODE_KSEG: MODE_TILE over a segmented reduction (the grouped input
// gradient: the operand pair changes at segment boundaries).  Separate kernels, so the register allocation of
// the tile kernel is not shared with the other paths.  The split modes run T256 tiles only.
template <int EPI, int MODE, class C, int NS>
__device__ __forceinline__ void gemm_tile(const GemmArgsN<NS>& p, int64_t lid, int kbeg, int nk);

template <int EPI, int MODE, class C, int NS>
__global__ __launch_bounds__(GT, C::WPC) __attribute__((amdgpu_waves_per_eu(2 * C::WPC, 2 * C::WPC)))
void gemm_nt_kernel(GemmArgsN<NS> p) {
  const int64_t nk_full = p.kbytes / SBK;
  if constexpr (MODE == MODE_FIXUP) {
    gemm_tile<EPI, MODE, C, NS>(p, p.dp_tiles + blockIdx.x, 0, (int)nk_full);
  } else if constexpr (MODE == MODE_PIECE) {   // pieces cover whole stage pairs
    const int sl = (int)blockIdx.x / p.sk_rem;
    const int np = (int)(nk_full / 2);
    const int kbeg = 2 * (sl * np / p.sk_s);
    gemm_tile<EPI, MODE, C, NS>(p, p.dp_tiles + (int)blockIdx.x % p.sk_rem, kbeg,
                                2 * ((sl + 1) * np / p.sk_s) - kbeg);
  } else {
    const int64_t me = xcd_remap((int)blockIdx.x, p.nwg);
    for (int64_t base = 0; base + me < p.dp_tiles; base += p.nwg) {
      if (base > 0) lds_barrier();   // every wave is done with the previous tile's LDS
      gemm_tile<EPI, MODE, C, NS>(p, base + me, 0, (int)nk_full);
    }
  }
}

// One output tile (linear id lid) over reduction stages kbeg .. kbeg+nk-1, then its epilogue (MODE_TILE,
// MODE_FIXUP) or its parked accumulators (MODE_PIECE).
template <int EPI, int MODE, class C, int NS>
__device__ __forceinline__ void gemm_tile(const GemmArgsN<NS>& p0, int64_t lid, int kbeg, int nk) {
  constexpr bool BF16 = (EPI == EPI_DX || EPI == EPI_LIN || EPI == EPI_DXLIN);
  constexpr bool SCALED = (EPI == EPI_W8 || EPI == EPI_LIN);   // per-row scale / bias epilogue
  // MFMA block: 16 x 16 (v_mfma_i32_16x16x64_i8) for the int8 256 x 320 tiles, 32 x 32 (v_mfma_i32_32x32x32_i8,
  // v_mfma_f32_32x32x16_bf16) for the rest.  Register-only loops of the two int8 forms sustain 4.18 and 3.54
  // POP/s on this board (the 16 x 16 one moves fewer accumulator bytes per MAC, and the clock is set by
  // power); inside the GEMM the 16 x 16 main loop below measured faster on the 256 x 320 tiles and slower on
  // the 256 x 256 and 128 x 128 ones, and the bf16 16 x 16 form gained nothing.  Per wave the output is NA x
  // NB such blocks.
  constexpr int MB = (!BF16 && C::TB == 320) ? 16 : 32;
  constexpr int NA = C::ARW / MB, NB = C::BRW / MB, TA = C::TA, TB = C::TB;
  using Acc = std::conditional_t<MB == 32, v16i, v4i>;
  static_assert(EPI != EPI_DX || C::ARW == 128, "the rotating epilogue runs a 128-row FWHT per wave");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];  // [2][A stage | B stage], then epilogue
  // The thread index through an empty asm: values derived from it are then computed per tile, not hoisted
  // out of the tile loop of MODE_TILE (where they would stay live through the main loop and spill).
  int tid = (int)threadIdx.x;
  asm volatile("" : "+v"(tid));

  const int64_t tiles_a = (p0.rows_a + TA - 1) / TA;
  const int64_t tiles_b = (p0.rows_b + TB - 1) / TB;
  int64_t ta, tb;
  group_coords(lid, tiles_a, tiles_b, p0.gb > 0 ? p0.gb : 8, ta, tb);
  int64_t A0 = ta * TA;
  const int64_t B0 = tb * TB;
  // A grouped forward: the tile's segment supplies the operands (workgroup-uniform, scalar registers); A0
  // becomes the row within the segment.  Constant segment indices keep every field a plain argument load.
  // Grouped launches run full-K tiles only (no split pieces), so the piece and fixup kernels, at their
  // register limit, carry none of this.  Segments start on multiples of TA (the launch checks it).
  GemmBase p = p0;
  if constexpr (EPI == EPI_W8 && MODE == MODE_TILE && NS > 0) {
    if (p0.nseg > 0) {
      int s = 0;
#pragma unroll
      for (int i = 1; i < MAX_SEG; ++i) s = (i < p0.nseg && A0 >= p0.seg[i].start) ? i : s;
#pragma unroll
      for (int i = 0; i < MAX_SEG; ++i) {
        if (i != s) continue;
        const GemmSeg& g = p0.seg[i];
        p.a = g.a;
        p.sw = g.sw;
        p.bias = g.bias;
        p.lora_ra = g.lora_ra;
        p.lora_rb = g.lora_ra ? p0.lora_rb + g.rb_off : nullptr;
        p.lora_scale = g.lora_scale;
        p.out = g.out;
        p.rows_a = g.rows;
        p.ldo = g.ldo;
        A0 -= g.start;
      }
    }
  }

  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wa = wave % C::WVA, wb = wave / C::WVA;
  const int h = lane >> 5, c32 = lane & 31;   // 32 x 32 C layout: lane l owns B-row l%32, A-rows 8j+4(l/32)+i
  const int q4 = lane >> 4, c16 = lane & 15;  // 16 x 16 C layout: lane l owns B-row l%16, A-rows 4(l/16)+i

  Acc acc[NA][NB];
#pragma unroll
  for (int i = 0; i < NA; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = Acc{0};

  // Epilogue operands of this tile, fetched now so their latency hides under the main loop:
  // thread t < TB holds s_x of B-row B0+t (times 2^-7), thread t < TA s_w and bias of A-row A0+t.
  float pre_sx = 0.f, pre_sw = 0.f, pre_bi = 0.f;
  if constexpr (SCALED) {
    const int t = tid;
    const int64_t rb = B0 + t < p.rows_b ? B0 + t : p.rows_b - 1;
    const int64_t ra = A0 + t < p.rows_a ? A0 + t : p.rows_a - 1;
    if constexpr (EPI == EPI_W8) {
      if (t < TB) pre_sx = p.sx[rb] * 0.0078125f;  // 2^-7: the two unnormalised rotations
      if (t < TA) pre_sw = p.sw[ra];
    } else {
      pre_sx = 1.f;                    // fma(acc, 1, bias) = acc + bias, rounded once
      pre_sw = 1.f;
    }
    if (t < TA) pre_bi = p.bias ? p.bias[ra] : 0.f;
  }

  // DMA sources.  Instruction i of wave w fills LDS rows 8 (D w + i) + lane/8 with the logical chunks
  // (lane%8) ^ swz(row) of those rows, so its per-lane byte offset from the tile's first row is V[(D w + i) & 1]
  // + 8 i ld: one vector register per parity of 8-row group (the swizzle flips with bit 3 of the row), the
  // 8 i ld part scalar, like the stage offset.  The copies go through buffer resources over the tile's rows:
  // rows past the matrix end lie past the resource's range, read as zero and only feed outputs that are never
  // stored.
  uint32_t va[2], vb[2];
  int lda_s = 0, ldb_s = 0;
  __amdgpu_buffer_rsrc_t rsa, rsb;
  auto bind = [&](const uint8_t* a, const uint8_t* b, int64_t lda, int64_t ldb) {
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      // the 16 x 16 main loop's layout swizzles by row & 7 only (see swz16)
      const int ca = (lane & 7) ^ (lane >> 3) ^ (MB == 16 ? 0 : ((C::DA * wave + par) & 1));
      const int cb = (lane & 7) ^ (lane >> 3) ^ (MB == 16 ? 0 : ((C::DB * wave + par) & 1));
      va[par] = (uint32_t)((8 * C::DA * wave + (lane >> 3)) * lda) + 16u * (uint32_t)ca;
      vb[par] = (uint32_t)((8 * C::DB * wave + (lane >> 3)) * ldb) + 16u * (uint32_t)cb;
    }
    lda_s = __builtin_amdgcn_readfirstlane((int)lda);
    ldb_s = __builtin_amdgcn_readfirstlane((int)ldb);
    const int64_t na = p.rows_a - A0 < TA ? p.rows_a - A0 : TA;
    const int64_t nb = p.rows_b - B0 < TB ? p.rows_b - B0 : TB;
    rsa = k2q_rsrc(a + A0 * lda + (int64_t)kbeg * SBK, na * lda - (int64_t)kbeg * SBK);
    rsb = k2q_rsrc(b + B0 * ldb + (int64_t)kbeg * SBK, nb * ldb - (int64_t)kbeg * SBK);
  };
  // Segmented reduction (full-K tiles of EPI_DXLIN only): stage st of segment j reads its operands at stage
  // st - kbase; seek(st) moves to st's segment.  The stages passed to seek increase by at most one per call
  // and every segment holds at least one stage, so one step per call reaches it.
  constexpr bool KSEGS = (MODE == MODE_KSEG);
  int kseg = 0, kbase = 0, kend = 0x7fffffff;
  auto bind_seg = [&](int j) {   // j is workgroup-uniform; constant indices keep the fields argument loads
    if constexpr (NS > 0) {
      const KSeg* sp = &p0.ks[0];
#pragma unroll
      for (int i = 1; i < NS; ++i) sp = j == i ? &p0.ks[i] : sp;
      bind(sp->a, sp->b, sp->lda_b, sp->ldb_b);
      kend = sp->end;
    }
  };
  if constexpr (KSEGS && NS > 0) {
    if (p0.nks > 0) bind_seg(0);
    else bind(p.a, p.b, p.lda_b, p.ldb_b);
  } else {
    bind(p.a, p.b, p.lda_b, p.ldb_b);
  }
  auto seek = [&](int st) {
    if constexpr (KSEGS) {
      if (st >= kend) {
        kbase = kend;
        bind_seg(++kseg);
      }
    }
  };
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);   // the LDS destinations (M0) in scalar registers
  uint8_t* ldsa = smem + 1024 * C::DA * wave_s;            // this wave's DMA rows inside a stage
  uint8_t* ldsb = smem + TA * WBK + 1024 * C::DB * wave_s;

  // DMA of stage st (128 reduction bytes) into LDS slot `slot`.  Cache policy sc0 (K2Q_DMA_CPOL): nothing
  // here is re-read through this CU's L1, and the copies measured 0.3-2.3 % faster with it on every GEMM shape
  // (nt, which also stops the L2 from keeping the operand strips other tiles re-read, 8-48 % slower).
  auto issue = [&](int st, int slot) {
    const int so = (st - kbase) * WBK;
#pragma unroll
    for (int i = 0; i < C::DA; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, K2Q_LPTR(ldsa + slot * C::STAGE + 1024 * i), 16, (int)va[i & 1],
                                               so + 8 * i * lda_s, 0, K2Q_DMA_CPOL);
#pragma unroll
    for (int i = 0; i < C::DB; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsb, K2Q_LPTR(ldsb + slot * C::STAGE + 1024 * i), 16, (int)vb[i & 1],
                                               so + 8 * i * ldb_s, 0, K2Q_DMA_CPOL);
  };
  // Fragments of substep kk (32 reduction bytes) of the stage in LDS slot `slot`.
  // A lane's fragment rows are c32 plus multiples of 32, which share the chunk swizzle (swz looks at the row's
  // low four bits), so each substep's reads take one per-lane address per operand and constant offsets of
  // 32 rows (immediate ds_read offsets) instead of an address per fragment.
  const int fsw = swz(c32);
  const uint8_t* fra = smem + (C::ARW * wa + c32) * BKB;
  const uint8_t* frb = smem + TA * WBK + (C::BRW * wb + c32) * BKB;
  auto read_frags = [&](int slot, int kk, v4i (&fa)[NA], v4i (&fb)[NB]) {
    const int co = slot * C::STAGE + 16 * ((2 * kk + h) ^ fsw);
    const uint8_t* tA = fra + co;
    const uint8_t* tB = frb + co;
#pragma unroll
    for (int i = 0; i < NA; ++i) fa[i] = *reinterpret_cast<const v4i*>(tA + 32 * BKB * i);
#pragma unroll
    for (int i = 0; i < NB; ++i) fb[i] = *reinterpret_cast<const v4i*>(tB + 32 * BKB * i);
  };
  auto mfmas = [&](const v4i (&fa)[NA], const v4i (&fb)[NB]) {
#pragma unroll
    for (int ia = 0; ia < NA; ++ia)
#pragma unroll
      for (int ib = 0; ib < NB; ++ib) mma<BF16>(fa[ia], fb[ib], acc[ia][ib]);
  };

  // Software pipeline, per stage s (slot s & 1) in four substeps of 32 bytes:
  //   substeps 0-2 : read the next substep's fragments | NA NB MFMAs
  //   end of stage : wait for stage s+1's DMA and for this wave's own fragment reads, s_barrier (every
  //                  wave is done with slot s & 1), DMA stage s+2 into it
  //   substep 3    : read stage s+1 substep-0 fragments | NA NB MFMAs, the DMA instructions interleaved
  // so fragments are always in registers before their MFMAs and each stage's DMA is in flight for one
  // stage before its wait.  The body has no branches: past the last stage the DMA re-loads the last stage
  // into the freed slot (never one still in use) and the extra fragment reads are discarded, which keeps
  // the count of outstanding DMA instructions fixed at the waits.  nk counts 64-byte halves and is even
  // (every reduction length is a multiple of 128 bytes).
  constexpr int G = C::DA + C::DB;   // DMA instructions per wave per stage
  constexpr int NR = NA + NB;        // fragment reads per substep
  constexpr int NM = NA * NB;        // MFMAs per substep
  // Accumulator storage of a piece in part: 16-byte unit ((ia * NB + ib) * 4 + q) of thread t at byte
  // 8 KB * unit + 16 t, so each wave instruction moves 1 KB of consecutive bytes.  The per-unit base is
  // workgroup-uniform (scalar registers) and the thread offset a 32-bit vector register.
  constexpr int64_t PIECE_BYTES = (int64_t)TA * TB * 4;
  const uint32_t toff = 16u * tid;
  if constexpr (MODE == MODE_FIXUP) {
    for (int sl = 0; sl < p.sk_s; ++sl) {
      const uint8_t* pc = reinterpret_cast<const uint8_t*>(p.part) + ((int64_t)sl * p.sk_rem + blockIdx.x) * PIECE_BYTES;
#pragma unroll
      for (int ia = 0; ia < NA; ++ia)
#pragma unroll
        for (int ib = 0; ib < NB; ++ib) {
          if constexpr (MB == 16) {   // one 16-byte unit per block
            acc[ia][ib] += *reinterpret_cast<const v4i*>(pc + (int64_t)(ia * NB + ib) * GT * 16 + toff);
          } else {
            const uint8_t* u = pc + (int64_t)(ia * NB + ib) * 4 * GT * 16;
            const v4i q0 = *reinterpret_cast<const v4i*>(u + toff);
            const v4i q1 = *reinterpret_cast<const v4i*>(u + GT * 16 + toff);
            const v4i q2 = *reinterpret_cast<const v4i*>(u + 2 * GT * 16 + toff);
            const v4i q3 = *reinterpret_cast<const v4i*>(u + 3 * GT * 16 + toff);
            const v16i v = __builtin_shufflevector(__builtin_shufflevector(q0, q1, 0, 1, 2, 3, 4, 5, 6, 7),
                                                   __builtin_shufflevector(q2, q3, 0, 1, 2, 3, 4, 5, 6, 7), 0, 1,
                                                   2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
            if constexpr (BF16)
              acc[ia][ib] = __builtin_bit_cast(v16i, __builtin_bit_cast(v16f, acc[ia][ib]) + __builtin_bit_cast(v16f, v));
            else
              acc[ia][ib] += v;
          }
        }
    }
  } else if constexpr (MB == 16) {
    // int8 main loop on 16 x 16 blocks.  A stage is two 64-byte windows; a window is a grid of NA x NB
    // v_mfma_i32_16x16x64_i8 (a lane's fragment: 16 bytes of one row, row c16 of the block, chunk 4 w + q4 of
    // window w).  The operand with fewer blocks per wave is "held" (all NH fragments of a window in
    // registers); the other is "streamed": one fragment per micro-step, read P micro-steps ahead, and each
    // micro-step is its NH MFMAs against the held fragments.  The stage barrier sits P micro-steps before
    // the stage's end: every read of the stage's slot is issued before it (the streamed reads run P ahead)
    // and every read after it belongs to the next stage (the other slot, whose copies that barrier
    // publishes), so the MFMAs run on across the barrier.  Live fragments: the two windows' held sets for P
    // micro-steps, plus P + 1 streamed ones: (2 NH + P + 1) x 4 VGPRs (44 on the 256 x 320 tile, against 56
    // for the two substep sets of the 32 x 32 loop).
    constexpr bool STRB = NB >= NA;             // stream the B side (it has more blocks)
    constexpr int NH = STRB ? NA : NB, NSB = STRB ? NB : NA;
#ifndef K2Q_MS_P
#define K2Q_MS_P 5
#endif
    constexpr int P = K2Q_MS_P < NSB - 1 ? K2Q_MS_P : NSB - 1;
    constexpr int NU = 2 * NSB;                  // micro-steps per stage
    constexpr int RING = (NU % (P + 1) == 0) ? P + 1 : (NU % (P + 2) == 0) ? P + 2 : (NU % (P + 3) == 0) ? P + 3 : NU;
    static_assert(NSB > P && RING > P && NU % RING == 0, "micro-step pipeline");
    const int fsw16 = swz16(c16);               // the block's rows are c16 + 16 i: one swizzle per lane
    const uint8_t* fha = smem + (STRB ? (C::ARW * wa + c16) * BKB : TA * WBK + (C::BRW * wb + c16) * BKB);
    const uint8_t* fsa = smem + (STRB ? TA * WBK + (C::BRW * wb + c16) * BKB : (C::ARW * wa + c16) * BKB);
    const int cw0 = 16 * (q4 ^ fsw16), cw1 = 16 * ((4 + q4) ^ fsw16);
    v4i hf[2][NH];   // held fragments of windows 0 and 1
    v4i sf[RING];    // streamed fragments, micro-step u in sf[u % RING]
    auto rd_held = [&](int slot, int w, v4i (&f)[NH]) {
      const uint8_t* b = fha + slot * C::STAGE + (w ? cw1 : cw0);
#pragma unroll
      for (int i = 0; i < NH; ++i) f[i] = *reinterpret_cast<const v4i*>(b + 16 * BKB * i);
    };
    auto rd_str = [&](int slot, int w, int j) -> v4i {
      return *reinterpret_cast<const v4i*>(fsa + slot * C::STAGE + (w ? cw1 : cw0) + 16 * BKB * j);
    };
    auto mstep = [&](const v4i (&hv)[NH], v4i sv, auto J) {
      constexpr int j = decltype(J)::value;
#pragma unroll
      for (int i = 0; i < NH; ++i) {
        if constexpr (STRB) mma<false>(hv[i], sv, acc[i][j]);
        else mma<false>(sv, hv[i], acc[j][i]);
      }
    };
    const int ns = nk / 2;   // stages
    issue(0, 0);
    seek(ns > 1 ? 1 : 0);
    issue(ns > 1 ? 1 : 0, 1);
    wait_vmcnt<G>();           // stage 0 (stage 1 may be in flight)
    lds_barrier();
    rd_held(0, 0, hf[0]);
#pragma unroll
    for (int u = 0; u < P; ++u) sf[u] = rd_str(0, 0, u);
    // One micro-step u of stage st in LDS slot sl.
    auto mu = [&](int st, int sl, auto U) {
      constexpr int u = decltype(U)::value;
      constexpr int w = u / NSB, j = u % NSB, v = u + P;
      if constexpr (u == NU - P) {
        seek(st + 2 < ns ? st + 2 : ns - 1);
        wait_vmcnt<0>();                                      // stage st+1
        lds_barrier();                                        // every read of slot sl has landed (lgkmcnt(0))
        __builtin_amdgcn_s_setprio(2);
        issue(st + 2 < ns ? st + 2 : ns - 1, sl);
      }
      if constexpr (v < NU) sf[v % RING] = rd_str(sl, v / NSB, v % NSB);
      else sf[v % RING] = rd_str(sl ^ 1, 0, v - NU);       // the next stage's window 0
      if constexpr (u == NSB - P) rd_held(sl, 1, hf[1]);
      if constexpr (u == NU - P) rd_held(sl ^ 1, 0, hf[0]);
      mstep(hf[w], sf[u % RING], std::integral_constant<int, j>{});
      constexpr int NRD = 1 + ((u == NSB - P || u == NU - P) ? NH : 0);   // reads issued in this micro-step
      if constexpr (u >= NU - P) {   // after the barrier: the DMA instructions and reads between the MFMAs
        constexpr int GQ = (G + P - 1) / P;                   // DMA instructions per post-barrier micro-step
        constexpr int g0 = (u - (NU - P)) * GQ;
        constexpr int GN = g0 >= G ? 0 : (G - g0 < GQ ? G - g0 : GQ);
        static_for<0, NH>([&](auto I) {
          constexpr int i = decltype(I)::value;
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                     // MFMA
          constexpr int nd = (NRD * (i + 1)) / NH - (NRD * i) / NH;
          if constexpr (nd > 0) __builtin_amdgcn_sched_group_barrier(0x100, nd, 0);              // DS read
          constexpr int nv = (GN * (i + 1)) / NH - (GN * i) / NH;
          if constexpr (nv > 0) __builtin_amdgcn_sched_group_barrier(0x020, nv, 0);              // VMEM
        });
      } else {
        static_for<0, NH>([&](auto I) {
          constexpr int i = decltype(I)::value;
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                     // MFMA
          constexpr int nd = (NRD * (i + 1)) / NH - (NRD * i) / NH;
          if constexpr (nd > 0) __builtin_amdgcn_sched_group_barrier(0x100, nd, 0);              // DS read
        });
      }
    };
    // The loop is rotated: an iteration runs from one stage barrier to the next (the post-barrier micro-steps of
    // stage st, then the pre-barrier ones of stage st + 1), so its back-edge sits at the barrier's own
    // lgkmcnt(0).  Entered anywhere else, the rolled loop made the compiler wait for every fragment read in
    // flight at the back-edge (unrolled by two stages, the 256 x 320 tile spills ~100 registers).
    auto pre = [&](int st, int sl) { static_for<0, NU - P>([&](auto U) { mu(st, sl, U); }); };
    auto post = [&](int st, int sl) {
      static_for<NU - P, NU>([&](auto U) { mu(st, sl, U); });
      __builtin_amdgcn_s_setprio(0);
    };
    pre(0, 0);
    for (int st = 0; st + 1 < ns; ++st) {
      post(st, st & 1);
      pre(st + 1, (st + 1) & 1);
    }
    post(ns - 1, (ns - 1) & 1);
    wait_vmcnt<0>();   // no LDS-DMA may still be in flight when the workgroup's LDS is released
  } else {
    v4i f0a[NA], f0b[NB], f1a[NA], f1b[NB];
    const int ns = nk / 2;   // stages
    // MFMAs of one substep interleaved with the next substep's fragment reads, two reads per MFMA (with exact
    // lgkmcnt waits, reads issued early measured 0.4-1.6 % faster than one per MFMA on 8 of 9 shapes).
    auto sub = [&](const v4i (&fa)[NA], const v4i (&fb)[NB]) {
      mfmas(fa, fb);
      constexpr int H = (NR + 1) / 2;
      static_for<0, H>([&](auto I) {
        constexpr int i = decltype(I)::value;
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                            // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, (2 * i + 2 <= NR) ? 2 : 1, 0);   // DS read
      });
      if constexpr (NM > H) __builtin_amdgcn_sched_group_barrier(0x008, NM - H, 0);
    };
    issue(0, 0);
    seek(ns > 1 ? 1 : 0);
    issue(ns > 1 ? 1 : 0, 1);
    wait_vmcnt<G>();           // stage 0 (stage 1 may be in flight)
    lds_barrier();
    read_frags(0, 0, f0a, f0b);
    // Unrolled by two stages so that the LDS slot, and with it every fragment address, is a constant.
    // Wave priority (below): the builtin bounds the compiler's scheduling region, which on the bf16 256 x 320
    // tiles made it spill ~100 bytes per lane; those raise it inside the barrier's own asm statement instead
    // (no new region boundary; the drop at the end of the stage sits on the rolled loop's latch).
    constexpr bool PRIO_ASM = C::TB == 320 && (EPI == EPI_LIN || EPI == EPI_DXLIN);
    constexpr bool PRIO = !PRIO_ASM;
    auto stage = [&](int st, auto SLC) {
      const int sl = static_cast<int>(SLC);
      seek(st + 2 < ns ? st + 2 : ns - 1);   // the segment of the stage this iteration's DMA fetches
      read_frags(sl, 1, f1a, f1b);
      sub(f0a, f0b);
      read_frags(sl, 2, f0a, f0b);
      sub(f1a, f1b);
      read_frags(sl, 3, f1a, f1b);
      sub(f0a, f0b);
      wait_vmcnt<0>();                                      // stage st+1
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // this wave's reads of slot sl have landed
      if constexpr (PRIO_ASM) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier\n\ts_setprio 2" ::: "memory");
      else lds_barrier();
      // Raised wave priority from the barrier to the end of the stage: the waves past the barrier issue
      // their DMA and MFMAs ahead of waves still in the pre-barrier substeps (0.3-2.3 % faster on the 8
      // large shapes; raising it for the pre-barrier substeps instead measured 0.7-2.4 % slower).
      if constexpr (PRIO) __builtin_amdgcn_s_setprio(2);
      issue(st + 2 < ns ? st + 2 : ns - 1, sl);
      read_frags(sl ^ 1, 0, f0a, f0b);
      mfmas(f1a, f1b);
      constexpr int GI = G < NM ? G : NM;
#pragma unroll
      for (int i = 0; i < GI; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM (LDS-DMA)
      }
      if constexpr (G > GI) __builtin_amdgcn_sched_group_barrier(0x020, G - GI, 0);
#pragma unroll
      for (int i = 0; i < NR; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      if constexpr (NM > GI) __builtin_amdgcn_sched_group_barrier(0x008, NM - GI, 0);
      if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
      if constexpr (PRIO_ASM) asm volatile("s_setprio 0");
    };
    if constexpr (C::TB == 320) {   // the 256 x 320 tile keeps the rolled loop (unrolled, it spills registers)
      for (int st = 0; st < ns; ++st) stage(st, st & 1);
    } else {
      int st = 0;
      for (; st + 1 < ns; st += 2) {
        stage(st, std::integral_constant<int, 0>{});
        stage(st + 1, std::integral_constant<int, 1>{});
      }
      if (st < ns) stage(st, std::integral_constant<int, 0>{});
    }
    wait_vmcnt<0>();   // no LDS-DMA may still be in flight when the workgroup's LDS is released
  }
  if constexpr (MODE == MODE_PIECE) {   // park the accumulators for the fixup launch
    uint8_t* dst = reinterpret_cast<uint8_t*>(p.part) + (int64_t)blockIdx.x * PIECE_BYTES;
#pragma unroll
    for (int ia = 0; ia < NA; ++ia)
#pragma unroll
      for (int ib = 0; ib < NB; ++ib) {
        if constexpr (MB == 16) {
          *reinterpret_cast<v4i*>(dst + (int64_t)(ia * NB + ib) * GT * 16 + toff) = acc[ia][ib];
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<v4i*>(dst + (int64_t)((ia * NB + ib) * 4 + q) * GT * 16 + toff) =
                v4i{acc[ia][ib][4 * q], acc[ia][ib][4 * q + 1], acc[ia][ib][4 * q + 2], acc[ia][ib][4 * q + 3]};
        }
      }
    return;
  }

  const int64_t a0 = A0 + C::ARW * wa;   // first A-row of this wave
  const int64_t b0 = B0 + C::BRW * wb;   // first B-row of this wave

  if constexpr (EPI == EPI_ACC) {
    int32_t* out = static_cast<int32_t*>(p.out);
#pragma unroll
    for (int ia = 0; ia < NA; ++ia)
#pragma unroll
      for (int ib = 0; ib < NB; ++ib) {
        if constexpr (MB == 16) {
          const int64_t m = b0 + 16 * ib + c16, n = a0 + 16 * ia + 4 * q4;
          if (m < p.rows_b && n < p.rows_a) *reinterpret_cast<v4i*>(out + m * p.ldo + n) = acc[ia][ib];
        } else {
          const int64_t m = b0 + 32 * ib + c32;
          if (m >= p.rows_b) continue;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int64_t n = a0 + 32 * ia + 8 * j + 4 * h;
            if (n >= p.rows_a) continue;
            int4 v = make_int4(acc[ia][ib][4 * j], acc[ia][ib][4 * j + 1], acc[ia][ib][4 * j + 2],
                               acc[ia][ib][4 * j + 3]);
            *reinterpret_cast<int4*>(out + m * p.ldo + n) = v;
          }
        }
      }
    return;
  } else {
    // Epilogue:
    //   A  dequantize in registers, in place of the accumulators (W8/LIN: f32 = s acc + bias; DX: inverse
    //      FWHT, 2^-7)
    //   B  LoRA: bf16 MFMAs accumulate the adapter term straight onto those f32 values (the factor rows
    //      staged in LDS per 16-rank chunk); base + adapter is rounded to bf16 once
    //   C  the bf16 tile goes to LDS (CROWS rows of CROW bytes at a time), then out with coalesced 16-byte
    //      stores, 2 TA contiguous bytes per output row segment.
    // This thread's share of the LoRA factor rows for the staging below (A-side row A0 + t/2 for t/2 < TA,
    // B-side rows B0 + t/2 + 256 i, ranks 8 (t&1) .. +8 of each 16-rank chunk): the first chunk is fetched
    // now, so its latency hides under pass A, and each later chunk while the previous one is multiplied.  The
    // input-gradient epilogues read their A-side factors straight from LoRA A (r x rows_a): 8 loads of 4
    // bytes, rank by rank, consecutive threads on consecutive columns.
    constexpr bool RA_T = (EPI == EPI_DX || EPI == EPI_DXLIN);
    constexpr int NBR = C::NBR;
    const bool lora = p.lora_rb != nullptr && p.r > 0;
    const int srow = tid >> 1, shalf = tid & 1;
    const bool a_side = srow < TA;
    const float* pra = nullptr;
    const float* prb[NBR];
    v4f lfa[2], lfb[NBR][2];
    auto load_ra = [&](int c0) {
      if constexpr (RA_T) {
        const float* q = pra + (int64_t)c0 * p.rows_a;
#pragma unroll
        for (int j = 0; j < 8; ++j) lfa[j >> 2][j & 3] = q[(int64_t)j * p.rows_a];
      } else {
        lfa[0] = *reinterpret_cast<const v4f*>(pra + c0);
        lfa[1] = *reinterpret_cast<const v4f*>(pra + c0 + 4);
      }
    };
    auto load_rb = [&](int c0) {
#pragma unroll
      for (int i = 0; i < NBR; ++i) {
        lfb[i][0] = *reinterpret_cast<const v4f*>(prb[i] + c0);
        lfb[i][1] = *reinterpret_cast<const v4f*>(prb[i] + c0 + 4);
      }
      if constexpr (EPI == EPI_W8) {
        for (int q = 1; q < p.rb_parts; ++q) {   // ((part 0 + part 1) + part 2) ..., as lora_reduce_kernel adds
#pragma unroll
          for (int i = 0; i < NBR; ++i) {
            lfb[i][0] += *reinterpret_cast<const v4f*>(prb[i] + q * p.rb_pstride + c0);
            lfb[i][1] += *reinterpret_cast<const v4f*>(prb[i] + q * p.rb_pstride + c0 + 4);
          }
        }
      }
    };
    if (lora) {
      int64_t ra = A0 + (a_side ? srow : 0);
      ra = ra < p.rows_a ? ra : p.rows_a - 1;
      pra = RA_T ? p.lora_ra + (int64_t)(8 * shalf) * p.rows_a + ra : p.lora_ra + ra * p.r + 8 * shalf;
#pragma unroll
      for (int i = 0; i < NBR; ++i) {
        int64_t rb = B0 + srow + (GT / 2) * i;
        rb = rb < p.rows_b ? rb : p.rows_b - 1;
        prb[i] = p.lora_rb + rb * p.ldr + 8 * shalf;
      }
      load_ra(0);
      load_rb(0);
    }
    lds_barrier();   // every wave is done with the LDS ring
    float* s_sx = reinterpret_cast<float*>(smem + C::SCALE_OFF);
    float* s_sw = s_sx + TB;
    float* s_bi = s_sw + TA;
    if constexpr (SCALED) {
      if (tid < TB) s_sx[tid] = pre_sx;
      if (tid < TA) {
        s_sw[tid] = pre_sw;
        s_bi[tid] = pre_bi;
      }
    }
    lds_barrier();
    uint8_t* ctile = smem;
    if constexpr (SCALED && MB == 16) {   // a lane's 4 values: A-rows 4 q4 .. +3 of one B-row
#pragma unroll
      for (int ia = 0; ia < NA; ++ia) {
        const int nl = C::ARW * wa + 16 * ia + 4 * q4;
        const v4f sw = *reinterpret_cast<const v4f*>(s_sw + nl);
        const v4f bi = *reinterpret_cast<const v4f*>(s_bi + nl);
#pragma unroll
        for (int ib = 0; ib < NB; ++ib) {
          const float sxm = s_sx[C::BRW * wb + 16 * ib + c16];
          const v4f a = __builtin_convertvector(acc[ia][ib], v4f);
          v4f f;
#pragma unroll
          for (int i = 0; i < 4; ++i) f[i] = __builtin_fmaf(a[i], sxm * sw[i], bi[i]);
          acc[ia][ib] = __builtin_bit_cast(v4i, f);
        }
      }
    } else if constexpr (SCALED) {
#pragma unroll
      for (int ia = 0; ia < NA; ++ia) {
        v4f sw[4], bi[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int nl = C::ARW * wa + 32 * ia + 8 * j + 4 * h;
          sw[j] = *reinterpret_cast<const v4f*>(s_sw + nl);
          bi[j] = *reinterpret_cast<const v4f*>(s_bi + nl);
        }
#pragma unroll
        for (int ib = 0; ib < NB; ++ib) {
          const float sxm = s_sx[C::BRW * wb + 32 * ib + c32];
          v16f a;   // whole-vector conversions (element-wise bit casts of vector lanes have miscompiled here)
          if constexpr (BF16)
            a = __builtin_bit_cast(v16f, acc[ia][ib]);
          else
            a = __builtin_convertvector(acc[ia][ib], v16f);
          v16f f;
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) f[4 * j + i] = __builtin_fmaf(a[4 * j + i], sxm * sw[j][i], bi[j][i]);
          acc[ia][ib] = __builtin_bit_cast(v16i, f);   // in place: the f32 tile reuses the accumulators
        }
      }
    } else if constexpr (EPI == EPI_DX) {  // one 32-column slice (ib) at a time; the FWHT needs all 4 row slices
#pragma unroll
      for (int ib = 0; ib < NB; ++ib) {
        v16f f[4];
#pragma unroll
        for (int ia = 0; ia < 4; ++ia) f[ia] = __builtin_bit_cast(v16f, acc[ia][ib]);
        fwht128_rows(f, h);
#pragma unroll
        for (int ia = 0; ia < 4; ++ia) acc[ia][ib] = __builtin_bit_cast(v16i, f[ia]);
      }
    }   // EPI_DXLIN: the accumulators are the f32 values already
    // Pin the dequantized tile in registers here: otherwise the compiler sinks pass A's arithmetic past the
    // LoRA branch (to the stores) and keeps its scale operands live across it, which spills.
#pragma unroll
    for (int ia = 0; ia < NA; ++ia)
#pragma unroll
      for (int ib = 0; ib < NB; ++ib) asm volatile("" : "+v"(acc[ia][ib]));
    if (lora) {
      // Per 16-rank chunk the workgroup stages the tile's TA A-side and TB B-side factor rows in LDS as
      // bf16 (B side times lora_scale), each f32 read once: thread t converts 8 ranks of its rows.
      uint8_t* sla = smem + C::LORA_OFF;
      uint8_t* slb = sla + TA * LROW;
      for (int c0 = 0; c0 < p.r; c0 += 16) {
        if (a_side) *reinterpret_cast<v8bf*>(sla + srow * LROW + 16 * shalf) = f32x8_to_bf16v(lfa[0], lfa[1], 1.f);
#pragma unroll
        for (int i = 0; i < NBR; ++i) {
          const int row = srow + (GT / 2) * i;
          if (row < TB)
            *reinterpret_cast<v8bf*>(slb + row * LROW + 16 * shalf) = f32x8_to_bf16v(lfb[i][0], lfb[i][1], p.lora_scale);
        }
        const int cn = c0 + 16 < p.r ? c0 + 16 : c0;   // next chunk (the last re-reads its own)
        load_ra(cn);
        load_rb(cn);
        lds_barrier();
        if constexpr (MB == 16) {   // v_mfma_f32_16x16x16_bf16: a lane's fragment is ranks 4 q4 .. +3 of row c16
          // (the 16x16x32 form over the chunk's 16 ranks and 16 zero ranks measured slower: twice the fragment
          // registers, and the 256 x 320 tile then spills)
          k2q_v4s fa[NA], fb[NB];
#pragma unroll
          for (int i = 0; i < NA; ++i)
            fa[i] = *reinterpret_cast<const k2q_v4s*>(sla + (C::ARW * wa + 16 * i + c16) * LROW + 8 * q4);
#pragma unroll
          for (int i = 0; i < NB; ++i)
            fb[i] = *reinterpret_cast<const k2q_v4s*>(slb + (C::BRW * wb + 16 * i + c16) * LROW + 8 * q4);
#pragma unroll
          for (int ia = 0; ia < NA; ++ia)
#pragma unroll
            for (int ib = 0; ib < NB; ++ib)
              acc[ia][ib] = __builtin_bit_cast(
                  v4i, __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(fa[ia], fb[ib], __builtin_bit_cast(v4f, acc[ia][ib]), 0, 0, 0));
        } else {
          v8bf fa[NA], fb[NB];
#pragma unroll
          for (int i = 0; i < NA; ++i)
            fa[i] = *reinterpret_cast<const v8bf*>(sla + (C::ARW * wa + 32 * i + c32) * LROW + 16 * h);
#pragma unroll
          for (int i = 0; i < NB; ++i)
            fb[i] = *reinterpret_cast<const v8bf*>(slb + (C::BRW * wb + 32 * i + c32) * LROW + 16 * h);
#pragma unroll
          for (int ia = 0; ia < NA; ++ia)
#pragma unroll
            for (int ib = 0; ib < NB; ++ib)
              acc[ia][ib] = __builtin_bit_cast(
                  v16i, __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[ia], fb[ib], __builtin_bit_cast(v16f, acc[ia][ib]), 0, 0, 0));
        }
        lds_barrier();   // every wave has its fragments before the next chunk overwrites them
      }
    }
    // Pass C, CROWS B-rows at a time: the waves owning those rows put their blocks into the LDS tile, then
    // wave w stores tile rows RPW w .. RPW w + RPW - 1, two rows (2 x 2 TA bytes) per instruction.
    // Non-temporal: the output is not read again by this launch, and streaming it keeps the operand strips
    // in L2.
    uint16_t* out = static_cast<uint16_t*>(p.out);
    constexpr int RPW = C::CROWS / GW;   // rows per wave per pass
    constexpr int CPR = TA / 8;          // 16-byte chunks per row
    const int chunk = lane & 31;
    const int64_t col = A0 + 8 * chunk;
#pragma unroll
    for (int pass = 0; pass < TB / C::CROWS; ++pass) {
      if (pass > 0) lds_barrier();       // the previous pass's rows have left the tile
      const int rbeg = pass * C::CROWS;
      if (C::BRW * wb >= rbeg && C::BRW * wb < rbeg + C::CROWS) {
#pragma unroll
        for (int ia = 0; ia < NA; ++ia)
#pragma unroll
          for (int ib = 0; ib < NB; ++ib) {
            if constexpr (MB == 16)
              ctile_put16<C::CROW>(ctile, C::BRW * wb - rbeg + 16 * ib, C::ARW * wa + 16 * ia, lane,
                                   __builtin_bit_cast(v4f, acc[ia][ib]));
            else
              ctile_put<C::CROW>(ctile, C::BRW * wb - rbeg + 32 * ib, C::ARW * wa + 32 * ia, lane,
                                 __builtin_bit_cast(v16f, acc[ia][ib]));
          }
      }
      lds_barrier();
      const int64_t R0 = B0 + rbeg;
      if ((p.ldo & 7) == 0) {        // rows are 16-byte aligned: one 16-byte store per lane
        const bool col_ok = chunk < CPR && col < p.rows_a;
#pragma unroll 4
        for (int i = 0; i < RPW / 2; ++i) {
          const int row = RPW * wave + 2 * i + (lane >> 5);
          const v4u v = *reinterpret_cast<const v4u*>(ctile + row * C::CROW + 16 * (chunk < CPR ? chunk : 0));
          if (col_ok && R0 + row < p.rows_b) __builtin_nontemporal_store(v, reinterpret_cast<v4u*>(out + (R0 + row) * p.ldo + col));
        }
      } else {                       // ragged widths: element stores
        for (int i = 0; i < RPW / 2; ++i) {
          const int row = RPW * wave + 2 * i + (lane >> 5);
          if (R0 + row >= p.rows_b || chunk >= CPR) continue;
          const uint16_t* src = reinterpret_cast<const uint16_t*>(ctile + row * C::CROW + 16 * chunk);
          for (int e = 0; e < 8 && col + e < p.rows_a; ++e) out[(R0 + row) * p.ldo + col + e] = src[e];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------
// W4A8: A operand = packed int4 weights (rows n, K/2 bytes per row), bf16 group scales sw4[g][n].
// Tile 128 (n) x 128 (m) per 256-thread workgroup, three workgroups per CU (166 VGPRs) so that one wave's
// per-group scaling runs while another's MFMAs do (wave priority follows the work left, see step()).
// Wave w owns the 32 n-rows 32w..32w+31 and all 128 m, so every
// packed weight byte is unpacked by exactly one wave.  The MFMA takes the x codes as its first operand, so
// a lane's 16 results share one n (the lane's column) and need one group scale.  A stage is 128 of K,
// double-buffered in LDS and filled by LDS-DMA from buffer resources (per-lane offsets fixed, the stage
// offset scalar): the packed A rows (64 B each, 16-byte chunk c of row r at c ^ ((r >> 2) & 3)), the int8
// B rows (the frag()/swz() layout) and the stage's two groups of 128 scales.  A lane's 8 packed bytes
// hold the 16 codes of one 16-wide K chunk; `w << 4 & 0xF0F0F0F0` and `w & 0xF0F0F0F0` give them as int8
// values 16*q in K order, so one v_mfma_i32_32x32x32_i8 per 32 of K sees 16x the true products (exact,
// |16 acc_g| <= 16*64*127*8 < 2^20).  Each 64-wide group is accumulated in int32, converted once and
// scaled: accf += float(acc_g) * s[g][n]; the 1/16 is folded into the final scale.  The per-group
// convert + FMA (2 VALU ops per output per group) bounds this kernel, not the MFMAs.
constexpr int W4_BA = 128;                // n rows per tile
constexpr int W4_BB = 128;                // m rows per tile
constexpr int W4_IB = 4;                  // 32-row m blocks per wave (one 32-row n block)
constexpr int W4_SA = W4_BA * 64;         // packed A bytes per stage (128 K codes per row)
constexpr int W4_SB = W4_BB * WBK;        // B bytes per stage
constexpr int W4_SS = 2 * W4_BA * 2;      // 2 groups x 128 n x bf16
constexpr int W4_STAGE = W4_SA + W4_SB + W4_SS;
constexpr int W4_G = 7;                   // DMA instructions per wave and stage: 2 A, 4 B, 1 scales
constexpr int W4_CROW = 2 * W4_BA + 16;   // epilogue bf16 tile row (padded: rows m and m + 4 on other banks)
static_assert(W4_BB * W4_CROW + 4 * W4_BB <= 2 * W4_STAGE, "epilogue tile and s_x fit the stage buffers");

struct W4Args {
  const uint8_t* a;      // N x K/2 packed
  const uint16_t* s4;    // K/64 x N bf16
  const int8_t* b;       // M x K int8
  int64_t N, M, K;
  void* out;             // bf16 y (EPI_W8) or f32 (EPI_ACC: sum_g s acc_g)
  const float* sx;
  const float* bias;
  const float* lora_rb;
  const float* lora_ra;
  int r;
  float lora_scale;
};

__device__ __forceinline__ int swz4(int row) { return (row >> 2) & 3; }

template <int EPI>
__global__ __launch_bounds__(256, 3) __attribute__((amdgpu_waves_per_eu(3, 3))) void gemm_w4_kernel(W4Args p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];   // [2][A | B | scales]

  const uint32_t tiles_a = (uint32_t)((p.N + W4_BA - 1) / W4_BA);
  const uint32_t tiles_b = (uint32_t)((p.M + W4_BB - 1) / W4_BB);
  uint32_t ta, tb;
  tile_coords(tiles_a, tiles_b, ta, tb);
  const int64_t A0 = (int64_t)ta * W4_BA, B0 = (int64_t)tb * W4_BB;

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int h = lane >> 5, c32 = lane & 31;
  const int64_t kb = p.K / 2;   // packed bytes per A row
  const int64_t na = (p.N - A0) < W4_BA ? (p.N - A0) : W4_BA;
  const int64_t nb = (p.M - B0) < W4_BB ? (p.M - B0) : W4_BB;

  v16f accf[W4_IB];
#pragma unroll
  for (int j = 0; j < W4_IB; ++j) accf[j] = v16f{0.f};

  // DMA sources, as offsets into buffer resources that start at the tile's first row (rows past the
  // matrix end clamped onto its last row; never stored).  A: wave w fills rows 32w + 16i + l/4, physical
  // chunk l%4; B: rows 32w + 8i + l/8, physical chunk l%8; scales: wave w copies group w/2, columns
  // 64 (w&1) + 2l, 2l+1 with lanes 0-31.
  const __amdgpu_buffer_rsrc_t ra = k2q_rsrc(p.a + A0 * kb, na * kb);
  const __amdgpu_buffer_rsrc_t rb = k2q_rsrc(reinterpret_cast<const uint8_t*>(p.b) + B0 * p.K, nb * p.K);
  const __amdgpu_buffer_rsrc_t rs = k2q_rsrc(p.s4, (p.K / 64) * p.N * 2);
  int offa[2], offb[4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int lrow = 32 * wave + 16 * i + (lane >> 2);
    const int rr = lrow < na ? lrow : (int)na - 1;
    offa[i] = (int)(rr * kb) + 16 * ((lane & 3) ^ swz4(lrow));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int lrow = 32 * wave + 8 * i + (lane >> 3);
    const int rr = lrow < nb ? lrow : (int)nb - 1;
    offb[i] = (int)(rr * p.K) + 16 * ((lane & 7) ^ swz(lrow));
  }
  int64_t ncol = A0 + 64 * (wave & 1) + 2 * (lane & 31);
  ncol = ncol < p.N ? ncol : p.N - 2;
  const int offs = (int)(((int64_t)(wave >> 1) * p.N + ncol) * 2);
  auto issue = [&](int st, int slot) {
    uint8_t* base = smem + slot * W4_STAGE;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, K2Q_LPTR(base + 1024 * (2 * wave + i)), 16, offa[i], st * 64, 0,
                                               0);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, K2Q_LPTR(base + W4_SA + 1024 * (4 * wave + i)), 16, offb[i],
                                               st * WBK, 0, 0);
    if (lane < 32)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, K2Q_LPTR(base + W4_SA + W4_SB + 256 * (wave >> 1) + 128 * (wave & 1)), 4, offs,
          (int)(st * 4 * p.N), 0, 0);
  };

  auto compute = [&](int slot) {
    const uint8_t* tA = smem + slot * W4_STAGE;
    const uint8_t* tB = tA + W4_SA;
    const uint16_t* tS = reinterpret_cast<const uint16_t*>(tB + W4_SB);
    const int arow = 32 * wave + c32;
#pragma unroll
    for (int grp = 0; grp < 2; ++grp) {
      v16i acc[W4_IB];
#pragma unroll
      for (int j = 0; j < W4_IB; ++j) acc[j] = v16i{0};
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        const int kk = 2 * grp + k2;
        const v2u w = *reinterpret_cast<const v2u*>(tA + arow * 64 + 16 * (kk ^ swz4(arow)) + 8 * h);
        const v4i fa = v4i{(int)((w[0] << 4) & 0xF0F0F0F0u), (int)((w[1] << 4) & 0xF0F0F0F0u),
                           (int)(w[0] & 0xF0F0F0F0u), (int)(w[1] & 0xF0F0F0F0u)};
        v4i fb[W4_IB];
#pragma unroll
        for (int i = 0; i < W4_IB; ++i) fb[i] = frag(tB, 32 * i + c32, 2 * kk + h);
#pragma unroll
        for (int ib = 0; ib < W4_IB; ++ib)   // rows m (x codes), columns n (weights): lane c32 is one n
          acc[ib] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fb[ib], fa, acc[ib], 0, 0, 0);
      }
      const float sv = bf16_bits_to_f32(tS[grp * W4_BA + arow]);
#pragma unroll
      for (int ib = 0; ib < W4_IB; ++ib)
#pragma unroll
        for (int e = 0; e < 16; ++e) accf[ib][e] = __builtin_fmaf((float)acc[ib][e], sv, accf[ib][e]);
      // One group's int32 accumulators live at a time: the scaled sums pass through here before the next
      // group's fragment reads (the memory clobber keeps those below), so its MFMAs cannot be hoisted
      // above this group's conversion.
      asm volatile("" : "+v"(accf[0]), "+v"(accf[1]), "+v"(accf[2]), "+v"(accf[3])::"memory");
    }
  };

  // Double-buffered: stage s+2 is fetched into stage s's slot once every wave is done with it.  Unrolled
  // by two so that the slot, and with it every LDS address, is a compile-time offset.
  const int ns = (int)(p.K / 128);
  auto step = [&](int st, int slot) {
    // Priority by work left (3 in the first quarter of the stages .. 0 in the last): under oldest-first
    // issue the three workgroups sharing a CU otherwise drift apart, and the last one finishes alone with
    // no other wave to fill its MFMA/VALU gaps.
    const int lvl = (4 * (ns - st) - 1) / ns;   // 3 .. 0
    if (lvl == 3) __builtin_amdgcn_s_setprio(3);
    else if (lvl == 2) __builtin_amdgcn_s_setprio(2);
    else if (lvl == 1) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
    compute(slot);
    wait_vmcnt<0>();                                       // stage st+1
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // this wave's reads of the slot have landed
    lds_barrier();
    if (st + 2 < ns) issue(st + 2, slot);
  };
  issue(0, 0);
  issue(ns > 1 ? 1 : 0, 1);
  wait_vmcnt<W4_G>();
  lds_barrier();
  for (int st = 0; st < ns; st += 2) {
    step(st, 0);
    if (st + 1 < ns) step(st + 1, 1);
  }
  wait_vmcnt<0>();   // no LDS-DMA may still be in flight when the workgroup's LDS is released

  // accf[ib][e]: n = a0 + c32, m = B0 + 32 ib + 8 (e / 4) + 4 h + e % 4.
  const int64_t a0 = A0 + 32 * wave;
  if constexpr (EPI == EPI_ACC) {
    float* out = static_cast<float*>(p.out);
    const int64_t n = a0 + c32;
    if (n < p.N) {
#pragma unroll
      for (int ib = 0; ib < W4_IB; ++ib)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int64_t m = B0 + 32 * ib + 8 * (e >> 2) + 4 * h + (e & 3);
          if (m < p.M) out[m * p.N + n] = accf[ib][e] * 0.0625f;
        }
    }
  } else {
    // s_x (times 2^-7 for the rotations and 1/16 for the nibble placement) staged in LDS for the tile's
    // 128 rows; scales, bias and LoRA applied in registers; then the bf16 tile goes through LDS (row m:
    // 128 n, W4_CROW bytes) for row-contiguous stores.
    uint16_t* ctile = reinterpret_cast<uint16_t*>(smem);
    float* sxs = reinterpret_cast<float*>(smem + W4_BB * W4_CROW);
    lds_barrier();   // every wave is past its last fragment read
    if (t < W4_BB) sxs[t] = p.sx[B0 + t < p.M ? B0 + t : p.M - 1] * (0.0078125f * 0.0625f);
    lds_barrier();
    const int64_t n = a0 + c32 < p.N ? a0 + c32 : p.N - 1;
    const float bi = p.bias ? p.bias[n] : 0.f;
#pragma unroll
    for (int ib = 0; ib < W4_IB; ++ib) {
      v16f f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const v4f sc = *reinterpret_cast<const v4f*>(sxs + 32 * ib + 8 * j + 4 * h);
#pragma unroll
        for (int i = 0; i < 4; ++i) f[4 * j + i] = __builtin_fmaf(accf[ib][4 * j + i], sc[i], bi);
      }
      if (p.lora_rb && p.r > 0)   // f[m][n] += u[m, :] . (scale lora_b[n, :])
        f = lora_block(p.lora_rb, p.lora_ra, p.r, p.lora_scale, p.M, p.N, B0 + 32 * ib, a0, lane, f);
      const int col = 32 * wave + c32;
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        const uint32_t v = pack_bf16x2(f[e], f[e + 1]);
        const int row = 32 * ib + 8 * (e >> 2) + 4 * h + (e & 3);
        ctile[(row * W4_CROW) / 2 + col] = (uint16_t)(v & 0xffffu);
        ctile[((row + 1) * W4_CROW) / 2 + col] = (uint16_t)(v >> 16);
      }
    }
    lds_barrier();
    const int cq = t & 31;                   // 4 n per thread, 8 rows per pass
    const int64_t n4 = A0 + 4 * cq;
    const int rows = (int)nb;
    if (n4 < p.N) {
      uint16_t* o = static_cast<uint16_t*>(p.out) + (B0 + (t >> 5)) * p.N + n4;
      const uint8_t* c = reinterpret_cast<const uint8_t*>(ctile) + (t >> 5) * W4_CROW + 8 * cq;
#pragma unroll 4
      for (int row = t >> 5; row < rows; row += 8) {
        __builtin_nontemporal_store(*reinterpret_cast<const v2u*>(c), reinterpret_cast<v2u*>(o));   // as in pass C
        o += 8 * p.N;
        c += 8 * W4_CROW;
      }
    }
  }
}

template <int EPI>
int launch_w4(const W4Args& p, hipStream_t st) {
  constexpr int lds = 2 * W4_STAGE;
  // Buffer-resource extents are 32-bit: a tile's rows of either operand and the whole scale array.
  if (p.K * W4_BB >= (int64_t(1) << 31) || (p.K / 64) * p.N * 2 >= (int64_t(1) << 31)) return K2Q_EUNSUPPORTED;
  static std::atomic<uint64_t> lds_set{0};
  if (k2q_lds_limit_once(gemm_w4_kernel<EPI>, lds, lds_set)) return K2Q_ELAUNCH;
  const int64_t tiles = ((p.N + W4_BA - 1) / W4_BA) * ((p.M + W4_BB - 1) / W4_BB);
  if (tiles > 0x7fffffff) return K2Q_EUNSUPPORTED;
  hipLaunchKernelGGL(gemm_w4_kernel<EPI>, dim3((unsigned)tiles), dim3(256), lds, st, p);
  return k2q_launch_status();
}

// Split plan for the tiles of the last, partly filled round of T256 tiles, in units of one reduction stage of
// one tile (measured on MI355X): a full-K tile costs nk + 8 (epilogue); cutting the rem remainder tiles into s
// pieces (one round of pieces when rem * s <= CUs) costs nk / s per piece plus ~12 (ramp and piece store),
// and the fixup launch ~20 + 3 per piece read back.  The s with the lowest cost is taken if it saves at least
// 10 %.
struct SplitPlan {
  int64_t dp_tiles;
  int rem, s;
  double cost;   // stage units of a T256 tile
};

SplitPlan split_plan(int64_t tiles, int nk, int cus) {
  SplitPlan q{tiles, 0, 1, 0.0};
  const int64_t full = tiles / cus, rem = tiles - full * cus;
  const double tile = nk + 8.0;
  q.cost = (double)((tiles + cus - 1) / cus) * tile;
  if (rem == 0) return q;
  double best = 0.9 * q.cost;
  for (int s = 2; s <= 8 && rem * s <= cus && nk / s >= 8; ++s) {
    const double t = (double)full * tile + (double)nk / s + 12.0 + 20.0 + 3.0 * s;
    if (t < best) {
      best = t;
      q.s = s;
    }
  }
  if (q.s > 1) {
    q.dp_tiles = full * cus;
    q.rem = (int)rem;
    q.cost = best;
  }
  return q;
}

// Split plan for a launch of 128 x 128 tiles (two workgroups per CU) that fits one round of workgroup slots:
// every tile cut along K into s pieces (whole stage pairs), then one fixup launch, when that is estimated at
// least 5 % faster.  Estimates in microseconds, fitted to MI355X timings of 11 launch shapes (M 256-2048,
// N 1024-6144, K 3072-16384; split or not, the plan's pick is within 6 % of the fastest measured): a full-K tile
// 0.62 per 128-byte stage + 6; s pieces 0.62 per stage of the longest piece, x 1.25 once pieces outnumber the
// CUs, + 10 + 0.035 per piece (piece stores and the fixup).  Long reductions over few tiles gain most: M = 1024,
// N = 3072, K = 12288 (cfg4's text-stream down projection) 70.5 -> 62.8 us with s = 2.
SplitPlan split_plan128(int64_t tiles, int nk, int cus) {
  SplitPlan q{tiles, 0, 1, 0.0};
  const int64_t slots = 2 * (int64_t)cus;
  if (tiles > slots) return q;
  const int np = nk / 2;   // 128-byte stages
  auto stages_us = [&](int stages, int64_t wgs) { return 0.62 * stages * (wgs > cus ? 1.25 : 1.0); };
  q.cost = stages_us(np, tiles) + 6.0;
  double best = 0.95 * q.cost;
  for (int s = 2; s <= 8 && tiles * s <= slots && np / s >= 4; ++s) {
    const double t = stages_us((np + s - 1) / s, tiles * s) + 10.0 + 0.035 * (double)(tiles * s);
    if (t < best) {
      best = t;
      q.s = s;
    }
  }
  if (q.s > 1) {
    q.dp_tiles = 0;
    q.rem = (int)tiles;
    q.cost = best;
  }
  return q;
}

// Tile shape of a launch: the one with the lowest estimated time, in units of one reduction stage of a T256 tile.
// A round of `active` tiles over `slots` = CUs x workgroups-per-CU costs nk x c x (0.7 + 0.3 active / slots) +
// epilogue: a partly filled round runs its stages faster (less HBM and L2 contention).  Per-stage costs relative
// to T256, fitted to the MI355X timings of 17 launch shapes (M 1024..16896, N 1536..16384, K 3072..16384; the
// fitted model picks the fastest measured shape on each): T320 1.25, T192 0.80, T128 0.60 with two workgroups
// sharing a CU and 0.30 with a CU to itself; epilogues 8 (T256, T320), 7 (T192), 4 (T128).  T256 may instead cut
// its last round's tiles along K (split_plan), and a launch of T128 tiles its one round (split_plan128).  The
// rotating input-gradient epilogue runs 128 A-rows per wave (T256 only); grouped launches need segments on tile
// boundaries (TA = 256 or 128).
struct TileChoice {
  int tile;
  SplitPlan split;   // T256 and T128
};

template <class C>
double tile_cost(int64_t rows_a, int64_t rows_b, int nk, int cus, double stage_cost, double alone_cost, double epi) {
  const int64_t tiles = ((rows_a + C::TA - 1) / C::TA) * ((rows_b + C::TB - 1) / C::TB);
  const int64_t slots = (int64_t)cus * C::WPC;
  const int64_t full = tiles / slots, rem = tiles - full * slots;
  auto round = [&](int64_t active) {
    const double c = (C::WPC > 1 && active <= cus) ? alone_cost : stage_cost;
    return nk * c * (0.7 + 0.3 * (double)active / (double)slots) + epi;
  };
  return (double)full * round(slots) + (rem ? round(rem) : 0.0);
}

// allowed: bit t set = tile shape t may be chosen; can_split: T256 may cut its last round along K.
TileChoice choose_tile(int epi, int64_t rows_a, int64_t rows_b, int64_t kbytes, unsigned allowed, bool can_split,
                       int forced, int cus) {
  const int nk = (int)(kbytes / SBK);
  const int64_t tiles256 = ((rows_a + 255) / 256) * ((rows_b + 255) / 256);
  TileChoice c{TILE_256, can_split ? split_plan(tiles256, nk, cus) : SplitPlan{tiles256, 0, 1, 0.0}};
  const int64_t tiles128 = ((rows_a + 127) / 128) * ((rows_b + 127) / 128);
  if (forced >= 0) {
    c.tile = forced;
    if (forced != TILE_256) c.split = SplitPlan{0, 0, 1, 0.0};
    if (forced == TILE_128 && can_split) c.split = split_plan128(tiles128, nk, cus);
    return c;
  }
  if (epi == EPI_DX) return c;
  double best = c.split.s > 1 ? c.split.cost : tile_cost<T256>(rows_a, rows_b, nk, cus, 1.0, 1.0, 8.0);
  const double t320 = allowed >> TILE_320 & 1 ? tile_cost<T320>(rows_a, rows_b, nk, cus, 1.25, 1.25, 8.0) : 1e300;
  const double t192 = allowed >> TILE_192 & 1 ? tile_cost<T192>(rows_a, rows_b, nk, cus, 0.80, 0.80, 7.0) : 1e300;
  const double t128 = allowed >> TILE_128 & 1 ? tile_cost<T128>(rows_a, rows_b, nk, cus, 0.60, 0.30, 4.0) : 1e300;
  if (t320 < best) { best = t320; c.tile = TILE_320; }
  if (t192 < best) { best = t192; c.tile = TILE_192; }
  if (t128 < best) { best = t128; c.tile = TILE_128; }
  if (c.tile != TILE_256) c.split = SplitPlan{0, 0, 1, 0.0};
  if (c.tile == TILE_128 && can_split) c.split = split_plan128(tiles128, nk, cus);
  return c;
}

// The tile shapes and split a launch may take: grouped forwards (row segments on 256- or 128-row boundaries)
// no 192-row tiles and no split; segmented reductions no split (a piece would start inside a segment) and no
// 256 x 320 tiles (that kernel variant spills registers).
constexpr unsigned ALL_TILES = (1u << TILE_COUNT) - 1;
unsigned allowed_tiles(bool grouped, bool ksegs) {
  unsigned m = ALL_TILES;
  if (grouped) m &= ~(1u << TILE_192);
  if (ksegs) m &= ~(1u << TILE_320);
  return m;
}

// Workspace for any schedule an entry may take: the larger of the T256 and T128 split plans' pieces (used when
// the launch runs that tile shape, chosen or forced; other shapes leave it untouched).
int64_t split_ws_bytes(int64_t rows_a, int64_t rows_b, int64_t kbytes) {
  const int cus = k2q_cu_count();
  const int nk = (int)(kbytes / SBK);
  const SplitPlan q = split_plan(((rows_a + 255) / 256) * ((rows_b + 255) / 256), nk, cus);
  const SplitPlan q128 = split_plan128(((rows_a + 127) / 128) * ((rows_b + 127) / 128), nk, cus);
  const int64_t b256 = q.s > 1 ? (int64_t)q.rem * q.s * 256 * 256 * 4 : 0;
  const int64_t b128 = q128.s > 1 ? (int64_t)q128.rem * q128.s * 128 * 128 * 4 : 0;
  return b256 > b128 ? b256 : b128;
}

template <int EPI, int MODE, class C, int NS>
int set_lds() {
  static std::atomic<uint64_t> lds_set{0};
  return k2q_lds_limit_once(gemm_nt_kernel<EPI, MODE, C, NS>, C::LDS, lds_set);
}

// The base of a launch's arguments, for the kernels that take no segment tables.
inline GemmArgsN<0> slim(const GemmArgs& p) {
  GemmArgsN<0> q;
  static_cast<GemmBase&>(q) = p;
  return q;
}

// Balanced persistent grid: as many rounds as the tiles need on this GPU's workgroup slots, and just enough
// workgroups for that many rounds, each taking the same number of tiles (3168 T256 tiles on 256 CUs: 244
// workgroups of 13), instead of a last round that leaves most CUs idle.  Launches with segments (a grouped
// forward, a segmented reduction) take the kernel that carries the tables; the others the slim one.
template <int EPI, class C, int MODE = MODE_TILE>
int launch_tiles(const GemmArgs& p, hipStream_t st) {
  const int64_t slots = (int64_t)k2q_cu_count() * C::WPC;
  const int64_t rounds = (p.dp_tiles + slots - 1) / slots;
  const dim3 grid((unsigned)((p.dp_tiles + rounds - 1) / rounds));
  constexpr bool kTables = MODE == MODE_KSEG || (EPI == EPI_W8 && MODE == MODE_TILE);
  if constexpr (kTables) {
    if (MODE == MODE_KSEG || p.nseg > 0) {
      if (int rc = set_lds<EPI, MODE, C, MAX_SEG>()) return rc;
      GemmArgs pt = p;
      pt.nwg = (int)grid.x;
      hipLaunchKernelGGL((gemm_nt_kernel<EPI, MODE, C, MAX_SEG>), grid, dim3(GT), C::LDS, st, pt);
      return K2Q_OK;
    }
  }
  if constexpr (MODE != MODE_KSEG) {
    if (int rc = set_lds<EPI, MODE, C, 0>()) return rc;
    GemmArgsN<0> ps = slim(p);
    ps.nwg = (int)grid.x;
    hipLaunchKernelGGL((gemm_nt_kernel<EPI, MODE, C, 0>), grid, dim3(GT), C::LDS, st, ps);
  }
  return K2Q_OK;
}

// Full-K tiles: the segmented-reduction kernel when the launch has reduction segments (EPI_DXLIN only).
template <int EPI, class C>
int launch_full(const GemmArgs& p, hipStream_t st) {
  if constexpr (EPI == EPI_DXLIN) {
    if (p.nks > 0) return launch_tiles<EPI, C, MODE_KSEG>(p, st);
  }
  return launch_tiles<EPI, C>(p, st);
}

// A split schedule: the pieces first (they fill the GPU for a short round), then the full tiles, then the fixup.
// Split launches carry no segments (the caller runs grouped launches as full-K tiles).
template <int EPI, class C>
int launch_split(const GemmArgs& p, const SplitPlan& q, hipStream_t st) {
  if (p.nseg > 0 || p.nks > 0) return K2Q_EINVAL;
  int rc;
  if ((rc = set_lds<EPI, MODE_PIECE, C, 0>()) || (rc = set_lds<EPI, MODE_FIXUP, C, 0>())) return rc;
  const GemmArgsN<0> ps = slim(p);
  hipLaunchKernelGGL((gemm_nt_kernel<EPI, MODE_PIECE, C, 0>), dim3((unsigned)(q.rem * q.s)), dim3(GT), C::LDS, st,
                     ps);
  if (q.dp_tiles > 0 && (rc = launch_full<EPI, C>(p, st))) return rc;
  hipLaunchKernelGGL((gemm_nt_kernel<EPI, MODE_FIXUP, C, 0>), dim3((unsigned)q.rem), dim3(GT), C::LDS, st, ps);
  return K2Q_OK;
}

// B-tiles per group of the tile order.  A launch whose tiles all run at once (one round of full-K tiles, or a
// split with pieces only) takes the width, of 8, 4 and 2, whose tiles on one XCD span the fewest operand rows
// (8 on a tie): an XCD holds the workgroups of consecutive remapped ids in the tile kernel, every 8th hardware
// id in the pieces kernel.  Those launches are short and feed on their operand strips: measured -5 to -21% on
// 1024-token shapes (128 x 128 tiles), no change on the others.  Launches of several rounds keep 8.
int group_width(int64_t rows_a, int64_t rows_b, int ta_rows, int tb_rows, int64_t dp_tiles, int64_t pieces,
                int64_t piece_tiles, int64_t slots) {
  const int64_t tiles_a = (rows_a + ta_rows - 1) / ta_rows, tiles_b = (rows_b + tb_rows - 1) / tb_rows;
  int64_t lids[64];
  int n = 0;
  if (pieces > 0) {
    if (dp_tiles > 0) return 8;
    const int64_t live = pieces < slots ? pieces : slots;
    for (int64_t b = 0; b < live && n < 64; b += 8) lids[n++] = b % piece_tiles;
  } else {
    if (dp_tiles > slots) return 8;
    const int64_t per = (dp_tiles + 7) / 8;
    for (int64_t i = 0; i < per && n < 64; ++i) lids[n++] = i;
  }
  int best = 8;
  int64_t best_rows = -1;
  for (int gb : {8, 4, 2}) {
    uint64_t seen_a[4] = {0, 0, 0, 0}, seen_b[4] = {0, 0, 0, 0};   // tile indices < 256 on the launches this applies to
    int na = 0, nb = 0;
    bool fits = true;
    for (int i = 0; i < n; ++i) {
      int64_t ta, tb;
      group_coords(lids[i], tiles_a, tiles_b, gb, ta, tb);
      if (ta >= 256 || tb >= 256) { fits = false; break; }
      if (!(seen_a[ta >> 6] >> (ta & 63) & 1)) { seen_a[ta >> 6] |= 1ull << (ta & 63); ++na; }
      if (!(seen_b[tb >> 6] >> (tb & 63) & 1)) { seen_b[tb >> 6] |= 1ull << (tb & 63); ++nb; }
    }
    if (!fits) return 8;
    const int64_t rows = (int64_t)na * ta_rows + (int64_t)nb * tb_rows;
    if (best_rows < 0 || rows < best_rows) { best_rows = rows; best = gb; }
  }
  return best;
}

template <int EPI>
int launch_gemm(GemmArgs p, void* ws, int64_t ws_bytes, hipStream_t st, int forced = TILE_AUTO) {
  if (p.ldr == 0) p.ldr = p.r;
  // A tile's operand rows are read through buffer resources with 31-bit byte offsets: 320 rows of either side
  int64_t ld_max = p.lda_b > p.ldb_b ? p.lda_b : p.ldb_b;
  for (int i = 0; i < p.nks; ++i) {
    ld_max = p.ks[i].lda_b > ld_max ? p.ks[i].lda_b : ld_max;
    ld_max = p.ks[i].ldb_b > ld_max ? p.ks[i].ldb_b : ld_max;
  }
  if (320 * ld_max >= 0x7fffffffLL) return K2Q_EUNSUPPORTED;
  if (forced >= TILE_COUNT || (EPI == EPI_DX && forced >= 0 && forced != TILE_256)) return K2Q_EINVAL;
  TileChoice c = choose_tile(EPI, p.rows_a, p.rows_b, p.kbytes, allowed_tiles(p.nseg > 0, p.nks > 0),
                             p.nseg == 0 && p.nks == 0, forced, k2q_cu_count());
  if (forced >= 0 && !(allowed_tiles(p.nseg > 0, p.nks > 0) >> forced & 1)) return K2Q_EINVAL;
  if (p.nseg > 0) {   // segments start on tile boundaries
    const int ta = c.tile == TILE_192 ? 192 : c.tile == TILE_128 ? 128 : 256;
    for (int i = 0; i < p.nseg; ++i)
      if (p.seg[i].start % ta || p.seg[i].rows % ta) return K2Q_EINVAL;
  }
  if (c.tile != TILE_256) {
    int64_t tiles;
    if (c.tile == TILE_320) tiles = ((p.rows_a + 255) / 256) * ((p.rows_b + 319) / 320);
    else if (c.tile == TILE_192) tiles = ((p.rows_a + 191) / 192) * ((p.rows_b + 255) / 256);
    else tiles = ((p.rows_a + 127) / 128) * ((p.rows_b + 127) / 128);
    if (tiles > 0x7fffffff) return K2Q_EUNSUPPORTED;
    p.dp_tiles = tiles;
    p.sk_rem = 0;
    p.sk_s = 1;
    SplitPlan q = c.split;
    if (c.tile != TILE_128 || (q.s > 1 && (!ws || ws_bytes < (int64_t)q.rem * q.s * 128 * 128 * 4 ||
                                           !k2q_aligned(ws, 16))))
      q = SplitPlan{tiles, 0, 1, 0.0};   // no split, or no room for the pieces: full-K tiles only
    {
      const int tar = c.tile == TILE_320 ? 256 : c.tile == TILE_192 ? 192 : 128;
      const int tbr = c.tile == TILE_320 ? 320 : c.tile == TILE_192 ? 256 : 128;
      const int wpc = c.tile == TILE_128 ? T128::WPC : c.tile == TILE_192 ? T192::WPC : T320::WPC;
      p.gb = q.s > 1 ? group_width(p.rows_a, p.rows_b, tar, tbr, q.dp_tiles, q.rem * q.s, q.rem,
                                   (int64_t)k2q_cu_count() * wpc)
                     : group_width(p.rows_a, p.rows_b, tar, tbr, tiles, 0, 1, (int64_t)k2q_cu_count() * wpc);
    }
    int rc;
    if constexpr (EPI == EPI_DX) {
      rc = K2Q_EINVAL;
    } else {
      if (c.tile == TILE_320) {
        rc = launch_full<EPI, T320>(p, st);
      } else if (c.tile == TILE_192) {
        rc = launch_full<EPI, T192>(p, st);
      } else if (q.s > 1) {
        p.dp_tiles = q.dp_tiles;
        p.sk_rem = q.rem;
        p.sk_s = q.s;
        p.part = static_cast<int32_t*>(ws);
        rc = launch_split<EPI, T128>(p, q, st);
      } else {
        rc = launch_full<EPI, T128>(p, st);
      }
    }
    return rc ? rc : k2q_launch_status();
  }
  SplitPlan q = c.split;
  const int64_t tiles = ((p.rows_a + 255) / 256) * ((p.rows_b + 255) / 256);
  if (tiles > 0x7fffffff) return K2Q_EUNSUPPORTED;
  if (q.s > 1 && (!ws || ws_bytes < (int64_t)q.rem * q.s * 256 * 256 * 4 || !k2q_aligned(ws, 16)))
    q = SplitPlan{tiles, 0, 1, 0.0};   // no room for the pieces: full-K tiles only
  p.dp_tiles = q.dp_tiles;
  p.sk_rem = q.rem;
  p.sk_s = q.s;
  p.part = static_cast<int32_t*>(ws);
  p.gb = group_width(p.rows_a, p.rows_b, 256, 256, q.dp_tiles, q.s > 1 ? q.rem * q.s : 0, q.rem > 0 ? q.rem : 1,
                     (int64_t)k2q_cu_count() * T256::WPC);
  int rc = q.s > 1 ? launch_split<EPI, T256>(p, q, st) : launch_full<EPI, T256>(p, st);
  return rc ? rc : k2q_launch_status();
}

int check_common(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || N < 1 || K < K2Q_HADAMARD || K % K2Q_HADAMARD) return K2Q_EINVAL;
  if (N % 4) return K2Q_EINVAL;
  return K2Q_OK;
}

// The epilogues take the LoRA term 16 ranks at a time, so any multiple of 16 up to K2Q_MAX_RANK works.
bool rank_ok(int64_t r) { return r >= 16 && r <= K2Q_MAX_RANK && r % 16 == 0; }

int check_lora(const float* u, const float* lb, int64_t r) {
  if (!u) return K2Q_OK;
  if (!lb || !rank_ok(r)) return K2Q_EINVAL;
  if (!k2q_aligned(u, 16) || !k2q_aligned(lb, 16)) return K2Q_EINVAL;
  return K2Q_OK;
}

}  // namespace

extern "C" int64_t k2q_gemm_w8a8_ws_bytes(int64_t M, int64_t N, int64_t K) {
  if (check_common(M, N, K) || M <= K2Q_GEMV_MAX_M) return 0;
  return split_ws_bytes(N, M, K);
}

extern "C" int64_t k2q_gemm_dx_ws_bytes(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || K < K2Q_HADAMARD || K % K2Q_HADAMARD || N < 64 || N % 64) return 0;
  return split_ws_bytes(K, M, 2 * N);
}

extern "C" int k2q_gemm_w8a8(const int8_t* qx, const float* sx, const int8_t* qw, const float* sw,
                             const float* bias, const float* u, const float* lora_b, int64_t r,
                             float lora_scale, int64_t M, int64_t N, int64_t K, uint16_t* y,
                             void* ws, int64_t ws_bytes, void* stream) {
  return k2q_gemm_w8a8_tile(qx, sx, qw, sw, bias, u, lora_b, r, lora_scale, M, N, K, y, ws, ws_bytes, -1, stream);
}

extern "C" int k2q_gemm_w8a8_tile(const int8_t* qx, const float* sx, const int8_t* qw, const float* sw,
                                  const float* bias, const float* u, const float* lora_b, int64_t r,
                                  float lora_scale, int64_t M, int64_t N, int64_t K, uint16_t* y,
                                  void* ws, int64_t ws_bytes, int tile, void* stream) {
  return gemm_w8a8_impl(qx, sx, qw, sw, bias, u, 1, 0, lora_b, r, lora_scale, M, N, K, y, ws, ws_bytes, tile,
                        static_cast<hipStream_t>(stream));
}

int gemm_w8a8_impl(const int8_t* qx, const float* sx, const int8_t* qw, const float* sw, const float* bias,
                   const float* u, int u_parts, int64_t u_pstride, const float* lora_b, int64_t r, float lora_scale,
                   int64_t M, int64_t N, int64_t K, uint16_t* y, void* ws, int64_t ws_bytes, int tile,
                   hipStream_t st) {
  int rc = check_common(M, N, K);
  if (rc) return rc;
  if (!k2q_aligned(y, 16)) return K2Q_EINVAL;
  if (!qx || !sx || !qw || !sw || !y) return K2Q_EINVAL;
  if (!k2q_aligned(qx, 16) || !k2q_aligned(qw, 16) || !k2q_aligned(sw, 16) || !k2q_aligned(y, 8))
    return K2Q_EINVAL;
  if (bias && !k2q_aligned(bias, 16)) return K2Q_EINVAL;
  if ((rc = check_lora(u, lora_b, r))) return rc;
  if (u_parts < 1 || (u_parts > 1 && (M <= K2Q_GEMV_MAX_M || u_pstride < M * r || u_pstride % 4))) return K2Q_EINVAL;
  if (M <= K2Q_GEMV_MAX_M)
    return k2q_launch_gemv_w8a8(qx, sx, qw, sw, bias, u, lora_b, (int)r, lora_scale, M, N, K, y, st);
  GemmArgs p{};
  p.a = reinterpret_cast<const uint8_t*>(qw);
  p.b = reinterpret_cast<const uint8_t*>(qx);
  p.rows_a = N; p.rows_b = M; p.kbytes = K; p.lda_b = K; p.ldb_b = K;
  p.out = y; p.ldo = N;
  p.sx = sx; p.sw = sw; p.bias = bias;
  p.lora_rb = u; p.lora_ra = lora_b; p.r = u ? (int)r : 0; p.lora_scale = lora_scale;
  p.rb_parts = u_parts; p.rb_pstride = u_pstride;
  return launch_gemm<EPI_W8>(p, ws, ws_bytes, st, tile);
}

extern "C" int k2q_gemm_w8a8_plan(int64_t M, int64_t N, int64_t K, int cus, int grouped, int* split_pieces) {
  if (M < 1 || N < 1 || K < K2Q_HADAMARD || K % K2Q_HADAMARD || cus < 1) return K2Q_EINVAL;
  if (M <= K2Q_GEMV_MAX_M) {
    if (grouped) return K2Q_EINVAL;
    if (split_pieces) *split_pieces = 1;
    return K2Q_TILE_GEMV;
  }
  const TileChoice c = choose_tile(EPI_W8, N, M, K, allowed_tiles(grouped != 0, false), grouped == 0, TILE_AUTO, cus);
  if (split_pieces) *split_pieces = c.tile == TILE_256 || c.tile == TILE_128 ? c.split.s : 1;
  return c.tile;
}

extern "C" int k2q_gemm_w8a8_grouped(const int8_t* qx, const float* sx, int64_t M, int64_t K,
                                     const k2q_w8a8_segment* seg, int64_t nseg, const float* u, int64_t r,
                                     int64_t ldu, void* ws, int64_t ws_bytes, void* stream) {
  if (!qx || !sx || !seg || nseg < 1 || nseg > MAX_SEG || M <= K2Q_GEMV_MAX_M) return K2Q_EINVAL;
  if (K < K2Q_HADAMARD || K % K2Q_HADAMARD || !k2q_aligned(qx, 16)) return K2Q_EINVAL;
  bool any_lora = false;
  int64_t start = 0;
  GemmArgs p{};
  for (int64_t i = 0; i < nseg; ++i) {
    const k2q_w8a8_segment& g = seg[i];
    if (!g.qw || !g.sw || !g.y || g.N < 256 || g.N % 256) return K2Q_EINVAL;
    if (!k2q_aligned(g.qw, 16) || !k2q_aligned(g.sw, 16) || !k2q_aligned(g.y, 16)) return K2Q_EINVAL;
    if (g.bias && !k2q_aligned(g.bias, 16)) return K2Q_EINVAL;
    if (g.lora_b) {
      if (!u || !k2q_aligned(g.lora_b, 16) || g.u_col < 0 || g.u_col + r > ldu || g.u_col % 4) return K2Q_EINVAL;
      any_lora = true;
    }
    GemmSeg& s = p.seg[i];
    s.a = reinterpret_cast<const uint8_t*>(g.qw);
    s.sw = g.sw;
    s.bias = g.bias;
    s.lora_ra = g.lora_b;
    s.out = g.y;
    s.start = start;
    s.rows = g.N;
    s.ldo = g.N;
    s.rb_off = g.u_col;
    s.lora_scale = g.lora_scale;
    start += g.N;
  }
  if (any_lora && (!rank_ok(r) || ldu % 4 || !k2q_aligned(u, 16))) return K2Q_EINVAL;
  p.nseg = (int)nseg;
  p.a = p.seg[0].a;   // unused by the tiles (each takes its segment's), set for completeness
  p.b = reinterpret_cast<const uint8_t*>(qx);
  p.rows_a = start; p.rows_b = M; p.kbytes = K; p.lda_b = K; p.ldb_b = K;
  p.sx = sx;
  p.lora_rb = any_lora ? u : nullptr;
  p.r = any_lora ? (int)r : 0;
  p.ldr = (int)ldu;
  (void)ws;
  (void)ws_bytes;   // full-K tiles only: the split schedule's kernels take no segments
  return launch_gemm<EPI_W8>(p, nullptr, 0, static_cast<hipStream_t>(stream));
}

extern "C" int k2q_gemm_w8a8_acc(const int8_t* qx, const int8_t* qw, int64_t M, int64_t N, int64_t K,
                                 int32_t* acc, void* ws, int64_t ws_bytes, int tile, void* stream) {
  int rc = check_common(M, N, K);
  if (rc) return rc;
  if (!qx || !qw || !acc || !k2q_aligned(qx, 16) || !k2q_aligned(qw, 16) || !k2q_aligned(acc, 16))
    return K2Q_EINVAL;
  GemmArgs p{};
  p.a = reinterpret_cast<const uint8_t*>(qw);
  p.b = reinterpret_cast<const uint8_t*>(qx);
  p.rows_a = N; p.rows_b = M; p.kbytes = K; p.lda_b = K; p.ldb_b = K;
  p.out = acc; p.ldo = N;
  return launch_gemm<EPI_ACC>(p, ws, ws_bytes, static_cast<hipStream_t>(stream), tile);
}

extern "C" int k2q_gemm_dx(const uint16_t* dy, const uint16_t* wt, int64_t M, int64_t N, int64_t K,
                           const float* g, const float* lora_a, int64_t r, uint16_t* dx, void* ws, int64_t ws_bytes,
                           void* stream) {
  if (M < 1 || K < K2Q_HADAMARD || K % K2Q_HADAMARD || N < 64 || N % 64) return K2Q_EINVAL;
  if (!dy || !wt || !dx || !k2q_aligned(dy, 16) || !k2q_aligned(wt, 16) || !k2q_aligned(dx, 16))
    return K2Q_EINVAL;
  int rc = check_lora(g, lora_a, r);
  if (rc) return rc;
  GemmArgs p{};
  p.a = reinterpret_cast<const uint8_t*>(wt);
  p.b = reinterpret_cast<const uint8_t*>(dy);
  p.rows_a = K; p.rows_b = M; p.kbytes = 2 * N; p.lda_b = 2 * N; p.ldb_b = 2 * N;
  p.out = dx; p.ldo = K;
  p.lora_rb = g; p.lora_ra = lora_a; p.r = g ? (int)r : 0; p.lora_scale = 1.f;
  return launch_gemm<EPI_DX>(p, ws, ws_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int64_t k2q_gemm_bf16_ws_bytes(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || N < 1 || N % 4 || K < 64 || K % 64) return 0;
  return split_ws_bytes(N, M, 2 * K);
}

extern "C" int k2q_gemm_bf16(const uint16_t* x, const uint16_t* w, const float* bias, const float* u,
                             const float* lora_b, int64_t r, float lora_scale, int64_t M, int64_t N, int64_t K,
                             uint16_t* y, void* ws, int64_t ws_bytes, void* stream) {
  if (M < 1 || N < 1 || N % 4 || K < 64 || K % 64) return K2Q_EINVAL;
  if (!x || !w || !y || !k2q_aligned(x, 16) || !k2q_aligned(w, 16) || !k2q_aligned(y, 16)) return K2Q_EINVAL;
  if (bias && !k2q_aligned(bias, 16)) return K2Q_EINVAL;
  int rc = check_lora(u, lora_b, r);
  if (rc) return rc;
  GemmArgs p{};
  p.a = reinterpret_cast<const uint8_t*>(w);
  p.b = reinterpret_cast<const uint8_t*>(x);
  p.rows_a = N; p.rows_b = M; p.kbytes = 2 * K; p.lda_b = 2 * K; p.ldb_b = 2 * K;
  p.out = y; p.ldo = N;
  p.bias = bias;
  p.lora_rb = u; p.lora_ra = lora_b; p.r = u ? (int)r : 0; p.lora_scale = lora_scale;
  return launch_gemm<EPI_LIN>(p, ws, ws_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int k2q_gemm_dx_lin(const uint16_t* dy, const uint16_t* wt, int64_t M, int64_t N, int64_t K,
                               const float* g, const float* lora_a, int64_t r, uint16_t* dx, void* ws, int64_t ws_bytes,
                               void* stream) {
  if (M < 1 || K < 64 || K % 64 || N < 64 || N % 64) return K2Q_EINVAL;
  if (!dy || !wt || !dx || !k2q_aligned(dy, 16) || !k2q_aligned(wt, 16) || !k2q_aligned(dx, 16))
    return K2Q_EINVAL;
  int rc = check_lora(g, lora_a, r);
  if (rc) return rc;
  GemmArgs p{};
  p.a = reinterpret_cast<const uint8_t*>(wt);
  p.b = reinterpret_cast<const uint8_t*>(dy);
  p.rows_a = K; p.rows_b = M; p.kbytes = 2 * N; p.lda_b = 2 * N; p.ldb_b = 2 * N;
  p.out = dx; p.ldo = K;
  p.lora_rb = g; p.lora_ra = lora_a; p.r = g ? (int)r : 0; p.lora_scale = 1.f;
  return launch_gemm<EPI_DXLIN>(p, ws, ws_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int k2q_gemm_dx_grouped(const k2q_dx_segment* seg, int64_t nseg, int64_t M, int64_t K, const float* g,
                                   int64_t ldg, const float* lora_a, int64_t r, uint16_t* dx, void* stream) {
  if (!seg || nseg < 1 || nseg > MAX_SEG || M < 1 || K < 64 || K % 64 || !dx || !k2q_aligned(dx, 16))
    return K2Q_EINVAL;
  GemmArgs p{};
  int64_t stages = 0;
  for (int64_t i = 0; i < nseg; ++i) {
    const k2q_dx_segment& sg = seg[i];
    if (!sg.dy || !sg.wt || sg.N < 64 || sg.N % 64 || sg.ldy < sg.N || sg.ldy % 8 || !k2q_aligned(sg.dy, 16) ||
        !k2q_aligned(sg.wt, 16))
      return K2Q_EINVAL;
    stages += 2 * sg.N / WBK;
    if (stages > 0x3fffffff) return K2Q_EUNSUPPORTED;
    p.ks[i] = KSeg{reinterpret_cast<const uint8_t*>(sg.wt), reinterpret_cast<const uint8_t*>(sg.dy), 2 * sg.N,
                   2 * sg.ldy, (int)stages};
  }
  int rc = check_lora(g, lora_a, r);
  if (rc) return rc;
  if (g && (ldg < r || ldg % 4)) return K2Q_EINVAL;
  p.nks = (int)nseg;
  p.a = p.ks[0].a; p.b = p.ks[0].b; p.lda_b = p.ks[0].lda_b; p.ldb_b = p.ks[0].ldb_b;
  p.rows_a = K; p.rows_b = M; p.kbytes = stages * WBK;
  p.out = dx; p.ldo = K;
  p.lora_rb = g; p.lora_ra = lora_a; p.r = g ? (int)r : 0; p.ldr = g ? (int)ldg : 0; p.lora_scale = 1.f;
  return launch_gemm<EPI_DXLIN>(p, nullptr, 0, static_cast<hipStream_t>(stream));
}

extern "C" int k2q_gemm_w4a8(const int8_t* qx, const float* sx, const uint8_t* qw4, const uint16_t* sw4,
                             const float* bias, const float* u, const float* lora_b, int64_t r,
                             float lora_scale, int64_t M, int64_t N, int64_t K, uint16_t* y, void* stream) {
  int rc = check_common(M, N, K);
  if (rc) return rc;
  if (!qx || !sx || !qw4 || !sw4 || !y) return K2Q_EINVAL;
  if (!k2q_aligned(qx, 16) || !k2q_aligned(qw4, 16) || !k2q_aligned(sw4, 8) || !k2q_aligned(y, 8))
    return K2Q_EINVAL;
  if (bias && !k2q_aligned(bias, 16)) return K2Q_EINVAL;
  if ((rc = check_lora(u, lora_b, r))) return rc;
  W4Args p{};
  p.a = qw4; p.s4 = sw4; p.b = qx; p.N = N; p.M = M; p.K = K;
  p.out = y; p.sx = sx; p.bias = bias;
  p.lora_rb = u; p.lora_ra = lora_b; p.r = u ? (int)r : 0; p.lora_scale = lora_scale;
  return launch_w4<EPI_W8>(p, static_cast<hipStream_t>(stream));
}

extern "C" int k2q_gemm_w4a8_f32(const int8_t* qx, const uint8_t* qw4, const uint16_t* sw4, int64_t M,
                                 int64_t N, int64_t K, float* out, void* stream) {
  int rc = check_common(M, N, K);
  if (rc) return rc;
  if (!qx || !qw4 || !sw4 || !out || !k2q_aligned(qx, 16) || !k2q_aligned(qw4, 16) ||
      !k2q_aligned(sw4, 8) || !k2q_aligned(out, 16))
    return K2Q_EINVAL;
  W4Args p{};
  p.a = qw4; p.s4 = sw4; p.b = qx; p.N = N; p.M = M; p.K = K; p.out = out;
  return launch_w4<EPI_ACC>(p, static_cast<hipStream_t>(stream));
}
