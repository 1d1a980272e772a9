// One quantized linear + LoRA forward per call: the C counterpart of Fp8Linear.forward followed by the adapter
// add of LoRALinear.forward (reference quantize.py:48-51, lora.py:43-48), with the ConvRot arithmetic of the
// other kernels.  The launches that make it up (rotate/quant, LoRA down-projection, GEMM with its epilogue) are
// issued from here, so a caller pays one foreign call per linear.
//
// Skinny M (M <= K2Q_GEMV_MAX_M: the adaLN modulation linears run at M = batch) has one more fusion: a prologue
// kernel computes the rows' int8 codes (one workgroup per row) and the LoRA factors u = x A^T (one workgroup
// per rank, its factor row kept in registers while the M rows stream past) in one launch, and the GEMV follows,
// so the linear is two launches.  Its codes are bit-identical to k2q_rotquant (same butterfly per 128-block,
// same quantizer); u is an f32 dot product per rank in a fixed order (x is bf16, so every product is exact in
// f32; the sums differ from the MFMA down-projection only by f32 rounding).
#include "rotation.h"

namespace {

using namespace k2q_rot;

constexpr int SK_T = 256;       // lanes per workgroup (four waves)
constexpr int SK_CW = SK_T * 16;   // elements per chunk

// Workgroups [0, ncode): row blockIdx.x's codes and scale (the row rotated in registers, one amax).
// Workgroups [ncode, ncode + r): rank j = blockIdx.x - ncode: u[m, j] = x[m, :] . A[j, :] for the M rows, each
// lane's 16 columns per chunk summed in column order, then the wave's lanes (shuffle tree), then the four
// waves in order.  kNCH chunks of 4096 elements cover K.
template <int kNCH>
__global__ __launch_bounds__(SK_T) void skinny_prologue_kernel(const __bf16* __restrict__ x, int64_t ldx, int K,
                                                               int M, const float* __restrict__ a, int r,
                                                               float* __restrict__ u, int ncode,
                                                               int8_t* __restrict__ q, float* __restrict__ s) {
  __shared__ float red[2][4];
  __shared__ float smax[4];
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int off = lane_offset(t);

  if ((int)blockIdx.x >= ncode) {
    const int j = (int)blockIdx.x - ncode;
    float w[kNCH][16];
#pragma unroll
    for (int c = 0; c < kNCH; ++c) {
      const int col = c * SK_CW + off;
      load16<float>(a + (int64_t)j * K + col, col < K, w[c]);
    }
    for (int m = 0; m < M; ++m) {
      float v[kNCH][16];
#pragma unroll
      for (int c = 0; c < kNCH; ++c) {
        const int col = c * SK_CW + off;
        load16<__bf16>(x + m * ldx + col, col < K, v[c]);
      }
      float p = 0.f;
#pragma unroll
      for (int c = 0; c < kNCH; ++c) {
        if (c * SK_CW + off >= K) continue;
#pragma unroll
        for (int e = 0; e < 16; ++e) p = __builtin_fmaf(v[c][e], w[c][e], p);
      }
      p = wave_sum(p);
      if (lane == 0) red[m & 1][wave] = p;
      __syncthreads();   // red[m & 1] is rewritten two rows later, after the next row's barrier
      if (t == 0) u[(int64_t)m * r + j] = ((red[m & 1][0] + red[m & 1][1]) + red[m & 1][2]) + red[m & 1][3];
    }
    return;
  }

  const int64_t row = blockIdx.x;
  const __bf16* xr = x + row * ldx;
  float v[kNCH][16];
#pragma unroll
  for (int c = 0; c < kNCH; ++c) {
    const int col = c * SK_CW + off;
    load16<__bf16>(xr + col, col < K, v[c]);
  }
  const int l = t & 15;
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
  if (lane == 0) smax[wave] = amax;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < 4; ++w) amax = fmaxf(amax, smax[w]);
  amax = fmaxf(amax, 1e-8f);
  const float inv = __fdiv_rn(127.f, amax);
  if (t == 0) s[row] = __fdiv_rn(amax, 127.f);
  const float mul = inv * sigma;
  int8_t* qr = q + row * (int64_t)K;
#pragma unroll
  for (int c = 0; c < kNCH; ++c) {
    const int col = c * SK_CW + off;
    if (col < K) store_codes16(qr + col, v[c], mul);
  }
}

int launch_skinny(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const float* a, int64_t r, float* u, int8_t* q,
                  float* s, hipStream_t st) {
  const __bf16* xp = reinterpret_cast<const __bf16*>(x);
  const int nch = (int)((K + SK_CW - 1) / SK_CW);
  const int ncode = q ? (int)M : 0;
  const dim3 grid((unsigned)(ncode + (a ? r : 0)));
  if (grid.x == 0) return K2Q_OK;
  switch (nch) {
#define K2Q_SK_CASE(NCH)                                                                                          \
  case NCH:                                                                                                      \
    hipLaunchKernelGGL(skinny_prologue_kernel<NCH>, grid, dim3(SK_T), 0, st, xp, ldx, (int)K, (int)M, a, (int)r, u, \
                       ncode, q, s);                                                                             \
    break;
    K2Q_SK_CASE(1) K2Q_SK_CASE(2) K2Q_SK_CASE(3) K2Q_SK_CASE(4)
#undef K2Q_SK_CASE
    default: return K2Q_EUNSUPPORTED;
  }
  return k2q_launch_status();
}

}  // namespace

namespace {

int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }

// Workspace layout of the forward (M > K2Q_GEMV_MAX_M): [u: M x r f32 when the caller passes no u]
// [the down-projection's K-slice partials] [the GEMM's split-K pieces].
struct FwdLayout {
  int64_t u_off, parts_off, gemm_off, total;
};

FwdLayout fwd_layout(int wmode, int64_t M, int64_t N, int64_t K, int64_t r) {
  FwdLayout L{};
  int64_t off = 0;
  if (r > 0 && M > K2Q_GEMV_MAX_M) {
    L.u_off = off;
    off += align256(M * r * 4);
    L.parts_off = off;
    const int64_t a = k2q_lora_down_ws_bytes(M, K, r), b = lora_down_parts_floats(M, K, r) * 4;
    off += align256(a > b ? a : b);
  }
  L.gemm_off = off;
  if (wmode == K2Q_WMODE_W8) off += align256(k2q_gemm_w8a8_ws_bytes(M, N, K));
  L.total = off;
  return L;
}

// Whether the GEMM epilogue should add the down-projection's K-slice partials itself instead of a reduce
// launch: every output-column tile reads the factor rows of its tokens, so the partials cost (slices - 1) x
// M x r x 4 bytes of extra reads per column of tiles.  Measured on MI355X: at cfg0 (M = 4096, N = K = 3072,
// r = 16; ~8 MB extra) the one-call forward gains ~9 us over the separate launches; at cfg2 (M = 16896,
// N = 12288; ~210 MB extra) it loses ~20 us.  The fold is taken up to 16 MB of extra reads.
bool fold_pays(int64_t M, int64_t N, int64_t K, int64_t r) {
  const int64_t parts = r > 0 ? lora_down_parts_floats(M, K, r) / (M * r) : 1;
  if (parts <= 1) return true;
  int pieces = 1;
  const int tile = k2q_gemm_w8a8_plan(M, N, K, k2q_cu_count(), 0, &pieces);
  const int64_t ta = tile == K2Q_TILE_192x256 ? 192 : tile == K2Q_TILE_128x128 ? 128 : 256;
  const int64_t extra = (parts - 1) * M * r * 4 * ((N + ta - 1) / ta);
  return extra <= ((int64_t)16 << 20);
}

// Whether the forward takes u from the rotate/quant pass (rotquant_lora_kernel) instead of a separate
// down-projection launch.  That kernel holds one 16-row tile per CU and streams A from L2 for every tile, so it
// is latency-bound once a CU has several tiles.  Measured on MI355X (K = 3072, 4 rotating inputs, rotate/quant
// + down-projection against the fused kernel): M = 1024 r = 16 24.7 -> 13.0 us, M = 4096 r = 16 25.5 -> 13.7,
// M = 8192 r = 16 27.1 -> 25.1, M = 16896 r = 16 46.9 -> 59.4, M = 16896 r = 32 50.7 -> 78.9, M = 4608 r = 64
// 27.6 -> 51.6.  So: at most one tile per CU for r <= 32, two for r = 16.
bool fuse_down(int64_t M, int64_t K, int64_t r) {
  if (r < 16 || r > 32 || !k2q_rotquant_lora_fits(K, r)) return false;
  const int64_t tiles = (M + 15) / 16, cus = k2q_cu_count();
  return tiles <= (r == 16 ? 2 * cus : cus);
}

}  // namespace

extern "C" int k2q_linear_fwd_fuses_down(int64_t M, int64_t K, int64_t r) {
  return M > K2Q_GEMV_MAX_M && fuse_down(M, K, r) ? 1 : 0;
}

extern "C" int64_t k2q_linear_fwd_ws_bytes(int wmode, int64_t M, int64_t N, int64_t K, int64_t r) {
  if (M < 1 || N < 1 || K < K2Q_HADAMARD || K % K2Q_HADAMARD) return 0;
  return fwd_layout(wmode, M, N, K, r).total;
}

extern "C" int k2q_linear_fwd(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, int8_t* qx, float* sx,
                              int codes_ready, const float* lora_a, const float* lora_b, int64_t r, float lora_scale,
                              float* u, int wmode, const void* qw, const void* sw, const float* bias, int64_t N,
                              uint16_t* y, void* ws, int64_t ws_bytes, void* stream) {
  if (!x || !qx || !sx || !qw || !sw || !y || M < 1 || N < 1 || K < K2Q_HADAMARD || K % K2Q_HADAMARD) return K2Q_EINVAL;
  if (K > 16384) return K2Q_EUNSUPPORTED;
  if (ldx < K || ldx % 8 || !k2q_aligned(x, 16) || !k2q_aligned(qx, 16)) return K2Q_EINVAL;
  if (wmode != K2Q_WMODE_W8 && wmode != K2Q_WMODE_W4) return K2Q_EINVAL;
  if (lora_a && (!lora_b || r < 16 || r > K2Q_MAX_RANK || r % 16 || !k2q_aligned(lora_a, 16) ||
                 (u && !k2q_aligned(u, 16))))
    return K2Q_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t rr = lora_a ? r : 0;
  const bool skinny = M <= K2Q_GEMV_MAX_M;
  const FwdLayout lay = fwd_layout(wmode, M, N, K, rr);
  // u from the rotate/quant pass straight into the caller's u leaves the factor region of ws unused
  const bool fused = !skinny && !codes_ready && lora_a && fuse_down(M, K, rr);
  const bool lora_ws = !skinny && rr > 0 && !(fused && u);
  if (lora_ws && (!ws || ws_bytes < lay.total)) return K2Q_EINVAL;
  if (ws && !k2q_aligned(ws, 256)) return K2Q_EINVAL;
  if (skinny && lora_a && !u) return K2Q_EINVAL;      // the prologue writes u
  uint8_t* w = static_cast<uint8_t*>(ws);
  // the GEMM's split pieces (without room for them it runs full-K tiles: the same output)
  void* gws = ws && ws_bytes > lay.gemm_off ? static_cast<void*>(w + lay.gemm_off) : nullptr;
  const int64_t gws_bytes = gws ? ws_bytes - lay.gemm_off : 0;
  int rc = K2Q_OK;
  const float* uu = nullptr;   // the factors the GEMM reads: u, or the down-projection's slice partials
  int parts = 1;
  if (skinny) {
    if (lora_a || !codes_ready)
      rc = launch_skinny(x, ldx, M, K, lora_a, rr, u, codes_ready ? nullptr : qx, sx, st);
    uu = lora_a ? u : nullptr;
  } else if (fused) {
    // u from the pass that rotates and quantizes x (one launch for both)
    float* ut = u ? u : reinterpret_cast<float*>(w + lay.u_off);
    rc = rotquant_lora_impl(x, M, K, ldx, qx, sx, lora_a, rr, ut, rr, st);
    uu = ut;
  } else {
    if (!codes_ready) rc = k2q_rotquant(x, K2Q_DTYPE_BF16, M, K, ldx, qx, sx, nullptr, stream);
    if (!rc && lora_a) {
      if (!u && wmode == K2Q_WMODE_W8 && rr <= 128 && fold_pays(M, N, K, rr)) {
        // nobody needs u itself: the GEMM epilogue adds the K-slice partials (no reduce launch)
        float* dst = reinterpret_cast<float*>(w + lay.parts_off);
        rc = lora_down_parts(x, M, K, ldx, lora_a, 1, 1.f, rr, dst, rr, &parts, st);
        uu = dst;
      } else {
        float* ut = u ? u : reinterpret_cast<float*>(w + lay.u_off);
        rc = lora_down_impl(x, M, K, ldx, lora_a, 1, 1.f, rr, w + lay.parts_off, lay.gemm_off - lay.parts_off, ut,
                            st);
        uu = ut;
      }
    }
  }
  if (rc) return rc;
  if (wmode == K2Q_WMODE_W8)
    return gemm_w8a8_impl(qx, sx, static_cast<const int8_t*>(qw), static_cast<const float*>(sw), bias, uu, parts,
                          M * rr, lora_a ? lora_b : nullptr, rr, lora_scale, M, N, K, y, gws, gws_bytes, -1, st);
  return k2q_gemm_w4a8(qx, sx, static_cast<const uint8_t*>(qw), static_cast<const uint16_t*>(sw), bias, uu,
                       lora_a ? lora_b : nullptr, rr, lora_scale, M, N, K, y, stream);
}
