// Skinny-M W8A8 forward (M <= 8 tokens): the adaLN modulation linears of the DiT run at M = batch
// (mmdit.py:314-317 modulate with one vector per sample), where the 256 x 256 MFMA tiles would hold 2
// valid rows out of 256 and a few dozen workgroups would have to stream the whole weight.  This path is
// HBM-bound on the weight read (N x K bytes, once): every wave streams GV_ROWS weight rows with 16-byte
// loads (a lane owns bytes 16 l + 1024 c of a row), dots them against the M token rows with
// v_dot4_i32_i8 (exact int32, the same sums as the MFMA path), and reduces across the wave with
// shuffles (integer adds: exact, order-free).
//
// The epilogue is the MFMA kernel's, term for term: f = fma(float(acc), (s_x 2^-7) s_w, bias); with LoRA,
// L = sum_j bf16(B[n,j]) bf16(s u[m,j]) in f32 is added to f; the result is rounded to bf16 once.  Without
// LoRA both paths give identical bits; with LoRA only L's summation order differs (the MFMA's internal
// order vs sequential here).
#include "k2q_common.h"

namespace {

constexpr int GV_ROWS = 4;    // weight rows per wave
constexpr int GV_WAVES = 4;   // waves per workgroup
constexpr int GV_CHUNK = 4;   // 1 KB row chunks per lane in flight (4 KB of every row per pass)

struct GemvArgs {
  const int8_t* qx;      // M x K
  const float* sx;       // M
  const int8_t* qw;      // N x K
  const float* sw;       // N
  const float* bias;     // N or null
  const float* u;        // M x r or null
  const float* lora_b;   // N x r
  int r;
  float lora_scale;
  int64_t M, N, K;
  uint16_t* y;           // M x N bf16
};

template <int MT>
__global__ __launch_bounds__(64 * GV_WAVES) void gemv_w8_kernel(GemvArgs p) {
  const int lane = threadIdx.x & 63;
  const int64_t n0 = ((int64_t)blockIdx.x * GV_WAVES + (threadIdx.x >> 6)) * GV_ROWS;
  if (n0 >= p.N) return;   // the kernel has no barriers: a wave past the end simply leaves

  const int8_t* wrow[GV_ROWS];
#pragma unroll
  for (int i = 0; i < GV_ROWS; ++i) {
    const int64_t n = n0 + i < p.N ? n0 + i : p.N - 1;
    wrow[i] = p.qw + n * p.K;
  }
  int acc[GV_ROWS][MT];
#pragma unroll
  for (int i = 0; i < GV_ROWS; ++i)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[i][m] = 0;

  for (int64_t kb = 0; kb < p.K; kb += 1024 * GV_CHUNK) {
    v4i w[GV_CHUNK][GV_ROWS];
#pragma unroll
    for (int c = 0; c < GV_CHUNK; ++c) {
      const int64_t k = kb + 1024 * c + 16 * lane;
#pragma unroll
      for (int i = 0; i < GV_ROWS; ++i)
        w[c][i] = k < p.K ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wrow[i] + k)) : v4i{0};
    }
#pragma unroll
    for (int c = 0; c < GV_CHUNK; ++c) {
      const int64_t k = kb + 1024 * c + 16 * lane;
      if (k >= p.K) break;
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const v4i xv = *reinterpret_cast<const v4i*>(p.qx + m * p.K + k);
#pragma unroll
        for (int i = 0; i < GV_ROWS; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[i][m] = __builtin_amdgcn_sdot4(w[c][i][e], xv[e], acc[i][m], false);
      }
    }
  }

  // Wave reduction: afterwards every lane holds every (row, token) sum.
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1)
#pragma unroll
    for (int i = 0; i < GV_ROWS; ++i)
#pragma unroll
      for (int m = 0; m < MT; ++m) acc[i][m] += __shfl_xor(acc[i][m], off, 64);

  // Lane i + GV_ROWS m writes y[m][n0 + i].
  if (lane >= GV_ROWS * MT) return;
  const int i = lane % GV_ROWS, m = lane / GV_ROWS;
  const int64_t n = n0 + i;
  if (n >= p.N) return;
  int a = 0;
#pragma unroll
  for (int ii = 0; ii < GV_ROWS; ++ii)
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) a = (ii == i && mm == m) ? acc[ii][mm] : a;

  const float sxm = p.sx[m] * 0.0078125f;   // 2^-7: the two unnormalised rotations
  const float bi = p.bias ? p.bias[n] : 0.f;
  float f = __builtin_fmaf((float)a, sxm * p.sw[n], bi);
  if (p.u) {
    const float* ub = p.u + (int64_t)m * p.r;
    const float* bb = p.lora_b + n * p.r;
    float l = 0.f;
    for (int j = 0; j < p.r; j += 4) {
      const v4f uv = *reinterpret_cast<const v4f*>(ub + j);
      const v4f bv = *reinterpret_cast<const v4f*>(bb + j);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        l = __builtin_fmaf(bf16_bits_to_f32(f32_to_bf16_bits(bv[e])),
                           bf16_bits_to_f32(f32_to_bf16_bits(uv[e] * p.lora_scale)), l);
    }
    f += l;
  }
  p.y[(int64_t)m * p.N + n] = (uint16_t)f32_to_bf16_bits(f);
}

template <int MT>
int launch_mt(const GemvArgs& p, hipStream_t st) {
  const int64_t rows_per_wg = (int64_t)GV_ROWS * GV_WAVES;
  const int64_t grid = (p.N + rows_per_wg - 1) / rows_per_wg;
  if (grid > 0x7fffffff) return K2Q_EUNSUPPORTED;
  hipLaunchKernelGGL(gemv_w8_kernel<MT>, dim3((unsigned)grid), dim3(64 * GV_WAVES), 0, st, p);
  return k2q_launch_status();
}

}  // namespace

// Called by k2q_gemm_w8a8 after its argument checks, for 1 <= M <= K2Q_GEMV_MAX_M.
int k2q_launch_gemv_w8a8(const int8_t* qx, const float* sx, const int8_t* qw, const float* sw, const float* bias,
                         const float* u, const float* lora_b, int r, float lora_scale, int64_t M, int64_t N,
                         int64_t K, uint16_t* y, hipStream_t st) {
  GemvArgs p{qx, sx, qw, sw, bias, u, lora_b, u ? r : 0, lora_scale, M, N, K, y};
  switch (M) {
    case 1: return launch_mt<1>(p, st);
    case 2: return launch_mt<2>(p, st);
    case 3: return launch_mt<3>(p, st);
    case 4: return launch_mt<4>(p, st);
    case 5: return launch_mt<5>(p, st);
    case 6: return launch_mt<6>(p, st);
    case 7: return launch_mt<7>(p, st);
    case 8: return launch_mt<8>(p, st);
    default: return K2Q_EINVAL;
  }
}
