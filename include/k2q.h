/* k2q — C ABI of the MI355X (gfx950) ConvRot QuantLinear + LoRA kernels.
 *
 * Every entry point takes raw device pointers, int64 shapes and a HIP stream passed as `void*`
 * (a hipStream_t; never the null stream in the module), launches asynchronously on that stream and
 * returns an int status (K2Q_OK or a negative K2Q_E* code).  No C++ exception crosses this boundary.
 * The caller (PyTorch's caching allocator) owns every buffer the other entry points use.  The library
 * holds one piece of device memory: the static scratch array of k2q_lora_grads_noalloc (K2Q_SCRATCH_BYTES
 * per GPU), whose per-device address it caches at that entry's first call on a device; that entry is not
 * re-entrant (overlapping calls on one GPU race for the scratch).  Beside it the library caches each
 * device's CU count (written once per device, read-only afterwards).  Every other entry point keeps no
 * state between calls, so its calls on different streams are re-entrant.
 *
 * Layouts (row-major, last index contiguous):
 *   x      M x K   bf16 activations (or f32 / bf16 weights for the weight quantizers)
 *   q      M x K   int8 codes, s M f32 per-row scales (s = absmax/127 of the rotated row)
 *   qw     N x K   int8 per-channel codes, sw N f32
 *   qw4    N x K/2 packed int4 codes (in every 16-wide K chunk, byte j = code j | code j+8 << 4),
 *          sw4 K/64 x N bf16 group scales, group-major (scales of one group are contiguous over n)
 *   u      M x r   f32 LoRA down-projection x A^T;  lora_a r x K f32, lora_b N x r f32
 *   y      M x N   bf16,  dy M x N bf16,  dx M x K bf16
 * Constraints checked before any launch: K % 128 == 0 (Hadamard block), r % 16 == 0 and 16 <= r <=
 * K2Q_MAX_RANK when a LoRA term is present (ranks run in chunks of 128 inside; a caller pads other ranks
 * with zero factor rows, which changes no result), pointers 16-byte aligned, M, N >= 1.
 */
#ifndef K2Q_H
#define K2Q_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define K2Q_OK 0
#define K2Q_EINVAL (-1)      /* bad shape, null or misaligned pointer */
#define K2Q_EARCH (-2)       /* current device is not gfx950 */
#define K2Q_ELAUNCH (-3)     /* kernel launch reported an error */
#define K2Q_EUNSUPPORTED (-4)/* shape outside what the kernels implement (e.g. K too large) */
#define K2Q_ESCRATCH (-5)    /* the shape needs more than the library's K2Q_SCRATCH_BYTES of device scratch */

#define K2Q_MAX_RANK 4096    /* largest LoRA rank any entry point takes */

#define K2Q_DTYPE_BF16 0
#define K2Q_DTYPE_F32 1

/* Library version string and device check (K2Q_OK when the current device is gfx950). */
const char* k2q_version(void);
int k2q_check_device(void);

/* (1) Rotate + per-row int8 quantize.
 * Replaces the point where Fp8Linear.forward receives x (reference quantize.py:48); the rotation and
 * the activation quantization have no reference code (north_star kernel (1)).  Also the int8 weight
 * quantizer of Fp8Linear.__init__'s ConvRot counterpart (quantize.py:34-37): call it on W's rows.
 * x_rot (nullable) receives bf16(FWHT(x)/sqrt(128)). */
int k2q_rotquant(const void* x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                 int8_t* q, float* s, uint16_t* x_rot, void* stream);

/* (1) + the LoRA down-projection from the same pass over x: the codes and scales of k2q_rotquant (bf16 x,
 * bit-identical) and u = x lora_a^T (lora_a r x K f32; u M rows of stride ldu f32, ranks 0 .. r-1), the first
 * product of LoRALinear.forward (reference lora.py:47) computed where Fp8Linear.forward receives x
 * (quantize.py:48).  One row per wave: K <= 3072 and K % 512 == 0, r in {16, 32, 48, 64}; other shapes return
 * K2Q_EUNSUPPORTED (k2q_lora_down then computes u in its own launch).  u is f32-accurate (A split into bf16
 * hi + lo on bf16 MFMA) in a fixed summation order, not bit-identical to k2q_lora_down's. */
int k2q_rotquant_lora(const void* x, int64_t M, int64_t K, int64_t ldx, int8_t* q, float* s,
                      const float* lora_a, int64_t r, float* u, int64_t ldu, void* stream);

/* int4 group-64 weight quantizer of W R (counterpart of Fp8Linear.__init__, quantize.py:34-39). */
int k2q_quant_weight_i4(const void* w, int w_dtype, int64_t N, int64_t K,
                        uint8_t* qw4, uint16_t* sw4, void* stream);

/* Producer-fused rotate/quant: the op that makes a quantized linear's input, computed in the same pass
 * that rotates and quantizes it.  Each writes h (M x K bf16, row stride K: the tensor the linear receives,
 * which its LoRA down-projection and backward read) and the codes / scales of k2q_rotquant(h), bit-identical
 * to a separate call on h.
 * k2q_swiglu_rotquant replaces `F.silu(self.gate(x)) * self.up(x)` of SwiGLU.forward (mmdit.py:177-178):
 *   h = bf16(bf16(silu(g)) * u), g / u the bf16 gate / up outputs (row strides ldg / ldu).
 * k2q_rmsmod_rotquant replaces `(1 + scale) * self.prenorm(x) + shift` of SingleStreamBlock.forward
 * (mmdit.py:314-317) with RMSNorm.forward (mmdit.py:156-161):
 *   n = bf16((x * rsqrt(mean_k x^2 + eps)) * (norm_scale + 1)),  h = bf16(bf16(bf16(1 + p) * n) + b),
 *   p / b = bf16 mod_scale / mod_shift at entry (row / rows_per_batch) * ld_mod (ld_mod 0: one entry).
 * k2q_swiglu_bwd is the autograd of the SwiGLU product (n bf16 elements, n % 8 == 0):
 *   du = bf16(dh * bf16(silu(g))),  dg = bf16((bf16(dh * u) * sig) * (1 + g (1 - sig))),  sig = sigmoid(g).
 * k2q_rmsmod_bwd is the autograd of the modulated RMSNorm for x (x, dh, dx contiguous M x K bf16, K % 8 == 0):
 *   g = bf16(dh * bf16(1 + p)) * (norm_scale + 1),  r = rsqrt(mean_k x^2 + eps),
 *   dx = bf16(g r - x (r^3 / K) sum_k g x),  p indexed as in k2q_rmsmod_rotquant. */
int k2q_swiglu_rotquant(const uint16_t* gate, int64_t ldg, const uint16_t* up, int64_t ldu, int64_t M, int64_t K,
                        uint16_t* h, int8_t* q, float* s, void* stream);
int k2q_rmsmod_rotquant(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const float* norm_scale, float eps,
                        const uint16_t* mod_scale, const uint16_t* mod_shift, int64_t ld_mod,
                        int64_t rows_per_batch, uint16_t* h, int8_t* q, float* s, void* stream);
int k2q_swiglu_bwd(const uint16_t* dh, const uint16_t* gate, const uint16_t* up, int64_t n, uint16_t* dgate,
                   uint16_t* dup, void* stream);
int k2q_rmsmod_bwd(const uint16_t* dh, const uint16_t* x, int64_t M, int64_t K, const float* norm_scale, float eps,
                   const uint16_t* mod_scale, int64_t ld_mod, int64_t rows_per_batch, uint16_t* dx, void* stream);

/* LoRA down-projection u = x.f32 @ A^T (lora.py:47, first product).  When the rows alone do not fill the
 * GPU, K is cut into slices whose partials meet in ws (k2q_lora_down_ws_bytes(M, K, r) bytes; 0 means none
 * is used) and are added in slice order; with ws == NULL or ws_bytes too small it runs unsliced. */
int64_t k2q_lora_down_ws_bytes(int64_t M, int64_t K, int64_t r);
int k2q_lora_down(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const float* lora_a, int64_t r,
                  void* ws, int64_t ws_bytes, float* u, void* stream);

/* LoRA gradients through the frozen base (the autograd of lora.py:47-48):
 *   g = scale * dy @ lora_b (M x r), dA = g^T x (r x K), dB = scale * dy^T u (N x r),
 * all f32 from bf16 dy (M x N) / x (M x K) and f32 u (M x r) / lora_b (N x r).  dA / dB nullable (x / u
 * then unused).  N % 128 == 0, K % 128 == 0.  ws: k2q_lora_grads_ws_bytes(M, N, K, r) bytes, 256-aligned. */
int64_t k2q_lora_grads_ws_bytes(int64_t M, int64_t N, int64_t K, int64_t r);
int k2q_lora_grads(const uint16_t* dy, const uint16_t* x, const float* u, const float* lora_b, int64_t r,
                   float scale, int64_t M, int64_t N, int64_t K, float* g, float* dA, float* dB, void* ws,
                   int64_t ws_bytes, void* stream);

/* One member of k2q_lora_grads_grouped: a linear that reads the group's shared input. */
typedef struct {
  const uint16_t* dy;    /* M x N bf16 output gradient, row stride ldy (a multiple of 8) */
  int64_t ldy;
  int64_t N;             /* out_features, a multiple of 128 */
  const float* lora_b;   /* N x r f32 */
  float scale;           /* the member's LoRA scale s_i */
  float* dB;             /* N x r f32 out (s_i dy_i^T u_i), or NULL */
} k2q_lora_member;

/* The LoRA gradients of n <= 8 linears with one rank r <= 128 that read one input x (M x K bf16): the
 * autograd of lora.py:47-48 for every member of a grouped node (the linears of Attention.forward that read
 * one tensor, mmdit.py:199; SwiGLU's gate and up, mmdit.py:178).  Member i: g_i = s_i dy_i B_i into columns
 * [i r, (i+1) r) of g (M x n r, row stride n r: the stacked layout k2q_gemm_dx_grouped reads); dA_i = g_i^T x
 * into rows [i r, (i+1) r) of dA (n r x K; NULL: none), computed over the stacked ranks in one pass over x per
 * 128 of them; dB_i from u_i = columns [i r, (i+1) r) of u (M x n r, the grouped forward's stacked factors).
 * Same arithmetic as k2q_lora_grads per member.  ws: k2q_lora_grads_grouped_ws_bytes bytes, 256-aligned. */
int64_t k2q_lora_grads_grouped_ws_bytes(const k2q_lora_member* members, int64_t n, int64_t M, int64_t K,
                                        int64_t r);
int k2q_lora_grads_grouped(const k2q_lora_member* members, int64_t n, const uint16_t* x, const float* u,
                           int64_t r, int64_t M, int64_t K, float* g, float* dA, void* ws, int64_t ws_bytes,
                           void* stream);

/* k2q_lora_grads without a workspace argument; allocates nothing.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving or training loops,
 * harnesses that forbid it).  The workspace comes from a device array inside the library, K2Q_SCRATCH_BYTES per
 * GPU, held until the process ends; a shape whose k2q_lora_grads_ws_bytes exceeds it returns K2Q_ESCRATCH
 * before any launch (cfg3's M = 4608, N = 3072, K = 12288, r = 64 needs ~34 MB).  Every call on one GPU shares
 * that GPU's scratch: calls that overlap on one GPU (two streams, two threads) race.  Results are bit-identical
 * to k2q_lora_grads. */
#define K2Q_SCRATCH_BYTES ((int64_t)64 << 20)
int k2q_lora_grads_noalloc(const uint16_t* dy, const uint16_t* x, const float* u, const float* lora_b, int64_t r,
                           float scale, int64_t M, int64_t N, int64_t K, float* g, float* dA, float* dB,
                           void* stream);

/* (2)+(3) W8A8 GEMM with the fused epilogue, replacing F.linear(x, W_deq, b) of quantize.py:49-51 and
 * the LoRA add of lora.py:47-48:
 *   y = bf16(2^-7 s_x[m] s_w[n] acc[m,n] + bias[n] + lora_scale * sum_j u[m,j] lora_b[n,j]).
 * bias, u, lora_b nullable (r ignored when u is null).  M <= 8 runs a GEMV.  When the 256 x 256 tiles
 * leave the last round of the GPU partly empty, the remainder tiles are cut along K into pieces whose
 * int32 sums meet in ws (k2q_gemm_w8a8_ws_bytes(M, N, K) bytes, 0 = not used); the result is identical.
 * ws == NULL or too small: full-K tiles only. */
int64_t k2q_gemm_w8a8_ws_bytes(int64_t M, int64_t N, int64_t K);
int k2q_gemm_w8a8(const int8_t* qx, const float* sx, const int8_t* qw, const float* sw, const float* bias,
                  const float* u, const float* lora_b, int64_t r, float lora_scale,
                  int64_t M, int64_t N, int64_t K, uint16_t* y, void* ws, int64_t ws_bytes, void* stream);

/* Grouped W8A8 forward: the linears that read one input (wq/wk/wv/gate of Attention.forward, mmdit.py:199,
 * each an Fp8Linear.forward + LoRA add, quantize.py:49-51 and lora.py:47-48) as one launch over the shared
 * codes qx / sx.  Segment i is k2q_gemm_w8a8 of its own weights into its own output y (M x N, row stride N)
 * with its factors u[:, u_col .. u_col + r) (u: M rows of ldu f32, r as for k2q_gemm_w8a8; lora_b NULL: no
 * adapter on that segment); the outputs are bit-identical to nseg separate k2q_gemm_w8a8 calls.
 * 1 <= nseg <= 4, every N a multiple of 256, M > 8.  The launch runs full-K tiles only: ws / ws_bytes are
 * accepted for symmetry with k2q_gemm_w8a8 and not used (pass NULL, 0). */
typedef struct {
  const int8_t* qw;       /* N x K int8 codes */
  const float* sw;        /* N f32 scales */
  const float* bias;      /* N f32, nullable */
  const float* lora_b;    /* N x r f32, nullable */
  uint16_t* y;            /* M x N bf16 */
  int64_t N;
  int64_t u_col;          /* first column of this segment's factors in u */
  float lora_scale;
} k2q_w8a8_segment;
int k2q_gemm_w8a8_grouped(const int8_t* qx, const float* sx, int64_t M, int64_t K, const k2q_w8a8_segment* seg,
                          int64_t nseg, const float* u, int64_t r, int64_t ldu, void* ws, int64_t ws_bytes,
                          void* stream);

/* One quantized linear + LoRA forward in one call: Fp8Linear.forward + the adapter add of LoRALinear.forward
 * (quantize.py:48-51, lora.py:43-48) with the ConvRot arithmetic, i.e. the launches of k2q_rotquant (skipped when
 * codes_ready: qx / sx already hold x's codes, e.g. from a producer kernel), k2q_lora_down (when lora_a) and
 * k2q_gemm_w8a8 / k2q_gemm_w4a8 issued from one call.  wmode K2Q_WMODE_W8: qw int8 N x K, sw f32 N;
 * K2Q_WMODE_W4: qw packed int4 N x K/2, sw bf16 K/64 x N.  x: M rows of ldx bf16; qx (M x K int8), sx (M f32)
 * and u (M x r f32, the LoRA factors the backward reuses) are caller buffers the call fills; y M x N bf16.
 * u may be NULL when nothing needs the factors afterwards (inference) and M > 8: then, for W8 and r <= 128,
 * the GEMM epilogue adds the down-projection's K-slice partials itself (no reduce launch; y is bit-identical).
 * M <= 8: one launch computes the codes and u, then the GEMV (two launches for the linear; u required).
 * Where k2q_linear_fwd_fuses_down(M, K, r) is 1 (codes not given, K <= 3072, a CU's worth or two of 16-row
 * tiles), the codes and u come from one k2q_rotquant_lora launch instead of k2q_rotquant + k2q_lora_down (u then
 * carries that kernel's summation order).
 * ws: k2q_linear_fwd_ws_bytes bytes (256-byte aligned): factors, their partials and the GEMM's split pieces.
 * It may be NULL when u is given and the call takes u from the rotate/quant pass (k2q_linear_fwd_fuses_down)
 * and, for W8, k2q_gemm_w8a8_ws_bytes(M, N, K) is 0: nothing of it is used then. */
#define K2Q_WMODE_W8 0
#define K2Q_WMODE_W4 1
int64_t k2q_linear_fwd_ws_bytes(int wmode, int64_t M, int64_t N, int64_t K, int64_t r);
/* Host only: 1 when k2q_linear_fwd with LoRA factors and codes not given computes u in the rotate/quant pass
 * (k2q_rotquant_lora), else 0 (no reference counterpart; lets callers and tests reproduce its launches). */
int k2q_linear_fwd_fuses_down(int64_t M, int64_t K, int64_t r);
int k2q_linear_fwd(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, int8_t* qx, float* sx, int codes_ready,
                   const float* lora_a, const float* lora_b, int64_t r, float lora_scale, float* u, int wmode,
                   const void* qw, const void* sw, const float* bias, int64_t N, uint16_t* y, void* ws,
                   int64_t ws_bytes, void* stream);

/* W4A8 variant: per-group int32 partials scaled by the bf16 group scales. */
int k2q_gemm_w4a8(const int8_t* qx, const float* sx, const uint8_t* qw4, const uint16_t* sw4,
                  const float* bias, const float* u, const float* lora_b, int64_t r, float lora_scale,
                  int64_t M, int64_t N, int64_t K, uint16_t* y, void* stream);

/* Output tile shapes of the MFMA GEMMs (A-rows x B-rows per workgroup).  Every entry point picks one per
 * launch with a cost model (K2Q_TILE_AUTO); the debug entries below take a shape explicitly so tests can run
 * each on any problem.  The result does not depend on the shape (int32 sums are exact; the f32 epilogue and
 * the LoRA term are computed per element in the same order). */
#define K2Q_TILE_AUTO (-1)
#define K2Q_TILE_256x256 0
#define K2Q_TILE_256x320 1
#define K2Q_TILE_192x256 2
#define K2Q_TILE_128x128 3
#define K2Q_TILE_GEMV 4      /* M <= K2Q_GEMV_MAX_M: the GEMV, no tiles */

/* The schedule k2q_gemm_w8a8 (and the W8 GEMM of k2q_linear_fwd) takes for an M x N x K problem on a GPU with
 * `cus` compute units: returns the K2Q_TILE_* shape (or K2Q_TILE_GEMV), and in *split_pieces (nullable) the
 * number of K-pieces its last round of 256x256 tiles is cut into (1 = none).  grouped != 0: the schedule of
 * k2q_gemm_w8a8_grouped with N the segments' total out_features.  Host only: no device call. */
int k2q_gemm_w8a8_plan(int64_t M, int64_t N, int64_t K, int cus, int grouped, int* split_pieces);

/* Debug entries: raw int32 accumulators acc[m,n] = sum_k qx[m,k] qw[n,k] (W8), and for W4 the f32
 * value sum_g sw4[n,g] * acc_g[m,n] without s_x, 2^-7, bias or LoRA.  k2q_gemm_w8a8_tile is k2q_gemm_w8a8
 * with the tile shape given (M <= 8 runs the GEMV whatever the shape). */
int k2q_gemm_w8a8_acc(const int8_t* qx, const int8_t* qw, int64_t M, int64_t N, int64_t K,
                      int32_t* acc, void* ws, int64_t ws_bytes, int tile, void* stream);   /* ws as k2q_gemm_w8a8 */
int k2q_gemm_w8a8_tile(const int8_t* qx, const float* sx, const int8_t* qw, const float* sw, const float* bias,
                       const float* u, const float* lora_b, int64_t r, float lora_scale,
                       int64_t M, int64_t N, int64_t K, uint16_t* y, void* ws, int64_t ws_bytes, int tile,
                       void* stream);
int k2q_gemm_w4a8_f32(const int8_t* qx, const uint8_t* qw4, const uint16_t* sw4,
                      int64_t M, int64_t N, int64_t K, float* out, void* stream);

/* (4) Input gradient through the frozen base (autograd of quantize.py:51 + lora.py:47-48):
 *   dx = bf16(2^-7 (dy W_hat) R + g A),   W_hat[n,k] = s_w[n] q[n,k] (or s_w4[n,k/64] q4[n,k]).
 * Two equivalent routes (same bar, different rounding points):
 * - k2q_dx_prep_eff writes wt = bf16(2^-7 W_hat R)^T (K x N), the effective weight of the straight-through
 *   forward with the rotation folded in, and k2q_gemm_dx_lin(dy, wt, ...) is then the whole gradient
 *   (the route the module's backward takes); for int8 codes each element is the exact product rounded once
 *   to f32 and once to bf16;
 * - k2q_dx_prep writes wt = bf16(W_hat)^T and k2q_gemm_dx applies the inverse rotation in its epilogue.
 * g = lora_scale * dy @ lora_b (M x r f32) is supplied by the caller, lora_a is the module's A (r x K
 * f32, lora.py:39); both nullable.  ws: as for k2q_gemm_w8a8 (f32 pieces, added in a fixed order),
 * k2q_gemm_dx_ws_bytes(M, N, K) bytes, for either GEMM. */
int k2q_dx_prep_eff(const int8_t* qw, const float* sw, const uint8_t* qw4, const uint16_t* sw4,
                    int64_t N, int64_t K, uint16_t* wt, void* stream);
int k2q_dx_prep(const int8_t* qw, const float* sw, const uint8_t* qw4, const uint16_t* sw4,
                int64_t N, int64_t K, uint16_t* wt, void* stream);
int64_t k2q_gemm_dx_ws_bytes(int64_t M, int64_t N, int64_t K);
int k2q_gemm_dx(const uint16_t* dy, const uint16_t* wt, int64_t M, int64_t N, int64_t K,
                const float* g, const float* lora_a, int64_t r, uint16_t* dx, void* ws, int64_t ws_bytes,
                void* stream);

/* fp8-e4m3 weight-only base, the reference's Fp8Linear (quantize.py:23-51).
 * k2q_quant_weight_fp8 replaces Fp8Linear.__init__ (quantize.py:34-37): s = max(amax_k |w[n,k]|, 1e-8) / 448,
 * q[n,k] = e4m3(clamp(w / s, +-448)) (round to nearest even), s written as bf16 bits.
 * k2q_dequant_fp8 replaces `weight_fp8.to(bf16) * scale.to(bf16)` (quantize.py:49): out = bf16(q * s), N x K,
 * or its transpose (K x N, for the input gradient) when transpose != 0.  K % 64 == 0.
 * k2q_gemm_bf16 replaces F.linear(x, w, b) (quantize.py:51) plus the LoRA add (lora.py:47-48):
 * y = bf16(x w^T + bias + LoRA), LoRA as in k2q_gemm_w8a8; bf16 MFMA with f32 accumulation.
 * k2q_gemm_dx_lin: dx = bf16(dy w + g A) (w given transposed, K x N; lora_a = A, r x K), the autograd of
 * the same. */
int k2q_quant_weight_fp8(const void* w, int w_dtype, int64_t N, int64_t K, uint8_t* q, uint16_t* s, void* stream);
int k2q_dequant_fp8(const uint8_t* q, const uint16_t* s, int64_t N, int64_t K, int transpose, uint16_t* out,
                    void* stream);
int64_t k2q_gemm_bf16_ws_bytes(int64_t M, int64_t N, int64_t K);
int k2q_gemm_bf16(const uint16_t* x, const uint16_t* w, const float* bias, const float* u, const float* lora_b,
                  int64_t r, float lora_scale, int64_t M, int64_t N, int64_t K, uint16_t* y, void* ws,
                  int64_t ws_bytes, void* stream);
int k2q_gemm_dx_lin(const uint16_t* dy, const uint16_t* wt, int64_t M, int64_t N, int64_t K, const float* g,
                    const float* lora_a, int64_t r, uint16_t* dx, void* ws, int64_t ws_bytes, void* stream);

/* Grouped input gradient: the linears that read one input (wq/wk/wv/gate of Attention.forward, mmdit.py:199;
 * gate/up of SwiGLU.forward, mmdit.py:178), whose input gradients autograd would add at the shared input, as
 * one GEMM whose reduction runs over the segments in turn:
 *   dx = bf16(sum_i dy_i wt_i^T + g A),
 * segment i the gradient dy_i of linear i's output (M x N_i bf16, rows of ldy_i elements) and its effective
 * weight wt_i (K x N_i bf16 from k2q_dx_prep_eff, row stride N_i); g (M x r f32, rows of ldg) and lora_a
 * (r x K f32) the members' LoRA terms stacked along the rank (nullable).  1 <= nseg <= 4, every N_i a
 * multiple of 64, ldy_i a multiple of 8, K % 64 == 0.  One f32 sum per output element, rounded once
 * (separate k2q_gemm_dx_lin calls round each member's dx to bf16 before autograd adds them). */
typedef struct {
  const uint16_t* dy;     /* M x N bf16, row stride ldy */
  int64_t ldy;
  const uint16_t* wt;     /* K x N bf16, row stride N */
  int64_t N;
} k2q_dx_segment;
int k2q_gemm_dx_grouped(const k2q_dx_segment* seg, int64_t nseg, int64_t M, int64_t K, const float* g, int64_t ldg,
                        const float* lora_a, int64_t r, uint16_t* dx, void* stream);


#ifdef __cplusplus
}
#endif

#endif /* K2Q_H */
