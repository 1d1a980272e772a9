"""CPU restatement of the ConvRot QuantLinear + LoRA arithmetic — TEST INFRASTRUCTURE ONLY.

Never imported by the product package.  Used by ``tests/`` as the parity checker, by ``__graft_entry__.smoke``
and by ``bench.py``'s ``cpu_baseline`` leg.

Sources restated
----------------
* The reference's quantized base is ``Fp8Linear`` (reference ``quantize.py:23-51``): per-output-row absmax
  scale floored at 1e-8 (``quantize.py:36``), codes clamped and cast (``quantize.py:37``), dequantized
  ``W_q * scale`` then ``F.linear`` (``quantize.py:48-51``).  :func:`fp8_weight_quant` /
  :func:`fp8_linear` restate it.
* The ConvRot arithmetic (block Walsh-Hadamard rotation, per-token int8 activations, int8 per-channel or
  int4 group-64 weights) has no code in the reference; its only specification is ``BASELINE.json``
  ``north_star``.  This module fixes every arithmetic choice the kernels must reproduce bit-for-bit:

  - FWHT over each 128-wide block of the last axis, float32, unnormalised (entries +-1), radix-2 butterfly,
    stage strides 1, 2, 4, ..., 64 in that order, pair ``(i, i+s)`` inside each ``2s`` chunk becomes
    ``(a+b, a-b)``.
  - Per-row absmax over the whole rotated row, floored at 1e-8 (mirrors ``quantize.py:36``),
    ``inv = 127/absmax`` (one correctly rounded float32 division), ``q = clamp(rint(v*inv), -127, 127)``
    with round-half-to-even, ``s = absmax/127`` (float32 division).
  - int4 weights: per (row, 64-wide group) absmax floored at 1e-8, ``s = bf16(absmax/7)`` (RNE),
    ``q = clamp(rint(v / float(s)), -7, 7)``; the bf16 scale is both the quantizer's and the dequantizer's.
  - int4 packing: inside every 16-wide chunk of K, byte ``j`` (0..7) holds code ``j`` in its low nibble and
    code ``j+8`` in its high nibble, two's complement.
  - GEMM accumulators are exact integers (int32 range is checked).
  - LoRA follows ``lora.py:43-48``: ``out + (scale*scale_mul) * ((x.f32 @ A^T) @ B^T)``.

Float outputs that the kernels are held to a tolerance on (the bf16 ``y`` and ``dX``) are computed here in
float64 from the exact integer accumulators and then rounded once to bf16.
"""
from __future__ import annotations

import math

import numpy as np

HADAMARD_BLOCK = 128
INT8_QMAX = 127
INT4_QMAX = 7
INT4_GROUP = 64
ABSMAX_FLOOR = np.float32(1e-8)      # quantize.py:36 clamp(min=1e-8)
INV_SQRT_BLOCK = np.float32(1.0 / math.sqrt(HADAMARD_BLOCK))
E4M3_MAX = 448.0                     # quantize.py:20


# ----------------------------------------------------------------------------------------------------------
# bf16 helpers (round-to-nearest-even, the rounding of torch's .to(bfloat16) and of the kernels' stores)
# ----------------------------------------------------------------------------------------------------------
def bf16_bits(a) -> np.ndarray:
    """float32 array -> uint16 bf16 bit patterns, round half to even, NaN kept quiet."""
    f = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = f.view(np.uint32)
    # no overflow for finite/inf inputs: u + 0x8000 < 2^32 whenever u <= 0xFF800000
    rounded = ((u + (np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)))) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        rounded[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return rounded


def bf16_to_f32(bits) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 values (exact)."""
    b = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16))
    return (b.astype(np.uint32) << 16).view(np.float32)


def bf16_round(a) -> np.ndarray:
    """Round float32 values to the nearest bf16 value (returned as float32)."""
    return bf16_to_f32(bf16_bits(a))


# ----------------------------------------------------------------------------------------------------------
# Rotation
# ----------------------------------------------------------------------------------------------------------
def fwht_blocks(v, block: int = HADAMARD_BLOCK) -> np.ndarray:
    """Unnormalised block-diagonal Walsh-Hadamard transform of the last axis, float32 butterfly.

    Spec: north_star "block-diagonal Walsh-Hadamard rotation of bf16 activations", block 128.  Stage order
    and pairing are fixed here (module docstring) because every stage rounds.
    """
    v = np.array(v, dtype=np.float32, copy=True)
    K = v.shape[-1]
    if K % block:
        raise ValueError(f"last dim {K} is not a multiple of {block}")
    lead = v.shape[:-1]
    s = 1
    while s < block:
        w = v.reshape(*lead, K // (2 * s), 2, s)
        a = w[..., 0, :]
        b = w[..., 1, :]
        v = np.stack((a + b, a - b), axis=-2).reshape(*lead, K)
        s *= 2
    return v


def fwht_blocks_f64(v, block: int = HADAMARD_BLOCK) -> np.ndarray:
    """The same transform in float64 (used where the kernels are held to a tolerance)."""
    v = np.array(v, dtype=np.float64, copy=True)
    K = v.shape[-1]
    lead = v.shape[:-1]
    s = 1
    while s < block:
        w = v.reshape(*lead, K // (2 * s), 2, s)
        v = np.stack((w[..., 0, :] + w[..., 1, :], w[..., 0, :] - w[..., 1, :]), axis=-2).reshape(*lead, K)
        s *= 2
    return v


# ----------------------------------------------------------------------------------------------------------
# Per-row int8 rotate + quantize (kernel 1; also the int8 weight quantizer, applied to W's rows)
# ----------------------------------------------------------------------------------------------------------
def rotquant(x, want_xrot: bool = False):
    """Rotate each 128-block of every row, then quantize the row to int8 with one float32 scale.

    Returns ``(q int8 (M,K), s float32 (M,), xrot_bits uint16 (M,K) or None)``.  ``xrot`` is
    ``bf16(v * float32(1/sqrt(128)))``, the normalised rotation.  Spec: north_star (1); the absmax floor
    mirrors ``quantize.py:36``.
    """
    v = fwht_blocks(x)
    absmax = np.max(np.abs(v), axis=-1)
    absmax = np.maximum(absmax, ABSMAX_FLOOR).astype(np.float32)
    inv = (np.float32(INT8_QMAX) / absmax).astype(np.float32)
    q = np.clip(np.rint(v * inv[..., None]), -INT8_QMAX, INT8_QMAX).astype(np.int8)
    s = (absmax / np.float32(INT8_QMAX)).astype(np.float32)
    xrot = bf16_bits(v * INV_SQRT_BLOCK) if want_xrot else None
    return q, s, xrot


def quant_weight_i8(w):
    """int8 symmetric per-output-channel weight quantization of the rotated weight ``W R``.

    Counterpart of ``Fp8Linear.__init__`` (``quantize.py:34-37``) with the rotation of the north_star.
    Returns ``(q int8 (N,K), s float32 (N,))``.
    """
    q, s, _ = rotquant(w)
    return q, s


def quant_weight_i4(w, group: int = INT4_GROUP):
    """int4 symmetric group-wise quantization of ``W R``: one bf16 scale per (row, 64-wide K group).

    Returns ``(q int8 codes in [-7,7] (N,K), s_bits uint16 bf16 (N, K//group))``.  Spec: north_star
    "packed group-wise int4 weights with per-group scales", BASELINE.json configs[1].
    """
    v = fwht_blocks(w)
    N, K = v.shape
    if K % group:
        raise ValueError(f"K={K} is not a multiple of the int4 group {group}")
    vg = v.reshape(N, K // group, group)
    absmax = np.maximum(np.max(np.abs(vg), axis=-1), ABSMAX_FLOOR).astype(np.float32)
    s_bits = bf16_bits(absmax / np.float32(INT4_QMAX))
    s = bf16_to_f32(s_bits)
    q = np.clip(np.rint(vg / s[..., None]), -INT4_QMAX, INT4_QMAX).astype(np.int8).reshape(N, K)
    return q, s_bits


def pack_i4(q) -> np.ndarray:
    """Pack int4 codes (N,K) into (N,K/2) bytes: in each 16-wide chunk, byte j = code j | code j+8 << 4."""
    q = np.asarray(q, dtype=np.int8)
    N, K = q.shape
    if K % 16:
        raise ValueError("K must be a multiple of 16 for int4 packing")
    c = q.reshape(N, K // 16, 2, 8).astype(np.uint8) & 0x0F
    return (c[:, :, 0, :] | (c[:, :, 1, :] << 4)).reshape(N, K // 2).astype(np.uint8)


def unpack_i4(p) -> np.ndarray:
    """Inverse of :func:`pack_i4`."""
    p = np.asarray(p, dtype=np.uint8)
    N, H = p.shape
    b = p.reshape(N, H // 8, 8)
    lo = (b & 0x0F).astype(np.int16)
    hi = (b >> 4).astype(np.int16)
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    return np.concatenate((lo, hi), axis=-1).reshape(N, H * 2).astype(np.int8)


# ----------------------------------------------------------------------------------------------------------
# Integer GEMM (kernel 2) and the fused epilogue (kernel 3)
# ----------------------------------------------------------------------------------------------------------
def gemm_acc(qx, qw) -> np.ndarray:
    """Exact ``acc[m,n] = sum_k qx[m,k] * qw[n,k]`` as int32 (north_star (2): int32 accumulation)."""
    a = np.asarray(qx, dtype=np.int64) @ np.asarray(qw, dtype=np.int64).T
    if np.abs(a).max(initial=0) >= 2 ** 31:
        raise OverflowError("accumulator exceeds int32")
    return a.astype(np.int32)


def gemm_acc_fast(qx, qw) -> np.ndarray:
    """The same exact int32 accumulators through ``torch._int_mm`` (oneDNN int8 GEMM, int32 accumulate) —
    used where the oracle runs at benchmark sizes.  Equal to :func:`gemm_acc` bit for bit."""
    import torch
    a = torch.from_numpy(np.ascontiguousarray(qx, dtype=np.int8))
    b = torch.from_numpy(np.ascontiguousarray(np.asarray(qw, dtype=np.int8).T))
    return torch._int_mm(a, b).numpy()


def gemm_acc_groups(qx, qw, group: int = INT4_GROUP) -> np.ndarray:
    """Exact per-group partials ``acc[m,n,g] = sum_{k in g} qx[m,k] * qw[n,k]`` (int64)."""
    qx = np.asarray(qx, dtype=np.int64)
    qw = np.asarray(qw, dtype=np.int64)
    M, K = qx.shape
    N = qw.shape[0]
    G = K // group
    return np.einsum("mgk,ngk->mng", qx.reshape(M, G, group), qw.reshape(N, G, group))


def lora_down(x, A) -> np.ndarray:
    """``u = x.f32 @ A^T`` (``lora.py:47``), in float64."""
    return np.asarray(x, dtype=np.float64) @ np.asarray(A, dtype=np.float64).T


def forward(x, wq, ws, *, w4: bool = False, bias=None, lora_A=None, lora_B=None, lora_scale: float = 0.0,
            fast: bool = False):
    """ConvRot QuantLinear (+ LoRA) forward.  Returns a dict of every intermediate.

    ``x`` float32 (M,K) holding bf16 (or float32) values.  ``fast`` computes the W8 accumulators with
    :func:`gemm_acc_fast` (same integers).  ``wq``/``ws`` as returned by
    :func:`quant_weight_i8` (float32 per-row scale) or, with ``w4=True``, the int4 codes (unpacked) and the
    bf16 group-scale bits of :func:`quant_weight_i4`.  Epilogue (north_star (3)):
    ``y = bf16(2^-7 * s_x[m] * (s_w[n]*acc | sum_g s_w[n,g]*acc_g) + bias[n] + lora_scale * u @ B^T)``;
    the LoRA term is ``lora.py:47-48`` with ``lora_scale = scale * scale_mul``.
    """
    qx, sx, _ = rotquant(x)
    out = {"qx": qx, "sx": sx}
    if w4:
        accg = gemm_acc_groups(qx, wq)
        sg = bf16_to_f32(ws).astype(np.float64)
        base = np.einsum("mng,ng->mn", accg.astype(np.float64), sg)
        out["acc_groups"] = accg
    else:
        acc = gemm_acc_fast(qx, wq) if fast else gemm_acc(qx, wq)
        base = acc.astype(np.float64) * np.asarray(ws, dtype=np.float64)[None, :]
        out["acc"] = acc
    y = base * (2.0 ** -7) * sx.astype(np.float64)[:, None]
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)[None, :]
    if lora_A is not None and lora_scale != 0.0:
        u = lora_down(x, lora_A)
        out["u"] = u
        y = y + lora_scale * (u @ np.asarray(lora_B, dtype=np.float64).T)
    out["y64"] = y
    out["y"] = bf16_bits(y.astype(np.float32))
    return out


def dequant_weight(wq, ws, *, w4: bool = False, group: int = INT4_GROUP) -> np.ndarray:
    """``W_hat[n,k]`` in float64 (rotated domain): ``s_w[n]*q[n,k]`` or ``s_w[n,k//64]*q[n,k]``."""
    q = np.asarray(wq, dtype=np.float64)
    if w4:
        s = bf16_to_f32(ws).astype(np.float64)
        return q * np.repeat(s, group, axis=1)
    return q * np.asarray(ws, dtype=np.float64)[:, None]


def backward(dy, x, wq, ws, *, w4: bool = False, lora_A=None, lora_B=None, lora_scale: float = 0.0):
    """Input gradient through the frozen base plus the LoRA grads (north_star (4); autograd of
    ``lora.py:47-48``).

    Straight-through estimator over both quantizers: ``y = 2^-7 (x R) W_hat^T`` so
    ``dX = 2^-7 (dY W_hat) R`` (R is symmetric).  LoRA with ``g = lora_scale * dY @ B``:
    ``dX += g @ A``, ``dA = g^T x``, ``dB = lora_scale * dY^T u``.  float64 throughout.
    """
    dy = np.asarray(dy, dtype=np.float64)
    wh = dequant_weight(wq, ws, w4=w4)
    dx = fwht_blocks_f64(dy @ wh) * (2.0 ** -7)
    out = {"dx_base": dx}
    if lora_A is not None and lora_scale != 0.0:
        A = np.asarray(lora_A, dtype=np.float64)
        B = np.asarray(lora_B, dtype=np.float64)
        x64 = np.asarray(x, dtype=np.float64)
        u = x64 @ A.T
        g = lora_scale * (dy @ B)
        dx = dx + g @ A
        out["g"] = g
        out["dA"] = g.T @ x64
        out["dB"] = lora_scale * (dy.T @ u)
    out["dx64"] = dx
    out["dx"] = bf16_bits(dx.astype(np.float32))
    return out


# ----------------------------------------------------------------------------------------------------------
# The reference's own quantized base: fp8 e4m3 weight-only (quantize.py:33-51)
# ----------------------------------------------------------------------------------------------------------
def fp8_weight_quant(w):
    """``Fp8Linear.__init__`` (``quantize.py:34-39``): returns ``(codes float8_e4m3fn torch tensor,
    scale bf16 torch tensor (N,1))``.  Uses torch's CPU e4m3 cast, the one the reference calls."""
    import torch
    wt = torch.as_tensor(np.asarray(w, dtype=np.float32))
    scale = wt.abs().amax(dim=1, keepdim=True).clamp(min=1e-8) / E4M3_MAX
    wq = (wt / scale).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return wq, scale.to(torch.bfloat16)


def fp8_linear(x_bf16, wq, scale_bf16, bias=None):
    """``Fp8Linear.forward`` (``quantize.py:48-51``) on the CPU: bf16 dequant then ``F.linear``."""
    import torch
    import torch.nn.functional as F
    w = wq.to(torch.bfloat16) * scale_bf16.to(torch.bfloat16)
    b = bias.to(torch.bfloat16) if bias is not None else None
    return F.linear(x_bf16, w, b)


# ----------------------------------------------------------------------------------------------------------
# Producers of the quantized linears' inputs (fused into rotate/quant by the kernels)
# ----------------------------------------------------------------------------------------------------------
def _sigmoid_f32(g) -> np.ndarray:
    g = np.asarray(g, dtype=np.float32)
    with np.errstate(over="ignore"):
        return np.float32(1.0) / (np.float32(1.0) + np.exp(-g))


def swiglu(g, u) -> np.ndarray:
    """``F.silu(self.gate(x)) * self.up(x)`` of ``SwiGLU.forward`` (reference ``mmdit.py:177-178``) on bf16
    tensors: ``F.silu`` computes ``g / (1 + exp(-g))`` in float32 and returns bf16, the product rounds to bf16
    again.  ``g``, ``u`` float32 arrays holding bf16 values; returns float32 holding the bf16 result ``h``."""
    g = np.asarray(g, dtype=np.float32)
    u = np.asarray(u, dtype=np.float32)
    with np.errstate(over="ignore"):
        s = bf16_round(g / (np.float32(1.0) + np.exp(-g)))
    return bf16_round(s * u)


def swiglu_backward(dh, g, u):
    """Autograd of :func:`swiglu` with the reference's eager bf16 roundings: the product's backward gives
    ``du = bf16(dh * s)`` and ``ds = bf16(dh * u)`` (``s = bf16(silu(g))``), and silu's backward gives
    ``dg = bf16((ds * sig) * (1 + g (1 - sig)))`` with ``sig = 1 / (1 + exp(-g))`` in float32 — the
    derivative of ``g * sig(g)``.  Returns ``(dg, du)`` as float32 holding bf16 values."""
    dh = np.asarray(dh, dtype=np.float32)
    g = np.asarray(g, dtype=np.float32)
    u = np.asarray(u, dtype=np.float32)
    sig = _sigmoid_f32(g)
    with np.errstate(over="ignore"):
        s = bf16_round(g / (np.float32(1.0) + np.exp(-g)))
    du = bf16_round(dh * s)
    ds = bf16_round(dh * u)
    dg = bf16_round((ds * sig) * (np.float32(1.0) + g * (np.float32(1.0) - sig)))
    return dg, du


def rmsmod(x, norm_scale, eps: float, mod_scale, mod_shift, rows_per_batch: int) -> np.ndarray:
    """The modulated RMSNorm that feeds ``attn`` and ``mlp`` in ``SingleStreamBlock.forward`` (reference
    ``mmdit.py:314-317``), with ``RMSNorm.forward`` (``mmdit.py:156-161``):

    ``n = bf16((x * rsqrt(mean(x^2) + eps)) * (scale + 1))`` in float32 over the whole row (``F.rms_norm`` on
    ``x.float()`` with weight ``scale.float() + 1``, then ``.to(x.dtype)``), and
    ``h = bf16(bf16(bf16(1 + p) * n) + b)`` — each eager bf16 op rounds — with ``p``, ``b`` the modulation
    scale / shift entry of the row's batch (``row // rows_per_batch``; one entry for every row when there
    is one).  ``x`` float32 (M,K) holding bf16 values, ``norm_scale`` float32 (K,), ``mod_scale`` /
    ``mod_shift`` float32 (B,K) holding bf16 values.  Returns float32 holding the bf16 result ``h``."""
    x = np.asarray(x, dtype=np.float32)
    M, K = x.shape
    w1 = np.asarray(norm_scale, dtype=np.float32) + np.float32(1.0)
    ms = np.asarray(mod_scale, dtype=np.float32).reshape(-1, K)
    mb = np.asarray(mod_shift, dtype=np.float32).reshape(-1, K)
    b = np.zeros(M, dtype=np.int64) if ms.shape[0] == 1 else np.arange(M) // int(rows_per_batch)
    mean = np.sum(x * x, axis=1, dtype=np.float32) / np.float32(K)
    r = np.float32(1.0) / np.sqrt(mean + np.float32(eps))
    n = bf16_round((x * r[:, None]) * w1[None, :])
    p1 = bf16_round(np.float32(1.0) + ms[b])
    return bf16_round(bf16_round(p1 * n) + mb[b])


def rmsmod_backward_x(dh, x, norm_scale, eps: float, mod_scale, rows_per_batch: int) -> np.ndarray:
    """The input gradient of :func:`rmsmod` for ``x`` under the reference's eager ops: the modulation's
    product backward rounds ``dn = bf16(dh * bf16(1 + p))`` (bf16 tensors), the cast ``.to(x.dtype)`` passes it
    to float32, and ``F.rms_norm``'s backward (``mmdit.py:158-160``) with ``g = dn * (scale + 1)`` is
    ``dx = g r - x (r^3 / K) sum_k(g x)``, ``r = rsqrt(mean(x^2) + eps)``, rounded to bf16 at the end.
    Evaluated in float64 here (the kernels' float32 differs by rounding only)."""
    x = np.asarray(x, dtype=np.float32)
    M, K = x.shape
    dh = np.asarray(dh, dtype=np.float32)
    ms = np.asarray(mod_scale, dtype=np.float32).reshape(-1, K)
    b = np.zeros(M, dtype=np.int64) if ms.shape[0] == 1 else np.arange(M) // int(rows_per_batch)
    p1 = bf16_round(np.float32(1.0) + ms[b])
    g = bf16_round(dh * p1).astype(np.float64) * (np.asarray(norm_scale, np.float32) + np.float32(1.0))[None, :]
    x64 = x.astype(np.float64)
    r = 1.0 / np.sqrt((x64 * x64).mean(axis=1) + eps)
    dot = (g * x64).sum(axis=1)
    dx = g * r[:, None] - x64 * (r ** 3 * dot / K)[:, None]
    return bf16_round(dx.astype(np.float32))
