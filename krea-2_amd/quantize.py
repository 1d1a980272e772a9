"""ConvRot quantized frozen base: the drop-in counterpart of the reference's ``Fp8Linear``.

Reference interface followed (``quantize.py:23-68``): built from an existing ``nn.Linear``
(``quantize.py:33``), class attribute ``is_quant_linear = True`` (``:31``, checked by ``lora.py:100,107``),
``in_features`` / ``out_features`` (``:42``), a ``weight`` property used only as a device probe (``:44-46``),
``bias`` Parameter or None (``:40-41``), every tensor an ``nn.Parameter(requires_grad=False)`` so block swap
pages it (``mmdit.py:409-414``), and a walker that replaces the Linears of ``dit.blocks`` and returns the count
(``quantize.py:54-68``).

What differs is the arithmetic: activations are rotated by a block Walsh-Hadamard
transform and quantized per token to int8 on the fly; weights are stored rotated and quantized, int8 per output
channel (``w8a8``) or packed int4 with one bf16 scale per 64-wide group (``w4a8``); the GEMM runs on int8
MFMA with int32 accumulation.  All of it runs in the HIP library ``libk2q.so``; nothing here computes on the
CPU.  Scales are stored as integer bit patterns (f32 bits in int32, bf16 bits in int16) so that
``Module.to(dtype)`` — which casts floating Parameters — leaves them exact.
"""
from __future__ import annotations

import weakref

import torch
import torch.nn as nn

from . import _lib

MODES = ("w8a8", "w4a8")


class _SharedInputQuant:
    """The last activation's int8 codes and scales, reused when the next ConvRot layer receives the very same
    tensor: the DiT feeds one tensor to ``wq/wk/wv/gate`` (``mmdit.py:199``) and another to ``mlp.gate/up``
    (``mmdit.py:178``), so the rotation + quantization runs once per input instead of 4 / 2 times.

    A hit needs the same tensor object (held by weak reference, so a freed tensor never matches), the same
    version counter (any in-place write bumps it), data pointer, shape, strides and CUDA stream.  The
    codes are a pure function of the input, so a hit returns exactly what a fresh call would."""

    enabled = True

    def __init__(self):
        self.ref = None
        self.key = None
        self.val = None
        self.misses = 0

    @staticmethod
    def _key(x: torch.Tensor):
        return (x._version, x.data_ptr(), tuple(x.shape), tuple(x.stride()), x.device, _lib._stream(x.device))

    def lookup(self, x: torch.Tensor, x2: torch.Tensor):
        key = self._key(x)
        if self.enabled and self.ref is not None and self.ref() is x and self.key == key:
            return self.val
        self.misses += 1
        qx, sx, _ = _lib.rotquant(x2)
        if self.enabled:
            self.ref, self.key, self.val = weakref.ref(x), key, (qx, sx)
        return qx, sx

    def find(self, x: torch.Tensor):
        """``(key, codes)``: the codes kept for exactly this tensor, or None; the key goes back to :meth:`keep`."""
        key = self._key(x)
        if self.enabled and self.ref is not None and self.ref() is x and self.key == key:
            return key, self.val
        self.misses += 1
        return key, None

    def keep(self, x: torch.Tensor, key, qx: torch.Tensor, sx: torch.Tensor) -> None:
        """Record the codes a fused forward wrote for ``x`` (``key`` from :meth:`find`, taken before that call)."""
        if self.enabled:
            self.ref, self.key, self.val = weakref.ref(x), key, (qx, sx)

    def clear(self) -> None:
        """Forget the kept codes (their memory returns to the allocator)."""
        self.ref = self.key = self.val = None

    def seed(self, x: torch.Tensor, qx: torch.Tensor, sx: torch.Tensor) -> None:
        """Record codes a producer-fused kernel computed for ``x`` (exactly those ``rotquant`` gives), so the
        ConvRot layers that receive ``x`` next skip their own rotate/quant."""
        if self.enabled:
            self.ref, self.key, self.val = weakref.ref(x), self._key(x), (qx, sx)


shared_input_quant = _SharedInputQuant()


def _check_out_features(N: int) -> None:
    """The input-gradient GEMM reads dY in 64-column steps, so a layer that trains through its backward needs
    ``out_features % 64 == 0`` (every Krea 2 linear has it); reject others when the layer is built, not in the
    middle of a training step."""
    if N < 64 or N % 64:
        raise ValueError(f"out_features={N} must be a positive multiple of 64 (the input-gradient GEMM's step)")


class _ConvRotLinearFn(torch.autograd.Function):
    """Forward: one library call (``k2q_linear_fwd``): rotate+quantize x (unless its codes are given), LoRA
    down-projection, fused GEMM + epilogue.
    Backward (straight-through over both quantizers): ``dX = 2^-7 (dY W_hat) R + g A`` with
    ``g = s dY B``; ``dA = g^T x``, ``dB = s dY^T u`` — the autograd of ``lora.py:47-48`` through a frozen base.
    Deterministic (no atomics, fixed reduction order), so checkpoint recompute reproduces the forward."""

    @staticmethod
    def forward(ctx, x2, lora_A, lora_B, qweight, wscale, bias, w4, lora_scale, qx, sx, codes_ready, owner):
        y, u = _lib.linear_fwd(x2, qx, sx, codes_ready, lora_A, lora_B, lora_scale, qweight, wscale, bias, w4)
        ctx.w4 = w4
        ctx.lora_scale = lora_scale
        ctx.owner = owner
        ctx.save_for_backward(x2 if lora_A is not None else None, u, lora_A, lora_B, qweight, wscale)
        return y

    @staticmethod
    def backward(ctx, dy):
        x2, u, A, B, qweight, wscale = ctx.saved_tensors
        dy = dy.contiguous()
        if dy.dtype != torch.bfloat16:
            dy = dy.to(torch.bfloat16)
        g = dA = dB = None
        if A is not None:
            g, dA, dB = _lib.lora_grads(dy, x2 if ctx.needs_input_grad[1] else None,
                                        u if ctx.needs_input_grad[2] else None, B, ctx.lora_scale)
        dx = None
        if ctx.needs_input_grad[0]:
            dx = _lib.gemm_dx(dy, qweight, wscale, w4=ctx.w4, g=g, lora_a=A if g is not None else None,
                              wt=ctx.owner.dx_weight())
        return dx, dA, dB, None, None, None, None, None, None, None, None, None


class ConvRotLinear(nn.Module):
    """Frozen ``nn.Linear`` with the ConvRot W8A8 / W4A8 base, computed by gfx950 HIP kernels.

    ``y = bf16(2^-7 s_x[m] s_w[n] (q_x q_w^T)[m,n] + bias[n])`` with ``q_x`` the per-token int8 codes of
    ``x R`` and ``q_w`` the codes of ``W R`` (R = blockdiag of 128x128 +-1 Hadamards).  Exposes
    ``in_features`` / ``out_features`` / ``weight`` / ``bias`` so it drops in as a ``LoRALinear`` base.
    """

    is_quant_linear = True

    def __init__(self, lin: nn.Linear | None = None, mode: str = "w8a8"):
        super().__init__()
        if mode not in MODES:
            raise ValueError(f"mode must be one of {MODES}, got {mode!r}")
        self.mode = mode
        self.keep_dx_weight = False   # build the backward's effective weight per call (see dx_weight)
        self._dx_kept = None          # (source key, effective weight) while the cache is on: not a parameter
        if lin is None:  # filled by from_quantized
            return
        w = lin.weight.data
        N, K = w.shape
        _lib._check_k(K)
        _check_out_features(N)
        home = w.device
        if home.type != "cuda":
            if not torch.cuda.is_available():
                raise RuntimeError("ConvRotLinear quantizes on the GPU (libk2q, gfx950); no GPU is available")
            w = w.to("cuda")
        w = w.contiguous()
        if w.dtype not in (torch.bfloat16, torch.float32):
            w = w.float()
        if mode == "w8a8":
            q, s = _lib.quant_weight_i8(w)
            s_bits = s.view(torch.int32)
        else:
            q, s4 = _lib.quant_weight_i4(w)
            s_bits = s4.view(torch.int16)
        self.qweight = nn.Parameter(q.to(home), requires_grad=False)
        self.wscale = nn.Parameter(s_bits.to(home), requires_grad=False)
        self.bias = (nn.Parameter(lin.bias.data.clone(), requires_grad=False)
                     if lin.bias is not None else None)
        self.in_features, self.out_features = K, N

    @classmethod
    def from_quantized(cls, qweight: torch.Tensor, wscale_bits: torch.Tensor, bias: torch.Tensor | None,
                       mode: str = "w8a8") -> "ConvRotLinear":
        """Wrap already-quantized tensors (e.g. loaded from disk): ``qweight`` int8 (N,K) with ``wscale_bits``
        int32 (N,) f32 bits, or uint8 (N,K/2) packed int4 with int16 (K/64,N) bf16 bits."""
        m = cls(None, mode)
        if mode == "w8a8":
            if qweight.dtype != torch.int8 or wscale_bits.dtype != torch.int32:
                raise ValueError("w8a8 expects int8 codes and int32 scale bits")
            N, K = qweight.shape
            if wscale_bits.shape != (N,):
                raise ValueError("w8a8 scale bits must be (N,)")
        else:
            if qweight.dtype != torch.uint8 or wscale_bits.dtype != torch.int16:
                raise ValueError("w4a8 expects uint8 packed codes and int16 bf16 scale bits")
            N, K = qweight.shape[0], qweight.shape[1] * 2
            if wscale_bits.shape != (K // _lib.INT4_GROUP, N):
                raise ValueError("w4a8 scale bits must be (K/64, N)")
        _lib._check_k(K)
        _check_out_features(N)
        m.qweight = nn.Parameter(qweight, requires_grad=False)
        m.wscale = nn.Parameter(wscale_bits, requires_grad=False)
        m.bias = nn.Parameter(bias, requires_grad=False) if bias is not None else None
        m.in_features, m.out_features = K, N
        return m

    @property
    def weight(self) -> torch.Tensor:  # device probe for LoRALinear (quantize.py:44-46)
        return self.qweight

    def dx_weight(self) -> torch.Tensor:
        """The effective weight ``bf16(2^-7 W_hat R)^T`` (K x N bf16) that the input-gradient GEMM reads.

        By default every backward builds it (one pass over the codes: 1 byte read and 2 written per weight) and
        lets it go, so the layer holds only its codes and scales: 1 byte per weight resident and paged by block
        swap, as the reference's fp8 base (``quantize.py:8-11``; ``mmdit.py:409-414``).

        With ``keep_dx_weight`` on (:func:`set_dx_weight_cache`) it is built at the first backward and kept,
        trading 2 bytes per weight of HBM (24 GB for Krea 2's 12.2e9 block weights) for that pass.  The kept
        weight is a plain attribute, not a parameter: block swap does not page it and ``state_dict`` does not
        hold it.  It belongs to the codes' current storage (pointer, version, device), so a layer whose codes
        were paged out or re-pointed rebuilds it on its next backward, and every build first releases the
        weights kept for layers whose codes have left the device they were built on (a block paged out by
        block swap keeps nothing resident past the next backward of any layer).  An edit through ``.data``
        that keeps the pointer bumps no version: turn the cache off and on after one."""
        q, s = self.qweight, self.wscale
        if not getattr(self, "keep_dx_weight", False):
            self._dx_kept = None
            return _lib.dx_weight(q, self.weight_scale, w4=self.mode == "w4a8")
        key = _dx_key(self)
        kept = self._dx_kept
        if kept is not None and kept[0] == key:
            return kept[1]
        self._dx_kept = None
        _release_stale_dx_weights()
        wt = _lib.dx_weight(q, self.weight_scale, w4=self.mode == "w4a8")
        self._dx_kept = (key, wt)
        _dx_holders.add(self)
        return wt

    @property
    def dx_weight_kept(self) -> torch.Tensor | None:
        """The effective weight this layer keeps resident now, or None (cache off, or nothing built yet)."""
        kept = self.__dict__.get("_dx_kept")
        return None if kept is None else kept[1]

    @property
    def weight_scale(self) -> torch.Tensor:
        """The scales as floats: f32 (N,) for w8a8, bf16 (K/64, N) for w4a8 (views, no copy)."""
        return self.wscale.view(torch.float32 if self.mode == "w8a8" else torch.bfloat16)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, mode={self.mode}, " \
               f"bias={self.bias is not None}"

    def _bias_f32(self):
        if self.bias is None:
            return None
        b = self.bias
        return b if b.dtype == torch.float32 and b.is_contiguous() else b.float().contiguous()

    def forward_lora(self, x: torch.Tensor, lora_A: torch.Tensor | None, lora_B: torch.Tensor | None,
                     lora_scale: float) -> torch.Tensor:
        """``base(x) + lora_scale * (x.f32 @ A^T) @ B^T`` in one fused pass (``lora.py:47-48``)."""
        if x.shape[-1] != self.in_features:
            raise ValueError(f"x has {x.shape[-1]} features, layer expects {self.in_features}")
        if x.dtype != torch.bfloat16:
            raise NotImplementedError(f"ConvRotLinear runs bf16 activations (the DiT dtype); got {x.dtype}")
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.in_features)
        if not x2.is_contiguous() or x2.data_ptr() % 16:
            x2 = x2.contiguous()
        M = x2.shape[0]
        if M == 0:
            return x.new_empty(*lead, self.out_features)
        key, codes = shared_input_quant.find(x)
        ready = codes is not None
        if ready:
            qx, sx = codes
        else:
            qx = torch.empty((M, self.in_features), dtype=torch.int8, device=x2.device)
            sx = torch.empty((M,), dtype=torch.float32, device=x2.device)
        w4 = self.mode == "w4a8"
        grad = torch.is_grad_enabled() and (x2.requires_grad or (lora_A is not None and
                                                                  (lora_A.requires_grad or lora_B.requires_grad)))
        if grad:
            y = _ConvRotLinearFn.apply(x2, lora_A, lora_B, self.qweight, self.weight_scale, self._bias_f32(), w4,
                                       float(lora_scale), qx, sx, ready, self)
        else:   # nothing to differentiate: no autograd node, the one library call (u stays internal)
            y, _ = _lib.linear_fwd(x2, qx, sx, ready, lora_A, lora_B, float(lora_scale), self.qweight,
                                   self.weight_scale, self._bias_f32(), w4, need_u=False)
        if not ready:
            shared_input_quant.keep(x, key, qx, sx)
        return y.reshape(*lead, self.out_features)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.forward_lora(x, None, None, 0.0)


def quantize_dit_convrot(dit, mode: str = "w8a8") -> int:
    """Replace the transformer blocks' ``nn.Linear`` with :class:`ConvRotLinear` in place.

    Same walk as ``quantize_dit_fp8`` (``quantize.py:54-68``): collect every ``nn.Linear`` child of every
    module in ``dit.blocks`` first, then ``setattr``; the stages outside the blocks stay bf16.  Returns the
    number of layers quantized.  Call BEFORE ``inject_lora`` (the adapters then wrap the quantized bases).
    """
    targets = []
    for block in dit.blocks:
        for mod in block.modules():
            for name, child in mod.named_children():
                if isinstance(child, nn.Linear):
                    targets.append((mod, name, child))
    for mod, name, child in targets:
        setattr(mod, name, ConvRotLinear(child, mode))
    return len(targets)


# layers holding a kept effective weight (weak: a dropped layer takes its weight with it)
_dx_holders: "weakref.WeakSet[ConvRotLinear]" = weakref.WeakSet()


def _dx_key(m: "ConvRotLinear"):
    """What a kept effective weight was built from: the codes' and scales' storage, versions and device."""
    q, s = m.qweight, m.wscale
    return (q.data_ptr(), q._version, s.data_ptr(), s._version, q.device, tuple(q.shape))


def _release_stale_dx_weights() -> None:
    """Drop the effective weights kept for layers whose codes no longer sit where the weight was built (paged
    to the host by block swap, re-pointed, moved to another device, or rewritten in place)."""
    for m in list(_dx_holders):
        kept = m.__dict__.get("_dx_kept")
        if kept is None or kept[0] != _dx_key(m):
            m._dx_kept = None
            _dx_holders.discard(m)


def set_dx_weight_cache(model: nn.Module, enable: bool = True) -> int:
    """Keep or drop (the default) the resident input-gradient weight of every :class:`ConvRotLinear` in
    ``model`` (:meth:`ConvRotLinear.dx_weight`).  On keeps 2 more bytes per weight of HBM beside the 1-byte codes
    and saves one weight pass per backward; off frees the kept weights.  Returns the number of layers set."""
    n = 0
    for m in model.modules():
        if isinstance(m, ConvRotLinear):
            m.keep_dx_weight = bool(enable)
            if not enable:
                m._dx_kept = None
                _dx_holders.discard(m)
            n += 1
    return n


# ----------------------------------------------------------------------------------------------------------
# fp8-e4m3 weight-only base: the reference's own quantized Linear (quantize.py:23-51), on the same kernels
# ----------------------------------------------------------------------------------------------------------
class _Fp8LinearFn(torch.autograd.Function):
    """Forward ``quantize.py:48-51`` (dequantize to bf16, bf16 GEMM with f32 accumulation, bias) with the LoRA
    term of ``lora.py:47-48`` fused; backward ``dX = dY W_deq + g A``, ``dA = g^T x``, ``dB = s dY^T u``."""

    @staticmethod
    def forward(ctx, x2, lora_A, lora_B, q, scale, bias, lora_scale):
        w = _lib.dequant_fp8(q, scale)            # the reference's per-forward bf16 temporary
        u = _lib.lora_down(x2, lora_A) if lora_A is not None else None
        y = _lib.gemm_bf16(x2, w, bias, u, lora_B, lora_scale)
        ctx.lora_scale = lora_scale
        ctx.save_for_backward(x2 if lora_A is not None else None, u, lora_A, lora_B, q, scale)
        return y

    @staticmethod
    def backward(ctx, dy):
        x2, u, A, B, q, scale = ctx.saved_tensors
        dy = dy.contiguous()
        if dy.dtype != torch.bfloat16:
            dy = dy.to(torch.bfloat16)
        g = dA = dB = None
        if A is not None:
            g, dA, dB = _lib.lora_grads(dy, x2 if ctx.needs_input_grad[1] else None,
                                        u if ctx.needs_input_grad[2] else None, B, ctx.lora_scale)
        dx = None
        if ctx.needs_input_grad[0]:
            dx = _lib.gemm_dx_fp8(dy, q, scale, g=g, lora_a=A if g is not None else None)
        return dx, dA, dB, None, None, None, None


class Fp8Linear(nn.Module):
    """Frozen ``nn.Linear`` with the weight in fp8 (e4m3) and a per-output-row bf16 scale: the reference's
    ``Fp8Linear`` (``quantize.py:23-51``) with the same attributes (``weight_fp8``, ``scale``, ``bias``,
    ``in_features``, ``out_features``, the ``weight`` probe) and the same numerics, run by gfx950 kernels:
    quantization ``q = e4m3(clamp(W / s, +-448))`` with ``s = max(amax, 1e-8)/448``; forward
    ``F.linear(x, bf16(q) * bf16(s), bias.bf16)`` on bf16 MFMA with f32 accumulation."""

    is_quant_linear = True

    def __init__(self, lin: nn.Linear):
        super().__init__()
        w = lin.weight.data
        N, K = w.shape
        if K % 64:
            raise ValueError(f"Fp8Linear needs in_features % 64 == 0, got {K}")
        _check_out_features(N)
        home = w.device
        if home.type != "cuda":
            if not torch.cuda.is_available():
                raise RuntimeError("Fp8Linear quantizes on the GPU (libk2q, gfx950); no GPU is available")
            w = w.to("cuda")
        w = w.contiguous()
        if w.dtype not in (torch.bfloat16, torch.float32):
            w = w.float()
        q, s = _lib.quant_weight_fp8(w)
        self.weight_fp8 = nn.Parameter(q.to(home), requires_grad=False)
        self.scale = nn.Parameter(s.to(home), requires_grad=False)
        self.bias = (nn.Parameter(lin.bias.data.clone(), requires_grad=False)
                     if lin.bias is not None else None)
        self.in_features, self.out_features = K, N

    @classmethod
    def from_quantized(cls, weight_fp8: torch.Tensor, scale: torch.Tensor, bias: torch.Tensor | None) -> "Fp8Linear":
        """Wrap already-quantized tensors (e.g. loaded from disk): float8_e4m3fn codes (N,K) and bf16 scales."""
        if weight_fp8.dtype != torch.float8_e4m3fn or weight_fp8.dim() != 2:
            raise ValueError("weight_fp8 must be a 2-D float8_e4m3fn tensor")
        N, K = weight_fp8.shape
        if K % 64:
            raise ValueError(f"Fp8Linear needs in_features % 64 == 0, got {K}")
        _check_out_features(N)
        if scale.dtype != torch.bfloat16 or scale.numel() != N:
            raise ValueError("scale must hold one bf16 value per output row")
        m = cls.__new__(cls)
        nn.Module.__init__(m)
        m.weight_fp8 = nn.Parameter(weight_fp8, requires_grad=False)
        m.scale = nn.Parameter(scale.reshape(N, 1), requires_grad=False)
        m.bias = nn.Parameter(bias, requires_grad=False) if bias is not None else None
        m.in_features, m.out_features = K, N
        return m

    @property
    def weight(self) -> torch.Tensor:  # device probe for LoRALinear (quantize.py:44-46)
        return self.weight_fp8

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, fp8=e4m3, " \
               f"bias={self.bias is not None}"

    def forward_lora(self, x: torch.Tensor, lora_A: torch.Tensor | None, lora_B: torch.Tensor | None,
                     lora_scale: float) -> torch.Tensor:
        if x.shape[-1] != self.in_features:
            raise ValueError(f"x has {x.shape[-1]} features, layer expects {self.in_features}")
        if x.dtype != torch.bfloat16:
            raise NotImplementedError(f"Fp8Linear runs bf16 activations (the DiT dtype); got {x.dtype}")
        lead = x.shape[:-1]
        x2 = x.reshape(-1, self.in_features)
        if not x2.is_contiguous() or x2.data_ptr() % 16:
            x2 = x2.contiguous()
        if x2.shape[0] == 0:
            return x.new_empty(*lead, self.out_features)
        # the reference adds the bias in x.dtype (quantize.py:50): round it to bf16 first
        b = self.bias.to(torch.bfloat16).float().contiguous() if self.bias is not None else None
        scale = self.scale.to(torch.bfloat16).contiguous()
        y = _Fp8LinearFn.apply(x2, lora_A, lora_B, self.weight_fp8, scale, b, float(lora_scale))
        return y.reshape(*lead, self.out_features)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.forward_lora(x, None, None, 0.0)


def quantize_dit_fp8(dit) -> int:
    """Replace the transformer blocks' ``nn.Linear`` with :class:`Fp8Linear` in place: the walk and return
    value of the reference's ``quantize_dit_fp8`` (``quantize.py:54-68``).  Call BEFORE ``inject_lora``."""
    targets = []
    for block in dit.blocks:
        for mod in block.modules():
            for name, child in mod.named_children():
                if isinstance(child, nn.Linear):
                    targets.append((mod, name, child))
    for mod, name, child in targets:
        setattr(mod, name, Fp8Linear(child))
    return len(targets)
