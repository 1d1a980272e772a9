"""Producer fusion: the ops that make the quantized linears' inputs, fused with their rotate/quant.

In a Krea 2 block every ConvRot linear receives one of three tensors (reference ``mmdit.py:310-319``):
the modulated RMSNorm output ``(1 + scale) * norm(x) + shift`` (read by ``wq/wk/wv/gate`` and by
``mlp.gate/up``), the attention output (read by ``wo``) and the SwiGLU product ``silu(gate) * up`` (read by
``mlp.down``).  The two producers here compute that tensor AND its int8 codes in one gfx950 pass
(``k2q_rmsmod_rotquant`` / ``k2q_swiglu_rotquant``), then hand the codes to the shared-input cache, so the
layers that read the tensor run no rotate/quant of their own.  Outputs are the reference's eager bf16
results (same rounding points), and the codes equal a separate rotate/quant of them bit for bit.

:func:`fuse_producers` patches a DiT's blocks in place (call it after ``quantize_dit_convrot`` and
``inject_lora``); :func:`modulated_rmsnorm` and :func:`swiglu` are the two operations for model code that
calls them directly.  :func:`group_siblings` makes the linears that read one tensor (``wq / wk / wv / gate``)
run as one grouped GEMM launch.
"""
from __future__ import annotations

import types
import weakref

import torch
import torch.nn as nn

from . import _lib
from .quantize import ConvRotLinear, shared_input_quant


def _rows(t: torch.Tensor, K: int) -> torch.Tensor:
    t2 = t.reshape(-1, K)
    if t2.stride(1) != 1 or t2.stride(0) % 8 or t2.data_ptr() % 16:
        t2 = t2.contiguous()
    return t2


class _SwiGLUQuantFn(torch.autograd.Function):
    """Forward ``h = bf16(bf16(silu(g)) * u)`` (``mmdit.py:178``) with the codes of ``h``; backward
    ``k2q_swiglu_bwd`` (the autograd of the two eager bf16 ops)."""

    @staticmethod
    def forward(ctx, g2, u2):
        h, q, s = _lib.swiglu_rotquant(g2, u2)
        ctx.save_for_backward(g2, u2)
        ctx.mark_non_differentiable(q, s)
        return h, q, s

    @staticmethod
    def backward(ctx, dh, _dq, _ds):
        g2, u2 = ctx.saved_tensors
        dh = dh.contiguous()
        if dh.dtype != torch.bfloat16:
            dh = dh.to(torch.bfloat16)
        g2, u2 = g2.contiguous(), u2.contiguous()
        dg, du = _lib.swiglu_bwd(dh, g2, u2)
        return dg, du


def swiglu(gate_out: torch.Tensor, up_out: torch.Tensor) -> torch.Tensor:
    """``F.silu(gate_out) * up_out`` (bf16), with the result's int8 codes recorded for the next ConvRot layer
    that receives it (``SwiGLU.forward``, ``mmdit.py:177-178``)."""
    if gate_out.shape != up_out.shape:
        raise ValueError(f"gate {tuple(gate_out.shape)} and up {tuple(up_out.shape)} differ in shape")
    if gate_out.dtype != torch.bfloat16 or up_out.dtype != torch.bfloat16:
        raise NotImplementedError("the fused SwiGLU runs bf16 tensors (the DiT dtype)")
    K = gate_out.shape[-1]
    h, q, s = _SwiGLUQuantFn.apply(_rows(gate_out, K), _rows(up_out, K))
    h = h.reshape(gate_out.shape)
    shared_input_quant.seed(h, q, s)
    return h


class _RmsModQuantFn(torch.autograd.Function):
    """Forward: the modulated RMSNorm of ``mmdit.py:314-317`` with the codes of its output (one gfx950 pass).
    Backward: the input gradient ``k2q_rmsmod_bwd``.  Only ``x`` can need one: in LoRA training the norm scale
    and the modulation tensors are frozen (the conditioning vector is ``tproj(t)``, ``mmdit.py:446``), and
    :func:`modulated_rmsnorm` refuses them as gradient inputs before launching anything."""

    @staticmethod
    def forward(ctx, x2, norm_scale, mod_scale, mod_shift, eps, rows_per_batch):
        h, q, s = _lib.rmsmod_rotquant(x2, norm_scale, eps, mod_scale, mod_shift, rows_per_batch)
        ctx.eps, ctx.rpb = eps, rows_per_batch
        ctx.save_for_backward(x2, norm_scale, mod_scale, mod_shift)
        ctx.mark_non_differentiable(q, s)
        return h, q, s

    @staticmethod
    def backward(ctx, dh, _dq, _ds):
        x2, ns, ms, mb = ctx.saved_tensors
        if not ctx.needs_input_grad[0]:
            return None, None, None, None, None, None
        M = x2.shape[0]
        rpb = ctx.rpb if ms.shape[0] > 1 else M
        dh = dh.contiguous()
        if dh.dtype != torch.bfloat16:
            dh = dh.to(torch.bfloat16)
        dx = _lib.rmsmod_bwd(dh, x2.contiguous(), ns, ctx.eps, ms, rpb)
        return dx, None, None, None, None, None


def _norm_scale_f32(norm: nn.Module) -> torch.Tensor:
    """The norm's (frozen) scale as the kernels take it, f32 and contiguous, kept on the module and rebuilt when
    the scale changes (in place: version; re-pointed, e.g. paged by block swap: pointer or device)."""
    t = norm.scale
    key = (t._version, t.data_ptr(), t.device, t.dtype, tuple(t.shape))
    kept = norm.__dict__.get("_k2q_scale_f32")
    if kept is None or kept[0] != key:
        kept = (key, t.detach().float().contiguous())
        norm.__dict__["_k2q_scale_f32"] = kept
    return kept[1]


def modulated_rmsnorm(norm: nn.Module, x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor) -> torch.Tensor:
    """``(1 + scale) * norm(x) + shift`` for the reference's ``RMSNorm`` module ``norm`` (attributes ``scale``,
    ``eps``; ``mmdit.py:146-161``), computed with its int8 codes in one pass and the codes recorded for the
    ConvRot layers that receive the result.  ``x`` (B, L, K) or (M, K) bf16; ``scale`` / ``shift`` bf16 with one
    entry per batch row of ``x`` broadcast over the tokens ((B, 1, K), as ``DoubleSharedModulation`` yields) or
    a single entry."""
    if x.dtype != torch.bfloat16 or scale.dtype != torch.bfloat16 or shift.dtype != torch.bfloat16:
        raise NotImplementedError("the fused modulated RMSNorm runs bf16 tensors (the DiT dtype)")
    K = x.shape[-1]
    if scale.shape != shift.shape or scale.shape[-1] != K:
        raise ValueError(f"scale {tuple(scale.shape)} / shift {tuple(shift.shape)} do not match {K} features")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (norm.scale, scale, shift)):
        raise NotImplementedError("the fused modulated RMSNorm computes the gradient of its input only; the norm "
                                  "scale and the modulation must be frozen (as in LoRA training) or the block left "
                                  "unfused")
    x2 = _rows(x, K)
    M = x2.shape[0]
    ms, mb = scale.reshape(-1, K), shift.reshape(-1, K)
    B = ms.shape[0]
    if B > 1:
        if x.dim() < 2 or x.shape[0] != B or scale.numel() // K != B or any(d != 1 for d in scale.shape[1:-1]):
            raise ValueError(f"scale {tuple(scale.shape)} does not broadcast over x {tuple(x.shape)} per batch row")
    # the kernel reads both with one row stride (the chunks of one modulation tensor share theirs)
    if not (ms.stride(1) == 1 and mb.stride(1) == 1 and ms.stride(0) == mb.stride(0) and ms.stride(0) % 8 == 0
            and ms.data_ptr() % 16 == 0 and mb.data_ptr() % 16 == 0):
        ms, mb = ms.contiguous(), mb.contiguous()
    h, q, s = _RmsModQuantFn.apply(x2, _norm_scale_f32(norm), ms, mb, float(norm.eps), M // B)
    h = h.reshape(x.shape)
    shared_input_quant.seed(h, q, s)
    return h


# ----------------------------------------------------------------------------------------------------------
# In-place patch of a DiT's blocks
# ----------------------------------------------------------------------------------------------------------
def _convrot(m) -> bool:
    return isinstance(m, ConvRotLinear) or isinstance(getattr(m, "base", None), ConvRotLinear)


def _fused_swiglu_forward(self, x):
    # SwiGLU.forward (mmdit.py:177-178) with the product and its codes from one pass
    return self.down(swiglu(self.gate(x), self.up(x)))


def _block_norms_train(blk, vec) -> bool:
    """Whether the block's forward would need gradients of its norm scales or its modulation (a full fine-tune):
    the modulation's chunks need one when ``vec`` or the modulation's own parameters do."""
    if not torch.is_grad_enabled():
        return False
    return (blk.prenorm.scale.requires_grad or blk.postnorm.scale.requires_grad
            or (isinstance(vec, torch.Tensor) and vec.requires_grad)
            or any(p.requires_grad for p in blk.mod.parameters()))


def _fused_block_forward(self, x, vec, freqs, mask=None):
    # SingleStreamBlock.forward (mmdit.py:310-319) with both modulated norms and their codes from one pass.  The
    # fused norm differentiates its input only, so a block whose norm scales or modulation train runs the block
    # class's own forward (its quantized linears still run on the library's kernels).
    if _block_norms_train(self, vec):
        return type(self).forward(self, x, vec, freqs, mask)
    prescale, preshift, pregate, postscale, postshift, postgate = self.mod(vec)
    x = x + pregate * self.attn(modulated_rmsnorm(self.prenorm, x, prescale, preshift), freqs, mask)
    x = x + postgate * self.mlp(modulated_rmsnorm(self.postnorm, x, postscale, postshift))
    return x


def fuse_producers(dit) -> int:
    """Patch the blocks of ``dit.blocks`` in place so their quantized linears' inputs come from the fused
    producers: a block with ``mod / prenorm / postnorm / attn / mlp`` (``SingleStreamBlock``,
    ``mmdit.py:294-319``) whose attention and MLP input linears are ConvRot gets the fused modulated RMSNorm;
    an MLP with ``gate / up / down`` (``SwiGLU``) whose ``down`` is ConvRot gets the fused product.  A patched
    block whose norm scales or modulation need gradients when it runs (a full fine-tune rather than LoRA
    training) runs its class's own forward for that call.  Call after ``quantize_dit_convrot`` and
    ``inject_lora``.  Returns the number of forwards patched."""
    n = 0
    for blk in dit.blocks:
        mlp = getattr(blk, "mlp", None)
        if mlp is not None and all(hasattr(mlp, a) for a in ("gate", "up", "down")) and _convrot(mlp.down):
            mlp.forward = types.MethodType(_fused_swiglu_forward, mlp)
            n += 1
        attn = getattr(blk, "attn", None)
        if (all(hasattr(blk, a) for a in ("mod", "prenorm", "postnorm", "attn", "mlp"))
                and all(hasattr(nm, "scale") and hasattr(nm, "eps") for nm in (blk.prenorm, blk.postnorm))
                and _convrot(getattr(attn, "wq", None)) and _convrot(getattr(mlp, "gate", None))):
            blk.forward = types.MethodType(_fused_block_forward, blk)
            n += 1
    return n


# ----------------------------------------------------------------------------------------------------------
# Linears that read one tensor, computed in one grouped launch
# ----------------------------------------------------------------------------------------------------------
def _lora_state(m):
    """(A, B, effective scale) of a member's adapter as its forward would apply it now (the factors as the
    kernels take them: f32, rank padded to a multiple of 16), or None (exact base)."""
    if isinstance(m, ConvRotLinear) or m.scale * m.scale_mul == 0.0:
        return None
    A, B = m._kernel_factors()
    return A, B, float(m.scale * m.scale_mul)


def _state_key(m):
    """Identity of what a member's adapter would add now: its parameters (object and version) and scale."""
    if isinstance(m, ConvRotLinear) or m.scale * m.scale_mul == 0.0:
        return None
    A, B = m.lora_A, m.lora_B
    return (id(A), A._version, id(B), B._version, float(m.scale * m.scale_mul))


class _GroupedFn(torch.autograd.Function):
    """Forward: one LoRA down-projection over the stacked adapters (``u = x [A_0; A_1; ..]^T``) and one grouped
    GEMM (``k2q_gemm_w8a8_grouped``) giving every member's output, each bit-identical to the member's own
    fused forward.  Backward: the members' LoRA gradients in one call (``k2q_lora_grads_grouped``: the same
    arithmetic as ``_ConvRotLinearFn``'s per member, dA of every member from one pass over x per 128 stacked
    ranks, g written in the stacked layout; per member when an output got no gradient or the rank is above 128);
    ``dX`` of all members in one GEMM (``k2q_gemm_dx_grouped``) whose reduction runs over every member's output
    gradient and effective weight, with the members' LoRA terms stacked along the rank: the sum autograd would
    form at the shared input, in f32 and rounded once."""

    @staticmethod
    def forward(ctx, x2, qx, sx, bases, scales, a_stack, *ab):
        As, Bs = ab[0::2], ab[1::2]
        u = _lib.lora_down(x2, a_stack) if As else None
        r = As[0].shape[0] if As else 0
        segs, li = [], 0
        for base, sc in zip(bases, scales):
            if sc is None:
                segs.append((base.qweight, base.weight_scale, base._bias_f32(), None, 0, 0.0))
            else:
                segs.append((base.qweight, base.weight_scale, base._bias_f32(), Bs[li], li * r, sc))
                li += 1
        ys = _lib.gemm_w8a8_grouped(qx, sx, segs, u)
        ctx.set_materialize_grads(False)    # an output nothing used gets no gradient pass (None, not zeros)
        ctx.bases, ctx.scales, ctx.r, ctx.nl = bases, scales, r, len(As)
        ctx.save_for_backward(x2 if As else None, u, a_stack, *As, *Bs)
        return tuple(ys)

    @staticmethod
    def backward(ctx, *dys):
        x2, u, a_stack, *ab = ctx.saved_tensors
        nl, r = ctx.nl, ctx.r
        As, Bs = ab[:nl], ab[nl:]
        grads = [None] * (2 * nl)
        dys = [None if dy is None else (dy.contiguous() if dy.dtype == torch.bfloat16
                                        else dy.to(torch.bfloat16).contiguous()) for dy in dys]
        adapted = [i for i, sc in enumerate(ctx.scales) if sc is not None]
        need_a = [ctx.needs_input_grad[6 + 2 * li] for li in range(nl)]
        need_b = [ctx.needs_input_grad[7 + 2 * li] for li in range(nl)]
        g = a = None
        if nl and r <= 128 and all(dys[i] is not None for i in adapted):
            # every adapter's gradients in one call: dA of all members from one pass over x per 128 stacked
            # ranks, g already in the stacked layout the grouped input gradient reads
            g, dA, dBs = _lib.lora_grads_grouped([dys[i] for i in adapted], x2 if any(need_a) else None, u, Bs,
                                                 [ctx.scales[i] for i in adapted], need_b)
            for li in range(nl):
                grads[2 * li] = dA[li * r:(li + 1) * r] if need_a[li] else None
                grads[2 * li + 1] = dBs[li]
            a = a_stack
        elif nl:
            gs, ga, li = [], [], 0
            for i, sc in enumerate(ctx.scales):
                if sc is None:
                    continue
                if dys[i] is not None:
                    u_i = u[:, li * r:(li + 1) * r].contiguous() if need_b[li] else None
                    gi, grads[2 * li], grads[2 * li + 1] = _lib.lora_grads(dys[i], x2 if need_a[li] else None, u_i,
                                                                           Bs[li], sc)
                    gs.append(gi)
                    ga.append(As[li])
                li += 1
            g = torch.cat(gs, dim=1) if len(gs) > 1 else (gs[0] if gs else None)
            a = torch.cat(ga) if len(ga) > 1 else (ga[0] if ga else None)
        dx = None
        segs = [(dys[i], base.dx_weight()) for i, base in enumerate(ctx.bases) if dys[i] is not None] \
            if ctx.needs_input_grad[0] else []
        if segs:
            # one GEMM over the members' reductions: the sum autograd would form at the shared input
            dx = _lib.gemm_dx_grouped(segs, g, a)
        return (dx, None, None, None, None, None, *grads)


class _SiblingGroup:
    """Linears that receive the same tensor (``wq / wk / wv / gate`` of ``Attention.forward``, ``mmdit.py:199``).
    The first member called with a tensor computes every member's output in one grouped launch and keeps the
    others; each later member called with that same tensor (same object, version, pointer, shape, strides and
    stream) and an unchanged adapter takes its output.  Anything else runs the member's own forward.  Kept
    outputs a member never asks for stay referenced until the group's next launch replaces them."""

    def __init__(self, members):
        self.members = list(members)
        self.ref = self.key = None
        self.kept = {}
        self.stack = None   # (key, the adapted members' stacked LoRA A rows)

    def _a_stack(self, As):
        """The members' A factors stacked along the rank.  Kept while every factor is the adapter's own
        parameter (a leaf the module holds, so its object, version and pointer identify its values: an optimizer
        step or a re-pointed parameter rebuilds the stack); padded or converted factors are new tensors every
        call and are stacked every call."""
        if not As:
            return None
        if not all(a.is_leaf for a in As):
            with torch.no_grad():
                return torch.cat(As) if len(As) > 1 else As[0].detach()
        key = tuple((id(a), a._version, a.data_ptr(), a.device) for a in As)
        if self.stack is None or self.stack[0] != key:
            with torch.no_grad():
                self.stack = (key, torch.cat(As) if len(As) > 1 else As[0].detach())
        return self.stack[1]

    @staticmethod
    def _key(x):
        return (x._version, x.data_ptr(), tuple(x.shape), tuple(x.stride()), x.device, _lib._stream(x.device))

    def call(self, idx: int, x: torch.Tensor):
        key = self._key(x)
        if self.ref is not None and self.ref() is x and self.key == key and idx in self.kept:
            out, sk = self.kept.pop(idx)
            if sk == _state_key(self.members[idx]):
                return out
        K = x.shape[-1]
        if x.dtype != torch.bfloat16 or x.numel() // max(K, 1) <= 8:
            return None
        x2 = _rows(x, K)
        with torch.no_grad():
            qx, sx = shared_input_quant.lookup(x, x2)
        states = [_lora_state(m) for m in self.members]
        bases = tuple(m if isinstance(m, ConvRotLinear) else m.base for m in self.members)
        ab = [t for st in states if st is not None for t in st[:2]]
        ys = _GroupedFn.apply(x2, qx, sx, bases, tuple(None if st is None else st[2] for st in states),
                              self._a_stack(ab[0::2]), *ab)
        lead = x.shape[:-1]
        outs = [y.reshape(*lead, b.out_features) for y, b in zip(ys, bases)]
        self.ref, self.key = weakref.ref(x), key
        self.kept = {i: (o, _state_key(m)) for i, (o, m) in enumerate(zip(outs, self.members)) if i != idx}
        return outs[idx]


def _grouped_member_forward(self, x):
    group, idx = self._k2q_group
    out = group.call(idx, x)
    return out if out is not None else type(self).forward(self, x)


def _groupable(m) -> bool:
    base = m if isinstance(m, ConvRotLinear) else getattr(m, "base", None)
    if not isinstance(base, ConvRotLinear) or base.mode != "w8a8" or base.out_features % _lib.GROUP_ALIGN:
        return False
    return base is m or hasattr(m, "_kernel_factors")


def group_siblings(dit, groups=(("attn", ("wq", "wk", "wv", "gate")), ("mlp", ("gate", "up")))) -> int:
    """Make the ConvRot linears that read one tensor run as one grouped launch, in place: for every block of
    ``dit.blocks`` and every ``(parent, names)`` of ``groups`` (default: the attention inputs of
    ``mmdit.py:199`` and the SwiGLU gate / up of ``mmdit.py:178``: each group's forward is one launch and its
    input gradient one GEMM), patch the members' forwards.  Members must be w8a8 ConvRot bases (or adapters over them with the fused
    rank rules), ``out_features`` multiples of 256, one adapter rank.  Call after ``quantize_dit_convrot`` and
    ``inject_lora``.  Returns the number of groups formed."""
    n = 0
    for blk in dit.blocks:
        for parent_name, names in groups:
            parent = getattr(blk, parent_name, None)
            mods = [getattr(parent, nm, None) for nm in names] if parent is not None else []
            if not mods or len(mods) > _lib.GROUP_MAX or not all(m is not None and _groupable(m) for m in mods):
                continue
            bases = [m if isinstance(m, ConvRotLinear) else m.base for m in mods]
            ranks = {m.rank for m in mods if not isinstance(m, ConvRotLinear)}
            if len({b.in_features for b in bases}) != 1 or len(ranks) > 1:
                continue
            group = _SiblingGroup(mods)
            for i, m in enumerate(mods):
                m._k2q_group = (group, i)
                m.forward = types.MethodType(_grouped_member_forward, m)
            n += 1
    return n
