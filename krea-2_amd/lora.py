"""LoRA adapters over the ConvRot base, with the reference's module API unchanged.

Mirrors ``lora.py`` of the reference: ``LoRALinear`` (``lora.py:27-48``) with the same attributes
(``base, rank, scale, scale_mul, lora_A, lora_B``), init (``:30-41``) and maths
``base(x) + (scale*scale_mul) * ((x.f32 @ A^T) @ B^T)`` (``:43-48``); ``lora_scaled`` / ``lora_disabled``
(``:51-70``); ``inject_lora`` with the same duck-typed base check (``:81-116``); ``lora_parameters``
(``:119-123``); ``save_lora`` / ``load_lora_weights`` / ``load_lora`` with the same safetensors keys and
metadata (``:154-222``).

The one behavioural addition: when ``base`` is a :class:`~.quantize.ConvRotLinear` or
:class:`~.quantize.Fp8Linear` and the rank fits the fused
kernels (a multiple of 16, at most 128; ``out_features`` a multiple of 128), ``forward`` runs base + LoRA as
one fused HIP pass (the LoRA down-projection on bf16 MFMA, the up-projection inside the GEMM epilogue) instead
of three extra GEMMs and three elementwise kernels, and the backward computes the LoRA gradients with the
library's own kernels.  ``scale_mul == 0`` still returns exactly ``base(x)`` (``lora.py:45-46``).
"""
from __future__ import annotations

import contextlib
import math
import os

import torch
import torch.nn as nn

from .quantize import ConvRotLinear, Fp8Linear

DEFAULT_TARGETS = ("attn.wq", "attn.wk", "attn.wv", "attn.wo", "attn.gate",
                   "mlp.gate", "mlp.up", "mlp.down")


class LoRALinear(nn.Module):
    """``base(x) + scale * (x @ A^T) @ B^T`` with ``A:(rank,in)``, ``B:(out,rank)``, ``B`` init 0."""

    def __init__(self, base: nn.Module, rank: int, alpha: float):
        super().__init__()
        self.base = base
        for p in self.base.parameters():
            p.requires_grad_(False)
        self.rank = rank
        self.scale = alpha / rank
        self.scale_mul = 1.0
        dev = base.weight.device
        self.lora_A = nn.Parameter(torch.empty(rank, base.in_features, device=dev, dtype=torch.float32))
        self.lora_B = nn.Parameter(torch.zeros(base.out_features, rank, device=dev, dtype=torch.float32))
        nn.init.kaiming_uniform_(self.lora_A, a=math.sqrt(5))

    def _fusable(self) -> bool:
        return (isinstance(self.base, (ConvRotLinear, Fp8Linear)) and self.rank % 16 == 0 and self.rank <= 128
                and self.base.in_features % 128 == 0 and self.base.out_features % 128 == 0
                and self.lora_A.dtype == torch.float32 and self.lora_B.dtype == torch.float32)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.scale_mul == 0.0:
            return self.base(x)
        if self._fusable():
            return self.base.forward_lora(x, self.lora_A, self.lora_B, self.scale * self.scale_mul)
        out = self.base(x)
        delta = (x.to(self.lora_A.dtype) @ self.lora_A.t()) @ self.lora_B.t()
        return out + (self.scale * self.scale_mul) * delta.to(out.dtype)


@contextlib.contextmanager
def lora_scaled(model: nn.Module, factor: float):
    """Temporarily multiply every adapter's effect by ``factor`` (may be negative or 0)."""
    mods = [m for m in model.modules() if isinstance(m, LoRALinear)]
    prev = [m.scale_mul for m in mods]
    try:
        for m in mods:
            m.scale_mul = float(factor)
        yield
    finally:
        for m, p in zip(mods, prev):
            m.scale_mul = p


def lora_disabled(model: nn.Module):
    """Context manager: run with all adapters off (frozen-base prediction)."""
    return lora_scaled(model, 0.0)


def _resolve(parent: nn.Module, dotted: str):
    obj = parent
    parts = dotted.split(".")
    for p in parts[:-1]:
        obj = getattr(obj, p)
    return obj, parts[-1]


def _adaptable(base) -> bool:
    return isinstance(base, nn.Linear) or getattr(base, "is_quant_linear", False)


def inject_lora(dit, rank: int, alpha: float | None = None, *, targets=DEFAULT_TARGETS,
                include_txtfusion: bool = True, include_txtmlp: bool = True) -> dict:
    """Freeze the DiT and wrap each target Linear (or quantized base) with :class:`LoRALinear`."""
    alpha = alpha if alpha is not None else float(rank)
    dit.requires_grad_(False)
    groups = [("blocks", dit.blocks)]
    if include_txtfusion and hasattr(dit, "txtfusion"):
        groups.append(("txtfusion.layerwise_blocks", dit.txtfusion.layerwise_blocks))
        groups.append(("txtfusion.refiner_blocks", dit.txtfusion.refiner_blocks))
    adapters: dict[str, LoRALinear] = {}
    for prefix, modlist in groups:
        for i, blk in enumerate(modlist):
            for tgt in targets:
                try:
                    parent, leaf = _resolve(blk, tgt)
                    base = getattr(parent, leaf)
                except AttributeError:
                    continue
                if not _adaptable(base):
                    continue
                lora = LoRALinear(base, rank, alpha)
                setattr(parent, leaf, lora)
                adapters[f"{prefix}.{i}.{tgt}"] = lora
    if include_txtmlp and hasattr(dit, "txtmlp"):
        for name, base in list(dit.txtmlp.named_modules()):
            if not name or not _adaptable(base):
                continue
            parent = dit.txtmlp.get_submodule(name.rsplit(".", 1)[0]) if "." in name else dit.txtmlp
            leaf = name.rsplit(".", 1)[-1]
            lora = LoRALinear(base, rank, alpha)
            setattr(parent, leaf, lora)
            adapters[f"txtmlp.{name}"] = lora
    if not adapters:
        raise RuntimeError("inject_lora matched no Linear targets; check target names vs mmdit.py")
    return adapters


def lora_parameters(adapters: dict) -> list:
    params = []
    for m in adapters.values():
        params.extend([m.lora_A, m.lora_B])
    return params


def save_lora(adapters: dict, path: str, *, rank: int, alpha: float, metadata: dict | None = None,
              key_prefix: str = "diffusion_model") -> None:
    """Save adapters as bf16 safetensors, keys ``<key_prefix>.<name>.lora_{A,B}.weight``, written atomically."""
    from safetensors.torch import save_file

    sd = {}
    for name, m in adapters.items():
        sd[f"{key_prefix}.{name}.lora_A.weight"] = m.lora_A.detach().to(torch.bfloat16).cpu().contiguous()
        sd[f"{key_prefix}.{name}.lora_B.weight"] = m.lora_B.detach().to(torch.bfloat16).cpu().contiguous()
    meta = {"format": "krea2-lora", "rank": str(rank), "alpha": str(alpha)}
    if metadata:
        meta.update({k: str(v) for k, v in metadata.items()})
    tmp = path + ".tmp"
    save_file(sd, tmp, metadata=meta)
    os.replace(tmp, path)


def load_lora_weights(adapters: dict, path: str, *, key_prefix: str = "diffusion_model") -> int:
    """Copy saved ``lora_{A,B}`` into already-injected adapters; returns how many had no saved weights."""
    from safetensors.torch import load_file

    sd = load_file(path)
    missing = 0
    for name, m in adapters.items():
        a = sd.get(f"{key_prefix}.{name}.lora_A.weight")
        b = sd.get(f"{key_prefix}.{name}.lora_B.weight")
        if a is None or b is None:
            missing += 1
            continue
        with torch.no_grad():
            m.lora_A.copy_(a.to(m.lora_A.dtype))
            m.lora_B.copy_(b.to(m.lora_B.dtype))
    return missing


def load_lora(dit, path: str) -> dict:
    """Inject adapters matching a saved LoRA (rank and text-side stages inferred from its keys) and load it."""
    from safetensors.torch import load_file

    sd = load_file(path)
    rank = None
    has_txtfusion = has_txtmlp = False
    for k, v in sd.items():
        name = k[len("diffusion_model."):].rsplit(".lora_", 1)[0]
        has_txtfusion |= "txtfusion" in name
        has_txtmlp |= "txtmlp" in name
        if k.endswith("lora_A.weight") and rank is None:
            rank = v.shape[0]
    if rank is None:
        raise ValueError(f"no lora_A weights found in {path}")
    adapters = inject_lora(dit, rank, include_txtfusion=has_txtfusion, include_txtmlp=has_txtmlp)
    missing = load_lora_weights(adapters, path)
    if missing:
        print(f"[load_lora] warning: {missing} injected adapters had no saved weights")
    return adapters
