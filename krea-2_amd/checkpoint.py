"""On-disk format for a quantized frozen base, so a trainer can skip re-quantizing at every start.

The reference re-quantizes all 224 block Linears (12.2e9 weights) each time a run starts
(``train_t2i_lora_cached.py:83-88``) and has no file format for the result.  This one is a single
safetensors file:

- keys ``<module path>.<tensor>`` for every quantized Linear under ``dit.blocks``, with the module path as the
  walker of ``quantize.py:54-68`` reaches it (``blocks.3.attn.wq``; a LoRA wrapper's ``.base`` is not part of
  it, so a file saved before or after ``inject_lora`` is the same);
- tensors exactly as the modules hold them: ConvRot ``qweight`` (int8 N x K, or uint8 N x K/2 packed int4:
  in every 16-wide K chunk byte j = code j | code j+8 << 4) and ``wscale`` (int32 f32 bits (N,), or int16 bf16
  bits (K/64, N) group-major); fp8 ``weight_fp8`` (float8_e4m3fn N x K) and ``scale`` (bf16 (N, 1)); ``bias``
  as stored;
- metadata ``format = krea2-quantized-base``, ``version``, ``modes`` (w8a8 / w4a8 / fp8, comma-separated),
  ``hadamard_block = 128``, ``int4_group = 64``, ``count``.

Loading builds the modules from the stored tensors directly (no GPU work, no bf16 weights needed).
"""
from __future__ import annotations

import os

import torch
import torch.nn as nn

from .quantize import ConvRotLinear, Fp8Linear

FORMAT = "krea2-quantized-base"
VERSION = "1"


def _quantized_modules(dit):
    """(path, module) for every quantized base under ``dit.blocks``, paths without a LoRA wrapper's ``.base``."""
    out = []
    for name, mod in dit.blocks.named_modules(prefix="blocks"):
        if isinstance(mod, (ConvRotLinear, Fp8Linear)):
            path = name[: -len(".base")] if name.endswith(".base") else name
            out.append((path, mod))
    return out


def save_quantized_base(dit, path: str, metadata: dict | None = None) -> int:
    """Write every quantized Linear of ``dit.blocks`` to ``path`` (atomically); returns how many."""
    from safetensors.torch import save_file

    sd, modes = {}, set()
    mods = _quantized_modules(dit)
    if not mods:
        raise ValueError("no quantized Linear under dit.blocks (run quantize_dit_convrot / quantize_dit_fp8 first)")
    for p, m in mods:
        if isinstance(m, ConvRotLinear):
            sd[f"{p}.qweight"] = m.qweight.detach().cpu().contiguous()
            sd[f"{p}.wscale"] = m.wscale.detach().cpu().contiguous()
            modes.add(m.mode)
        else:
            sd[f"{p}.weight_fp8"] = m.weight_fp8.detach().cpu().contiguous()
            sd[f"{p}.scale"] = m.scale.detach().cpu().contiguous()
            modes.add("fp8")
        if m.bias is not None:
            sd[f"{p}.bias"] = m.bias.detach().cpu().contiguous()
    meta = {"format": FORMAT, "version": VERSION, "modes": ",".join(sorted(modes)), "hadamard_block": "128",
            "int4_group": "64", "count": str(len(mods))}
    if metadata:
        meta.update({k: str(v) for k, v in metadata.items()})
    tmp = path + ".tmp"
    save_file(sd, tmp, metadata=meta)
    os.replace(tmp, path)
    return len(mods)


def load_quantized_base(dit, path: str, device=None) -> int:
    """Replace the ``nn.Linear`` children of ``dit.blocks`` with the quantized modules stored in ``path``
    (the same walk as ``quantize.py:54-68``; call before ``inject_lora``).  Shapes must match the Linears being
    replaced; every one of them must be in the file.  Returns how many were replaced."""
    from safetensors import safe_open

    with safe_open(path, framework="pt") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT:
            raise ValueError(f"{path} is not a {FORMAT} file (format={meta.get('format')!r})")
        if meta.get("hadamard_block", "128") != "128" or meta.get("int4_group", "64") != "64":
            raise ValueError(f"{path}: unsupported block sizes {meta.get('hadamard_block')}/{meta.get('int4_group')}")
        keys = set(f.keys())
        targets = []
        for bi, block in enumerate(dit.blocks):
            for name, mod in block.named_modules(prefix=f"blocks.{bi}"):
                for cname, child in mod.named_children():
                    if isinstance(child, nn.Linear):
                        targets.append((mod, cname, child, f"{name}.{cname}"))

        def get(k):
            t = f.get_tensor(k)
            return t.to(device) if device is not None else t

        new = []
        for mod, cname, child, p in targets:
            bias = get(f"{p}.bias") if f"{p}.bias" in keys else None
            if f"{p}.qweight" in keys:
                q, s = get(f"{p}.qweight"), get(f"{p}.wscale")
                mode = "w8a8" if q.dtype == torch.int8 else "w4a8"
                m = ConvRotLinear.from_quantized(q, s, bias, mode)
            elif f"{p}.weight_fp8" in keys:
                m = Fp8Linear.from_quantized(get(f"{p}.weight_fp8"), get(f"{p}.scale"), bias)
            else:
                raise KeyError(f"{path} has no quantized weights for {p}")
            if (m.in_features, m.out_features) != (child.in_features, child.out_features):
                raise ValueError(f"{p}: file holds {m.out_features}x{m.in_features}, model has "
                                 f"{child.out_features}x{child.in_features}")
            if (bias is None) != (child.bias is None):
                raise ValueError(f"{p}: bias presence differs between file and model")
            new.append((mod, cname, m))
    for mod, cname, m in new:
        setattr(mod, cname, m)
    return len(new)
