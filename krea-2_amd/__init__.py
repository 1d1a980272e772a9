"""krea-2_amd — MI355X (gfx950) ConvRot QuantLinear + LoRA for the Krea 2 DiT.

Drop-in for the reference's quantized-base / LoRA module API (``quantize.py``, ``lora.py``):
:class:`ConvRotLinear` replaces ``Fp8Linear``, :func:`quantize_dit_convrot` replaces ``quantize_dit_fp8``,
:class:`Fp8Linear` / :func:`quantize_dit_fp8` are the reference's fp8 weight-only base on the same kernels, and
:mod:`.lora` mirrors the adapter API, and :mod:`.fused` computes the quantized linears' inputs (modulated RMSNorm,
SwiGLU product) together with their int8 codes.  The arithmetic runs in hand-written gfx950 HIP kernels behind the C ABI
of ``include/k2q.h`` (``libk2q.so``, built by ``build.py``), reached through :mod:`._lib`.

The directory name is not a Python identifier; load it with ``__graft_entry__.load_package()``, which
registers it as ``krea2_amd``.
"""
from . import _lib
from .lora import (DEFAULT_TARGETS, QWEN_TE_TARGETS, LoRALinear, inject_lora, inject_lora_te, load_lora,
                   load_lora_weights, lora_disabled, lora_parameters, lora_scaled, save_lora)
from .checkpoint import load_quantized_base, save_quantized_base
from .quantize import (MODES, ConvRotLinear, Fp8Linear, quantize_dit_convrot, quantize_dit_fp8,
                       set_dx_weight_cache)
from .fused import fuse_producers, group_siblings, modulated_rmsnorm, swiglu

__all__ = ["ConvRotLinear", "quantize_dit_convrot", "set_dx_weight_cache", "MODES", "Fp8Linear", "quantize_dit_fp8",
           "save_quantized_base", "load_quantized_base", "fuse_producers", "group_siblings", "modulated_rmsnorm",
           "swiglu", "LoRALinear", "inject_lora", "inject_lora_te", "QWEN_TE_TARGETS", "lora_scaled", "lora_disabled",
           "lora_parameters", "save_lora", "load_lora_weights", "load_lora", "DEFAULT_TARGETS", "_lib"]
