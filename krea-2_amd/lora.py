"""LoRA adapters for the DiT, with the module API of the reference's ``lora.py`` and the adapter maths run in the
fused HIP kernels whenever the base is one of this package's quantized linears.

Interface kept from the reference (callers and saved files depend on it):

* ``LoRALinear(base, rank, alpha)`` with attributes ``base, rank, scale, scale_mul, lora_A, lora_B``, the init of
  ``lora.py:30-41`` (frozen base, ``scale = alpha / rank``, ``A`` kaiming-uniform, ``B`` zeros) and the output
  ``base(x) + (scale * scale_mul) * ((x.f32 @ A^T) @ B^T)`` of ``lora.py:43-48``; ``scale_mul == 0`` returns
  exactly ``base(x)``.
* ``lora_scaled`` / ``lora_disabled`` (``lora.py:51-70``), ``inject_lora`` with the duck-typed base test
  (``lora.py:81-116``), ``lora_parameters`` (``:119-123``), ``QWEN_TE_TARGETS`` / ``inject_lora_te`` for the
  text encoder's language-model projections (``:126-151``), ``save_lora`` / ``load_lora_weights`` /
  ``load_lora`` with the key format ``<prefix>.<module path>.lora_{A,B}.weight`` and metadata
  ``{format: krea2-lora, rank, alpha}`` (``:154-222``).

Every name the reference's trainers import from ``lora`` is here (``train_t2i_lora_cached.py:22``,
``train_slider.py:28``, ``sample.py:23``), and a trainer must import all of them from this module together:
``lora_scaled`` / ``lora_disabled`` find adapters by ``isinstance`` against this module's :class:`LoRALinear`,
so the reference's own context managers do not see adapters injected here (and the reverse).

Over a :class:`~.quantize.ConvRotLinear` or :class:`~.quantize.Fp8Linear` base every rank runs on the library's
kernels: the down-projection on bf16 MFMA, the up-projection in the GEMM epilogue, the backward in the LoRA
gradient kernels.  The kernels take ranks in multiples of 16, so other ranks are padded with zero factor rows,
which adds exact zeros and changes no result.  Over a plain ``nn.Linear`` (the unquantized stages outside the
hot path) the adapter is the reference's own torch expression.
"""
from __future__ import annotations

import contextlib
import math
import os
import stat
import uuid
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from .quantize import ConvRotLinear, Fp8Linear

DEFAULT_TARGETS = ("attn.wq", "attn.wk", "attn.wv", "attn.wo", "attn.gate",
                   "mlp.gate", "mlp.up", "mlp.down")

_LORA_FORMAT = "krea2-lora"
_HIP_BASES = (ConvRotLinear, Fp8Linear)


def _is_adaptable(mod) -> bool:
    """The reference's test for a wrappable base: an ``nn.Linear`` or anything flagged ``is_quant_linear``."""
    return isinstance(mod, nn.Linear) or bool(getattr(mod, "is_quant_linear", False))


def _padded_rank(rank: int) -> int:
    return -(-rank // _lib.RANK_ALIGN) * _lib.RANK_ALIGN


class LoRALinear(nn.Module):
    """``base(x) + scale * (x @ A^T) @ B^T`` with ``A:(rank,in)``, ``B:(out,rank)``, ``B`` init 0."""

    def __init__(self, base: nn.Module, rank: int, alpha: float):
        super().__init__()
        if rank < 1:
            raise ValueError(f"LoRA rank must be positive, got {rank}")
        if isinstance(base, _HIP_BASES):
            # what the library's LoRA gradient kernels take (the dims of every Krea 2 linear qualify)
            if base.in_features % _lib.HADAMARD_BLOCK or base.out_features % _lib.HADAMARD_BLOCK:
                raise ValueError(f"a LoRA over a quantized base needs in/out features that are multiples of "
                                 f"{_lib.HADAMARD_BLOCK}, got {base.in_features} -> {base.out_features}")
            if rank > _lib.MAX_RANK:
                raise ValueError(f"LoRA rank {rank} exceeds the library's {_lib.MAX_RANK}")
        self.base = base
        base.requires_grad_(False)
        self.rank = rank
        self.scale = alpha / rank
        self.scale_mul = 1.0
        home = base.weight.device
        self.lora_A = nn.Parameter(torch.empty(rank, base.in_features, device=home, dtype=torch.float32))
        self.lora_B = nn.Parameter(torch.zeros(base.out_features, rank, device=home, dtype=torch.float32))
        nn.init.kaiming_uniform_(self.lora_A, a=math.sqrt(5))

    def _kernel_factors(self):
        """``(A, B)`` as the kernels take them: f32, the rank padded with zeros to a multiple of 16.  Both are
        autograd functions of the parameters, so the padded ranks' gradients are dropped on the way back."""
        A, B = self.lora_A, self.lora_B
        if A.dtype != torch.float32:
            A, B = A.float(), B.float()
        extra = _padded_rank(self.rank) - self.rank
        if extra:
            A = F.pad(A, (0, 0, 0, extra))
            B = F.pad(B, (0, extra))
        return A.contiguous(), B.contiguous()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        s = self.scale * self.scale_mul
        if isinstance(self.base, _HIP_BASES):
            if s == 0.0:
                return self.base(x)
            A, B = self._kernel_factors()
            return self.base.forward_lora(x, A, B, s)
        y = self.base(x)
        if s == 0.0:
            return y
        return y + s * ((x.to(self.lora_A.dtype) @ self.lora_A.t()) @ self.lora_B.t()).to(y.dtype)


def _adapters_in(model: nn.Module) -> list[LoRALinear]:
    return [m for m in model.modules() if isinstance(m, LoRALinear)]


@contextlib.contextmanager
def lora_scaled(model: nn.Module, factor: float):
    """Within the ``with`` body every adapter of ``model`` acts ``factor`` times as strongly (negative flips the
    direction, 0 turns it off); each adapter's own multiplier comes back afterwards."""
    saved = {m: m.scale_mul for m in _adapters_in(model)}
    for m in saved:
        m.scale_mul = float(factor)
    try:
        yield
    finally:
        for m, v in saved.items():
            m.scale_mul = v


def lora_disabled(model: nn.Module):
    """Context manager: the frozen base alone (every adapter's multiplier 0)."""
    return lora_scaled(model, 0.0)


@dataclass
class _Site:
    name: str          # adapter name: the module path under the DiT
    owner: nn.Module   # module holding the linear as an attribute
    attr: str
    base: nn.Module


def _target_sites(prefix: str, stack, targets):
    for i, blk in enumerate(stack):
        for tgt in targets:
            owner_path, _, attr = tgt.rpartition(".")
            try:
                owner = blk.get_submodule(owner_path) if owner_path else blk
            except AttributeError:
                continue
            base = getattr(owner, attr, None)
            if _is_adaptable(base):
                yield _Site(f"{prefix}.{i}.{tgt}", owner, attr, base)


def _module_sites(prefix: str, root: nn.Module):
    for path, mod in list(root.named_modules()):
        if path and _is_adaptable(mod):
            owner_path, _, attr = path.rpartition(".")
            yield _Site(f"{prefix}.{path}", root.get_submodule(owner_path) if owner_path else root, attr, mod)


def inject_lora(dit, rank: int, alpha: float | None = None, *, targets=DEFAULT_TARGETS,
                include_txtfusion: bool = True, include_txtmlp: bool = True) -> dict:
    """Freeze ``dit`` and put a :class:`LoRALinear` around every targeted linear (or quantized base): the
    ``targets`` paths inside each of ``dit.blocks`` and, when asked for and present, inside the text-fusion
    layerwise / refiner blocks, plus every linear of ``dit.txtmlp``.  Returns ``{module path: adapter}``;
    raises ``RuntimeError`` when nothing matched.  ``alpha`` defaults to ``rank`` (scale 1)."""
    alpha = float(rank) if alpha is None else alpha
    dit.requires_grad_(False)
    sites = list(_target_sites("blocks", dit.blocks, targets))
    fusion = getattr(dit, "txtfusion", None) if include_txtfusion else None
    if fusion is not None:
        for stage in ("layerwise_blocks", "refiner_blocks"):
            sites += _target_sites(f"txtfusion.{stage}", getattr(fusion, stage), targets)
    txtmlp = getattr(dit, "txtmlp", None) if include_txtmlp else None
    if txtmlp is not None:
        sites += _module_sites("txtmlp", txtmlp)
    if not sites:
        raise RuntimeError(f"inject_lora: no linear of {type(dit).__name__} matches the targets {tuple(targets)}")
    adapters = {}
    for site in sites:
        adapter = LoRALinear(site.base, rank, alpha)
        setattr(site.owner, site.attr, adapter)
        adapters[site.name] = adapter
    return adapters


def lora_parameters(adapters: dict) -> list:
    """The trainable tensors, ``[A_0, B_0, A_1, B_1, ...]`` in adapter order."""
    return [p for m in adapters.values() for p in (m.lora_A, m.lora_B)]


# the language-model projections of the Qwen3-VL text encoder that TE-LoRA adapts (reference ``lora.py:127``)
QWEN_TE_TARGETS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

# path components that mark the encoder's vision tower, which TE-LoRA leaves unadapted
_VISION_MARKS = ("visual", "vision")


def inject_lora_te(qwen: nn.Module, rank: int, alpha: float | None = None, *, targets=QWEN_TE_TARGETS) -> dict:
    """Freeze the text encoder ``qwen`` and put a :class:`LoRALinear` around every ``nn.Linear`` whose own name
    (the last path component) is one of ``targets``, skipping any whose path mentions the vision tower
    (reference ``lora.py:130-151``).  Matching by leaf name keeps it independent of how a transformers version
    nests the decoder layers.  The encoder's linears are plain bf16 ``nn.Linear`` (it is never quantized), so
    these adapters compute the reference's own torch expression.  Returns ``{module path: adapter}``; raises
    ``RuntimeError`` when nothing matched.  ``alpha`` defaults to ``rank`` (scale 1)."""
    alpha = float(rank) if alpha is None else alpha
    wanted = frozenset(targets)
    qwen.requires_grad_(False)
    sites = []
    for path, mod in qwen.named_modules():
        owner_path, _, attr = path.rpartition(".")
        if not isinstance(mod, nn.Linear) or attr not in wanted:
            continue
        if any(mark in path for mark in _VISION_MARKS):
            continue
        sites.append(_Site(path, qwen.get_submodule(owner_path) if owner_path else qwen, attr, mod))
    if not sites:
        raise RuntimeError(f"inject_lora_te: no nn.Linear of {type(qwen).__name__} is named one of {tuple(targets)} "
                           f"outside the vision tower")
    adapters = {}
    for site in sites:
        adapter = LoRALinear(site.base, rank, alpha)
        setattr(site.owner, site.attr, adapter)
        adapters[site.name] = adapter
    return adapters


def _key(prefix: str, name: str, which: str) -> str:
    return f"{prefix}.{name}.lora_{which}.weight"


def save_lora(adapters: dict, path: str, *, rank: int, alpha: float, metadata: dict | None = None,
              key_prefix: str = "diffusion_model") -> None:
    """Write the adapters to ``path`` as safetensors: bf16 ``lora_A`` / ``lora_B`` per adapter under
    ``<key_prefix>.<name>.lora_{A,B}.weight``, metadata ``format / rank / alpha`` plus ``metadata``.
    ``key_prefix`` is ``diffusion_model`` for DiT adapters and ``text_encoder`` for TE-LoRA.  The file appears
    atomically (written next to ``path``, then renamed), with the permissions a plainly created file gets (the
    process umask applied to 0o666; safetensors alone would leave it readable by its owner only)."""
    from safetensors.torch import save_file

    tensors = {_key(key_prefix, name, w): t.detach().to(torch.bfloat16).cpu().contiguous()
               for name, m in adapters.items() for w, t in (("A", m.lora_A), ("B", m.lora_B))}
    meta = {"format": _LORA_FORMAT, "rank": str(rank), "alpha": str(alpha)}
    meta.update({k: str(v) for k, v in (metadata or {}).items()})
    # a fresh name beside the target, created the way open() creates files (0o666 less the umask); safetensors
    # writes its files owner-only, so that mode is put back before the rename and the result is as readable as a
    # plainly created file
    tmp = f"{os.path.abspath(path)}.{os.getpid()}.{uuid.uuid4().hex[:12]}.tmp"
    os.close(os.open(tmp, os.O_WRONLY | os.O_CREAT | os.O_EXCL, 0o666))
    try:
        mode = stat.S_IMODE(os.stat(tmp).st_mode)
        save_file(tensors, tmp, metadata=meta)
        os.chmod(tmp, mode)
        os.replace(tmp, path)
    except BaseException:
        if os.path.exists(tmp):
            os.remove(tmp)
        raise


def load_lora_weights(adapters: dict, path: str, *, key_prefix: str = "diffusion_model") -> int:
    """Copy the factors saved in ``path`` into already-injected ``adapters`` (in place, cast to the parameters'
    dtype).  Returns how many adapters found no saved pair (0: everything loaded)."""
    from safetensors.torch import load_file

    saved = load_file(path)
    missing = 0
    with torch.no_grad():
        for name, m in adapters.items():
            pair = [saved.get(_key(key_prefix, name, w)) for w in ("A", "B")]
            if any(t is None for t in pair):
                missing += 1
                continue
            for param, t in zip((m.lora_A, m.lora_B), pair):
                param.copy_(t.to(param.dtype))
    return missing


def load_lora(dit, path: str) -> dict:
    """Inject adapters shaped like the ones saved in ``path`` and load them.  The rank comes from the first
    saved ``lora_A``; text-fusion and text-MLP adapters are injected when the file holds any."""
    from safetensors.torch import load_file

    saved = load_file(path)
    prefix = "diffusion_model."
    names = {k[len(prefix):].rsplit(".lora_", 1)[0] for k in saved if k.startswith(prefix)}
    ranks = [t.shape[0] for k, t in saved.items() if k.endswith("lora_A.weight")]
    if not ranks:
        raise ValueError(f"{path} holds no lora_A tensors")
    adapters = inject_lora(dit, ranks[0], include_txtfusion=any("txtfusion" in n for n in names),
                           include_txtmlp=any("txtmlp" in n for n in names))
    missing = load_lora_weights(adapters, path)
    if missing:
        print(f"[load_lora] {missing} of {len(adapters)} injected adapters have no weights in {path}")
    return adapters
