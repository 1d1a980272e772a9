"""End-to-end LoRA training step through a restated Krea 2 single-stream block at the real width.

The block restates the structure of ``mmdit.py:163-212,293-319``: modulation from a conditioning vector,
RMSNorm, attention with ``wq/wk/wv/gate/wo`` (48 heads of 128, 12 KV heads for ``wk/wv``: 6144 -> 1536, the
sigmoid output gate), and the SwiGLU MLP 6144 -> 16384 -> 6144 (``mlp.gate/up/down``); QK-norm and RoPE are left
out (they touch no Linear).  The trainer wiring of ``train_t2i_lora_cached.py:84-97`` is followed: quantize the
blocks, inject LoRA, train only the adapters under gradient checkpointing (``mmdit.py:479-481``), with block
swap paging the frozen parameters (``mmdit.py:409-414``), and save / load the adapters (``lora.py:154-222``).
The reference point is the same block on unquantized bf16 Linears with the reference's LoRA maths.
"""
import copy

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

FEAT, HEADS, KVHEADS, HID = 6144, 48, 12, 16384


class RMSNorm(nn.Module):
    def __init__(self, n):
        super().__init__()
        self.n = n

    def forward(self, x):
        return F.rms_norm(x.float(), (self.n,), eps=1e-6).to(x.dtype)


class Attention(nn.Module):
    def __init__(self):
        super().__init__()
        hd = FEAT // HEADS
        self.wq = nn.Linear(FEAT, FEAT, bias=False)
        self.wk = nn.Linear(FEAT, hd * KVHEADS, bias=False)
        self.wv = nn.Linear(FEAT, hd * KVHEADS, bias=False)
        self.gate = nn.Linear(FEAT, FEAT, bias=False)
        self.wo = nn.Linear(FEAT, FEAT, bias=False)

    def forward(self, x):
        B, L, _ = x.shape
        hd = FEAT // HEADS
        q = self.wq(x).view(B, L, HEADS, hd).transpose(1, 2)
        k = self.wk(x).view(B, L, KVHEADS, hd).transpose(1, 2)
        v = self.wv(x).view(B, L, KVHEADS, hd).transpose(1, 2)
        g = self.gate(x)
        k = k.repeat_interleave(HEADS // KVHEADS, dim=1)
        v = v.repeat_interleave(HEADS // KVHEADS, dim=1)
        # attention in f32 (reference attention math is kept off the bf16 batched-product path)
        o = F.scaled_dot_product_attention(q.float(), k.float(), v.float()).to(x.dtype)
        o = o.transpose(1, 2).reshape(B, L, FEAT)
        return self.wo(o * torch.sigmoid(g))


class SwiGLU(nn.Module):
    def __init__(self):
        super().__init__()
        self.gate = nn.Linear(FEAT, HID, bias=False)
        self.up = nn.Linear(FEAT, HID, bias=False)
        self.down = nn.Linear(HID, FEAT, bias=False)

    def forward(self, x):
        return self.down(F.silu(self.gate(x)) * self.up(x))


class Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.prenorm, self.postnorm = RMSNorm(FEAT), RMSNorm(FEAT)
        self.attn, self.mlp = Attention(), SwiGLU()

    def forward(self, x, mod):
        prescale, preshift, pregate, postscale, postshift, postgate = mod.chunk(6, dim=-1)
        x = x + pregate * self.attn((1 + prescale) * self.prenorm(x) + preshift)
        return x + postgate * self.mlp((1 + postscale) * self.postnorm(x) + postshift)


class Dit(nn.Module):
    def __init__(self):
        super().__init__()
        self.blocks = nn.ModuleList([Block()])


def _init(dit, seed):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in sorted(dit.named_parameters()):
            p.copy_(torch.randn(p.shape, generator=g) * (1.0 / np.sqrt(p.shape[-1])))


def _run(dit, x, mod, dy, ckpt):
    blk = dit.blocks[0]
    if ckpt:
        y = torch.utils.checkpoint.checkpoint(blk, x, mod, use_reentrant=False)
    else:
        y = blk(x, mod)
    y.backward(dy)
    return y.detach()


def _cos(a, b):
    a, b = a.double().flatten(), b.double().flatten()
    return float(a @ b / (a.norm() * b.norm()))


@pytest.mark.timeout(300)
def test_lora_training_step_on_restated_block(k2, dev, tmp_path):
    torch.manual_seed(0)
    ref = Dit().to(torch.bfloat16)
    _init(ref, 1)
    ref = ref.to(dev)
    dit = copy.deepcopy(ref)
    assert k2.quantize_dit_convrot(dit, "w8a8") == 8
    ad_q = k2.inject_lora(dit, 32, include_txtfusion=False, include_txtmlp=False)
    ad_r = k2.inject_lora(ref, 32, include_txtfusion=False, include_txtmlp=False)
    assert sorted(ad_q) == sorted(ad_r) and len(ad_q) == 8
    g = torch.Generator().manual_seed(2)
    with torch.no_grad():
        for name in sorted(ad_q):
            A = torch.randn(ad_q[name].lora_A.shape, generator=g) * 0.01
            B = torch.randn(ad_q[name].lora_B.shape, generator=g) * 0.01
            for m in (ad_q[name], ad_r[name]):
                m.lora_A.copy_(A)
                m.lora_B.copy_(B)
    assert all(isinstance(m.base, k2.ConvRotLinear) for m in ad_q.values())   # all on the fused kernels

    L = 512
    x = (torch.randn(1, L, FEAT, generator=g)).to(torch.bfloat16).to(dev)
    mod = (torch.randn(1, 1, 6 * FEAT, generator=g) * 0.1).to(torch.bfloat16).to(dev)
    dy = (torch.randn(1, L, FEAT, generator=g) * 1e-2).to(torch.bfloat16).to(dev)

    # quantized block under checkpointing vs the bf16 reference: the ConvRot error stays small
    y_q = _run(dit, x, mod, dy, ckpt=True)
    y_r = _run(ref, x, mod, dy, ckpt=False)
    rel = float((y_q.float() - y_r.float()).norm() / (y_r.float() - x.float()).norm())
    assert rel < 0.05, rel                                  # of the block's update x -> y
    for name in sorted(ad_q):
        assert _cos(ad_q[name].lora_B.grad, ad_r[name].lora_B.grad) > 0.99, name
        assert _cos(ad_q[name].lora_A.grad, ad_r[name].lora_A.grad) > 0.98, name

    # the checkpoint recompute is bit-identical: same gradients without checkpointing
    grads = {n: (m.lora_A.grad.clone(), m.lora_B.grad.clone()) for n, m in ad_q.items()}
    for m in ad_q.values():
        m.lora_A.grad = m.lora_B.grad = None
    y_q2 = _run(dit, x, mod, dy, ckpt=False)
    assert torch.equal(y_q2, y_q)
    for n, m in ad_q.items():
        assert torch.equal(m.lora_A.grad, grads[n][0]) and torch.equal(m.lora_B.grad, grads[n][1])

    # one optimizer step on the adapters only, then block swap: page the frozen params out and back
    opt = torch.optim.AdamW(k2.lora_parameters(ad_q), lr=1e-3)
    opt.step()
    with torch.no_grad():
        y_after = dit.blocks[0](x, mod)
    assert not torch.equal(y_after, y_q)
    for p in dit.blocks[0].parameters():
        if not p.requires_grad:
            p.data = p.data.to("cpu")
    for p in dit.blocks[0].parameters():
        if not p.requires_grad:
            p.data = p.data.to(dev, non_blocking=True)
    with torch.no_grad():
        assert torch.equal(dit.blocks[0](x, mod), y_after)

    # adapters saved and loaded into a freshly quantized copy reproduce the trained block
    f = str(tmp_path / "lora.safetensors")
    k2.save_lora(ad_q, f, rank=32, alpha=32.0)
    fresh = copy.deepcopy(ref)
    wrapped = [(m, cname, child) for m in fresh.modules() for cname, child in m.named_children()
               if isinstance(child, k2.LoRALinear)]
    for m, cname, child in wrapped:                         # back to plain Linears before quantizing
        setattr(m, cname, child.base)
    assert len(wrapped) == 8
    assert k2.quantize_dit_convrot(fresh, "w8a8") == 8
    assert len(k2.load_lora(fresh, f)) == 8
    # adapters are stored in bf16 (lora.py:161-164): the reloaded block equals the trained one with its
    # adapters rounded to bf16, bit for bit (same quantized base, deterministic kernels)
    with torch.no_grad():
        for m in ad_q.values():
            m.lora_A.copy_(m.lora_A.to(torch.bfloat16).float())
            m.lora_B.copy_(m.lora_B.to(torch.bfloat16).float())
        y_rounded = dit.blocks[0](x, mod)
        y_loaded = fresh.blocks[0](x, mod)
    assert torch.equal(y_loaded, y_rounded)
