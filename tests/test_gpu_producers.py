"""GPU parity of the producer-fused rotate/quant kernels (through the C ABI) and of the patched block.

* ``k2q_swiglu_rotquant`` / ``k2q_rmsmod_rotquant``: the bf16 output ``h`` within one bf16 step of the oracle's
  restatement of the reference's eager ops (``mmdit.py:156-161,177-178,314-317``) and equal to it almost
  everywhere (the exp / reduction orders differ only in the last float32 bits); the int8 codes and scales
  bit-exact against the oracle's rotate/quant of the kernel's own ``h`` and against ``k2q_rotquant(h)``.
* ``k2q_swiglu_bwd``: within two bf16 steps of the oracle's autograd restatement (each output is two roundings
  deep), equal almost everywhere.
* ``fuse_producers`` on a restated reference block (``mmdit.py:104-115,146-212,294-319``): outputs and gradients
  against the same block without fusion, one rotate/quant per block left (the attention output), and a
  checkpointed backward equal to a plain one.
"""
import copy
import gc

import numpy as np
import pytest
import torch

from oracle import convrot as orc
from restated_block import FEAT, Dit

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


def _steps(a, b):
    """bf16 steps between two arrays of bf16 values (+0 == -0)."""
    def line(x):
        u = orc.bf16_bits(x).astype(np.int32)
        return np.where(u & 0x8000, -(u & 0x7FFF), u)
    return np.abs(line(a) - line(b))


def _bf16(shape, g, scale=1.0):
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def _check_rmsmod(h, x, ns, eps, ms, mb, rpb):
    """h within one bf16 step of the modulated product bf16((1 + p) n) plus one of the result (the shift is
    added after the product rounds, so a last-bit difference in n moves h by up to a step of the product
    where the sum cancels), and equal to the oracle almost everywhere."""
    ho = orc.rmsmod(_np(x), _np(ns), eps, _np(ms), _np(mb), rpb)
    zero = np.zeros_like(_np(ms))
    n = orc.rmsmod(_np(x), _np(ns), eps, zero, zero, rpb)          # p = b = 0 leaves n
    rows = np.arange(n.shape[0]) // rpb if ms.shape[0] > 1 else np.zeros(n.shape[0], np.int64)
    prod = orc.bf16_round(orc.bf16_round(1.0 + _np(ms))[rows] * n)
    hk = _np(h)
    assert np.all(np.abs(hk - ho) <= (np.abs(prod) + np.abs(ho)) * 2.0 ** -7)
    assert (hk == ho).mean() > 0.999


def _check_codes(k2, h, q, s):
    qo, so, _ = orc.rotquant(_np(h))
    assert np.array_equal(q.cpu().numpy(), qo)
    assert np.array_equal(s.cpu().numpy(), so)
    q2, s2, _ = k2._lib.rotquant(h)
    assert torch.equal(q2, q) and torch.equal(s2, s)


@pytest.mark.parametrize("M,K,strided", [(5, 128, False), (37, 3072, False), (96, 6144, True), (64, 12288, False),
                                         (16, 16384, True)])
def test_swiglu_rotquant(k2, dev, M, K, strided):
    g = torch.Generator().manual_seed(M + K)
    if strided:   # gate / up as the two halves of one (M, 2K) tensor
        gu = _bf16((M, 2 * K), g, 3.0).to(dev)
        gd, ud = gu[:, :K], gu[:, K:]
    else:
        gd, ud = _bf16((M, K), g, 3.0).to(dev), _bf16((M, K), g).to(dev)
    h, q, s = k2._lib.swiglu_rotquant(gd, ud)
    torch.cuda.synchronize()
    # bf16(silu(g)) may sit one step off the oracle's where exp / reciprocal differ in the last float32 bits
    # at a rounding boundary; h = bf16(s u) then moves by up to a step of the product plus one of its own
    gn, un = _np(gd), _np(ud)
    ho = orc.swiglu(gn, un)
    so = orc.swiglu(gn, np.ones_like(un))                      # bf16(silu(g))
    hk = _np(h)
    assert np.all(np.abs(hk - ho) <= (np.abs(so * un) + np.abs(ho)) * 2.0 ** -7)
    assert (hk == ho).mean() > 0.999
    _check_codes(k2, h, q, s)


@pytest.mark.parametrize("B,L,K", [(1, 40, 3072), (2, 48, 6144), (2, 16, 16384), (3, 7, 128)])
def test_rmsmod_rotquant(k2, dev, B, L, K):
    g = torch.Generator().manual_seed(B * L + K)
    x = _bf16((B * L, K), g, 2.0).to(dev)
    ns = (torch.randn(K, generator=g) * 0.1).to(dev)
    vec = _bf16((B, 1, 6 * K), g, 0.3).to(dev)       # DoubleSharedModulation output, chunked as the block does
    ps, sh = vec.chunk(6, dim=-1)[0], vec.chunk(6, dim=-1)[1]
    ms, mb = ps.reshape(B, K), sh.reshape(B, K)
    assert B == 1 or ms.stride(0) == 6 * K            # strided views go to the kernel as they are
    h, q, s = k2._lib.rmsmod_rotquant(x, ns, 1e-5, ms, mb, L)
    torch.cuda.synchronize()
    _check_rmsmod(h, x, ns, 1e-5, ms, mb, L)
    _check_codes(k2, h, q, s)


def test_rmsmod_rotquant_single_entry_and_zero_row(k2, dev):
    """One modulation entry for every row; an all-zero row gives n = 0, h = bf16(shift), and the codes of h."""
    g = torch.Generator().manual_seed(5)
    M, K = 20, 1024
    x = _bf16((M, K), g).to(dev)
    x[3] = 0
    ns = torch.zeros(K, device=dev)
    ms, mb = _bf16((1, K), g, 0.5).to(dev), _bf16((1, K), g, 0.5).to(dev)
    h, q, s = k2._lib.rmsmod_rotquant(x, ns, 1e-6, ms, mb, M)
    torch.cuda.synchronize()
    _check_rmsmod(h, x, ns, 1e-6, ms, mb, M)
    assert torch.equal(h[3], mb[0])
    _check_codes(k2, h, q, s)


def test_producer_argument_checks(k2, dev):
    x = torch.zeros(4, 256, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        k2._lib.swiglu_rotquant(x, x[:, :128])
    with pytest.raises(ValueError):
        k2._lib.rmsmod_rotquant(x, torch.zeros(128, device=dev), 1e-5, x[:1], x[:1], 4)
    with pytest.raises(ValueError):   # 3 entries cannot split 4 rows
        m = torch.zeros(3, 256, dtype=torch.bfloat16, device=dev)
        k2._lib.rmsmod_rotquant(x, torch.zeros(256, device=dev), 1e-5, m, m, 1)


@pytest.mark.parametrize("M,K", [(8, 128), (333, 3072)])
def test_swiglu_bwd(k2, dev, M, K):
    g = torch.Generator().manual_seed(M)
    gd, ud = _bf16((M, K), g, 3.0).to(dev), _bf16((M, K), g).to(dev)
    dh = _bf16((M, K), g, 1e-3).to(dev)
    dg, du = k2._lib.swiglu_bwd(dh, gd, ud)
    torch.cuda.synchronize()
    og, ou = orc.swiglu_backward(_np(dh), _np(gd), _np(ud))
    d_u, d_g = _steps(_np(du), ou), _steps(_np(dg), og)
    assert d_u.max() <= 2 and (d_u == 0).mean() > 0.999    # du = bf16(dh * bf16(silu(g))): two roundings
    assert d_g.max() <= 2 and (d_g == 0).mean() > 0.99


@pytest.mark.parametrize("B,L,K", [(1, 40, 3072), (2, 48, 6144), (2, 16, 16384), (3, 7, 128), (1, 9, 12288)])
def test_rmsmod_bwd(k2, dev, B, L, K):
    """Input gradient of the modulated RMSNorm against the oracle's float64 restatement of the reference's
    autograd: relative Frobenius < 1e-3 and equal in > 99% of elements."""
    g = torch.Generator().manual_seed(B * L + K + 1)
    x = _bf16((B * L, K), g, 2.0).to(dev)
    ns = (torch.randn(K, generator=g) * 0.1).to(dev)
    vec = _bf16((B, 1, 6 * K), g, 0.3).to(dev)
    ms = vec[..., :K].reshape(B, K)
    dh = _bf16((B * L, K), g, 1e-2).to(dev)
    dx = k2._lib.rmsmod_bwd(dh, x, ns, 1e-5, ms, L)
    torch.cuda.synchronize()
    ref = orc.rmsmod_backward_x(_np(dh), _np(x), _np(ns), 1e-5, _np(ms), L)
    dk = _np(dx)
    assert np.linalg.norm(dk - ref) / np.linalg.norm(ref) < 1e-3
    assert (dk == ref).mean() > 0.99


# ------------------------------------------------------------------------------------------- patched block

def _build(k2, dev):
    g = torch.Generator().manual_seed(3)
    dit = Dit()
    with torch.no_grad():
        for name, p in sorted(dit.named_parameters()):
            sc = 0.1 if ("scale" in name or "lin" in name) else 1.0 / np.sqrt(p.shape[-1])
            p.copy_(torch.randn(p.shape, generator=g) * sc)
    dit = dit.to(torch.bfloat16).to(dev)
    assert k2.quantize_dit_convrot(dit, "w8a8") == 16
    ad = k2.inject_lora(dit, 16, include_txtfusion=False, include_txtmlp=False)
    with torch.no_grad():
        for m in ad.values():
            m.lora_B.copy_(torch.randn(m.lora_B.shape, generator=g) * 0.01)
    return dit, ad


def _step(dit, ad, x, vec, dy, ckpt=False):
    for m in ad.values():
        m.lora_A.grad = m.lora_B.grad = None
    xr = x.clone().requires_grad_(True)
    h = xr
    for blk in dit.blocks:
        h = torch.utils.checkpoint.checkpoint(blk, h, vec, None, use_reentrant=False) if ckpt else blk(h, vec, None)
    h.backward(dy)
    grads = {k: (m.lora_A.grad.clone(), m.lora_B.grad.clone()) for k, m in ad.items()}
    return h.detach(), xr.grad.detach(), grads


def _rel(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm())


@pytest.mark.timeout(300)
def test_fused_block_matches_unfused(k2, dev):
    from krea2_amd.quantize import shared_input_quant
    dit, ad = _build(k2, dev)
    fdit = copy.deepcopy(dit)
    fad = {k: fdit.get_submodule(k) for k in ad}
    assert k2.fuse_producers(fdit) == 4      # 2 blocks x (block forward + SwiGLU forward)
    g = torch.Generator().manual_seed(4)
    B, L = 2, 256
    x = _bf16((B, L, FEAT), g).to(dev)
    vec = _bf16((B, 1, 6 * FEAT), g, 0.3).to(dev)
    dy = _bf16((B, L, FEAT), g, 1e-2).to(dev)

    m0 = shared_input_quant.misses
    y0, dx0, gr0 = _step(dit, ad, x, vec, dy)
    m1 = shared_input_quant.misses
    y1, dx1, gr1 = _step(fdit, fad, x, vec, dy)
    m2 = shared_input_quant.misses
    torch.cuda.synchronize()
    assert m1 - m0 == 8        # unfused: prenorm output, attention output, postnorm output, SwiGLU product
    assert m2 - m1 == 2        # fused: only the attention output is rotated/quantized by its layer
    # torch's rms_norm and silu can differ from the kernel's in the last bit of an element of h; that flips
    # int8 codes of the row, which moves its outputs by the quantization noise: the bf16 bar of 1e-2 applies
    assert _rel(y1, y0) < 1e-2
    assert _rel(dx1, dx0) < 1e-2
    for k in gr0:
        assert _rel(gr1[k][0], gr0[k][0]) < 2e-2 and _rel(gr1[k][1], gr0[k][1]) < 2e-2, k

    # gradient checkpointing recomputes the fused forward bit for bit
    y2, dx2, gr2 = _step(fdit, fad, x, vec, dy, ckpt=True)
    assert torch.equal(y2, y1) and torch.equal(dx2, dx1)
    for k in gr1:
        assert torch.equal(gr2[k][0], gr1[k][0]) and torch.equal(gr2[k][1], gr1[k][1]), k


@pytest.mark.timeout(300)
def test_fused_block_full_finetune_runs_unfused(k2, dev):
    """A patched block whose norm scale trains (a full fine-tune, not LoRA training) runs its class's own forward
    instead of raising: the output and the norm scale's gradient match the unpatched block's (the patched SwiGLU
    product still runs fused, so within the bf16 bar), and with the scale frozen again the fused norms are taken
    (fewer rotate/quant misses)."""
    from krea2_amd.quantize import shared_input_quant
    dit, ad = _build(k2, dev)
    fdit = copy.deepcopy(dit)
    assert k2.fuse_producers(fdit) == 4
    g = torch.Generator().manual_seed(5)
    B, L = 2, 128
    x = _bf16((B, L, FEAT), g).to(dev)
    vec = _bf16((B, 1, 6 * FEAT), g, 0.3).to(dev)
    dy = _bf16((B, L, FEAT), g, 1e-2).to(dev)
    outs = []
    for d in (dit, fdit):
        blk = d.blocks[0]
        blk.prenorm.scale.requires_grad_(True)
        blk.prenorm.scale.grad = None
        y = blk(x, vec, None)
        y.backward(dy)
        outs.append((y.detach(), blk.prenorm.scale.grad.detach().clone()))
        blk.prenorm.scale.requires_grad_(False)
    torch.cuda.synchronize()
    assert _rel(outs[1][0], outs[0][0]) < 1e-2
    assert _rel(outs[1][1], outs[0][1]) < 2e-2
    m0 = shared_input_quant.misses
    with torch.no_grad():
        dit.blocks[0](x, vec, None)
        m1 = shared_input_quant.misses
        fdit.blocks[0](x, vec, None)
        m2 = shared_input_quant.misses
    assert m2 - m1 < m1 - m0
    del dit, fdit, outs   # the patched blocks hold bound methods of themselves: a cycle for the collector
    gc.collect()
