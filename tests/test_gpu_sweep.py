"""Seeded shape sweep of the producer-fused kernels, their backward kernels, the grouped GEMM, the one-call
forward and the backward through the frozen base: ragged M, K with and without a partial chunk (K a multiple
of 128 that is not a multiple of the 1024 / 2048 / 4096 chunk width), row strides above K, one to four
segments, M from 1 to a few thousand with every rank the module pads to.  The bars are those of the dedicated
tests: codes and scales bit-exact against rotate/quant of the kernel's own h (or the oracle's for the
forward), h within the stated bf16 steps of the oracle, grouped outputs bit-identical to the per-segment GEMM,
the forward and the backward within the float64 formulas' bars."""
import numpy as np
import pytest
import torch

from oracle import convrot as orc

pytestmark = pytest.mark.gpu

_RNG = np.random.default_rng(2024)
_K = [128, 384, 1152, 3072, 4992, 6144, 9088, 12288, 16384]
_PROD_CASES = [(int(_RNG.integers(1, 700)), int(k), int(_RNG.integers(0, 3))) for k in _RNG.choice(_K, 12)]


def _np(t):
    return t.detach().float().cpu().numpy()


def _codes_match(k2, h, q, s):
    q2, s2, _ = k2._lib.rotquant(h)
    assert torch.equal(q2, q) and torch.equal(s2, s)
    qo, so, _ = orc.rotquant(_np(h))
    assert np.array_equal(q.cpu().numpy(), qo) and np.array_equal(s.cpu().numpy(), so)


@pytest.mark.parametrize("M,K,pad", _PROD_CASES)
def test_swiglu_sweep(k2, dev, M, K, pad):
    g = torch.Generator().manual_seed(M * 7 + K)
    ld = K + 128 * pad
    buf = (torch.randn(M, 2 * ld, generator=g) * 3).to(torch.bfloat16).to(dev)
    gt, ut = buf[:, :K], buf[:, ld:ld + K]
    h, q, s = k2._lib.swiglu_rotquant(gt, ut)
    dh = (torch.randn(M, K, generator=g) * 1e-2).to(torch.bfloat16).to(dev)
    dg, du = k2._lib.swiglu_bwd(dh, gt.contiguous(), ut.contiguous())
    torch.cuda.synchronize()
    gn, un = _np(gt), _np(ut)
    ho, so = orc.swiglu(gn, un), orc.swiglu(gn, np.ones_like(un))
    hk = _np(h)
    assert np.all(np.abs(hk - ho) <= (np.abs(so * un) + np.abs(ho)) * 2.0 ** -7)
    assert (hk == ho).mean() > 0.999
    _codes_match(k2, h, q, s)
    og, ou = orc.swiglu_backward(_np(dh), gn, un)
    assert np.linalg.norm(_np(dg) - og) <= 1e-2 * np.linalg.norm(og)
    assert np.linalg.norm(_np(du) - ou) <= 1e-2 * np.linalg.norm(ou)


@pytest.mark.parametrize("M,K,pad", _PROD_CASES)
def test_rmsmod_sweep(k2, dev, M, K, pad):
    g = torch.Generator().manual_seed(M * 11 + K)
    B = 1 + pad % 2 + (M % 3 == 0)
    Mb = max(B, M - M % B)
    L = Mb // B
    ld = K + 128 * pad
    x = (torch.randn(Mb, ld, generator=g) * 2).to(torch.bfloat16).to(dev)[:, :K]
    ns = (torch.randn(K, generator=g) * 0.1).to(dev)
    vec = (torch.randn(B, 1, 6 * K, generator=g) * 0.3).to(torch.bfloat16).to(dev)
    ms, mb = vec[..., :K].reshape(B, K), vec[..., K:2 * K].reshape(B, K)
    h, q, s = k2._lib.rmsmod_rotquant(x, ns, 1e-5, ms, mb, L)
    dh = (torch.randn(Mb, K, generator=g) * 1e-2).to(torch.bfloat16).to(dev)
    dx = k2._lib.rmsmod_bwd(dh, x.contiguous(), ns, 1e-5, ms, L)
    torch.cuda.synchronize()
    xn = _np(x)
    ho = orc.rmsmod(xn, _np(ns), 1e-5, _np(ms), _np(mb), L)
    zero = np.zeros_like(_np(ms))
    n = orc.rmsmod(xn, _np(ns), 1e-5, zero, zero, L)
    rows = np.arange(Mb) // L if B > 1 else np.zeros(Mb, np.int64)
    prod = orc.bf16_round(orc.bf16_round(1.0 + _np(ms))[rows] * n)
    hk = _np(h)
    assert np.all(np.abs(hk - ho) <= (np.abs(prod) + np.abs(ho)) * 2.0 ** -7)
    assert (hk == ho).mean() > 0.999
    _codes_match(k2, h, q, s)
    ref = orc.rmsmod_backward_x(_np(dh), xn, _np(ns), 1e-5, _np(ms), L)
    assert np.linalg.norm(_np(dx) - ref) <= 1e-3 * np.linalg.norm(ref)


_GROUP_CASES = [(int(_RNG.integers(9, 1200)), int(_RNG.choice([128, 640, 3072, 6144])),
                 tuple(int(256 * v) for v in _RNG.integers(1, 9, size=int(_RNG.integers(1, 5)))),
                 int(_RNG.choice([16, 32, 64]))) for _ in range(10)]


@pytest.mark.parametrize("M,K,Ns,r", _GROUP_CASES)
def test_grouped_sweep(k2, dev, M, K, Ns, r):
    L = k2._lib
    g = torch.Generator().manual_seed(M + K + sum(Ns))
    qx = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(dev)
    sx = (torch.rand(M, generator=g) * 0.05 + 1e-3).to(dev)
    u = torch.randn(M, len(Ns) * r, generator=g).to(dev)
    segs = []
    for i, N in enumerate(Ns):
        qw = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
        sw = (torch.rand(N, generator=g) * 0.01 + 1e-4).to(dev)
        b = (torch.randn(N, generator=g) * 0.1).to(dev) if i % 2 else None
        lb = (torch.randn(N, r, generator=g) * 0.05).to(dev) if (i + M) % 3 else None
        segs.append((qw, sw, b, lb, i * r, 0.5 + i))
    ys = L.gemm_w8a8_grouped(qx, sx, segs, u)
    for (qw, sw, b, lb, c, sc), y in zip(segs, ys):
        uc = u[:, c:c + r].contiguous() if lb is not None else None
        assert torch.equal(y, L.gemm_w8a8(qx, sx, qw, sw, b, uc, lb, sc, split=False))


def _lin_case(rng):
    band = int(rng.integers(0, 4))
    M = int(rng.integers(1, 9)) if band == 0 else int(rng.integers(9, 300)) if band == 1 else \
        int(rng.integers(300, 1500)) if band == 2 else int(rng.integers(1500, 4200))
    K = int(rng.choice([128, 384, 1152, 3072, 4992, 6144]))
    N = 32 * int(rng.integers(1, 48)) + int(rng.choice([0, 4, 12]))
    r = int(rng.choice([0, 16, 32, 48, 64, 128]))
    return M, K, N, r, bool(rng.integers(0, 4) == 0), bool(rng.integers(0, 2))


_LIN_CASES = [_lin_case(_RNG) for _ in range(14)]


@pytest.mark.parametrize("M,K,N,r,w4,bias", _LIN_CASES)
def test_linear_fwd_sweep(k2, dev, M, K, N, r, w4, bias):
    """The module's one-call forward (``k2q_linear_fwd``) over seeded random shapes, which take its different
    routes (GEMV for M <= 8, A.x in the rotate/quant pass or its own launch, each output tile shape and split the
    chooser picks): codes and scales bit-exact against the oracle, u within 1e-5 and y within the forward bar of
    the float64 formula, and the inference form (no factors returned) the same bits as the training form."""
    L = k2._lib
    g = torch.Generator().manual_seed(M * 31 + K + N + r)
    x = torch.randn(M, K, generator=g)
    x[:, torch.randperm(K, generator=g)[: max(1, K // 100)]] *= 20
    x = x.to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(N, generator=g) * 0.02 if bias else None
    A = torch.randn(r, K, generator=g) * 0.01 if r else None
    B = torch.randn(N, r, generator=g) * 0.01 if r else None
    xd = x.to(dev)
    if w4:
        qw, sw = L.quant_weight_i4(w.to(dev))
        qw_o, sw_o = orc.quant_weight_i4(w.float().numpy())
    else:
        qw, sw = L.quant_weight_i8(w.to(dev))
        qw_o, sw_o = orc.quant_weight_i8(w.float().numpy())
    qx = torch.empty(M, K, dtype=torch.int8, device=dev)
    sx = torch.empty(M, device=dev)
    Ad = A.to(dev) if r else None
    Bd = B.to(dev) if r else None
    bd = b.to(dev) if bias else None
    y, u = L.linear_fwd(xd, qx, sx, False, Ad, Bd, 0.75, qw, sw, bd, w4)
    y2, u2 = L.linear_fwd(xd, qx, sx, False, Ad, Bd, 0.75, qw, sw, bd, w4, need_u=False)
    torch.cuda.synchronize()
    ref = orc.forward(x.float().numpy(), qw_o, sw_o, w4=w4, bias=None if b is None else b.numpy(),
                      lora_A=None if A is None else A.numpy(), lora_B=None if B is None else B.numpy(),
                      lora_scale=0.75, fast=not w4)
    assert np.array_equal(qx.cpu().numpy(), ref["qx"]) and np.array_equal(sx.cpu().numpy(), ref["sx"])
    yk = _np(y).astype(np.float64)
    assert np.linalg.norm(yk - ref["y64"]) <= 4e-3 * np.linalg.norm(ref["y64"])
    if r:
        assert np.linalg.norm(_np(u) - ref["u"]) <= 1e-5 * np.linalg.norm(ref["u"])
    assert u2 is None and torch.equal(y2, y)


def _bwd_case(rng):
    band = int(rng.integers(0, 3))
    M = int(rng.integers(1, 64)) if band == 0 else int(rng.integers(64, 900)) if band == 1 else \
        int(rng.integers(900, 4000))
    return (M, 128 * int(rng.integers(1, 40)), 128 * int(rng.integers(1, 30)), int(rng.choice([0, 16, 32, 48, 64, 128])),
            bool(rng.integers(0, 4) == 0))


_BWD_CASES = [_bwd_case(_RNG) for _ in range(12)]


@pytest.mark.parametrize("M,K,N,r,w4", _BWD_CASES)
def test_backward_sweep(k2, dev, M, K, N, r, w4):
    """The backward through the frozen base (``gemm_dx``: the effective weight, each tile shape and split, the
    LoRA term in the epilogue) and the LoRA gradients (``lora_grads``) over seeded random shapes, against the
    float64 formulas: dx within the forward's bar, g, dA and dB within 2e-5 relative Frobenius."""
    L = k2._lib
    gen = torch.Generator().manual_seed(M * 13 + K + N + r)
    w = (torch.randn(N, K, generator=gen) * 0.02).to(torch.bfloat16)
    x = torch.randn(M, K, generator=gen).to(torch.bfloat16)
    dy = (torch.randn(M, N, generator=gen) * 1e-3).to(torch.bfloat16)
    A = torch.randn(r, K, generator=gen) * 0.01 if r else None
    B = torch.randn(N, r, generator=gen) * 0.01 if r else None
    u = (x.float() @ A.t()) if r else None
    s = 0.75
    if w4:
        qw, sw = L.quant_weight_i4(w.to(dev))
        qo, so = orc.quant_weight_i4(w.float().numpy())
    else:
        qw, sw = L.quant_weight_i8(w.to(dev))
        qo, so = orc.quant_weight_i8(w.float().numpy())
    g = dA = dB = None
    if r:
        g, dA, dB = L.lora_grads(dy.to(dev), x.to(dev), u.to(dev), B.to(dev), s)
    dx = L.gemm_dx(dy.to(dev), qw, sw, w4=w4, g=g, lora_a=A.to(dev) if r else None)
    torch.cuda.synchronize()
    ref = orc.backward(_np(dy), _np(x), qo, so, w4=w4, lora_A=None if A is None else A.numpy(),
                       lora_B=None if B is None else B.numpy(), lora_scale=s)
    assert np.linalg.norm(_np(dx) - ref["dx64"]) <= 4e-3 * np.linalg.norm(ref["dx64"])
    if r:
        for got, want in ((g, ref["g"]), (dA, ref["dA"]), (dB, ref["dB"])):
            assert np.linalg.norm(_np(got) - want) <= 2e-5 * np.linalg.norm(want)
