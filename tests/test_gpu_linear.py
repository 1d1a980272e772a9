"""GPU tests of ``k2q_linear_fwd``: one library call per quantized linear + LoRA forward (the module's path).

* M > 8: the call issues the same launches as the separate entry points (rotate/quant, LoRA down-projection,
  GEMM; or, where ``k2q_linear_fwd_fuses_down`` says so, rotate/quant with the down-projection in the same pass,
  then the GEMM), so codes, scales, u and y are bit-identical to calling them one by one.
* M <= 8: one prologue launch computes the codes (bit-identical to ``k2q_rotquant``) and u (an f32 dot product
  per rank: within f32 rounding of the down-projection kernel and of the float64 product), then the GEMV;
  y within the forward bar of the oracle.
* ``codes_ready``: codes computed elsewhere (a producer kernel) are used as given.
* No factors requested (inference): the GEMM epilogue adds the down-projection's K-slice partials itself
  (W8, r <= 128) or u stays in the workspace; y is bit-identical to the separate launches either way.
* W4A8 through the same call.
"""
import numpy as np
import pytest
import torch

from oracle import convrot as orc

pytestmark = pytest.mark.gpu


def rel_frob(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def _case(M, K, N, r, seed, dev, w4=False, bias=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    x[:, torch.randperm(K, generator=g)[: max(1, K // 100)]] *= 20
    x = x.to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(N, generator=g) * 0.02 if bias else None
    A = torch.randn(r, K, generator=g) * 0.01 if r else None
    B = torch.randn(N, r, generator=g) * 0.01 if r else None
    return x, w, b, A, B


@pytest.mark.parametrize("M,K,N,r,w4", [(512, 3072, 1024, 32, False), (300, 640, 384, 0, False),
                                        (1024, 12288, 3072, 16, False), (256, 512, 384, 48, True),
                                        (4096, 3072, 3072, 16, False), (700, 1024, 512, 128, False),
                                        (200, 2048, 256, 256, False), (64, 16384, 512, 64, False),
                                        (8192, 3072, 12288, 16, False), (4096, 3072, 3072, 16, True),
                                        (16896, 3072, 1024, 32, False), (1024, 2048, 512, 32, False)])
def test_one_call_equals_separate_launches(k2, dev, M, K, N, r, w4):
    L = k2._lib
    x, w, b, A, B = _case(M, K, N, r, M + K, dev, w4)
    xd, wd = x.to(dev), w.to(dev)
    bd = b.to(dev) if b is not None else None
    Ad = A.to(dev) if A is not None else None
    Bd = B.to(dev) if B is not None else None
    qw, sw = L.quant_weight_i4(wd) if w4 else L.quant_weight_i8(wd)
    qx = torch.empty(M, K, dtype=torch.int8, device=dev)
    sx = torch.empty(M, device=dev)
    y, u = L.linear_fwd(xd, qx, sx, False, Ad, Bd, 0.75, qw, sw, bd, w4)
    fused = bool(r) and L.linear_fwd_fuses_down(M, K, r)
    if fused:
        q0, s0, u0 = L.rotquant_lora(xd, Ad)
    else:
        q0, s0, _ = L.rotquant(xd)
        u0 = L.lora_down(xd, Ad) if r else None
    gemm = L.gemm_w4a8 if w4 else L.gemm_w8a8
    y0 = gemm(q0, s0, qw, sw, bd, u0, Bd, 0.75)
    assert torch.equal(qx, q0) and torch.equal(sx, s0) and torch.equal(y, y0)
    if r:
        assert torch.equal(u, u0)
        ref = orc.lora_down(x.float().numpy(), A.numpy())
        assert rel_frob(u.cpu().numpy(), ref) < 1e-5
    # codes given (as a producer kernel leaves them): the call uses them as they are, u from the down-projection
    y1, _ = L.linear_fwd(xd, q0, s0, True, Ad, Bd, 0.75, qw, sw, bd, w4)
    ud = L.lora_down(xd, Ad) if r else None
    assert torch.equal(y1, gemm(q0, s0, qw, sw, bd, ud, Bd, 0.75))
    # no factors requested (inference): W8 with r <= 128 folds the down-projection's reduce into the GEMM
    # epilogue, the other cases keep u in the workspace; y is the same bits either way
    y2, u2 = L.linear_fwd(xd, qx, sx, False, Ad, Bd, 0.75, qw, sw, bd, w4, need_u=False)
    assert u2 is None and torch.equal(y2, y0)


def test_fused_down_plan(k2):
    """The one-call forward takes u from the rotate/quant pass for K <= 3072 (K % 512 == 0) with r 16 or 32 when
    the 16-row tiles fit one round of CUs (two for r = 16), and issues the separate down-projection otherwise."""
    f = k2._lib.linear_fwd_fuses_down
    assert f(4096, 3072, 16) and f(1024, 3072, 16) and f(8192, 3072, 16) and f(4096, 3072, 32) and f(16, 1024, 32)
    assert not f(16896, 3072, 32) and not f(8208, 3072, 16) and not f(4112, 3072, 32)
    assert not f(4096, 6144, 16) and not f(4096, 3072, 64) and not f(4096, 640, 16) and not f(8, 3072, 16)
    assert not f(16, 512, 32)     # 32 ranks of wave partials do not fit where 16 rows of 512 sat in LDS


@pytest.mark.parametrize("M,K,N,r", [(1, 3072, 18432, 16), (2, 3072, 18432, 16), (5, 12288, 3072, 64),
                                     (8, 16384, 256, 128), (3, 640, 512, 0), (2, 6144, 2048, 256)])
def test_skinny_prologue_codes_and_factors(k2, dev, M, K, N, r):
    L = k2._lib
    x, w, b, A, B = _case(M, K, N, r, 3 * M + K, dev)
    xd = x.to(dev)
    qw, sw = L.quant_weight_i8(w.to(dev))
    Ad = A.to(dev) if A is not None else None
    Bd = B.to(dev) if B is not None else None
    qx = torch.full((M, K), 99, dtype=torch.int8, device=dev)
    sx = torch.zeros(M, device=dev)
    y, u = L.linear_fwd(xd, qx, sx, False, Ad, Bd, 1.0, qw, sw, b.to(dev), False)
    q0, s0, _ = L.rotquant(xd)
    assert torch.equal(qx, q0) and torch.equal(sx, s0)                       # bit-identical codes
    if r:
        u64 = orc.lora_down(x.float().numpy(), A.numpy())
        assert rel_frob(u.cpu().numpy(), u64) < 1e-6
    ref = orc.forward(x.float().numpy(), qw.cpu().numpy(), sw.cpu().numpy(), bias=b.numpy(),
                      lora_A=None if A is None else A.numpy(), lora_B=None if B is None else B.numpy(), lora_scale=1.0)
    assert rel_frob(y.float().cpu().numpy(), ref["y64"]) < 4e-3
    # LoRA factors only (codes given)
    if r:
        y2, u2 = L.linear_fwd(xd, q0, s0, True, Ad, Bd, 1.0, qw, sw, b.to(dev), False)
        assert torch.equal(u2, u) and torch.equal(y2, y)


def test_skinny_w4(k2, dev):
    L = k2._lib
    M, K, N, r = 2, 3072, 1024, 16
    x, w, b, A, B = _case(M, K, N, r, 77, dev, w4=True)
    q4, s4 = L.quant_weight_i4(w.to(dev))
    qx = torch.empty(M, K, dtype=torch.int8, device=dev)
    sx = torch.empty(M, device=dev)
    y, u = L.linear_fwd(x.to(dev), qx, sx, False, A.to(dev), B.to(dev), 1.0, q4, s4, b.to(dev), True)
    qo, so = orc.quant_weight_i4(w.float().numpy())
    ref = orc.forward(x.float().numpy(), qo, so, w4=True, bias=b.numpy(), lora_A=A.numpy(), lora_B=B.numpy(),
                      lora_scale=1.0)
    assert rel_frob(y.float().cpu().numpy(), ref["y64"]) < 4e-3


def test_workspace_only_where_used(k2, dev):
    """``k2q_linear_fwd`` takes ws = NULL where nothing of it is used (u given, u from the rotate/quant pass, no
    GEMM split) with the same output as with the full workspace, and refuses NULL where the factors need it."""
    L = k2._lib
    lib = L.load()
    M, K, N, r = 4096, 3072, 3072, 16
    assert L.linear_fwd_fuses_down(M, K, r) and lib.k2q_gemm_w8a8_ws_bytes(M, N, K) == 0
    x, w, b, A, B = _case(M, K, N, r, 91, dev)
    xd, Ad, Bd, bd = x.to(dev), A.to(dev), B.to(dev), b.to(dev)
    qw, sw = L.quant_weight_i8(w.to(dev))
    st = L._stream(dev)
    nws = lib.k2q_linear_fwd_ws_bytes(0, M, N, K, r)
    ws = torch.empty(nws, dtype=torch.uint8, device=dev)
    outs = []
    for wsp, wsb in ((ws.data_ptr(), nws), (None, 0)):
        qx = torch.empty(M, K, dtype=torch.int8, device=dev)
        sx = torch.empty(M, device=dev)
        u = torch.empty(M, r, device=dev)
        y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        assert lib.k2q_linear_fwd(xd.data_ptr(), K, M, K, qx.data_ptr(), sx.data_ptr(), 0, Ad.data_ptr(),
                                  Bd.data_ptr(), r, 0.5, u.data_ptr(), 0, qw.data_ptr(), sw.data_ptr(), bd.data_ptr(),
                                  N, y.data_ptr(), wsp, wsb, st) == 0
        outs.append((qx, sx, u, y))
    for a, c in zip(*outs):
        assert torch.equal(a, c)
    y2 = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    qx, sx, u = outs[0][:3]
    # codes given: the down-projection's partials live in ws, so NULL is refused; so is u = NULL without ws
    assert lib.k2q_linear_fwd(xd.data_ptr(), K, M, K, qx.data_ptr(), sx.data_ptr(), 1, Ad.data_ptr(), Bd.data_ptr(),
                              r, 0.5, u.data_ptr(), 0, qw.data_ptr(), sw.data_ptr(), bd.data_ptr(), N, y2.data_ptr(),
                              None, 0, st) == -1
    assert lib.k2q_linear_fwd(xd.data_ptr(), K, M, K, qx.data_ptr(), sx.data_ptr(), 0, Ad.data_ptr(), Bd.data_ptr(),
                              r, 0.5, None, 0, qw.data_ptr(), sw.data_ptr(), bd.data_ptr(), N, y2.data_ptr(),
                              None, 0, st) == -1
    torch.cuda.synchronize()
