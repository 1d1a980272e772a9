"""GPU tests of the grouped W8A8 forward (``k2q_gemm_w8a8_grouped``), the grouped input gradient
(``k2q_gemm_dx_grouped``) and of ``group_siblings``.

* Forward kernel: every segment's output is bit-identical to ``k2q_gemm_w8a8`` of that segment alone on the
  same codes (full-K tiles), with and without bias / adapter per segment, ragged M, and the Krea 2
  attention-input shapes (6144 -> 6144 | 1536 | 1536 | 6144).
* Input-gradient kernel: the segmented reduction equals ``k2q_gemm_dx_lin`` over the concatenated operands
  bit for bit (same stage order, full-K tiles), one-stage segments and row-strided output gradients included,
  and the float64 sum within bf16 rounding.
* LoRA gradients (``k2q_lora_grads_grouped``): every member's g bit-identical to ``k2q_lora_grads`` of that
  member alone, written in the stacked layout; the stacked dA (one pass over x per 128 stacked ranks, a shorter
  last chunk in its own launch) and each member's dB against float64, with ragged widths, row-strided output
  gradients, eight members and dB requested for some members only.
* Module: a restated block's attention inputs and SwiGLU gate / up grouped against the same block ungrouped:
  forward within one bf16 rounding (the stacked LoRA down-projection may add in another order), gradients
  within the bars of the per-layer path, one grouped launch per group, a checkpointed backward equal to a
  plain one, and a member whose adapter changed between the calls running its own forward.
"""
import copy

import pytest
import torch

from restated_block import FEAT, Dit

pytestmark = pytest.mark.gpu


def _codes(M, N, K, g, dev):
    q = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(dev)
    s = (torch.rand(M, generator=g) * 0.05 + 0.01).to(dev)
    return q, s


def _segment(N, K, r, g, dev, bias, lora):
    qw = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
    sw = (torch.rand(N, generator=g) * 0.01 + 0.001).to(dev)
    b = (torch.randn(N, generator=g) * 0.1).to(dev) if bias else None
    lb = (torch.randn(N, r, generator=g) * 0.05).to(dev) if lora else None
    return qw, sw, b, lb


@pytest.mark.parametrize("M,K,Ns,r", [(300, 768, (512, 256, 256, 512), 16), (1000, 1024, (256, 768), 32),
                                      (4608, 6144, (6144, 1536, 1536, 6144), 16)])
def test_grouped_equals_separate(k2, dev, M, K, Ns, r):
    L = k2._lib
    g = torch.Generator().manual_seed(M + K)
    qx, sx = _codes(M, sum(Ns), K, g, dev)
    segs = [_segment(N, K, r, g, dev, bias=(i % 2 == 0), lora=(i != 1)) for i, N in enumerate(Ns)]
    nl = sum(lb is not None for *_, lb in segs)
    u = torch.randn(M, nl * r, generator=g).to(dev)
    args, col = [], 0
    for i, (qw, sw, b, lb) in enumerate(segs):
        scale = 0.5 + 0.25 * i
        args.append((qw, sw, b, lb, col if lb is not None else 0, scale))
        col += r if lb is not None else 0
    ys = L.gemm_w8a8_grouped(qx, sx, args, u)
    for (qw, sw, b, lb, c, scale), y in zip(args, ys):
        uc = u[:, c:c + r].contiguous() if lb is not None else None
        ref = L.gemm_w8a8(qx, sx, qw, sw, b, uc, lb, scale, split=False)
        assert torch.equal(y, ref)


def test_grouped_argument_checks(k2, dev):
    L = k2._lib
    g = torch.Generator().manual_seed(1)
    qx, sx = _codes(64, 512, 256, g, dev)
    seg = _segment(384, 256, 16, g, dev, False, False)        # 384 is not a multiple of 256
    with pytest.raises(ValueError):
        L.gemm_w8a8_grouped(qx, sx, [(*seg, 0, 1.0)])
    ok = _segment(256, 256, 16, g, dev, False, False)
    with pytest.raises(ValueError):
        L.gemm_w8a8_grouped(qx, sx, [(*ok, 0, 1.0)] * 5)      # at most 4 segments
    with pytest.raises(ValueError):
        L.gemm_w8a8_grouped(qx[:8], sx[:8], [(*ok, 0, 1.0)])  # skinny M runs the GEMV per linear


@pytest.mark.parametrize("M,K,Ns,r,strided", [(300, 640, (512, 64, 128, 256), 48, True),
                                               (1000, 1024, (64, 64), 16, False),
                                               (4608, 6144, (6144, 1536, 1536, 6144), 64, False),
                                               (257, 384, (1024,), 0, True)])
def test_dx_grouped_equals_concatenated(k2, dev, M, K, Ns, r, strided):
    L = k2._lib
    g = torch.Generator().manual_seed(M + K + len(Ns))
    big = (torch.randn(M, sum(Ns) + 64 * strided, generator=g) * 1e-2).to(torch.bfloat16).to(dev)
    dys, col = [], 0
    for N in Ns:                                       # strided: every dy a column slice of one wider tensor
        d = big[:, col:col + N]
        dys.append(d if strided else d.contiguous())
        col += N
    wts = [(torch.randn(K, N, generator=g) * 0.02).to(torch.bfloat16).to(dev) for N in Ns]
    gg = (torch.randn(M, r, generator=g) * 1e-3).to(dev) if r else None
    A = (torch.randn(r, K, generator=g) * 0.01).to(dev) if r else None
    dx = L.gemm_dx_grouped(list(zip(dys, wts)), gg, A)
    dy_cat = torch.cat([d.contiguous() for d in dys], dim=1)
    wt_cat = torch.cat(wts, dim=1).contiguous()
    N = dy_cat.shape[1]
    dummy_q = torch.zeros(N, K, dtype=torch.int8, device=dev)
    ref = L.gemm_dx(dy_cat, dummy_q, torch.ones(N, device=dev), g=gg, lora_a=A, wt=wt_cat, split=False)
    assert torch.equal(dx, ref)
    ref64 = dy_cat.double() @ wt_cat.double().t()
    if r:
        ref64 += gg.double() @ A.double()
    err = (dx.double() - ref64).norm() / ref64.norm()
    assert err < 4e-3


@pytest.mark.parametrize("M,K,Ns,r,want", [(700, 1024, (512, 256, 256, 512), 16, None),
                                           (333, 768, (384, 640), 64, None),
                                           (64, 512, (128,) * 8, 16, None),
                                           (1024, 640, (256, 384, 128), 128, (True, False, True)),
                                           (200, 512, (256, 256, 256), 48, (False, True, False)),
                                           (4608, 6144, (6144, 1536, 1536, 6144), 16, None)])
def test_lora_grads_grouped_matches_members(k2, dev, M, K, Ns, r, want):
    """g_i = s_i dY_i B_i, dA_i = g_i^T x, dB_i = s_i dY_i^T u_i for linears sharing x, in one grouped call:
    g bit-identical to each member's own ``k2q_lora_grads`` (same down-projection and slice sums), dA and dB
    within 2e-5 of float64 (their slice plans differ from the single calls').  The last case is the Krea 2
    attention-input group at full size (dA and dB checked against the single calls there)."""
    g = torch.Generator().manual_seed(M + K + r)
    n = len(Ns)
    x = (torch.randn(M, K, generator=g)).to(torch.bfloat16)
    u = torch.randn(M, n * r, generator=g)
    # the members' output gradients as column blocks of one wider tensor: rows of stride sum(Ns) + 128
    wide = (torch.randn(M, sum(Ns) + 128, generator=g) * 1e-3).to(torch.bfloat16).to(dev)
    offs = [sum(Ns[:i]) for i in range(n)]
    dys = [wide[:, o:o + N] for o, N in zip(offs, Ns)]
    Bs = [torch.randn(N, r, generator=g).mul(0.01).to(dev) for N in Ns]
    scales = [0.5 + 0.25 * i for i in range(n)]
    xd, ud = x.to(dev), u.to(dev)
    gst, dA, dBs = k2._lib.lora_grads_grouped(dys, xd, ud, Bs, scales, want)
    big = M * K > 10 ** 7
    for i in range(n):
        gi, dAi, dBi = k2._lib.lora_grads(dys[i].contiguous(), xd, ud[:, i * r:(i + 1) * r].contiguous(), Bs[i],
                                          scales[i])
        assert torch.equal(gst[:, i * r:(i + 1) * r], gi), i
        if want is not None and not want[i]:
            assert dBs[i] is None
        if big:
            assert _rel(dA[i * r:(i + 1) * r], dAi) < 1e-5 and _rel(dBs[i], dBi) < 1e-5, i
            continue
        dy64 = dys[i].double().cpu()
        g64 = scales[i] * (dy64 @ Bs[i].double().cpu())
        assert _rel(dA[i * r:(i + 1) * r].cpu(), g64.t() @ x.double()) < 2e-5, i
        if dBs[i] is not None:
            assert _rel(dBs[i].cpu(), scales[i] * (dy64.t() @ u[:, i * r:(i + 1) * r].double())) < 2e-5, i
    # without x: no dA, the same g
    g2, dA2, _ = k2._lib.lora_grads_grouped(dys, None, ud, Bs, scales, want)
    assert dA2 is None and torch.equal(g2, gst)


def test_lora_grads_grouped_argument_checks(k2, dev):
    M, K, r = 64, 256, 16
    x = torch.zeros(M, K, dtype=torch.bfloat16, device=dev)
    u = torch.zeros(M, 2 * r, device=dev)
    dys = [torch.zeros(M, 128, dtype=torch.bfloat16, device=dev)] * 2
    Bs = [torch.zeros(128, r, device=dev)] * 2
    with pytest.raises(ValueError, match="members"):
        k2._lib.lora_grads_grouped(dys * 5, x, torch.zeros(M, 10 * r, device=dev), Bs * 5, [1.0] * 10)
    with pytest.raises(ValueError, match="rank"):
        k2._lib.lora_grads_grouped(dys, x, torch.zeros(M, 2 * 256, device=dev),
                                   [torch.zeros(128, 256, device=dev)] * 2, [1.0] * 2)
    with pytest.raises(ValueError, match="lora_B"):
        k2._lib.lora_grads_grouped(dys, x, u, [Bs[0], torch.zeros(128, 32, device=dev)], [1.0] * 2)
    with pytest.raises(ValueError, match="stacked"):
        k2._lib.lora_grads_grouped(dys, x, torch.zeros(M, r, device=dev), Bs, [1.0] * 2)
    lib = k2._lib.load()
    assert lib.k2q_lora_grads_grouped_ws_bytes(None, 2, M, K, r) == 0
    assert lib.k2q_lora_grads_grouped(None, 2, x.data_ptr(), u.data_ptr(), r, M, K, u.data_ptr(), None, None, 0,
                                      torch.cuda.current_stream(dev).cuda_stream) == -1


def test_dx_grouped_argument_checks(k2, dev):
    L = k2._lib
    dy = torch.zeros(64, 128, dtype=torch.bfloat16, device=dev)
    wt = torch.zeros(256, 128, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        L.gemm_dx_grouped([(dy, wt)] * 5)                                   # at most 4 segments
    with pytest.raises(ValueError):
        L.gemm_dx_grouped([(dy[:, :96], wt[:, :96])])                      # N % 64
    with pytest.raises(ValueError):
        L.gemm_dx_grouped([(dy, wt), (dy[:32], wt)])                       # M differs
    with pytest.raises(ValueError):
        L.gemm_dx_grouped([(dy, wt)], torch.zeros(64, 16, device=dev), torch.zeros(16, 100, device=dev))


def _build(k2, dev, rank=16):
    g = torch.Generator().manual_seed(3)
    dit = Dit()
    with torch.no_grad():
        for name, p in sorted(dit.named_parameters()):
            sc = 0.1 if ("scale" in name or "lin" in name) else 1.0 / p.shape[-1] ** 0.5
            p.copy_(torch.randn(p.shape, generator=g) * sc)
    dit = dit.to(torch.bfloat16).to(dev)
    assert k2.quantize_dit_convrot(dit, "w8a8") == 16
    ad = k2.inject_lora(dit, rank, include_txtfusion=False, include_txtmlp=False)
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
    return h.detach(), xr.grad.detach(), {k: (m.lora_A.grad.clone(), m.lora_B.grad.clone()) for k, m in ad.items()}


def _rel(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm())


@pytest.mark.timeout(300)
def test_group_siblings_matches_ungrouped(k2, dev, monkeypatch):
    dit, ad = _build(k2, dev)
    gdit = copy.deepcopy(dit)
    gad = {k: gdit.get_submodule(k) for k in ad}
    assert k2.group_siblings(gdit) == 4           # (wq, wk, wv, gate) and (gate, up) per block
    calls = []
    real = k2._lib.gemm_w8a8_grouped
    monkeypatch.setattr(k2._lib, "gemm_w8a8_grouped", lambda *a, **kw: calls.append(1) or real(*a, **kw))
    g = torch.Generator().manual_seed(4)
    B, Lt = 2, 256
    x = (torch.randn(B, Lt, FEAT, generator=g)).to(torch.bfloat16).to(dev)
    vec = (torch.randn(B, 1, 6 * FEAT, generator=g) * 0.3).to(torch.bfloat16).to(dev)
    dy = (torch.randn(B, Lt, FEAT, generator=g) * 1e-2).to(torch.bfloat16).to(dev)

    y0, dx0, gr0 = _step(dit, ad, x, vec, dy)
    y1, dx1, gr1 = _step(gdit, gad, x, vec, dy)
    torch.cuda.synchronize()
    assert len(calls) == 4                        # one grouped launch per group and block forward
    # u differs in the last bits between the routes (ungrouped, the first linear on a tensor takes u from the
    # rotate/quant pass at these sizes, the others from the down-projection; grouped, one stacked
    # down-projection), which moves a few bf16 outputs by one step; the next layers requantize those outputs, so
    # a moved element can flip an int8 code, and through attention's backward that moves the upstream gradients:
    # hence the block-level bars (the layer-level test below is tighter)
    assert _rel(y1, y0) < 5e-3
    assert _rel(dx1, dx0) < 1e-2
    for k in gr0:
        assert _rel(gr1[k][0], gr0[k][0]) < 2e-2 and _rel(gr1[k][1], gr0[k][1]) < 2e-2, k

    # checkpoint recompute runs the grouped forward again, bit for bit
    y2, dx2, gr2 = _step(gdit, gad, x, vec, dy, ckpt=True)
    assert torch.equal(y2, y1) and torch.equal(dx2, dx1)
    for k in gr1:
        assert torch.equal(gr2[k][0], gr1[k][0]) and torch.equal(gr2[k][1], gr1[k][1]), k


@pytest.mark.parametrize("rank", [16, 32, 64, 24])
def test_grouped_layer_gradients(k2, dev, rank):
    """The four attention inputs on one tensor with fixed output gradients: grouped against each member's own
    forward / backward (same codes; only the stacked LoRA down-projection's summation order differs).  The
    stacked rank is 4 x rank: 64 .. 256 (the reference's default rank 64 stacks to 256, two 128-rank chunks of
    the down-projection); rank 24 is padded to 32 per member."""
    dit, ad = _build(k2, dev, rank)
    gdit = copy.deepcopy(dit)
    assert k2.group_siblings(gdit) == 4
    names = ("wq", "wk", "wv", "gate")
    g = torch.Generator().manual_seed(6)
    x = (torch.randn(2, 192, FEAT, generator=g)).to(torch.bfloat16).to(dev)
    res = []
    for d in (dit, gdit):
        attn = d.blocks[0].attn
        mods = [getattr(attn, n) for n in names]
        for m in mods:
            m.lora_A.grad = m.lora_B.grad = None
        xr = x.clone().requires_grad_(True)
        ys = [m(xr) for m in mods]
        gg = torch.Generator().manual_seed(7)
        loss = sum((y.float() * (torch.randn(y.shape, generator=gg) * 1e-2).to(dev)).sum() for y in ys)
        loss.backward()
        res.append((ys, xr.grad, [(m.lora_A.grad, m.lora_B.grad) for m in mods]))
    (ys0, dx0, g0), (ys1, dx1, g1) = res
    for a, b in zip(ys1, ys0):
        assert (a.float() - b.float()).abs().max() <= b.float().abs().max() * 2 ** -7
    # dX: four bf16 gradients added at the shared input in bf16, by autograd ungrouped and by the grouped
    # backward in member order; the two orders differ by that rounding noise (~0.3%), inside the 1e-2 bar
    assert _rel(dx1, dx0) < 1e-2
    for (a1, b1), (a0, b0) in zip(g1, g0):
        assert _rel(a1, a0) < 1e-3 and _rel(b1, b0) < 1e-4


def test_grouped_forward_follows_adapter_updates(k2, dev):
    """The group keeps its members' stacked LoRA A rows between launches; an in-place update of the adapters
    (what an optimizer step does) must reach the next grouped forward: after the same update on both models,
    grouped outputs match the ungrouped ones again, and differ from the pre-update outputs."""
    dit, _ = _build(k2, dev)
    gdit = copy.deepcopy(dit)
    assert k2.group_siblings(gdit) == 4
    names = ("wq", "wk", "wv", "gate")
    g = torch.Generator().manual_seed(17)
    xs = [(torch.randn(2, 96, FEAT, generator=g)).to(torch.bfloat16).to(dev) for _ in range(3)]
    outs = []
    for step, x in enumerate(xs):
        if step:
            for d in (dit, gdit):
                for n in names:
                    m = getattr(d.blocks[0].attn, n)
                    with torch.no_grad():
                        m.lora_A.add_(0.01 * step)
                        m.lora_B.add_(0.002 * step)
        with torch.no_grad():
            y0 = [getattr(dit.blocks[0].attn, n)(x) for n in names]
            y1 = [getattr(gdit.blocks[0].attn, n)(x) for n in names]
        for a, b in zip(y1, y0):
            assert (a.float() - b.float()).abs().max() <= b.float().abs().max() * 2 ** -7
        outs.append(y1)
    # the updates changed what the adapters add
    assert not torch.equal(outs[2][0], getattr(gdit.blocks[0].attn, "wq").base(xs[2]))


def test_grouped_unused_outputs_get_no_gradient_pass(k2, dev):
    """Members whose outputs reach no loss (here wk and wv) get no backward work in the grouped node, as
    ungrouped autograd would skip their nodes: their adapters get no gradient, and dX and the used members'
    gradients match the ungrouped block's."""
    dit, ad = _build(k2, dev)
    gdit = copy.deepcopy(dit)
    assert k2.group_siblings(gdit) == 4
    names = ("wq", "wk", "wv", "gate")
    g = torch.Generator().manual_seed(16)
    x = (torch.randn(2, 160, FEAT, generator=g)).to(torch.bfloat16).to(dev)
    w = (torch.randn(2, 160, FEAT, generator=g) * 1e-2).to(dev)
    res = []
    for d in (dit, gdit):
        mods = [getattr(d.blocks[0].attn, n) for n in names]
        for m in mods:
            m.lora_A.grad = m.lora_B.grad = None
        xr = x.clone().requires_grad_(True)
        q, _k, _v, gt = (m(xr) for m in mods)
        ((q.float() * torch.sigmoid(gt.float())) * w).sum().backward()
        res.append((xr.grad, [(m.lora_A.grad, m.lora_B.grad) for m in mods]))
    (dx0, g0), (dx1, g1) = res
    assert _rel(dx1, dx0) < 1e-2
    for i in (1, 2):
        assert g0[i] == (None, None) and g1[i] == (None, None), names[i]
    for i in (0, 3):
        assert _rel(g1[i][0], g0[i][0]) < 1e-3 and _rel(g1[i][1], g0[i][1]) < 1e-4, names[i]


def test_group_member_with_changed_adapter_runs_alone(k2, dev):
    dit, _ = _build(k2, dev)
    assert k2.group_siblings(dit) == 4
    attn = dit.blocks[0].attn
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(2, 64, FEAT, generator=g)).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        q = attn.wq(x)                                 # runs the group, keeps wk / wv / gate
        attn.wk.scale_mul = 0.0                        # wk's kept output no longer applies
        k = attn.wk(x)
        v = attn.wv(x)
        ref_k = type(attn.wk).forward(attn.wk, x)      # the member's own forward: exactly base(x)
        ref_v = type(attn.wv).forward(attn.wv, x)
        ref_q = type(attn.wq).forward(attn.wq, x)
    assert torch.equal(k, ref_k)
    assert torch.equal(k, attn.wk.base(x))
    assert (v.float() - ref_v.float()).abs().max() <= ref_v.float().abs().max() * 2 ** -7
    assert (q.float() - ref_q.float()).abs().max() <= ref_q.float().abs().max() * 2 ** -7


@pytest.mark.timeout(300)
def test_producers_and_grouping_together(k2, dev):
    """fuse_producers and group_siblings on the same blocks: the patched block forward feeds the grouped
    attention inputs the codes its fused RMSNorm produced (no rotate/quant for them), outputs and gradients
    stay within the bf16 bars of the plain block, and a checkpointed backward equals a plain one bit for bit."""
    from krea2_amd.quantize import shared_input_quant
    dit, ad = _build(k2, dev)
    fdit = copy.deepcopy(dit)
    fad = {k: fdit.get_submodule(k) for k in ad}
    assert k2.fuse_producers(fdit) == 4 and k2.group_siblings(fdit) == 4
    g = torch.Generator().manual_seed(8)
    B, Lt = 2, 128
    x = (torch.randn(B, Lt, FEAT, generator=g)).to(torch.bfloat16).to(dev)
    vec = (torch.randn(B, 1, 6 * FEAT, generator=g) * 0.3).to(torch.bfloat16).to(dev)
    dy = (torch.randn(B, Lt, FEAT, generator=g) * 1e-2).to(torch.bfloat16).to(dev)
    y0, dx0, gr0 = _step(dit, ad, x, vec, dy)
    m0 = shared_input_quant.misses
    y1, dx1, gr1 = _step(fdit, fad, x, vec, dy)
    assert shared_input_quant.misses - m0 == 2    # only the attention output (wo's input), once per block
    assert _rel(y1, y0) < 1e-2 and _rel(dx1, dx0) < 1e-2
    for k in gr0:
        assert _rel(gr1[k][0], gr0[k][0]) < 2e-2 and _rel(gr1[k][1], gr0[k][1]) < 2e-2, k
    y2, dx2, gr2 = _step(fdit, fad, x, vec, dy, ckpt=True)
    assert torch.equal(y2, y1) and torch.equal(dx2, dx1)
    for k in gr1:
        assert torch.equal(gr2[k][0], gr1[k][0]) and torch.equal(gr2[k][1], gr1[k][1]), k


@pytest.mark.timeout(300)
def test_fusions_at_krea_width(k2, dev):
    """One block at the real Krea 2 widths (6144, 48 heads of 128 with 12 KV heads, SwiGLU 16384): the fused
    producers at K = 6144 / 16384 and the grouped 6144 | 1536 | 1536 | 6144 attention inputs against the same
    quantized block without them, within the bf16 bars, and a bit-identical checkpointed recompute."""
    dims = dict(feat=6144, heads=48, kvheads=12, hid=16384)
    g = torch.Generator().manual_seed(9)
    dit = Dit(1, **dims)
    with torch.no_grad():
        for name, p in sorted(dit.named_parameters()):
            sc = 0.1 if ("scale" in name or "lin" in name) else 1.0 / p.shape[-1] ** 0.5
            p.copy_(torch.randn(p.shape, generator=g) * sc)
    dit = dit.to(torch.bfloat16).to(dev)
    assert k2.quantize_dit_convrot(dit, "w8a8") == 8
    ad = k2.inject_lora(dit, 16, include_txtfusion=False, include_txtmlp=False)
    with torch.no_grad():
        for m in ad.values():
            m.lora_B.copy_(torch.randn(m.lora_B.shape, generator=g) * 0.01)
    fdit = copy.deepcopy(dit)
    fad = {k: fdit.get_submodule(k) for k in ad}
    assert k2.fuse_producers(fdit) == 2 and k2.group_siblings(fdit) == 2
    B, Lt, D = 2, 256, dims["feat"]
    x = torch.randn(B, Lt, D, generator=g).to(torch.bfloat16).to(dev)
    vec = (torch.randn(B, 1, 6 * D, generator=g) * 0.3).to(torch.bfloat16).to(dev)
    dy = (torch.randn(B, Lt, D, generator=g) * 1e-2).to(torch.bfloat16).to(dev)
    y0, dx0, gr0 = _step(dit, ad, x, vec, dy)
    y1, dx1, gr1 = _step(fdit, fad, x, vec, dy)
    assert _rel(y1, y0) < 1e-2 and _rel(dx1, dx0) < 1e-2
    for k in gr0:
        assert _rel(gr1[k][0], gr0[k][0]) < 2e-2 and _rel(gr1[k][1], gr0[k][1]) < 2e-2, k
    y2, dx2, gr2 = _step(fdit, fad, x, vec, dy, ckpt=True)
    assert torch.equal(y2, y1) and torch.equal(dx2, dx1)
    for k in gr1:
        assert torch.equal(gr2[k][0], gr1[k][0]) and torch.equal(gr2[k][1], gr1[k][1]), k


@pytest.mark.timeout(300)
def test_block_forward_replays_in_a_hip_graph(k2, dev):
    """A fused, grouped block forward (producers, grouped attention inputs, every ConvRot GEMM and LoRA
    kernel) captured once in a HIP graph and replayed three times on new input data, with eager work and
    synchronizations between the replays: every replay equals the eager forward bit for bit."""
    dit, _ = _build(k2, dev)
    assert k2.fuse_producers(dit) == 4 and k2.group_siblings(dit) == 4
    g = torch.Generator().manual_seed(10)
    B, Lt = 2, 128
    vec = (torch.randn(B, 1, 6 * FEAT, generator=g) * 0.3).to(torch.bfloat16).to(dev)
    xs = [torch.randn(B, Lt, FEAT, generator=g).to(torch.bfloat16).to(dev) for _ in range(3)]

    def fwd(x):
        h = x
        for blk in dit.blocks:
            h = blk(h, vec, None)
        return h

    static_x = xs[0].clone()
    with torch.no_grad():
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                fwd(static_x)                      # warm-up on the capture stream
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_y = fwd(static_x)
        for x in xs:
            static_x.copy_(x)
            graph.replay()
            torch.cuda.synchronize()
            got = static_y.clone()
            ref = fwd(x.clone())                   # eager, between the replays
            torch.cuda.synchronize()
            assert torch.equal(got, ref)
