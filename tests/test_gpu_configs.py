"""GPU parity at BASELINE.json's exact configuration shapes, and for every LoRA rank the reference accepts.

* Configs: cfg0 (W8A8, M=4096, K=N=3072, r=16, f32 bias), cfg1 (the same with int4 group-64 weights), cfg3's
  forward launch (M=4608, K=12288, N=3072, r=64: one round of full-K tiles) and all ten linears of cfg4's
  double-stream block (image M=8192 / text M=1024 x qkv 3072->9216, out 3072->3072, up 3072->12288,
  down 12288->3072, plus the adaLN modulation 3072->18432 at M=2 per stream), each run through the module path
  a user calls (``LoRALinear`` over ``ConvRotLinear``, split-K schedule and GEMV included).  Checked: weight and
  activation codes on sampled rows equal the oracle's; the int32 accumulators of every tile equal hipBLASLt's
  exact int8 GEMM (``torch._int_mm``); y on sampled rows within 4e-3 relative Frobenius of the oracle's float64
  forward (BASELINE bar 1e-2).  cfg2 is covered at full size in ``test_gpu_parity.py``.
* Ranks: ``LoRALinear`` (``lora.py:30-48``) at ranks 4, 8, 24 (padded to multiples of 16 with zero ranks) and
  256 (two 128-rank chunks) over the W8A8, W4A8 and fp8 bases runs on the library's kernels (the LoRA kernels
  are called; nothing falls back to torch matmuls) and matches the oracle forward and backward.
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


def synth_x(M, K, seed):
    """BASELINE.json activations: N(0,1) with 1% of the channels scaled x20, bf16."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    x[:, torch.randperm(K, generator=g)[: max(1, K // 100)]] *= 20
    return x.to(torch.bfloat16)


def build_layer(k2, dev, K, N, r, mode, bias, seed):
    """``LoRALinear`` (alpha = r, so scale 1) over a quantized base with BASELINE.json weights (N(0,0.02) bf16)
    and factors (N(0,0.01))."""
    g = torch.Generator().manual_seed(seed)
    lin = torch.nn.Linear(K, N, bias=bias, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_((torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16))
        if bias:
            lin.bias = torch.nn.Parameter(torch.randn(N, generator=g) * 0.02)     # f32 bias (cfg0)
    base = k2.Fp8Linear(lin.to(dev)) if mode == "fp8" else k2.ConvRotLinear(lin.to(dev), mode)
    layer = k2.LoRALinear(base, r, float(r))
    with torch.no_grad():
        layer.lora_A.copy_(torch.randn(r, K, generator=g) * 0.01)
        layer.lora_B.copy_(torch.randn(N, r, generator=g) * 0.01)
    return lin, base, layer


CONFIG_CASES = [
    # name, M, K, N, r, mode, bias
    ("cfg0", 4096, 3072, 3072, 16, "w8a8", True),
    ("cfg1", 4096, 3072, 3072, 16, "w4a8", True),
    ("cfg3.forward", 4608, 12288, 3072, 64, "w8a8", False),
    ("cfg4.image.qkv", 8192, 3072, 9216, 16, "w8a8", False),
    ("cfg4.image.out", 8192, 3072, 3072, 16, "w8a8", False),
    ("cfg4.image.up", 8192, 3072, 12288, 16, "w8a8", False),
    ("cfg4.image.down", 8192, 12288, 3072, 16, "w8a8", False),
    ("cfg4.image.adaln", 2, 3072, 18432, 16, "w8a8", False),
    ("cfg4.text.qkv", 1024, 3072, 9216, 16, "w8a8", False),
    ("cfg4.text.out", 1024, 3072, 3072, 16, "w8a8", False),
    ("cfg4.text.up", 1024, 3072, 12288, 16, "w8a8", False),
    ("cfg4.text.down", 1024, 12288, 3072, 16, "w8a8", False),
    ("cfg4.text.adaln", 2, 3072, 18432, 16, "w8a8", False),
]


@pytest.mark.timeout(300)
@pytest.mark.parametrize("name,M,K,N,r,mode,bias", CONFIG_CASES, ids=[c[0] for c in CONFIG_CASES])
def test_config_shape_module_forward(k2, dev, name, M, K, N, r, mode, bias):
    seed = M + 3 * K + 7 * N
    lin, base, layer = build_layer(k2, dev, K, N, r, mode, bias, seed)
    x = synth_x(M, K, seed + 1)
    xd = x.to(dev)
    with torch.no_grad():
        y = layer(xd)
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    L = k2._lib
    qx, sx, _ = L.rotquant(xd)
    rng = np.random.default_rng(seed)
    rows = np.arange(M) if M <= 32 else np.sort(np.concatenate([rng.choice(M - 1, 31, replace=False), [M - 1]]))
    w = lin.weight.detach().float().cpu().numpy()
    xs = x[torch.from_numpy(rows)].float().numpy()
    q0, s0, _ = orc.rotquant(xs)
    assert np.array_equal(qx.cpu().numpy()[rows], q0) and np.array_equal(sx.cpu().numpy()[rows], s0)
    if mode == "w8a8":
        qw0, sw0 = orc.quant_weight_i8(w)
        assert np.array_equal(base.qweight.cpu().numpy(), qw0)
        assert np.array_equal(base.weight_scale.cpu().numpy(), sw0)
        acc = L.gemm_w8a8_acc(qx, base.qweight)
        if M > 16:                                   # every tile against hipBLASLt's exact int8 GEMM
            assert torch.equal(acc, torch._int_mm(qx, base.qweight.t()))
        assert np.array_equal(acc.cpu().numpy()[rows], orc.gemm_acc(q0, qw0))
        qref, sref = qw0, sw0
    else:
        qw0, sb0 = orc.quant_weight_i4(w)
        assert np.array_equal(base.qweight.cpu().numpy(), orc.pack_i4(qw0))
        assert np.array_equal(base.wscale.cpu().numpy().view(np.uint16), np.ascontiguousarray(sb0.T))
        qref, sref = qw0, sb0
    bias_np = lin.bias.detach().float().cpu().numpy() if bias else None
    ref = orc.forward(xs, qref, sref, w4=mode == "w4a8", bias=bias_np, lora_A=layer.lora_A.detach().cpu().numpy(),
                      lora_B=layer.lora_B.detach().cpu().numpy(), lora_scale=1.0)
    err = rel_frob(y.float().cpu().numpy()[rows], ref["y64"])
    assert err < 4e-3, (name, err)


def _count_calls(monkeypatch, L, names):
    calls = {n: 0 for n in names}
    for n in names:
        real = getattr(L, n)

        def wrapped(*a, _real=real, _n=n, **kw):
            calls[_n] += 1
            return _real(*a, **kw)
        monkeypatch.setattr(L, n, wrapped)
    return calls


@pytest.mark.timeout(300)
@pytest.mark.parametrize("mode", ["w8a8", "w4a8", "fp8"])
@pytest.mark.parametrize("rank", [4, 8, 24, 256])
def test_lora_any_rank_runs_on_the_kernels(k2, dev, monkeypatch, mode, rank):
    """Forward and backward of ``LoRALinear`` at a rank the kernels do not take directly, against the oracle
    (ConvRot bases) or float64 autograd of the reference's dequantized fp8 weight (``quantize.py:48-51``)."""
    M, K, N = 320, 512, 384
    lin, base, layer = build_layer(k2, dev, K, N, rank, mode, True, 100 + rank)
    layer.scale_mul = -0.75                                          # a slider setting (lora.py:37)
    s = layer.scale * layer.scale_mul
    calls = _count_calls(monkeypatch, k2._lib, ("lora_down", "lora_grads"))
    real_fwd = k2._lib.linear_fwd

    def fwd(x2, qx, sx, ready, A, B, *rest):
        calls["lora_down"] += A is not None        # the one-call forward runs the down-projection inside
        return real_fwd(x2, qx, sx, ready, A, B, *rest)
    monkeypatch.setattr(k2._lib, "linear_fwd", fwd)
    x = synth_x(M, K, rank)
    dy = (torch.randn(M, N, generator=torch.Generator().manual_seed(rank)) * 1e-3).to(torch.bfloat16)
    xd = x.to(dev).requires_grad_(True)
    y = layer(xd)
    y.backward(dy.to(dev))
    assert calls["lora_down"] >= 1 and calls["lora_grads"] == 1       # the adapter ran on the HIP kernels
    A, B = layer.lora_A.detach().cpu(), layer.lora_B.detach().cpu()
    assert layer.lora_A.grad.shape == (rank, K) and layer.lora_B.grad.shape == (N, rank)
    bias = lin.bias.detach().float().cpu()
    if mode == "fp8":
        q0, s0 = orc.fp8_weight_quant(lin.weight.detach().float().cpu().numpy())
        yb = orc.fp8_linear(x, q0, s0, lin.bias.detach().cpu())
        y_ref = (yb.double() + s * ((x.double() @ A.double().t()) @ B.double().t())).numpy()
        wd = (q0.to(torch.bfloat16) * s0.to(torch.bfloat16)).double()
        x64 = x.double().requires_grad_(True)
        A64, B64 = A.double().requires_grad_(True), B.double().requires_grad_(True)
        (x64 @ wd.t() + s * (x64 @ A64.t()) @ B64.t()).backward(dy.double())
        dx_ref, dA_ref, dB_ref = x64.grad.numpy(), A64.grad.numpy(), B64.grad.numpy()
    else:
        w = lin.weight.detach().float().cpu().numpy()
        w4 = mode == "w4a8"
        qo, so = orc.quant_weight_i4(w) if w4 else orc.quant_weight_i8(w)
        fw = orc.forward(x.float().numpy(), qo, so, w4=w4, bias=bias.numpy(), lora_A=A.numpy(), lora_B=B.numpy(),
                         lora_scale=s)
        bw = orc.backward(dy.float().numpy(), x.float().numpy(), qo, so, w4=w4, lora_A=A.numpy(), lora_B=B.numpy(),
                          lora_scale=s)
        y_ref, dx_ref, dA_ref, dB_ref = fw["y64"], bw["dx64"], bw["dA"], bw["dB"]
    assert rel_frob(y.detach().float().cpu().numpy(), y_ref) < 4e-3
    assert rel_frob(xd.grad.float().cpu().numpy(), dx_ref) < 1e-2
    assert rel_frob(layer.lora_A.grad.cpu().numpy(), dA_ref) < 1e-3
    assert rel_frob(layer.lora_B.grad.cpu().numpy(), dB_ref) < 1e-3
