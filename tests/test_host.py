"""CPU tests of the boundary: the C-ABI library loads and exports every symbol ``include/k2q.h`` declares,
host-side validation rejects bad arguments before any launch, and the module satisfies the reference's
duck-typed contract (``quantize.py:31-46``, ``lora.py:27-116``, ``mmdit.py:409-414``).  No GPU needed."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import convrot as orc

ROOT = Path(__file__).resolve().parents[1]


def header_symbols():
    text = (ROOT / "include" / "k2q.h").read_text()
    return sorted(set(re.findall(r"^(?:const char\*|int|int64_t)\s+(k2q_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol(k2):
    lib = k2._lib.load()
    syms = header_symbols()
    assert len(syms) >= 12
    for name in syms:
        assert hasattr(lib, name), name
    assert sorted(k2._lib.EXPORTS) == syms
    assert k2._lib.version().startswith("k2q")


def test_library_is_gfx950_only():
    out = (ROOT / "krea-2_amd" / "libk2q.so").read_bytes()
    assert b"gfx950" in out
    for other in (b"gfx942", b"gfx90a", b"sm_"):
        assert other + b"\x00" not in out or other == b"sm_"


def test_status_codes_for_bad_arguments_without_gpu(k2):
    """Entry points reject invalid shapes/pointers with K2Q_EINVAL before touching the device."""
    lib = k2._lib.load()
    buf = ctypes.create_string_buffer(4096 + 16)
    p = (ctypes.addressof(buf) + 15) // 16 * 16
    assert lib.k2q_rotquant(p, 0, 4, 100, 100, p, p, None, None) == -1        # K % 128
    assert lib.k2q_rotquant(p, 7, 4, 128, 128, p, p, None, None) == -1        # dtype
    assert lib.k2q_rotquant(None, 0, 4, 128, 128, p, p, None, None) == -1     # null
    assert lib.k2q_rotquant(p + 2, 0, 4, 128, 128, p, p, None, None) == -1    # misaligned
    assert lib.k2q_rotquant(p, 0, 4, 32768, 32768, p, p, None, None) == -4    # K too large
    assert lib.k2q_gemm_w8a8(p, p, p, p, None, p, p, 8, 1.0, 4, 4, 128, p, None, 0, None) == -1   # rank 8
    assert lib.k2q_gemm_w8a8(p, p, p, p, None, None, None, 0, 0.0, 4, 6, 128, p, None, 0, None) == -1  # N % 4
    assert lib.k2q_gemm_dx(p, p, 4, 96, 128, None, None, 0, p, None, 0, None) == -1    # N % 64
    assert lib.k2q_lora_down(p, 4, 128, 128, p, 200, p, 0, p, None) == -1    # rank % 16
    assert lib.k2q_lora_down(p, 4, 128, 128, p, 8192, p, 0, p, None) == -1   # rank > K2Q_MAX_RANK
    assert lib.k2q_lora_down(p, 4, 100, 100, p, 16, None, 0, p, None) == -1  # K % 128
    assert lib.k2q_lora_down_ws_bytes(4, 128, 200) == 0                      # no plan for a bad rank
    # ranks above 128 run as 128-rank chunks sharing one workspace: the largest chunk's K-slice partials
    assert lib.k2q_lora_down_ws_bytes(4096, 3072, 256) == lib.k2q_lora_down_ws_bytes(4096, 3072, 128) > 0
    assert lib.k2q_lora_grads_ws_bytes(4096, 3072, 3072, 256) > lib.k2q_lora_grads_ws_bytes(4096, 3072, 3072, 128)
    assert lib.k2q_lora_grads_ws_bytes(4096, 3072, 3072, 8192) == 0
    # grouped LoRA gradients: members, ranks and widths are checked before any launch
    mem = (k2._lib.LoraMember * 2)(k2._lib.LoraMember(p, 3072, 3072, p, 1.0, None),
                                   k2._lib.LoraMember(p, 1536, 1536, p, 1.0, None))
    addr = ctypes.addressof(mem)
    assert lib.k2q_lora_grads_grouped_ws_bytes(addr, 2, 4608, 6144, 64) > 0
    assert lib.k2q_lora_grads_grouped_ws_bytes(addr, 2, 4608, 6144, 256) == 0     # rank above 128
    assert lib.k2q_lora_grads_grouped_ws_bytes(addr, 9, 4608, 6144, 64) == 0      # more than 8 members
    assert lib.k2q_lora_grads_grouped_ws_bytes(addr, 2, 4608, 100, 64) == 0       # K % 128
    mem[1].N = 1000                                                               # out_features % 128
    assert lib.k2q_lora_grads_grouped_ws_bytes(addr, 2, 4608, 6144, 64) == 0
    mem[1].N, mem[1].ldy = 1536, 1000                                             # row stride below N
    assert lib.k2q_lora_grads_grouped_ws_bytes(addr, 2, 4608, 6144, 64) == 0
    assert lib.k2q_lora_grads_grouped(addr, 2, p, p, 64, 4608, 6144, p, p, p, 0, None) == -1
    # a GEMM operand whose 320-row tile spans 2 GiB or more (the copies' buffer offsets are 31-bit): refused
    seg = k2._lib.DxSegment(p, 1 << 23, p, 64)        # dy rows 16 MiB apart
    assert lib.k2q_gemm_dx_grouped(ctypes.addressof(seg), 1, 4608, 6144, None, 0, None, 0, p, None) == -4


# MI355X timings (us, one GEMM launch incl. epilogue) of each output tile shape on the shapes the chooser was
# fitted to: (M, N, K) -> (fastest shape, its time, the 256x256 time).  The chooser must take the fastest.
TILE_TIMINGS = {
    (16896, 12288, 3072): ("256x320", 585.2, 609.1),     # cfg2
    (4096, 3072, 3072): ("192x256", 42.7, 43.7),         # cfg0
    (1024, 3072, 3072): ("128x128", 20.3, 36.8),         # cfg4 text out
    (1024, 9216, 3072): ("192x256", 36.1, 39.7),         # cfg4 text qkv
    (1024, 12288, 3072): ("192x256", 42.6, 43.1),        # cfg4 text up
    (1024, 3072, 12288): ("128x128", 65.4, 67.2),        # cfg4 text down
    (8192, 3072, 3072): ("192x256", 82.3, 84.4),         # cfg4 image out
    (8192, 9216, 3072): ("256x320", 227.3, 228.6),       # cfg4 image qkv
    (8192, 12288, 3072): ("256x256", 289.9, 289.9),      # cfg4 image up
    (8192, 3072, 12288): ("192x256", 269.6, 287.2),      # cfg4 image down
    (4608, 3072, 12288): ("256x256", 159.3, 159.3),      # cfg3 forward
    (4608, 1536, 6144): ("128x128", 56.1, 67.4),         # d=6144 wk/wv, 2304+2304 tokens
    (4608, 16384, 6144): ("256x320", 420.6, 422.1),      # d=6144 up
    (16896, 6144, 6144): ("256x320", 547.6, 582.8),      # d=6144 wq, 16896 tokens
}


@pytest.mark.parametrize("shape", list(TILE_TIMINGS), ids=["x".join(map(str, s)) for s in TILE_TIMINGS])
def test_gemm_plan_takes_the_fastest_measured_tile(k2, shape):
    M, N, K = shape
    tile, pieces = k2._lib.gemm_w8a8_plan(M, N, K, 256)
    assert tile == TILE_TIMINGS[shape][0] and pieces >= 1


def test_gemm_plan_edges(k2):
    L = k2._lib
    assert L.gemm_w8a8_plan(2, 18432, 3072) == ("gemv", 1)          # adaLN modulation: M <= 8
    assert L.gemm_w8a8_plan(9, 512, 128)[0] in L.TILES
    # a last round of 256x256 tiles that is cut along K: a GPU whose CUs the tiles fill a little over once
    assert L.gemm_w8a8_plan(1024, 4608, 16384, 256) == ("256x256", 3)
    # one round of 128x128 tiles over a long reduction is cut along K (measured 70.5 -> 62.8 us for cfg4's
    # text-stream down projection, 66.9 -> 46.9 us at N = 2048); a short one is not (text out: 23.6 -> 28.6)
    assert L.gemm_w8a8_plan(1024, 3072, 12288, 256) == ("128x128", 2)
    assert L.gemm_w8a8_plan(1024, 2048, 12288, 256) == ("128x128", 4)
    assert L.gemm_w8a8_plan(1024, 3072, 3072, 256) == ("128x128", 1)
    # grouped launches take no 192-row tiles (segments start on 256- or 128-row boundaries)
    assert L.gemm_w8a8_plan(4096, 3072, 3072) == ("192x256", 1)
    assert L.gemm_w8a8_plan(4096, 3072, 3072, grouped=True)[0] != "192x256"
    with pytest.raises(RuntimeError):
        L.gemm_w8a8_plan(4, 4, 100)


def test_forward_takes_down_projection_from_the_rotquant_pass_where_measured_faster(k2):
    """The one-call forward's route for u, decided on the host (the CU count is the MI355X's 256 without a GPU):
    the rotate/quant pass computes it for K <= 3072 (K % 512 == 0), r 16 or 32, while the 16-row tiles fit one
    round of CUs (two for r = 16); otherwise rotate/quant and the down-projection are separate launches."""
    f = k2._lib.linear_fwd_fuses_down
    assert f(4096, 3072, 16) and f(8192, 3072, 16) and f(4096, 3072, 32) and f(9, 1024, 32)   # cfg0/1, cfg4
    assert not f(16896, 3072, 32)        # cfg2: 1056 tiles, streaming A per tile measured slower
    assert not f(8193, 3072, 16) and not f(4097, 3072, 32)
    assert not f(4608, 12288, 64) and not f(4096, 6144, 16) and not f(4096, 3072, 64) and not f(8, 3072, 16)
    assert k2._lib.rotquant_lora_fits(3072, 64) and not k2._lib.rotquant_lora_fits(4096, 16)
    assert not k2._lib.rotquant_lora_fits(512, 32)      # 32 ranks of partials exceed 16 rows of 512 in LDS


def test_wrappers_validate_before_launch(k2):
    L = k2._lib
    # grouped LoRA gradients: member count and rank before anything touches a device
    dy = torch.zeros(4, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="members"):
        L.lora_grads_grouped([dy] * 9, None, None, [torch.zeros(128, 16)] * 9, [1.0] * 9)
    with pytest.raises(ValueError, match="above 128"):
        L.lora_grads_grouped([dy], None, None, [torch.zeros(128, 256)], [1.0])
    with pytest.raises(ValueError):
        L.lora_grads_grouped([dy], None, None, [torch.zeros(128, 24)], [1.0])       # rank % 16
    with pytest.raises(ValueError):
        L.rotquant(torch.zeros(4, 100, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        L.rotquant(torch.zeros(4, 256, dtype=torch.float16))
    with pytest.raises(ValueError):
        L.rotquant(torch.zeros(256, 4, dtype=torch.bfloat16).t())
    with pytest.raises(ValueError):
        L.gemm_w8a8(torch.zeros(4, 128, dtype=torch.int8), torch.zeros(4), torch.zeros(8, 256, dtype=torch.int8),
                    torch.zeros(8))
    with pytest.raises(ValueError):
        L.lora_down(torch.zeros(4, 128, dtype=torch.bfloat16), torch.zeros(12, 128))
    with pytest.raises(RuntimeError):          # valid shapes, CPU tensors: refuses, never computes on CPU
        L.rotquant(torch.zeros(4, 128, dtype=torch.bfloat16))


def _cpu_quantized(N=64, K=256, mode="w8a8", bias=True, seed=0):
    """A ConvRotLinear assembled from oracle-quantized tensors (CPU; no kernel runs)."""
    import __graft_entry__ as ge
    k2 = ge.load_package()
    rng = np.random.default_rng(seed)
    W = orc.bf16_round((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    b = torch.randn(N, dtype=torch.bfloat16) if bias else None
    if mode == "w8a8":
        q, s = orc.quant_weight_i8(W)
        return k2.ConvRotLinear.from_quantized(torch.from_numpy(q), torch.from_numpy(s).view(torch.int32), b, mode)
    q, s_bits = orc.quant_weight_i4(W)
    return k2.ConvRotLinear.from_quantized(torch.from_numpy(orc.pack_i4(q)),
                                           torch.from_numpy(np.ascontiguousarray(s_bits.T)).view(torch.int16), b,
                                           mode)


@pytest.mark.parametrize("mode", ["w8a8", "w4a8"])
def test_module_contract(k2, mode):
    m = _cpu_quantized(mode=mode)
    assert m.is_quant_linear is True and type(m).is_quant_linear is True
    assert (m.in_features, m.out_features) == (256, 64)
    assert m.weight is m.qweight and m.weight.device.type == "cpu"
    assert isinstance(m.bias, nn.Parameter)
    params = dict(m.named_parameters())
    assert set(params) == {"qweight", "wscale", "bias"}
    assert all(not p.requires_grad for p in params.values())
    # Module.to(dtype) casts floating parameters only: codes and scale bits stay exact
    before = {k: v.clone() for k, v in params.items()}
    m.to(torch.float16)
    assert m.qweight.dtype == before["qweight"].dtype and torch.equal(m.qweight, before["qweight"])
    assert torch.equal(m.wscale, before["wscale"])
    assert m.bias.dtype == torch.float16
    if mode == "w8a8":
        assert m.weight_scale.dtype == torch.float32 and m.weight_scale.shape == (64,)
    else:
        assert m.weight_scale.dtype == torch.bfloat16 and m.weight_scale.shape == (4, 64)


def test_block_swap_repoints_parameters(k2):
    """mmdit.py:409-414 pages with ``p.data = p.data.to(device)``; the module reads pointers per call."""
    m = _cpu_quantized()
    ptr = m.qweight.data_ptr()
    for p in m.parameters():
        p.data = p.data.clone()
    assert m.qweight.data_ptr() != ptr and m.weight is m.qweight


class _Block(nn.Module):
    """Block-shaped module with the reference's Linear names (mmdit.py:170-175, 188-194)."""

    def __init__(self, d=256, h=512):
        super().__init__()
        self.attn = nn.Module()
        for n, o in (("wq", d), ("wk", d // 2), ("wv", d // 2), ("gate", d), ("wo", d)):
            setattr(self.attn, n, nn.Linear(d, o, bias=False))
        self.mlp = nn.Module()
        self.mlp.gate = nn.Linear(d, h, bias=False)
        self.mlp.up = nn.Linear(d, h, bias=False)
        self.mlp.down = nn.Linear(h, d, bias=False)


class _Dit(nn.Module):
    def __init__(self, n=2):
        super().__init__()
        self.first = nn.Linear(64, 256)
        self.blocks = nn.ModuleList(_Block() for _ in range(n))


def test_inject_lora_accepts_quantized_bases_by_duck_typing(k2):
    dit = _Dit()
    for blk in dit.blocks:   # swap in pre-quantized bases the way the walker would
        for mod in list(blk.modules()):
            for name, child in list(mod.named_children()):
                if isinstance(child, nn.Linear):
                    setattr(mod, name, _cpu_quantized(child.out_features, child.in_features, bias=False))
    adapters = k2.inject_lora(dit, 16, include_txtfusion=False, include_txtmlp=False)
    assert len(adapters) == 16
    assert set(adapters) == {f"blocks.{i}.{t}" for i in range(2) for t in k2.DEFAULT_TARGETS}
    a = adapters["blocks.0.mlp.down"]
    assert isinstance(a.base, k2.ConvRotLinear) and a.lora_A.shape == (16, 512) and a.lora_B.shape == (256, 16)
    assert a.scale == 1.0 and a.scale_mul == 1.0 and torch.all(a.lora_B == 0)
    assert all(not p.requires_grad for p in a.base.parameters())
    assert next(dit.parameters()).dtype == torch.float32     # dtype probe stays the first Linear's
    with k2.lora_scaled(dit, -2.0):
        assert all(m.scale_mul == -2.0 for m in adapters.values())
    with k2.lora_disabled(dit):
        assert all(m.scale_mul == 0.0 for m in adapters.values())
    assert all(m.scale_mul == 1.0 for m in adapters.values())


def test_lora_over_quantized_base_rejects_shapes_the_kernels_do_not_take(k2):
    """A LoRA over a quantized base runs only on the library's kernels, which take in/out features in multiples
    of 128: other shapes are refused when the adapter is built (not with a torch fallback, not mid-step)."""
    base = _cpu_quantized(N=64, K=256)
    with pytest.raises(ValueError, match="multiples of 128"):
        k2.LoRALinear(base, 16, 16.0)
    with pytest.raises(ValueError, match="rank"):
        k2.LoRALinear(_cpu_quantized(N=128, K=256), 0, 1.0)
    with pytest.raises(ValueError, match="multiple of 64"):
        _cpu_quantized(N=96, K=256)


@pytest.mark.parametrize("rank", [4, 8, 16, 24, 200])
def test_lora_kernel_factors_pad_ranks_with_zeros(k2, rank):
    """The fused path hands the kernels the factors padded to a multiple of 16 ranks with zeros (an exact no-op
    in every sum); gradients reach the unpadded parameters only."""
    m = k2.LoRALinear(_cpu_quantized(N=128, K=256), rank, float(rank))
    nn.init.normal_(m.lora_B)
    A, B = m._kernel_factors()
    rp = -(-rank // 16) * 16
    assert A.shape == (rp, 256) and B.shape == (128, rp) and A.dtype == B.dtype == torch.float32
    assert torch.equal(A[:rank], m.lora_A) and torch.equal(B[:, :rank], m.lora_B)
    assert not A[rank:].any() and not B[:, rank:].any()
    (A.sum() + 2 * B.sum()).backward()
    assert m.lora_A.grad.shape == (rank, 256) and torch.all(m.lora_A.grad == 1)
    assert m.lora_B.grad.shape == (128, rank) and torch.all(m.lora_B.grad == 2)


def test_inject_lora_raises_without_targets(k2):
    dit = _Dit()
    for blk in dit.blocks:
        blk.attn = nn.Module()
        blk.mlp = nn.Module()
    with pytest.raises(RuntimeError):
        k2.inject_lora(dit, 16, include_txtfusion=False, include_txtmlp=False)


def test_save_load_lora_roundtrip(k2, tmp_path):
    dit = _Dit()
    adapters = k2.inject_lora(dit, 16, include_txtfusion=False, include_txtmlp=False)
    for m in adapters.values():
        nn.init.normal_(m.lora_B)
    path = str(tmp_path / "a.safetensors")
    k2.save_lora(adapters, path, rank=16, alpha=16.0)
    from safetensors import safe_open
    with safe_open(path, "pt") as f:
        assert f.metadata()["format"] == "krea2-lora"
        assert "diffusion_model.blocks.1.mlp.up.lora_A.weight" in f.keys()
    dit2 = _Dit()
    ad2 = k2.load_lora(dit2, path)
    for n, m in adapters.items():
        assert torch.equal(ad2[n].lora_B, m.lora_B.detach().to(torch.bfloat16).float())


def test_trainer_import_lines_resolve_from_the_package(k2):
    """Every name the reference's trainers and samplers import from ``lora`` (``train_t2i_lora_cached.py:22``,
    ``train_slider.py:28``, ``sample.py:23``, ``eval_t2i.py:27``) comes from the package, so the whole import line
    switches at once."""
    lines = {
        "train_t2i_lora_cached.py:22": "inject_lora, inject_lora_te, load_lora_weights, lora_parameters, save_lora",
        "train_slider.py:28": "inject_lora, lora_parameters, lora_scaled, lora_disabled, save_lora",
        "sample.py:23": "load_lora, lora_scaled",
    }
    for where, names in lines.items():
        ns = {}
        exec(f"from krea2_amd import {names}", ns)
        assert all(callable(ns[n.strip()]) for n in names.split(",")), where
    assert k2.QWEN_TE_TARGETS == ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


class _QwenLayer(nn.Module):
    """A decoder layer with the Qwen3 projection names (what ``inject_lora_te`` matches by leaf name)."""

    def __init__(self, d=32, h=64):
        super().__init__()
        self.self_attn = nn.Module()
        for n in ("q_proj", "k_proj", "v_proj", "o_proj"):
            setattr(self.self_attn, n, nn.Linear(d, d, bias=False))
        self.mlp = nn.Module()
        self.mlp.gate_proj = nn.Linear(d, h, bias=False)
        self.mlp.up_proj = nn.Linear(d, h, bias=False)
        self.mlp.down_proj = nn.Linear(h, d, bias=False)
        self.mlp.act = nn.SiLU()


class _ToyQwen(nn.Module):
    """Language model plus a vision tower that reuses the same projection names (which must stay unadapted)."""

    def __init__(self):
        super().__init__()
        self.model = nn.Module()
        self.model.language_model = nn.Module()
        self.model.language_model.layers = nn.ModuleList(_QwenLayer() for _ in range(2))
        self.model.language_model.embed_tokens = nn.Embedding(10, 32)
        self.model.visual = nn.Module()
        self.model.visual.blocks = nn.ModuleList(_QwenLayer() for _ in range(1))
        self.lm_head = nn.Linear(32, 10, bias=False)


def test_inject_lora_te_wraps_language_projections_and_skips_vision(k2):
    torch.manual_seed(0)
    qwen = _ToyQwen()
    x = torch.randn(3, 32)
    before = qwen.model.language_model.layers[0].mlp.down_proj(qwen.model.language_model.layers[0].mlp.up_proj(x))
    adapters = k2.inject_lora_te(qwen, 4)
    leaves = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj", "mlp.gate_proj",
              "mlp.up_proj", "mlp.down_proj")
    assert set(adapters) == {f"model.language_model.layers.{i}.{leaf}" for i in range(2) for leaf in leaves}
    for path, m in adapters.items():
        assert isinstance(m, k2.LoRALinear) and qwen.get_submodule(path) is m
        assert m.rank == 4 and m.scale == 1.0 and m.lora_A.dtype == torch.float32 and not m.lora_B.any()
    # the vision tower and the head are left as they were; every base parameter is frozen
    vis = qwen.model.visual.blocks[0]
    assert all(type(getattr(vis.self_attn, n)) is nn.Linear for n in ("q_proj", "k_proj", "v_proj", "o_proj"))
    assert type(vis.mlp.down_proj) is nn.Linear and type(qwen.lm_head) is nn.Linear
    assert not any(p.requires_grad for n, p in qwen.named_parameters() if "lora_" not in n)
    assert all(p.requires_grad for p in k2.lora_parameters(adapters))
    # B = 0: the wrapped layers compute what the plain ones did; then the reference's expression
    lay = qwen.model.language_model.layers[0].mlp
    assert torch.equal(lay.down_proj(lay.up_proj(x)), before)
    nn.init.normal_(lay.up_proj.lora_B)
    want = lay.up_proj.base(x) + ((x @ lay.up_proj.lora_A.t()) @ lay.up_proj.lora_B.t())
    torch.testing.assert_close(lay.up_proj(x), want, rtol=0, atol=0)
    with k2.lora_disabled(qwen):
        assert torch.equal(lay.up_proj(x), lay.up_proj.base(x))
    # a custom alpha and target subset; no match at all raises
    q2 = _ToyQwen()
    ad2 = k2.inject_lora_te(q2, 8, alpha=4.0, targets=("q_proj",))
    assert len(ad2) == 2 and all(m.scale == 0.5 for m in ad2.values())
    with pytest.raises(RuntimeError):
        k2.inject_lora_te(_ToyQwen(), 4, targets=("no_such_proj",))


def test_save_lora_file_gets_the_default_permissions(k2, tmp_path):
    """The adapter file is renamed into place with the mode a plainly created file gets (umask applied)."""
    import os
    import stat
    dit = _Dit()
    adapters = k2.inject_lora(dit, 16, include_txtfusion=False, include_txtmlp=False)
    path = tmp_path / "a.safetensors"
    k2.save_lora(adapters, str(path), rank=16, alpha=16.0, key_prefix="text_encoder")
    plain = tmp_path / "plain"
    plain.write_bytes(b"")
    assert stat.S_IMODE(os.stat(path).st_mode) == stat.S_IMODE(os.stat(plain).st_mode)
    assert sorted(p.name for p in tmp_path.iterdir()) == ["a.safetensors", "plain"]    # no temp file left
    from safetensors import safe_open
    with safe_open(str(path), "pt") as f:
        assert "text_encoder.blocks.0.attn.wq.lora_A.weight" in f.keys()


def test_effective_weight_cache_logic_on_cpu(k2, monkeypatch):
    """The effective input-gradient weight's cache, with the library's builder replaced by a CPU stand-in: off by
    default (built per call, nothing kept); on, kept as a plain attribute keyed to the codes' storage, rebuilt
    after they move, released by the next build anywhere once its layer's codes have left the device they were
    built on, and dropped when the cache is switched off.  Parameters are codes, scales and bias only."""
    builds = []

    def fake_dx_weight(q, s, w4=False):
        builds.append(q.data_ptr())
        return torch.zeros(q.shape[1], q.shape[0], dtype=torch.bfloat16, device=q.device)

    monkeypatch.setattr(k2._lib, "dx_weight", fake_dx_weight)
    a, b = _cpu_quantized(N=128, K=256), _cpu_quantized(N=128, K=256, seed=1)
    assert a.keep_dx_weight is False
    a.dx_weight()
    assert a.dx_weight_kept is None and len(builds) == 1                 # default: per call, nothing kept
    assert {n for n, _ in a.named_parameters()} == {"qweight", "wscale", "bias"}
    holder = nn.ModuleList([a, b])
    assert k2.set_dx_weight_cache(holder, True) == 2
    w1 = a.dx_weight()
    assert a.dx_weight() is w1 and len(builds) == 2                      # kept and reused
    assert not isinstance(w1, nn.Parameter) and not any("dx" in k for k in a.state_dict())
    assert {n for n, _ in a.named_parameters()} == {"qweight", "wscale", "bias"}
    for p in a.parameters():                                             # "paged out" (re-pointed elsewhere)
        p.data = p.data.clone()
    assert a.dx_weight_kept is w1                                        # stays until some build runs
    b.dx_weight()                                                        # another layer's build releases it
    assert a.dx_weight_kept is None and b.dx_weight_kept is not None
    w2 = a.dx_weight()
    assert w2 is not w1 and len(builds) == 4
    with torch.no_grad():
        a.qweight.add_(0)                                                # in-place write: version bump
    assert a.dx_weight() is not w2
    k2.set_dx_weight_cache(holder, False)
    assert a.dx_weight_kept is None and b.dx_weight_kept is None


def test_walker_requires_gpu_and_says_so(k2):
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    with pytest.raises(RuntimeError, match="GPU"):
        k2.quantize_dit_convrot(_Dit(), "w8a8")


# ------------------------------------------------------------------------------------------- on-disk base
def _tiny_dit():
    class Blk(nn.Module):
        def __init__(self):
            super().__init__()
            self.attn = nn.Module()
            self.attn.wq = nn.Linear(256, 128, bias=True, dtype=torch.bfloat16)
            self.mlp = nn.Module()
            self.mlp.up = nn.Linear(128, 256, bias=False, dtype=torch.bfloat16)

    class Dit(nn.Module):
        def __init__(self):
            super().__init__()
            self.first = nn.Linear(8, 128, dtype=torch.bfloat16)
            self.blocks = nn.ModuleList([Blk(), Blk()])
    return Dit()


def _fill_quantized(k2, dit, seed=0):
    """Replace the block Linears with quantized modules built from random stored tensors (no GPU needed)."""
    g = torch.Generator().manual_seed(seed)
    kinds = ["w8a8", "w4a8", "fp8", "w8a8"]
    i = 0
    for bi, blk in enumerate(dit.blocks):
        for parent, name in ((blk.attn, "wq"), (blk.mlp, "up")):
            lin = getattr(parent, name)
            N, K = lin.out_features, lin.in_features
            bias = torch.randn(N, generator=g) if lin.bias is not None else None
            kind = kinds[i % len(kinds)]
            i += 1
            if kind == "w8a8":
                m = k2.ConvRotLinear.from_quantized(torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8),
                                                    torch.rand(N, generator=g).view(torch.int32), bias, "w8a8")
            elif kind == "w4a8":
                m = k2.ConvRotLinear.from_quantized(torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.uint8),
                                                    torch.rand(K // 64, N, generator=g).to(torch.bfloat16).view(torch.int16),
                                                    bias, "w4a8")
            else:
                q = torch.randint(0, 256, (N, K), generator=g, dtype=torch.uint8)
                q[q == 0x7F] = 0
                q[q == 0xFF] = 0
                m = k2.Fp8Linear.from_quantized(q.view(torch.float8_e4m3fn),
                                                torch.rand(N, 1, generator=g).to(torch.bfloat16), bias)
            setattr(parent, name, m)


def _state(dit):
    return {k: v.view(torch.uint8) if v.dtype == torch.float8_e4m3fn else v for k, v in dit.state_dict().items()}


def test_quantized_base_save_load_roundtrip(k2, tmp_path):
    """Every mode (w8a8, w4a8 packed int4 with group-major scales, fp8) round-trips bit for bit, whether
    saved before or after inject_lora (the LoRA wrapper's `.base` is not part of the key)."""
    src = _tiny_dit()
    _fill_quantized(k2, src)
    f1 = str(tmp_path / "base.safetensors")
    assert k2.save_quantized_base(src, f1) == 4
    k2.inject_lora(src, 16, include_txtfusion=False, include_txtmlp=False)
    f2 = str(tmp_path / "base_after_lora.safetensors")
    assert k2.save_quantized_base(src, f2) == 4
    from safetensors import safe_open
    with safe_open(f1, framework="pt") as a, safe_open(f2, framework="pt") as b:
        assert sorted(a.keys()) == sorted(b.keys())
        assert "blocks.0.attn.wq.qweight" in a.keys() and "blocks.1.attn.wq.weight_fp8" in a.keys()
        assert a.metadata()["format"] == "krea2-quantized-base" and a.metadata()["modes"] == "fp8,w4a8,w8a8"
    dst = _tiny_dit()
    assert k2.load_quantized_base(dst, f1) == 4
    assert isinstance(dst.first, nn.Linear) and isinstance(dst.blocks[0].mlp.up, k2.ConvRotLinear)
    ref = _tiny_dit()
    _fill_quantized(k2, ref)
    s_ref, s_dst = _state(ref), _state(dst)
    assert s_ref.keys() == s_dst.keys()
    for k in s_ref:
        if k.startswith("blocks"):
            assert torch.equal(s_ref[k], s_dst[k]), k
    assert dst.blocks[0].mlp.up.mode == "w4a8" and dst.blocks[0].attn.wq.mode == "w8a8"


def test_quantized_base_load_rejects_mismatches(k2, tmp_path):
    src = _tiny_dit()
    _fill_quantized(k2, src)
    f = str(tmp_path / "base.safetensors")
    k2.save_quantized_base(src, f)
    wrong = _tiny_dit()
    wrong.blocks[1].mlp.up = nn.Linear(128, 384, bias=False, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        k2.load_quantized_base(wrong, f)
    extra = _tiny_dit()
    extra.blocks.append(extra.blocks[0].__class__())
    with pytest.raises(KeyError):
        k2.load_quantized_base(extra, f)
    from safetensors.torch import save_file
    g = str(tmp_path / "other.safetensors")
    save_file({"x": torch.zeros(1)}, g, metadata={"format": "krea2-lora"})
    with pytest.raises(ValueError):
        k2.load_quantized_base(_tiny_dit(), g)
    with pytest.raises(ValueError):
        k2.save_quantized_base(_tiny_dit(), str(tmp_path / "none.safetensors"))


def test_new_entry_points_reject_bad_arguments_without_gpu(k2):
    """The producer, producer-backward and grouped entry points return K2Q_EINVAL / K2Q_EUNSUPPORTED for invalid
    shapes and pointers before touching the device."""
    lib = k2._lib.load()
    buf = ctypes.create_string_buffer(8192 + 16)
    p = (ctypes.addressof(buf) + 15) // 16 * 16
    assert lib.k2q_swiglu_rotquant(p, 128, p, 128, 4, 100, p, p, p, None) == -1      # K % 128
    assert lib.k2q_swiglu_rotquant(p, 64, p, 128, 4, 128, p, p, p, None) == -1       # row stride < K
    assert lib.k2q_swiglu_rotquant(p, 32768, p, 32768, 4, 32768, p, p, p, None) == -4  # K too large
    assert lib.k2q_rmsmod_rotquant(p, 128, 4, 128, p, 1e-5, p, p, 0, 0, p, p, p, None) == -1   # rows per batch
    assert lib.k2q_rmsmod_rotquant(p, 128, 4, 128, p, -1.0, p, p, 0, 4, p, p, p, None) == -1   # eps
    assert lib.k2q_rmsmod_rotquant(p, 128, 4, 128, p, 1e-5, p + 2, p, 0, 4, p, p, p, None) == -1  # misaligned
    assert lib.k2q_rmsmod_bwd(p, p, 4, 12, p, 1e-5, p, 0, 4, p, None) == -1             # K % 8
    assert lib.k2q_rmsmod_bwd(p, p, 4, 32768, p, 1e-5, p, 0, 4, p, None) == -4          # K too large
    assert lib.k2q_swiglu_bwd(p, p, p, 12, p, p, None) == -1                           # n % 8
    seg = (k2._lib.W8A8Segment * 5)()
    for s in seg:
        s.qw = s.sw = s.y = p
        s.N, s.u_col, s.lora_scale = 256, 0, 1.0
    assert lib.k2q_gemm_w8a8_grouped(p, p, 64, 128, ctypes.cast(seg, ctypes.c_void_p), 5, None, 0, 0,
                                     None, 0, None) == -1                                # > 4 segments
    assert lib.k2q_gemm_w8a8_grouped(p, p, 8, 128, ctypes.cast(seg, ctypes.c_void_p), 1, None, 0, 0,
                                     None, 0, None) == -1                                # M <= 8
    seg[0].N = 384
    assert lib.k2q_gemm_w8a8_grouped(p, p, 64, 128, ctypes.cast(seg, ctypes.c_void_p), 1, None, 0, 0,
                                     None, 0, None) == -1                                # N % 256


def test_fusion_walkers_leave_unquantized_blocks_alone(k2):
    """fuse_producers / group_siblings patch only blocks whose linears are ConvRot (w8a8 for grouping):
    plain nn.Linear blocks are left untouched, and the host-side checks of the fused ops raise before any
    launch."""
    dit = _Dit()
    assert k2.fuse_producers(dit) == 0 and k2.group_siblings(dit) == 0
    assert "forward" not in vars(dit.blocks[0].attn.wq) and "forward" not in vars(dit.blocks[0])
    x = torch.zeros(2, 8, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        k2.swiglu(x, x[..., :128])
    with pytest.raises(NotImplementedError):
        k2.swiglu(x.float(), x.float())
    norm = nn.Module()
    norm.scale, norm.eps = nn.Parameter(torch.zeros(256), requires_grad=False), 1e-5
    sc = torch.zeros(3, 1, 256, dtype=torch.bfloat16)                    # 3 entries for a batch of 2
    with pytest.raises(ValueError):
        k2.modulated_rmsnorm(norm, x, sc, sc)
    with pytest.raises(ValueError):
        k2.modulated_rmsnorm(norm, x, sc[:2], sc[:2, :, :128])
    with pytest.raises(RuntimeError):                                    # valid shapes, CPU: refuses
        k2.modulated_rmsnorm(norm, x, sc[:2], sc[:2])
    # the fused norm differentiates its input only: a trainable norm scale or modulation is refused up front
    norm.scale.requires_grad_(True)
    with pytest.raises(NotImplementedError, match="frozen"):
        k2.modulated_rmsnorm(norm, x, sc[:2], sc[:2])
    norm.scale.requires_grad_(False)
    with pytest.raises(NotImplementedError, match="frozen"):
        k2.modulated_rmsnorm(norm, x, sc[:2].requires_grad_(True), sc[:2])
    with torch.no_grad(), pytest.raises(RuntimeError):                   # no autograd: only the CPU refusal
        k2.modulated_rmsnorm(norm, x, sc[:2].requires_grad_(True), sc[:2])


def test_fused_block_runs_its_own_forward_when_norms_train(k2):
    """A block patched by fuse_producers computes the gradients of its input only through the fused norm; when its
    norm scale or modulation needs a gradient it runs the block class's own forward instead (checked on the CPU,
    with the block's linears swapped back to plain ones after patching: the class forward then runs entirely
    here, while the fused forward would reach the library and refuse CPU tensors)."""
    from tests import restated_block as rb
    torch.manual_seed(0)
    blk = rb.Block(feat=256, heads=2, kvheads=1, hid=512)
    plain = {n: getattr(blk.attn, n) for n in ("wq",)} | {"gate": blk.mlp.gate}
    blk.attn.wq = _cpu_quantized(N=256, K=256, bias=False)
    blk.mlp.gate = _cpu_quantized(N=512, K=256, bias=False)
    blk.mlp.down = _cpu_quantized(N=256, K=512, bias=False)
    dit = nn.Module()
    dit.blocks = nn.ModuleList([blk])
    assert k2.fuse_producers(dit) == 2 and "forward" in vars(blk)
    blk.attn.wq, blk.mlp.gate = plain["wq"], plain["gate"]
    blk.mlp.down = nn.Linear(512, 256, bias=False)
    del blk.mlp.forward                       # the SwiGLU patch is not under test here
    blk.requires_grad_(False)
    x = torch.randn(2, 8, 256)
    vec = torch.randn(2, 1, 6 * 256) * 0.1
    blk.prenorm.scale.requires_grad_(True)
    y = blk(x, vec, None)
    torch.testing.assert_close(y, rb.Block.forward(blk, x, vec, None), rtol=0, atol=0)
    y.sum().backward()
    assert blk.prenorm.scale.grad is not None and blk.prenorm.scale.grad.abs().sum() > 0
    blk.prenorm.scale.requires_grad_(False)
    blk.mod.lin.requires_grad_(True)          # the modulation trains: the class forward again
    torch.testing.assert_close(blk(x, vec, None), rb.Block.forward(blk, x, vec, None), rtol=0, atol=0)
    blk.mod.lin.requires_grad_(False)
    with pytest.raises(RuntimeError):         # frozen norms: the fused path, which refuses CPU tensors
        blk(x.bfloat16(), vec.bfloat16(), None)


def test_grouped_wrapper_validates_before_launch(k2):
    L = k2._lib
    q = torch.zeros(64, 256, dtype=torch.int8)
    s = torch.zeros(64)
    seg = (torch.zeros(384, 256, dtype=torch.int8), torch.zeros(384), None, None, 0, 1.0)
    with pytest.raises(ValueError):                                      # N % 256
        L.gemm_w8a8_grouped(q, s, [seg])
    ok = (torch.zeros(256, 256, dtype=torch.int8), torch.zeros(256), None, torch.zeros(256, 16), 0, 1.0)
    with pytest.raises(ValueError):                                      # an adapter without u
        L.gemm_w8a8_grouped(q, s, [ok])
    with pytest.raises(ValueError):                                      # u columns out of range
        L.gemm_w8a8_grouped(q, s, [ok[:4] + (8, 1.0)], torch.zeros(64, 16))
