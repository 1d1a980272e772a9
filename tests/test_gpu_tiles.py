"""GPU tests of the GEMM's output tile shapes (256x256, 256x320, 192x256, 128x128; ``K2Q_TILE_*``).

Each launch picks a shape with a cost model; the result must not depend on the pick.  For every shape, forced
through the debug entries: the int32 accumulators equal hipBLASLt's exact int8 GEMM (``torch._int_mm``) on
ragged shapes and on BASELINE.json cfg2 at full size, and the W8A8 epilogue (scales, bias, LoRA r = 48, one
bf16 rounding) is bit-identical to the 256x256 tile's (every element is computed from the same operands in the
same order).  The shapes the automatic choice gives to the bf16 linear are checked against torch in float32.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

TILES = ("256x256", "256x320", "192x256", "128x128")


@pytest.mark.parametrize("M,N,K", [(300, 260, 384), (513, 1028, 1152), (1000, 640, 3072), (64, 128, 128),
                                   (4608, 1536, 6144), (16896, 12288, 3072)])
def test_every_tile_shape_exact_int32(k2, dev, M, N, K):
    L = k2._lib
    g = torch.Generator(device=dev).manual_seed(M + N + K)
    qx = torch.randint(-127, 128, (M, K), device=dev, dtype=torch.int8, generator=g)
    qw = torch.randint(-127, 128, (N, K), device=dev, dtype=torch.int8, generator=g)
    if M > 16 and N % 8 == 0:
        ref = torch._int_mm(qx, qw.t())
    else:   # exact in float64: every partial sum is below K * 127^2 < 2^53
        ref = (qx.double() @ qw.double().t()).to(torch.int32)
    for t in TILES:
        assert torch.equal(L.gemm_w8a8_acc(qx, qw, tile=t), ref), t
    assert torch.equal(L.gemm_w8a8_acc(qx, qw), ref)


@pytest.mark.parametrize("M,N,K,r", [(300, 384, 640, 48), (1000, 3072, 3072, 16), (4096, 3072, 3072, 16),
                                     (16896, 12288, 3072, 32)])
def test_every_tile_shape_same_w8_output(k2, dev, M, N, K, r):
    L = k2._lib
    g = torch.Generator(device=dev).manual_seed(M * 3 + N)
    qx = torch.randint(-127, 128, (M, K), device=dev, dtype=torch.int8, generator=g)
    qw = torch.randint(-127, 128, (N, K), device=dev, dtype=torch.int8, generator=g)
    sx = torch.rand(M, device=dev, generator=g) * 0.05 + 0.01
    sw = torch.rand(N, device=dev, generator=g) * 0.001 + 1e-4
    bias = torch.randn(N, device=dev, generator=g) * 0.02
    u = torch.randn(M, r, device=dev, generator=g)
    B = torch.randn(N, r, device=dev, generator=g) * 0.01
    y0 = L.gemm_w8a8(qx, sx, qw, sw, bias, u, B, 0.5, tile="256x256", split=False)
    for t in TILES[1:]:
        assert torch.equal(L.gemm_w8a8(qx, sx, qw, sw, bias, u, B, 0.5, tile=t), y0), t
    assert torch.equal(L.gemm_w8a8(qx, sx, qw, sw, bias, u, B, 0.5), y0)


@pytest.mark.parametrize("M,N,K", [(1024, 3072, 3072), (4096, 3072, 3072), (16896, 3072, 1024), (200, 384, 256)])
def test_bf16_linear_at_automatic_tile_shapes(k2, dev, M, N, K):
    """The bf16 GEMM (the fp8 base's linear and the input-gradient GEMM share it) at shapes whose automatic tile
    shape is not 256x256, against torch in float32 (f32 accumulation of bf16 products: order noise only)."""
    L = k2._lib
    g = torch.Generator(device=dev).manual_seed(N + K)
    x = torch.randn(M, K, device=dev, generator=g).bfloat16()
    w = (torch.randn(N, K, device=dev, generator=g) * 0.05).bfloat16()
    y = L.gemm_bf16(x, w).float()
    ref = x.float() @ w.float().t()
    err = float((y - ref).norm() / ref.norm())
    assert err < 4e-3, err
