"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle on the same seeded inputs.

Bars: int8 activation codes, scales and int32 accumulators bit-exact; the
rotated bf16 output within 2 bf16 ulp of the dense rotation (it is in fact bit-exact with the oracle);
bf16 outputs (y, dX) within 1e-2 relative Frobenius error of the oracle's float64 result.
At BASELINE.json's full sizes the oracle runs on sampled rows/columns (size-independent checks).
"""
import math

import numpy as np
import pytest
import torch

from oracle import convrot as orc

pytestmark = pytest.mark.gpu

REL_FROB_TOL = 1e-2


def rel_frob(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def make_x(M, K, seed=0, outliers=True, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    if outliers:
        idx = torch.randperm(K, generator=g)[: max(1, K // 100)]
        x[:, idx] *= 20
    return x.to(dtype)


def make_w(N, K, seed=1):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)


def bits16(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def ulp_dist_bf16(a_bits, b_bits):
    """Distance in bf16 ulps between bit patterns (sign-magnitude mapped to a line; +0 == -0)."""
    def line(b):
        b = np.asarray(b, np.int32)
        return np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(line(a_bits) - line(b_bits))


# ------------------------------------------------------------------------------------------- device
def test_device_is_gfx950(k2, dev):
    assert k2._lib.load().k2q_check_device() == 0
    assert "gfx950" in torch.cuda.get_device_properties(dev).gcnArchName


# ------------------------------------------------------------------------------------------- kernel (1)
@pytest.mark.parametrize("M,K", [(1, 128), (5, 640), (512, 3072), (64, 6144), (33, 12288), (16, 16384)])
def test_rotquant_bf16_bit_exact(k2, dev, M, K):
    x = make_x(M, K, seed=K + M)
    q, s, xr = k2._lib.rotquant(x.to(dev), want_xrot=True)
    q0, s0, xr0 = orc.rotquant(x.float().numpy(), want_xrot=True)
    assert np.array_equal(q.cpu().numpy(), q0)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s0.view(np.uint32))
    assert ulp_dist_bf16(bits16(xr), xr0).max() == 0      # equal values (a zero may differ in sign)


@pytest.mark.parametrize("N,K", [(64, 256), (96, 3072), (8, 16384)])
def test_rotquant_f32_weights_bit_exact(k2, dev, N, K):
    w = torch.randn(N, K, generator=torch.Generator().manual_seed(N)) * 0.02
    q, s = k2._lib.quant_weight_i8(w.to(dev))
    q0, s0 = orc.quant_weight_i8(w.numpy())
    assert np.array_equal(q.cpu().numpy(), q0)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s0.view(np.uint32))


def test_rotquant_special_rows(k2, dev):
    H = torch.from_numpy(np.kron(np.eye(2), __import__("scipy.linalg").linalg.hadamard(128)))
    v = torch.zeros(4, 256, dtype=torch.float64)
    v[0, :7] = torch.tensor([254, 1, 3, 5, -1, -3, 7], dtype=torch.float64)   # exact .5 ties
    v[2, 200] = 1e30                                                          # one huge value
    v[3] = torch.arange(256) - 127.5
    x = (v @ H / 128).float()
    x[1] = 0                                                                  # zero row -> floor
    q, s, _ = k2._lib.rotquant(x.to(dev))
    q0, s0, _ = orc.rotquant(x.numpy())
    assert np.array_equal(q.cpu().numpy(), q0) and np.array_equal(s.cpu().numpy(), s0)
    assert q[0, :7].tolist() == [127, 0, 2, 2, 0, -2, 4]
    assert torch.all(q[1] == 0)


def test_rotquant_xrot_within_two_ulp_of_dense(k2, dev):
    x = make_x(128, 1024, seed=3)
    _, _, xr = k2._lib.rotquant(x.to(dev), want_xrot=True)
    H = np.kron(np.eye(8), __import__("scipy.linalg").linalg.hadamard(128))
    dense = x.double().numpy() @ H / math.sqrt(128)
    assert ulp_dist_bf16(bits16(xr), orc.bf16_bits(dense.astype(np.float32))).max() <= 2


@pytest.mark.parametrize("N,K", [(64, 128), (256, 3072), (32, 12288)])
def test_quant_weight_i4_bit_exact(k2, dev, N, K):
    w = make_w(N, K, seed=N + K)
    q4, s4 = k2._lib.quant_weight_i4(w.to(dev))
    q0, sb0 = orc.quant_weight_i4(w.float().numpy())
    assert np.array_equal(q4.cpu().numpy(), orc.pack_i4(q0))
    assert np.array_equal(bits16(s4), np.ascontiguousarray(sb0.T))


# ------------------------------------------------------------------------------------------- kernel (2)
@pytest.mark.parametrize("M,N,K", [(256, 256, 128), (300, 260, 384), (1, 4, 128), (513, 1028, 1152)])
def test_gemm_int32_acc_bit_exact(k2, dev, M, N, K):
    rng = np.random.default_rng(M * N + K)
    qx = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    qw = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    acc = k2._lib.gemm_w8a8_acc(torch.from_numpy(qx).to(dev), torch.from_numpy(qw).to(dev))
    assert np.array_equal(acc.cpu().numpy(), orc.gemm_acc(qx, qw))


def test_gemm_int32_acc_extreme_codes(k2, dev):
    """All codes at +-127: the largest |acc| the path can produce at K=12288 (1.98e8) stays exact."""
    K = 12288
    qx = np.full((64, K), 127, np.int8)
    qx[1::2] = -127
    qw = np.full((64, K), -127, np.int8)
    acc = k2._lib.gemm_w8a8_acc(torch.from_numpy(qx).to(dev), torch.from_numpy(qw).to(dev))
    assert np.array_equal(acc.cpu().numpy(), orc.gemm_acc(qx, qw))


@pytest.mark.parametrize("M,N,K", [(256, 128, 128), (130, 132, 384)])
def test_gemm_w4_group_partials_exact(k2, dev, M, N, K):
    """With unit group scales the f32 sum of int32 group partials is an exact integer (< 2^24)."""
    rng = np.random.default_rng(M + N + K)
    qx = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    q4 = rng.integers(-7, 8, size=(N, K), dtype=np.int8)
    ones = torch.ones(K // 64, N, dtype=torch.bfloat16)
    out = k2._lib.gemm_w4a8_f32(torch.from_numpy(qx).to(dev), torch.from_numpy(orc.pack_i4(q4)).to(dev),
                                ones.to(dev))
    assert np.array_equal(out.cpu().numpy().astype(np.int64), orc.gemm_acc(qx, q4).astype(np.int64))
    s = (torch.rand(K // 64, N, generator=torch.Generator().manual_seed(1)) + 0.5).to(torch.bfloat16)
    out = k2._lib.gemm_w4a8_f32(torch.from_numpy(qx).to(dev), torch.from_numpy(orc.pack_i4(q4)).to(dev), s.to(dev))
    ref = np.einsum("mng,gn->mn", orc.gemm_acc_groups(qx, q4).astype(np.float64), s.double().numpy())
    assert rel_frob(out.cpu().numpy(), ref) < 1e-6


@pytest.mark.parametrize("M,N,K", [(256, 256, 3072), (130, 132, 12288)])
def test_gemm_w4_scale_exponents(k2, dev, M, N, K):
    """Group scales that exercise the integer chunks: every scale exponent from 2^-24 to 2^6 (windows left
    in both directions), zero and negative scales, runs of equal exponents longer than a chunk, and codes
    at -128 / -8 (the largest group sums).  Within the f32 bound of the float64 sum sum_g s_g acc_g."""
    rng = np.random.default_rng(M + N + K)
    qx = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    qx[: M // 4] = -128
    q4 = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    q4[: N // 4] = -8
    G = K // 64
    e = rng.integers(-24, 7, size=(G, N)).astype(np.float64)
    e[:, N // 2:] = -7.0                                        # long runs of one exponent
    s = (1.0 + rng.random((G, N))) * np.exp2(e)
    s[rng.random((G, N)) < 0.05] = 0.0
    s[rng.random((G, N)) < 0.2] *= -1.0
    s4 = torch.from_numpy(s).to(torch.bfloat16)
    out = k2._lib.gemm_w4a8_f32(torch.from_numpy(qx).to(dev), torch.from_numpy(orc.pack_i4(q4)).to(dev),
                                s4.to(dev)).double().cpu().numpy()
    pg = orc.gemm_acc_groups(qx, q4).astype(np.float64) * s4.double().numpy().T[None, :, :]
    ref, mag = pg.sum(axis=2), np.abs(pg).sum(axis=2)
    assert np.all(np.abs(out - ref) <= mag * (G * 2.0 ** -24) + 1e-30)


# ------------------------------------------------------------------------------------------- kernel (3)
def _forward_case(k2, dev, M, K, N, r, w4, bias, seed):
    x = make_x(M, K, seed=seed)
    w = make_w(N, K, seed=seed + 1)
    g = torch.Generator().manual_seed(seed + 2)
    b = torch.randn(N, generator=g) * 0.02 if bias else None
    A = torch.randn(r, K, generator=g) * 0.01 if r else None
    B = torch.randn(N, r, generator=g) * 0.01 if r else None
    xd = x.to(dev)
    qx, sx, _ = k2._lib.rotquant(xd)
    if w4:
        qw, sw = k2._lib.quant_weight_i4(w.to(dev))
        q0, s0 = orc.quant_weight_i4(w.float().numpy())
        qw_o, sw_o = q0, s0
    else:
        qw, sw = k2._lib.quant_weight_i8(w.to(dev))
        qw_o, sw_o = orc.quant_weight_i8(w.float().numpy())
    u = k2._lib.lora_down(xd, A.to(dev)) if r else None
    gemm = k2._lib.gemm_w4a8 if w4 else k2._lib.gemm_w8a8
    y = gemm(qx, sx, qw, sw, b.to(dev) if bias else None, u, B.to(dev) if r else None, 1.0)
    ref = orc.forward(x.float().numpy(), qw_o, sw_o, w4=w4, bias=None if b is None else b.numpy(),
                      lora_A=None if A is None else A.numpy(), lora_B=None if B is None else B.numpy(),
                      lora_scale=1.0)
    return y, u, ref


@pytest.mark.parametrize("M,K,N,r,bias", [(256, 256, 256, 0, False), (300, 384, 260, 16, True),
                                          (512, 3072, 1024, 32, True), (257, 1024, 512, 64, False),
                                          (64, 512, 128, 128, True), (384, 768, 512, 48, True),
                                          (130, 512, 384, 112, False)])
def test_forward_w8a8(k2, dev, M, K, N, r, bias):
    y, u, ref = _forward_case(k2, dev, M, K, N, r, False, bias, seed=M + N)
    assert rel_frob(y.float().cpu().numpy(), ref["y64"]) < REL_FROB_TOL
    # the bf16 output is the once-rounded f32 epilogue: far inside the bar
    assert rel_frob(y.float().cpu().numpy(), ref["y64"]) < 4e-3
    if r:
        assert rel_frob(u.cpu().numpy(), ref["u"]) < 1e-5


@pytest.mark.parametrize("M,K,N,r,bias", [(256, 256, 128, 0, False), (300, 384, 260, 16, True),
                                          (512, 3072, 1024, 32, False), (256, 768, 384, 48, True)])
def test_forward_w4a8(k2, dev, M, K, N, r, bias):
    y, _, ref = _forward_case(k2, dev, M, K, N, r, True, bias, seed=M + N + 7)
    assert rel_frob(y.float().cpu().numpy(), ref["y64"]) < 4e-3


@pytest.mark.parametrize("M,K,r", [(1, 512, 16), (15, 1024, 32), (17, 3072, 16), (4096, 3072, 16), (16896, 3072, 32),
                                   (1000, 3072, 64), (333, 2048, 48), (257, 1536, 32), (4111, 2560, 64), (8192, 3072, 16)])
def test_rotquant_lora_same_pass(k2, dev, M, K, r):
    """Rotate/quant with the LoRA down-projection from the same pass over x (``k2q_rotquant_lora``): the codes
    and scales equal the oracle's (and k2q_rotquant's) bit for bit, u is within 1e-5 of the f64 product, the
    columns of u past r and the rows of a longer buffer are left alone, and repeated calls are bit-identical."""
    x = make_x(M, K, seed=M + K + r)
    A = torch.randn(r, K, generator=torch.Generator().manual_seed(r + 1)) * 0.01
    xd, Ad = x.to(dev), A.to(dev)
    q, s, u = k2._lib.rotquant_lora(xd, Ad)
    q0, s0, _ = orc.rotquant(x.float().numpy())
    assert np.array_equal(q.cpu().numpy(), q0)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s0.view(np.uint32))
    ref = orc.lora_down(x.float().numpy(), A.numpy())
    assert rel_frob(u.cpu().numpy(), ref) < 1e-5
    q2, s2, u2 = k2._lib.rotquant_lora(xd, Ad)
    assert torch.equal(q2, q) and torch.equal(s2, s) and torch.equal(u2, u)
    # through the C ABI with a wider u (ldu = r + 16) inside a larger buffer: only rows < M, columns < r written
    ub = torch.full((M + 3, r + 16), 7.0, device=dev)
    qb = torch.empty(M, K, dtype=torch.int8, device=dev)
    sb = torch.empty(M, device=dev)
    lib = k2._lib.load()
    assert lib.k2q_rotquant_lora(xd.data_ptr(), M, K, K, qb.data_ptr(), sb.data_ptr(), Ad.data_ptr(), r,
                                 ub.data_ptr(), r + 16, torch.cuda.current_stream(dev).cuda_stream) == 0
    assert torch.equal(qb, q) and torch.equal(sb, s) and torch.equal(ub[:M, :r], u)
    assert torch.all(ub[:M, r:] == 7.0) and torch.all(ub[M:] == 7.0)
    # rows of a wider buffer (row stride ldx > K, as a strided view of a larger activation hands them over)
    xw = torch.zeros(M, K + 64, dtype=torch.bfloat16, device=dev)
    xw[:, :K] = xd
    qw_, sw_, uw_ = torch.empty_like(q), torch.empty_like(s), torch.empty_like(u)
    assert lib.k2q_rotquant_lora(xw.data_ptr(), M, K, K + 64, qw_.data_ptr(), sw_.data_ptr(), Ad.data_ptr(), r,
                                 uw_.data_ptr(), r, torch.cuda.current_stream(dev).cuda_stream) == 0
    assert torch.equal(qw_, q) and torch.equal(sw_, s) and torch.equal(uw_, u)


def test_rotquant_lora_refuses_other_shapes(k2, dev):
    """Shapes outside three chunks per lane (K > 3072), K not a multiple of 512, or ranks outside 16..64 are refused
    before launch (the module then runs the separate down-projection)."""
    lib = k2._lib.load()
    x = torch.zeros(4, 6144, dtype=torch.bfloat16, device=dev)
    A = torch.zeros(16, 6144, device=dev)
    q = torch.empty(4, 6144, dtype=torch.int8, device=dev)
    assert lib.k2q_rotquant_lora(x.data_ptr(), 4, 4096, 6144, q.data_ptr(), torch.empty(4, device=dev).data_ptr(),
                                 A.data_ptr(), 16, torch.empty(4, 16, device=dev).data_ptr(), 16,
                                 torch.cuda.current_stream(dev).cuda_stream) == -4
    s = torch.empty(4, device=dev)
    u = torch.empty(4, 128, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    assert lib.k2q_rotquant_lora(x.data_ptr(), 4, 6144, 6144, q.data_ptr(), s.data_ptr(), A.data_ptr(), 16,
                                 u.data_ptr(), 16, st) == -4
    assert lib.k2q_rotquant_lora(x.data_ptr(), 4, 640, 6144, q.data_ptr(), s.data_ptr(), A.data_ptr(), 16,
                                 u.data_ptr(), 16, st) == -4
    assert lib.k2q_rotquant_lora(x.data_ptr(), 4, 3072, 6144, q.data_ptr(), s.data_ptr(), A.data_ptr(), 128,
                                 u.data_ptr(), 128, st) == -4
    assert lib.k2q_rotquant_lora(x.data_ptr(), 4, 3072, 6144, q.data_ptr(), s.data_ptr(), A.data_ptr(), 24,
                                 u.data_ptr(), 24, st) == -1
    with pytest.raises(ValueError):
        k2._lib.rotquant_lora(x, A)


@pytest.mark.parametrize("M,K,r", [(2, 3072, 16), (1024, 12288, 16), (4608, 12288, 64), (100, 640, 48),
                                   (33, 1024, 128), (17, 2048, 80), (16896, 3072, 32), (1000, 3072, 256),
                                   (300, 1024, 144), (4608, 6144, 192)])
def test_lora_down_launch_plans(k2, dev, M, K, r):
    """Every launch plan of the down-projection (row tiles per workgroup, K slices summed in slice order)
    against the f64 product; the unsliced fallback (no workspace) too; repeated calls are bit-identical.  Ranks
    above 128 run as 128-rank chunks writing their columns of u (144 = 128 + 16, 192, 256)."""
    x = make_x(M, K, seed=M + r)
    A = torch.randn(r, K, generator=torch.Generator().manual_seed(r)) * 0.01
    xd, Ad = x.to(dev), A.to(dev)
    u = k2._lib.lora_down(xd, Ad)
    ref = orc.lora_down(x.float().numpy(), A.numpy())
    assert rel_frob(u.cpu().numpy(), ref) < 1e-5
    assert torch.equal(u, k2._lib.lora_down(xd, Ad))
    u1 = torch.empty_like(u)
    lib = k2._lib.load()
    assert lib.k2q_lora_down(xd.data_ptr(), M, K, K, Ad.data_ptr(), r, None, 0, u1.data_ptr(),
                             torch.cuda.current_stream(dev).cuda_stream) == 0
    assert rel_frob(u1.cpu().numpy(), ref) < 1e-5


@pytest.mark.parametrize("M,N,K,r", [(192, 256, 512, 16), (100, 128, 384, 48), (1, 384, 128, 128),
                                     (777, 640, 1280, 80), (4608, 3072, 12288, 64), (300, 384, 512, 256),
                                     (1000, 1024, 768, 144)])
def test_lora_grads(k2, dev, M, N, K, r):
    """g = s dY B, dA = g^T x, dB = s dY^T u (the autograd of lora.py:47-48) against float64; (4608, 3072,
    12288, 64) is BASELINE.json cfg3 at full size; ranks above 128 run as 128-rank chunks (rows of dA,
    columns of dB)."""
    gen = torch.Generator().manual_seed(M + N + r)
    dy = (torch.randn(M, N, generator=gen) * 1e-3).to(torch.bfloat16)
    x = make_x(M, K, seed=r)
    u = torch.randn(M, r, generator=gen)
    B = torch.randn(N, r, generator=gen) * 0.01
    s = 0.75
    g, dA, dB = k2._lib.lora_grads(dy.to(dev), x.to(dev), u.to(dev), B.to(dev), s)
    g64 = s * (dy.double() @ B.double())
    assert rel_frob(g.cpu().numpy(), g64.numpy()) < 2e-5
    assert rel_frob(dA.cpu().numpy(), (g64.t() @ x.double()).numpy()) < 2e-5
    assert rel_frob(dB.cpu().numpy(), (s * (dy.double().t() @ u.double())).numpy()) < 2e-5
    g2, dA2, dB2 = k2._lib.lora_grads(dy.to(dev), None, None, B.to(dev), s)
    assert dA2 is None and dB2 is None and torch.equal(g2, g)      # deterministic; optional outputs


@pytest.mark.parametrize("M,N,K,r", [(777, 640, 1280, 48), (64, 4096, 256, 16), (2048, 256, 4096, 32),
                                     (1000, 1024, 768, 144), (33, 512, 640, 96)])
def test_lora_grads_single_products(k2, dev, M, N, K, r):
    """dA alone and dB alone (the other gradient not requested) against float64: the workgroups of the shared
    wgrad launch and the slice count are planned for the products requested, so each subset runs its own
    schedule; g is the same bits in every mode."""
    gen = torch.Generator().manual_seed(3 * M + N + r)
    dy = (torch.randn(M, N, generator=gen) * 1e-3).to(torch.bfloat16)
    x = make_x(M, K, seed=r + 1)
    u = torch.randn(M, r, generator=gen)
    B = torch.randn(N, r, generator=gen) * 0.01
    s = 1.25
    g64 = s * (dy.double() @ B.double())
    dA64 = g64.t() @ x.double()
    dB64 = s * (dy.double().t() @ u.double())
    g, dA, dB = k2._lib.lora_grads(dy.to(dev), x.to(dev), u.to(dev), B.to(dev), s)
    ga, dAa, dBa = k2._lib.lora_grads(dy.to(dev), x.to(dev), None, B.to(dev), s)
    gb, dAb, dBb = k2._lib.lora_grads(dy.to(dev), None, u.to(dev), B.to(dev), s)
    assert dBa is None and dAb is None
    assert torch.equal(ga, g) and torch.equal(gb, g)
    for got, want in ((dA, dA64), (dAa, dA64), (dB, dB64), (dBb, dB64)):
        assert rel_frob(got.cpu().numpy(), want.numpy()) < 2e-5


# Skinny M (1 <= M <= 8: the adaLN modulation linears run at M = batch) takes the GEMV path.
@pytest.mark.parametrize("Ms,K,N,bias", [(1, 128, 4, False), (2, 3072, 1000, True), (5, 640, 260, False),
                                         (8, 12288, 256, True), (3, 16384, 36, False)])
def test_skinny_m_matches_mfma_rows_bit_exact(k2, dev, Ms, K, N, bias):
    """Without LoRA the GEMV's bf16 output equals the MFMA path's rows bit for bit (same int32 sums,
    same epilogue arithmetic); with LoRA the two differ by at most one bf16 ulp (summation order of L)."""
    x = make_x(300, K, seed=Ms + K)
    w = make_w(N, K, seed=N)
    g = torch.Generator().manual_seed(9)
    b = (torch.randn(N, generator=g) * 0.02).to(dev) if bias else None
    A = (torch.randn(16, K, generator=g) * 0.01).to(dev)
    B = (torch.randn(N, 16, generator=g) * 0.01).to(dev)
    qx, sx, _ = k2._lib.rotquant(x.to(dev))
    qw, sw = k2._lib.quant_weight_i8(w.to(dev))
    y_big = k2._lib.gemm_w8a8(qx, sx, qw, sw, b, None, None, 1.0)
    y_small = k2._lib.gemm_w8a8(qx[:Ms], sx[:Ms], qw, sw, b, None, None, 1.0)
    assert torch.equal(y_small.view(torch.int16), y_big[:Ms].view(torch.int16))
    u = k2._lib.lora_down(x.to(dev), A)
    y_big = k2._lib.gemm_w8a8(qx, sx, qw, sw, b, u, B, 0.5)
    y_small = k2._lib.gemm_w8a8(qx[:Ms], sx[:Ms], qw, sw, b, u[:Ms], B, 0.5)
    assert ulp_dist_bf16(bits16(y_small), bits16(y_big[:Ms])).max() <= 1


@pytest.mark.parametrize("M,K,N,r,bias", [(2, 3072, 18432, 16, False), (1, 256, 128, 128, True),
                                          (7, 1024, 520, 64, True)])
def test_forward_w8a8_skinny_m(k2, dev, M, K, N, r, bias):
    """(2, 3072, 18432): the adaLN modulation linear of a double-stream block at CFG batch 2."""
    y, u, ref = _forward_case(k2, dev, M, K, N, r, False, bias, seed=M + N)
    assert rel_frob(y.float().cpu().numpy(), ref["y64"]) < 4e-3
    assert rel_frob(u.cpu().numpy(), ref["u"]) < 1e-5


# ------------------------------------------------------------------------------------------- kernel (4)
@pytest.mark.parametrize("fold", [True, False])
@pytest.mark.parametrize("M,K,N,r,w4", [(256, 256, 256, 0, False), (200, 384, 320, 16, False),
                                        (512, 1024, 512, 64, False), (256, 512, 256, 32, True)])
def test_input_gradient(k2, dev, M, K, N, r, w4, fold):
    w = make_w(N, K, seed=M + K)
    g = torch.Generator().manual_seed(5)
    dy = (torch.randn(M, N, generator=g) * 1e-3).to(torch.bfloat16)
    A = torch.randn(r, K, generator=g) * 0.01 if r else None
    B = torch.randn(N, r, generator=g) * 0.01 if r else None
    if w4:
        qw, sw = k2._lib.quant_weight_i4(w.to(dev))
        qo, so = orc.quant_weight_i4(w.float().numpy())
    else:
        qw, sw = k2._lib.quant_weight_i8(w.to(dev))
        qo, so = orc.quant_weight_i8(w.float().numpy())
    gd = (dy.float() @ B).contiguous() if r else None
    dx = k2._lib.gemm_dx(dy.to(dev), qw, sw, w4=w4, g=gd.to(dev) if r else None, lora_a=A.to(dev) if r else None,
                         fold_rotation=fold)
    x_dummy = np.zeros((M, K))
    ref = orc.backward(dy.float().numpy(), x_dummy, qo, so, w4=w4, lora_A=None if A is None else A.numpy(),
                       lora_B=None if B is None else B.numpy(), lora_scale=1.0)
    assert rel_frob(dx.float().cpu().numpy(), ref["dx64"]) < REL_FROB_TOL


@pytest.mark.parametrize("N,K,w4", [(64, 128, False), (200, 384, False), (3072, 12288, False), (96, 512, True)])
def test_effective_weight_prep(k2, dev, N, K, w4):
    """k2q_dx_prep_eff: wt = bf16(2^-7 W_hat R)^T.  W8: the rotation of the integer codes is exact, so every
    element equals the float64 product rounded once to f32 and once to bf16, bit for bit (also with every code
    at -127, the largest sums).  W4 (a block mixes two group scales, so the codes are scaled first): against
    the dense block-Hadamard product in float32, one bf16 rounding apart at most (the butterfly and the matmul
    add in different orders)."""
    w = make_w(N, K, seed=N + K + 1)
    if w4:
        qw, sw = k2._lib.quant_weight_i4(w.to(dev))
        q = torch.from_numpy(orc.unpack_i4(qw.cpu().numpy())).to(dev).float()
        what = q * sw.float().t().repeat_interleave(64, dim=1)
    else:
        qw, sw = k2._lib.quant_weight_i8(w.to(dev))
        what = qw.float() * sw[:, None]
    lib = k2._lib.load()
    P = k2._lib._ptr

    def prep(q, s):
        wt = torch.empty(K, N, dtype=torch.bfloat16, device=dev)
        rc = lib.k2q_dx_prep_eff(None if w4 else P(q), None if w4 else P(s), P(q) if w4 else None,
                                 P(s) if w4 else None, N, K, P(wt), k2._lib._stream(dev))
        assert rc == 0
        torch.cuda.synchronize()
        return wt

    wt = prep(qw, sw)
    H64 = torch.from_numpy(__import__("scipy.linalg").linalg.hadamard(128).astype(np.float64)).to(dev)
    if not w4:
        for q in (qw, torch.full_like(qw, -127)):
            exact = ((q.double().view(N, K // 128, 128) @ H64).view(N, K) * sw.double()[:, None] * 2.0 ** -7).t()
            assert torch.equal(prep(q, sw), exact.float().to(torch.bfloat16))
        return
    ref = ((what.view(N, K // 128, 128) @ H64.float()).view(N, K) * 0.0078125).t()
    err = (wt.float() - ref).abs()
    tol = ref.abs() * 2 ** -8 + float(ref.abs().max()) * 2 ** -20   # plus f32 order noise near zero
    assert bool((err <= tol).all()), float((err - tol).max())


# ------------------------------------------------------------------------------------------- split schedule
@pytest.mark.parametrize("M,N,K", [(512, 768, 4096), (1024, 3072, 12288), (8192, 3072, 12288)])
def test_gemm_split_schedule_bit_exact(k2, dev, M, N, K):
    """Shapes whose last round of 256 x 256 tiles leaves the GPU partly empty (cfg4's text-stream and
    image-stream down projections are the last two): the remainder tiles are cut along K into pieces whose
    int32 sums a fixup launch adds.  Accumulators equal the exact product, and the bf16 outputs (bias,
    LoRA) equal those of the full-K schedule bit for bit."""
    assert k2._lib.load().k2q_gemm_w8a8_ws_bytes(M, N, K) > 0      # the split schedule is taken
    rng = np.random.default_rng(M + N + K)
    qx_h = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    qw_h = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    qx, qw = torch.from_numpy(qx_h).to(dev), torch.from_numpy(qw_h).to(dev)
    acc = k2._lib.gemm_w8a8_acc(qx, qw, tile="256x256")     # the split schedule runs 256 x 256 tiles
    assert torch.equal(acc, k2._lib.gemm_w8a8_acc(qx, qw, split=False, tile="256x256"))
    rows = np.arange(M) if M <= 1024 else np.array([0, 1, 255, 256, M // 2, M - 257, M - 1])
    assert np.array_equal(acc.cpu().numpy()[rows], orc.gemm_acc_fast(qx_h[rows], qw_h))
    g = torch.Generator().manual_seed(1)
    sx = (torch.rand(M, generator=g) * 0.01 + 1e-3).to(dev)
    sw = (torch.rand(N, generator=g) * 0.01 + 1e-3).to(dev)
    bias = (torch.randn(N, generator=g) * 0.02).to(dev)
    u = torch.randn(M, 16, generator=g).to(dev)
    B = (torch.randn(N, 16, generator=g) * 0.01).to(dev)
    y = k2._lib.gemm_w8a8(qx, sx, qw, sw, bias, u, B, 0.5, tile="256x256")
    y0 = k2._lib.gemm_w8a8(qx, sx, qw, sw, bias, u, B, 0.5, split=False, tile="256x256")
    assert torch.equal(y.view(torch.int16), y0.view(torch.int16))
    assert torch.equal(k2._lib.gemm_w8a8(qx, sx, qw, sw, bias, u, B, 0.5), y0)   # whatever tile is chosen


@pytest.mark.parametrize("M,N,K", [(1024, 3072, 12288), (512, 1536, 12288), (256, 6144, 6144), (1024, 2048, 12288)])
def test_gemm_split_schedule_128_bit_exact(k2, dev, M, N, K):
    """One round of 128 x 128 tiles over a long reduction (cfg4's text-stream down projection first): every
    tile cut along K into pieces (2 to 5 here) whose int32 sums a fixup launch adds in order.  Accumulators
    equal the exact product and the full-K schedule's, and the bf16 outputs (bias, LoRA) equal the full-K
    schedule's bit for bit."""
    tile, pieces = k2._lib.gemm_w8a8_plan(M, N, K)
    assert tile == "128x128" and pieces > 1                     # the split schedule is taken
    rng = np.random.default_rng(M + N + K + 1)
    qx_h = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    qw_h = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    qx, qw = torch.from_numpy(qx_h).to(dev), torch.from_numpy(qw_h).to(dev)
    acc = k2._lib.gemm_w8a8_acc(qx, qw, tile="128x128")
    assert torch.equal(acc, k2._lib.gemm_w8a8_acc(qx, qw, split=False, tile="128x128"))
    rows = np.array([0, 1, 127, 128, M // 2, M - 129, M - 1])
    assert np.array_equal(acc.cpu().numpy()[rows], orc.gemm_acc_fast(qx_h[rows], qw_h))
    g = torch.Generator().manual_seed(2)
    sx = (torch.rand(M, generator=g) * 0.01 + 1e-3).to(dev)
    sw = (torch.rand(N, generator=g) * 0.01 + 1e-3).to(dev)
    bias = (torch.randn(N, generator=g) * 0.02).to(dev)
    u = torch.randn(M, 16, generator=g).to(dev)
    B = (torch.randn(N, 16, generator=g) * 0.01).to(dev)
    y = k2._lib.gemm_w8a8(qx, sx, qw, sw, bias, u, B, 0.5)
    y0 = k2._lib.gemm_w8a8(qx, sx, qw, sw, bias, u, B, 0.5, split=False)
    assert torch.equal(y.view(torch.int16), y0.view(torch.int16))


def test_input_gradient_split_schedule(k2, dev):
    """dX with the remainder tiles cut along N (f32 pieces added in slice order): against the oracle, and
    within f32 summation-order noise of the full-N schedule; repeated calls are bit-identical."""
    M, K, N, r = 512, 768, 4096, 32
    assert k2._lib.load().k2q_gemm_dx_ws_bytes(M, N, K) > 0
    w = make_w(N, K, seed=7)
    g = torch.Generator().manual_seed(8)
    dy = (torch.randn(M, N, generator=g) * 1e-3).to(torch.bfloat16)
    A = torch.randn(r, K, generator=g) * 0.01
    B = torch.randn(N, r, generator=g) * 0.01
    qw, sw = k2._lib.quant_weight_i8(w.to(dev))
    qo, so = orc.quant_weight_i8(w.float().numpy())
    gd = (dy.float() @ B).contiguous().to(dev)
    dx = k2._lib.gemm_dx(dy.to(dev), qw, sw, g=gd, lora_a=A.to(dev))
    dx0 = k2._lib.gemm_dx(dy.to(dev), qw, sw, g=gd, lora_a=A.to(dev), split=False)
    ref = orc.backward(dy.float().numpy(), np.zeros((M, K)), qo, so, lora_A=A.numpy(), lora_B=B.numpy(),
                       lora_scale=1.0)
    assert rel_frob(dx.float().cpu().numpy(), ref["dx64"]) < 4e-3
    assert rel_frob(dx.float().cpu().numpy(), dx0.float().cpu().numpy()) < 1e-3
    assert torch.equal(dx, k2._lib.gemm_dx(dy.to(dev), qw, sw, g=gd, lora_a=A.to(dev)))


# ------------------------------------------------------------------------------------------- module
def _layers(k2, dev, K=512, N=384, r=32, mode="w8a8", seed=0, bias=False):
    lin = torch.nn.Linear(K, N, bias=bias, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(make_w(N, K, seed=seed))
        if bias:
            lin.bias.copy_(torch.randn(N, generator=torch.Generator().manual_seed(seed)) * 0.02)
    base = k2.ConvRotLinear(lin.to(dev), mode)
    lora = k2.LoRALinear(base, r, float(r))
    g = torch.Generator().manual_seed(seed + 9)
    with torch.no_grad():
        lora.lora_A.copy_(torch.randn(r, K, generator=g) * 0.01)
        lora.lora_B.copy_(torch.randn(N, r, generator=g) * 0.01)
    return lin, base, lora


@pytest.mark.parametrize("mode", ["w8a8", "w4a8"])
def test_module_fused_lora_matches_reference_formula(k2, dev, mode):
    _, base, lora = _layers(k2, dev, mode=mode, bias=True)
    x = make_x(3 * 100, 512, seed=11).reshape(3, 100, 512).to(dev)
    with torch.no_grad():
        y = lora(x)
        out = base(x)
        delta = (x.to(torch.float32) @ lora.lora_A.t()) @ lora.lora_B.t()       # lora.py:47-48
        ref = out + (lora.scale * lora.scale_mul) * delta.to(out.dtype)
        assert y.shape == (3, 100, 384) and y.dtype == torch.bfloat16
        assert rel_frob(y.float().cpu(), ref.float().cpu()) < REL_FROB_TOL
        with k2.lora_disabled(lora):
            assert torch.equal(lora(x), out)                                     # scale_mul 0 == base
        with k2.lora_scaled(lora, -2.0):
            yneg = lora(x)
        ref_neg = out + (-2.0 * lora.scale) * delta.to(out.dtype)
        assert rel_frob(yneg.float().cpu(), ref_neg.float().cpu()) < REL_FROB_TOL


def test_module_matches_oracle_and_unquantized_linear(k2, dev):
    lin, base, _ = _layers(k2, dev, K=1024, N=512)
    x = make_x(256, 1024, seed=12)
    q0, s0 = orc.quant_weight_i8(lin.weight.detach().float().cpu().numpy())
    assert np.array_equal(base.qweight.cpu().numpy(), q0)
    with torch.no_grad():
        y = base(x.to(dev)).float().cpu().numpy()
    ref = orc.forward(x.float().numpy(), q0, s0)
    assert rel_frob(y, ref["y64"]) < 4e-3
    dense = x.double().numpy() @ lin.weight.detach().double().cpu().numpy().T
    assert rel_frob(y, dense) < 0.03        # W8A8 quantization error on outlier-laden activations


@pytest.mark.parametrize("mode", ["w8a8", "w4a8"])
def test_module_backward_matches_oracle(k2, dev, mode):
    lin, base, lora = _layers(k2, dev, K=512, N=256, r=16, mode=mode)
    x = make_x(192, 512, seed=13)
    dy = (torch.randn(192, 256, generator=torch.Generator().manual_seed(3)) * 1e-3).to(torch.bfloat16)
    xd = x.to(dev).requires_grad_(True)
    lora(xd).backward(dy.to(dev))
    w = lin.weight.detach().float().cpu().numpy()
    qo, so = orc.quant_weight_i4(w) if mode == "w4a8" else orc.quant_weight_i8(w)
    ref = orc.backward(dy.float().numpy(), x.float().numpy(), qo, so, w4=mode == "w4a8",
                       lora_A=lora.lora_A.detach().cpu().numpy(), lora_B=lora.lora_B.detach().cpu().numpy(),
                       lora_scale=1.0)
    assert rel_frob(xd.grad.float().cpu().numpy(), ref["dx64"]) < REL_FROB_TOL
    assert rel_frob(lora.lora_A.grad.cpu().numpy(), ref["dA"]) < 1e-3
    assert rel_frob(lora.lora_B.grad.cpu().numpy(), ref["dB"]) < 1e-3
    assert base.qweight.grad is None


@pytest.mark.parametrize("mode", ["w8a8", "w4a8"])
def test_dx_weight_cache_and_block_swap(k2, dev, mode):
    """By default every backward builds the input-gradient weight and lets it go, so a ConvRot layer's
    parameters, which block swap pages (``mmdit.py:409-414``), are its codes, scales and bias only: 1 byte per
    weight resident and paged, as the reference's fp8 base.  With the cache on the weight is kept as a plain
    attribute (not a parameter, not in ``state_dict``), reused, rebuilt after the codes are paged out and back
    or written in place, and released when any later backward finds its layer's codes gone from the device.
    dX and the LoRA grads are bit-identical in every case."""
    _, base, lora = _layers(k2, dev, K=512, N=256, r=16, mode=mode)
    _, other_base, other = _layers(k2, dev, K=512, N=256, r=16, mode=mode, seed=9)
    x = make_x(160, 512, seed=21).to(dev)
    dy = (torch.randn(160, 256, generator=torch.Generator().manual_seed(5)) * 1e-3).to(torch.bfloat16).to(dev)

    def grads(layer=lora):
        layer.lora_A.grad = layer.lora_B.grad = None
        xr = x.clone().requires_grad_(True)
        layer(xr).backward(dy)
        return xr.grad.clone(), layer.lora_A.grad.clone(), layer.lora_B.grad.clone()

    paged = {"qweight", "wscale"} | ({"bias"} if base.bias is not None else set())
    assert base.keep_dx_weight is False                            # the default
    ref = grads()
    assert base.dx_weight_kept is None
    assert {n for n, _ in base.named_parameters()} == paged

    def swap(layer, device):                                       # mmdit.py:409-414, skip_trainable=True
        for p in layer.parameters():
            if not p.requires_grad:
                p.data = p.data.to(device, non_blocking=True)

    swap(lora, "cpu")                                              # default: block swap moves codes + scales only
    assert all(p.device.type == "cpu" for p in base.parameters())
    swap(lora, dev)
    assert all(torch.equal(a, b) for a, b in zip(grads(), ref))

    assert k2.set_dx_weight_cache(lora, True) == 1
    first = grads()
    w1 = base.dx_weight_kept
    assert w1 is not None and not isinstance(w1, torch.nn.Parameter) and w1.shape == (512, 256)
    assert {n for n, _ in base.named_parameters()} == paged        # still only codes, scales, bias
    assert not any("dx" in k for k in lora.state_dict())
    second = grads()
    assert base.dx_weight_kept is w1                               # reused
    swap(lora, "cpu")                                              # paged out: the kept weight stays behind ...
    assert base.dx_weight_kept is w1 and w1.device.type == "cuda"
    k2.set_dx_weight_cache(other, True)
    grads(other)                                                   # ... until any layer's next backward
    assert base.dx_weight_kept is None and other_base.dx_weight_kept is not None
    swap(lora, dev)
    third = grads()
    w3 = base.dx_weight_kept
    assert w3 is not None and w3 is not w1 and torch.equal(w3, w1)
    with torch.no_grad():
        base.qweight.copy_(base.qweight.clone())                   # an in-place write (same values)
    fourth = grads()
    assert base.dx_weight_kept is not w3 and torch.equal(base.dx_weight_kept, w1)
    for got in (first, second, third, fourth):
        assert all(torch.equal(a, b) for a, b in zip(got, ref))
    lora.load_state_dict(lora.state_dict())                        # strict load: no derived weight in it
    assert all(torch.equal(a, b) for a, b in zip(grads(), ref))
    k2.set_dx_weight_cache(lora, False)
    assert base.dx_weight_kept is None


def test_deterministic_and_checkpoint_recompute(k2, dev):
    _, _, lora = _layers(k2, dev)
    x = make_x(512, 512, seed=14).to(dev)
    with torch.no_grad():
        a, b = lora(x), lora(x)
    assert torch.equal(a, b)
    xa = x.clone().requires_grad_(True)
    xb = x.clone().requires_grad_(True)
    dy = torch.randn(512, 384, device=dev).to(torch.bfloat16)
    lora(xa).backward(dy)
    ga = (xa.grad.clone(), lora.lora_A.grad.clone())
    lora.lora_A.grad = None
    lora.lora_B.grad = None
    torch.utils.checkpoint.checkpoint(lora, xb, use_reentrant=False).backward(dy)
    assert torch.equal(xb.grad, ga[0]) and torch.equal(lora.lora_A.grad, ga[1])


def test_walker_and_block_swap_on_gpu(k2, dev):
    import torch.nn as nn

    class Blk(nn.Module):
        def __init__(self):
            super().__init__()
            self.mlp = nn.Module()
            self.mlp.up = nn.Linear(256, 512, bias=False, dtype=torch.bfloat16)
            self.mlp.down = nn.Linear(512, 256, bias=False, dtype=torch.bfloat16)

    class Dit(nn.Module):
        def __init__(self):
            super().__init__()
            self.first = nn.Linear(8, 256, dtype=torch.bfloat16)
            self.blocks = nn.ModuleList([Blk(), Blk()])

    dit = Dit().to(dev)
    assert k2.quantize_dit_convrot(dit, "w8a8") == 4
    ad = k2.inject_lora(dit, 16, include_txtfusion=False, include_txtmlp=False)
    assert len(ad) == 4
    blk = dit.blocks[1]
    x = make_x(64, 256, seed=15).to(dev)
    with torch.no_grad():
        ref = blk.mlp.down(blk.mlp.up(x))
    for p in blk.parameters():          # page out and back in, as mmdit.py:409-418 does
        if not p.requires_grad:
            p.data = p.data.to("cpu")
    for p in blk.parameters():
        if not p.requires_grad:
            p.data = p.data.to(dev, non_blocking=True)
    with torch.no_grad():
        assert torch.equal(blk.mlp.down(blk.mlp.up(x)), ref)


# ------------------------------------------------------------------------------------------- full size
def test_full_size_cfg2_sampled(k2, dev):
    """BASELINE.json configs[2] shapes (M=16896, K=3072, N=12288, r=32): sampled rows of the codes, scales
    and y against the oracle; sampled entries of the int32 accumulators exact."""
    M, K, N, r = 16896, 3072, 12288, 32
    x = make_x(M, K, seed=0)
    w = make_w(N, K, seed=1)
    g = torch.Generator().manual_seed(2)
    A = torch.randn(r, K, generator=g) * 0.01
    B = torch.randn(N, r, generator=g) * 0.01
    xd = x.to(dev)
    qx, sx, _ = k2._lib.rotquant(xd)
    qw, sw = k2._lib.quant_weight_i8(w.to(dev))
    u = k2._lib.lora_down(xd, A.to(dev))
    y = k2._lib.gemm_w8a8(qx, sx, qw, sw, None, u, B.to(dev), 1.0)
    acc = k2._lib.gemm_w8a8_acc(qx, qw)
    rows = np.sort(np.random.default_rng(0).choice(M, 48, replace=False))
    rows[-1] = M - 1
    cols = np.sort(np.random.default_rng(1).choice(N, 64, replace=False))
    xs = x[torch.from_numpy(rows)].float().numpy()
    q0, s0, _ = orc.rotquant(xs)
    assert np.array_equal(qx.cpu().numpy()[rows], q0) and np.array_equal(sx.cpu().numpy()[rows], s0)
    qw0, sw0 = orc.quant_weight_i8(w[torch.from_numpy(cols)].float().numpy())
    assert np.array_equal(qw.cpu().numpy()[cols], qw0)
    assert np.array_equal(acc.cpu().numpy()[np.ix_(rows, cols)], orc.gemm_acc(q0, qw0))
    qw_all, sw_all = qw.cpu().numpy(), sw.cpu().numpy()
    ref = orc.forward(xs, qw_all, sw_all, lora_A=A.numpy(), lora_B=B.numpy(), lora_scale=1.0)
    assert rel_frob(y.float().cpu().numpy()[rows], ref["y64"]) < 4e-3


def test_full_size_cfg3_input_gradient_sampled(k2, dev):
    """BASELINE.json configs[3] shapes (M=4608, K=12288, N=3072, r=64): dX on sampled rows."""
    M, K, N, r = 4608, 12288, 3072, 64
    w = make_w(N, K, seed=3)
    g = torch.Generator().manual_seed(4)
    dy = (torch.randn(M, N, generator=g) * 1e-3).to(torch.bfloat16)
    A = torch.randn(r, K, generator=g) * 0.01
    B = torch.randn(N, r, generator=g) * 0.01
    qw, sw = k2._lib.quant_weight_i8(w.to(dev))
    gd = (dy.float() @ B).contiguous()
    dx = k2._lib.gemm_dx(dy.to(dev), qw, sw, g=gd.to(dev), lora_a=A.to(dev))
    rows = np.sort(np.random.default_rng(2).choice(M, 16, replace=False))
    ref = orc.backward(dy.float().numpy()[rows], np.zeros((16, K)), qw.cpu().numpy(), sw.cpu().numpy(),
                       lora_A=A.numpy(), lora_B=B.numpy(), lora_scale=1.0)
    assert rel_frob(dx.float().cpu().numpy()[rows], ref["dx64"]) < REL_FROB_TOL


def test_full_size_cfg2_every_tile(k2, dev):
    """Every one of cfg2's 3168 tiles (the balanced persistent grid: 244 workgroups of 13 tiles): the int32
    accumulators equal hipBLASLt's exact int8 GEMM (torch._int_mm) element for element, and the W8 epilogue
    (2^-7 s_x s_w acc + bias + LoRA, one bf16 rounding) is within one bf16 rounding of the same formula
    evaluated in float32 by torch on the exact accumulators."""
    M, K, N, r = 16896, 3072, 12288, 32
    g = torch.Generator(device=dev).manual_seed(5)
    qx = torch.randint(-127, 128, (M, K), device=dev, dtype=torch.int8, generator=g)
    qw = torch.randint(-127, 128, (N, K), device=dev, dtype=torch.int8, generator=g)
    acc = k2._lib.gemm_w8a8_acc(qx, qw)
    ref = torch._int_mm(qx, qw.t())
    assert torch.equal(acc, ref)
    del ref
    sx = torch.rand(M, device=dev, generator=g) * 0.01 + 1e-3
    sw = torch.rand(N, device=dev, generator=g) * 0.01 + 1e-3
    bias = torch.randn(N, device=dev, generator=g) * 0.02
    u = torch.randn(M, r, device=dev, generator=g)
    B = torch.randn(N, r, device=dev, generator=g) * 0.01
    y = k2._lib.gemm_w8a8(qx, sx, qw, sw, bias, u, B, 1.0).float()
    lora = u.bfloat16().float() @ B.bfloat16().float().t()
    yr = acc.float() * ((sx * 0.0078125)[:, None] * sw[None, :]) + bias[None, :] + lora
    err = (y - yr).abs()
    tol = yr.abs() * 2 ** -8 + 1e-6                        # one bf16 rounding (2^-9 relative) plus the
    assert bool((err <= tol).all()), float((err - tol).max())   # f32 ordering differences


@pytest.mark.parametrize("M,N", [(4096, 3072), (16896, 12288)])
def test_full_size_w4_every_tile(k2, dev, M, N):
    """W4A8 at full size, every tile (cfg1's shape and the cfg2 shape with int4 weights; codes -8..7, so
    the unpacking of -8 is covered too).  Group partials come from torch._int_mm per 64-wide group (exact
    int32).  Unit scales: the f32 result is the exact integer sum.  Random bf16 scales: within the f32
    accumulation bound of the float64 sum.  The forward epilogue (2^-7 s_x sum_g s acc_g + bias + LoRA,
    one bf16 rounding) within one bf16 rounding of the same formula in float64."""
    K, r = 3072, 32
    g = torch.Generator(device=dev).manual_seed(11)
    qx = torch.randint(-127, 128, (M, K), device=dev, dtype=torch.int8, generator=g)
    q = torch.randint(-8, 8, (N, K), device=dev, dtype=torch.int8, generator=g)
    q4 = torch.from_numpy(orc.pack_i4(q.cpu().numpy())).to(dev)
    G = K // 64
    s4 = (torch.rand(G, N, device=dev, generator=g) * 0.02 + 1e-3).bfloat16()
    exact = torch.zeros(M, N, dtype=torch.float64, device=dev)
    ref = torch.zeros(M, N, dtype=torch.float64, device=dev)
    mag = torch.zeros(M, N, dtype=torch.float64, device=dev)
    for i in range(G):
        pg = torch._int_mm(qx[:, 64 * i:64 * i + 64].contiguous(), q[:, 64 * i:64 * i + 64].t().contiguous()).double()
        exact += pg
        pg *= s4[i].double()[None, :]
        ref += pg
        mag += pg.abs()
    out = k2._lib.gemm_w4a8_f32(qx, q4, torch.ones(G, N, dtype=torch.bfloat16, device=dev))
    assert torch.equal(out.double(), exact)
    del exact
    out = k2._lib.gemm_w4a8_f32(qx, q4, s4).double()
    assert bool(((out - ref).abs() <= mag * (G * 2.0 ** -24) + 1e-6).all())
    del out
    sx = torch.rand(M, device=dev, generator=g) * 0.01 + 1e-3
    bias = torch.randn(N, device=dev, generator=g) * 0.02
    u = torch.randn(M, r, device=dev, generator=g)
    B = torch.randn(N, r, device=dev, generator=g) * 0.01
    y = k2._lib.gemm_w4a8(qx, sx, q4, s4, bias, u, B, 1.0).double()
    lora = (u.bfloat16().double() @ B.bfloat16().double().t())
    yr = ref * (sx.double() * 0.0078125)[:, None] + bias.double()[None, :] + lora
    err = (y - yr).abs()
    tol = yr.abs() * 2 ** -8 + mag * (sx.double() * 0.0078125)[:, None] * (G * 2.0 ** -24) + 1e-6
    assert bool((err <= tol).all()), float((err - tol).max())


@pytest.mark.parametrize("fold", [True, False])
def test_full_size_cfg3_input_gradient_every_tile(k2, dev, fold):
    """Every tile of cfg3's input gradient (864 tiles on 216 workgroups) against torch in float32: the dense
    product dY W_hat, then the inverse rotation as a block-diagonal Hadamard matmul, times 2^-7, plus g A."""
    M, K, N, r = 4608, 12288, 3072, 64
    w = make_w(N, K, seed=6)
    g = torch.Generator(device=dev).manual_seed(7)
    dy = (torch.randn(M, N, device=dev, generator=g) * 1e-3).to(torch.bfloat16)
    A = torch.randn(r, K, device=dev, generator=g) * 0.01
    gd = torch.randn(M, r, device=dev, generator=g) * 1e-3
    qw, sw = k2._lib.quant_weight_i8(w.to(dev))
    dx = k2._lib.gemm_dx(dy, qw, sw, g=gd, lora_a=A, fold_rotation=fold).float()
    w_hat = (qw.float() * sw[:, None]).bfloat16().float()           # bf16(s_w q_w), N x K
    t = dy.float() @ w_hat                                          # M x K, f32
    H = torch.from_numpy(__import__("scipy.linalg").linalg.hadamard(128).astype(np.float32)).to(dev)
    t = (t.view(M, K // 128, 128) @ H).view(M, K) * 0.0078125
    ref = t + gd.bfloat16().float() @ A.bfloat16().float()
    assert rel_frob(dx.cpu().numpy(), ref.cpu().numpy()) < 3e-3   # bf16 output rounding: ~1.1e-3 RMS


# ------------------------------------------------------------------------------------------- fp8 base (f3)
def _fp8_special_rows(K):
    """Rows whose amax is 448 (scale 1): RNE ties in the normal range (17 -> 16, 1.0625 -> 1, 1.1875 -> 1.25,
    248 -> 256 with the carry into the exponent), subnormal ties (2.5 * 2^-9 -> 2 * 2^-9, 7.5 * 2^-9 -> the
    smallest normal), -0, and a zero row (scale floor 1e-8/448)."""
    v = torch.zeros(3, K)
    ties = [448.0, 17.0, 1.0625, 1.1875, 248.0, 2.5 * 2 ** -9, 7.5 * 2 ** -9, -0.0, -17.0, 0.5 * 2 ** -9, 300.0]
    v[0, : len(ties)] = torch.tensor(ties)
    v[1] = torch.linspace(-448, 448, K)
    return v                                               # row 2 stays zero


@pytest.mark.parametrize("N,K,dtype", [(64, 256, torch.bfloat16), (33, 3072, torch.float32), (8, 12288, torch.bfloat16)])
def test_fp8_weight_quant_bit_exact(k2, dev, N, K, dtype):
    """Fp8Linear.__init__ (quantize.py:34-37) on the GPU: e4m3 codes and bf16 scale bits equal torch's CPU
    computation (the oracle calls the same cast the reference does)."""
    w = torch.randn(N, K, generator=torch.Generator().manual_seed(N + K)) * 0.02
    w[:3] = _fp8_special_rows(K)
    w = w.to(dtype)
    q, s = k2._lib.quant_weight_fp8(w.to(dev))
    q0, s0 = orc.fp8_weight_quant(w.float().numpy())
    assert torch.equal(q.cpu().view(torch.uint8), q0.view(torch.uint8))
    assert torch.equal(s.cpu().view(torch.int16), s0.view(torch.int16))
    assert q.cpu().view(torch.uint8)[0, :11].tolist() == [0x7E, 0x58, 0x38, 0x3A, 0x78, 0x02, 0x08, 0x80, 0xD8, 0x00, 0x79]


def test_fp8_dequant_exact(k2, dev):
    """bf16(q * s) per element, as `weight_fp8.to(bf16) * scale.to(bf16)` (quantize.py:49), and transposed."""
    w = torch.randn(96, 640, generator=torch.Generator().manual_seed(5)) * 0.02
    w[:3] = _fp8_special_rows(640)
    q, s = k2._lib.quant_weight_fp8(w.to(dev))
    ref = q.cpu().to(torch.bfloat16) * s.cpu().to(torch.bfloat16)
    assert torch.equal(k2._lib.dequant_fp8(q, s).cpu().view(torch.int16), ref.view(torch.int16))
    assert torch.equal(k2._lib.dequant_fp8(q, s, transpose=True).cpu().view(torch.int16), ref.t().contiguous().view(torch.int16))


@pytest.mark.parametrize("M,K,N,bias", [(256, 256, 256, False), (300, 640, 320, True), (1000, 3072, 1024, True)])
def test_fp8_linear_matches_reference(k2, dev, M, K, N, bias):
    """The Fp8Linear module against the reference's forward restated on the CPU (dequantize, bf16 F.linear):
    the same bf16 weights and bias, so only the f32 summation order differs."""
    lin = torch.nn.Linear(K, N, bias=bias, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(make_w(N, K, seed=K))
        if bias:
            lin.bias.copy_(torch.randn(N, generator=torch.Generator().manual_seed(2)) * 0.02)
    base = k2.Fp8Linear(lin.to(dev))
    x = make_x(M, K, seed=M)
    with torch.no_grad():
        y = base(x.to(dev)).float().cpu()
    q0, s0 = orc.fp8_weight_quant(lin.weight.detach().float().cpu().numpy())
    ref = orc.fp8_linear(x, q0, s0, None if not bias else lin.bias.detach().cpu()).float()
    assert rel_frob(y.numpy(), ref.numpy()) < 1e-3


def test_fp8_lora_forward_backward(k2, dev):
    """LoRALinear over the fp8 base (fused path): forward against lora.py:47-48 on the reference forward, and
    dX, dA, dB against float64 autograd of the same dequantized weights."""
    M, K, N, r = 192, 512, 384, 32
    lin = torch.nn.Linear(K, N, bias=True, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(make_w(N, K, seed=3))
        lin.bias.copy_(torch.randn(N, generator=torch.Generator().manual_seed(4)) * 0.02)
    base = k2.Fp8Linear(lin.to(dev))
    lora = k2.LoRALinear(base, r, float(r))
    g = torch.Generator().manual_seed(6)
    with torch.no_grad():
        lora.lora_A.copy_(torch.randn(r, K, generator=g) * 0.01)
        lora.lora_B.copy_(torch.randn(N, r, generator=g) * 0.01)
    x = make_x(M, K, seed=7)
    dy = (torch.randn(M, N, generator=g) * 1e-3).to(torch.bfloat16)
    xd = x.to(dev).requires_grad_(True)
    y = lora(xd)
    y.backward(dy.to(dev))
    q0, s0 = orc.fp8_weight_quant(lin.weight.detach().float().cpu().numpy())
    A, B = lora.lora_A.detach().cpu(), lora.lora_B.detach().cpu()
    base_ref = orc.fp8_linear(x, q0, s0, lin.bias.detach().cpu())
    ref = base_ref + (((x.float() @ A.t()) @ B.t()).to(torch.bfloat16))   # lora.py:47-48, scale 1
    assert rel_frob(y.detach().float().cpu().numpy(), ref.float().numpy()) < 4e-3
    wd = (q0.to(torch.bfloat16) * s0.to(torch.bfloat16)).double()
    x64 = x.double().requires_grad_(True)
    A64, B64 = A.double().requires_grad_(True), B.double().requires_grad_(True)
    y64 = x64 @ wd.t() + (x64 @ A64.t()) @ B64.t()
    y64.backward(dy.double())
    assert rel_frob(xd.grad.float().cpu().numpy(), x64.grad.numpy()) < REL_FROB_TOL
    assert rel_frob(lora.lora_A.grad.cpu().numpy(), A64.grad.numpy()) < 1e-3
    assert rel_frob(lora.lora_B.grad.cpu().numpy(), B64.grad.numpy()) < 1e-3


def test_quantize_dit_fp8_walker(k2, dev):
    """quantize_dit_fp8 (quantize.py:54-68): same walk and count; the blocks then run on the fp8 kernels."""
    import torch.nn as nn

    class Blk(nn.Module):
        def __init__(self):
            super().__init__()
            self.attn = nn.Module()
            self.attn.wq = nn.Linear(256, 256, bias=False, dtype=torch.bfloat16)
            self.mlp = nn.Module()
            self.mlp.up = nn.Linear(256, 512, bias=False, dtype=torch.bfloat16)

    class Dit(nn.Module):
        def __init__(self):
            super().__init__()
            self.first = nn.Linear(8, 256, dtype=torch.bfloat16)
            self.blocks = nn.ModuleList([Blk(), Blk(), Blk()])

    dit = Dit().to(dev)
    w_up = dit.blocks[0].mlp.up.weight.detach().float().cpu().numpy()
    assert k2.quantize_dit_fp8(dit) == 6
    assert isinstance(dit.blocks[0].mlp.up, k2.Fp8Linear) and isinstance(dit.first, nn.Linear)
    x = make_x(32, 256, seed=1)
    with torch.no_grad():
        y = dit.blocks[0].mlp.up(x.to(dev)).float().cpu()
    q0, s0 = orc.fp8_weight_quant(w_up)
    assert rel_frob(y.numpy(), orc.fp8_linear(x, q0, s0).float().numpy()) < 1e-3


# ------------------------------------------------------------------------------------------- on-disk base (f4)
@pytest.mark.parametrize("mode", ["w8a8", "w4a8", "fp8"])
def test_quantized_base_file_reproduces_outputs(k2, dev, mode, tmp_path):
    """Quantize on the GPU, save, load into a fresh model (no re-quantization): bit-identical outputs."""
    import torch.nn as nn

    def make():
        torch.manual_seed(0)
        blk = nn.Module()
        blk.mlp = nn.Module()
        blk.mlp.up = nn.Linear(256, 512, bias=True, dtype=torch.bfloat16)
        dit = nn.Module()
        dit.blocks = nn.ModuleList([blk])
        return dit.to(dev)

    src = make()
    if mode == "fp8":
        k2.quantize_dit_fp8(src)
    else:
        k2.quantize_dit_convrot(src, mode)
    f = str(tmp_path / "q.safetensors")
    assert k2.save_quantized_base(src, f) == 1
    dst = make()
    assert k2.load_quantized_base(dst, f, device=dev) == 1
    x = make_x(64, 256, seed=2).to(dev)
    with torch.no_grad():
        assert torch.equal(src.blocks[0].mlp.up(x).view(torch.int16), dst.blocks[0].mlp.up(x).view(torch.int16))


# ------------------------------------------------------------------------------------------- shared input (f1)
def test_shared_input_quantized_once(k2, dev):
    """wq/wk/wv/gate of one attention read the same tensor (mmdit.py:199): it is rotated and quantized once,
    and every output equals the one computed with its own quantization; an in-place write to the input or a
    different tensor forces a fresh quantization."""
    import importlib
    cache = importlib.import_module("krea2_amd.quantize").shared_input_quant
    layers = [_layers(k2, dev, K=512, N=384, r=16, seed=s)[2] for s in range(4)]
    x = make_x(96, 512, seed=21).to(dev)
    with torch.no_grad():
        m0 = cache.misses
        ys = [l(x) for l in layers]
        assert cache.misses == m0 + 1
        cache.enabled = False
        try:
            ref = [l(x) for l in layers]
        finally:
            cache.enabled = True
        for a, b in zip(ys, ref):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16))
        m1 = cache.misses
        x.mul_(2)                                   # in-place write: version bump
        y2 = layers[0](x)
        assert cache.misses == m1 + 1
        cache.enabled = False
        try:
            assert torch.equal(y2.view(torch.int16), layers[0](x).view(torch.int16))
        finally:
            cache.enabled = True
        m2 = cache.misses
        layers[1](x)                                # same tensor, unchanged since: reused
        assert cache.misses == m2
        layers[1](x.clone())                        # another tensor with equal values: quantized afresh
        assert cache.misses == m2 + 1


def test_mfma_probe_runs_and_counts(k2, dev):
    """The same-run MFMA ceiling bench.py reports (its own library, libk2q_probe.so): the probe writes one
    checksum per thread (not all equal: the operands differ per lane) and reports 2*32^3 ops per MFMA, 64 MFMAs
    per wave and iteration."""
    import bench
    ops = bench.mfma_probe_i8(3, 4, dev)
    torch.cuda.synchronize()
    assert ops == 4 * 8 * 3 * 64 * 2 * 32 * 32 * 32
    out = bench._probe[dev][: 4 * 512].cpu()
    assert len(set(out.tolist())) > 1
