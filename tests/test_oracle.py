"""Pins of the CPU oracle (``oracle/convrot.py``) — CPU only.

The reference holds no golden vectors or tests for this path, so every oracle function is pinned here by
an independent route: a library routine (``scipy.linalg.hadamard``), a closed form, hand-computed known
answers, brute force on tiny inputs, or torch autograd.  Each pin is chosen so that a plausible mistake (a
dropped term, a wrong sign or index, a transposed operand, a wrong rounding mode) fails it.
"""
import math

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import convrot as orc

H128 = scipy.linalg.hadamard(128).astype(np.float64)


def R_block(K):
    return np.kron(np.eye(K // 128), H128)


# ---------------------------------------------------------------------------------------------- rotation
def test_fwht_matches_sylvester_hadamard_exactly_on_small_integers():
    rng = np.random.default_rng(1)
    x = rng.integers(-8, 9, size=(5, 384)).astype(np.float32)   # every partial sum exact in f32
    assert np.array_equal(orc.fwht_blocks(x).astype(np.float64), x.astype(np.float64) @ R_block(384))


def test_fwht_invariants():
    K = 256
    e = np.zeros((1, K), np.float32)
    e[0, 130] = 1.0
    assert np.array_equal(orc.fwht_blocks(e)[0, 128:], H128[2])          # unit vector -> its row
    assert np.all(orc.fwht_blocks(e)[0, :128] == 0)                        # block diagonal
    c = np.full((1, 128), 3.0, np.float32)
    out = orc.fwht_blocks(c)[0]
    assert out[0] == 384.0 and np.all(out[1:] == 0)                        # constant -> 128c at 0
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, K)).astype(np.float32)
    twice = orc.fwht_blocks_f64(orc.fwht_blocks_f64(x))
    np.testing.assert_allclose(twice, 128.0 * x, rtol=1e-12, atol=1e-9)     # H H = 128 I


def test_fwht_f32_stage_order_is_fixed():
    """The f32 butterfly is not the dense product in general; it must equal a loop restatement of
    strides 1, 2, ..., 64 with (a+b, a-b) pairs (written here as explicit Python loops)."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(128) * np.array([1e4 if i % 7 == 0 else 1.0 for i in range(128)])).astype(np.float32)
    v = [np.float32(t) for t in x]
    s = 1
    while s < 128:
        for base in range(0, 128, 2 * s):
            for i in range(base, base + s):
                a, b = v[i], v[i + s]
                v[i], v[i + s] = np.float32(a + b), np.float32(a - b)
        s *= 2
    assert np.array_equal(orc.fwht_blocks(x[None])[0], np.array(v, np.float32))


def test_xrot_within_two_bf16_ulp_of_dense_rotation():
    rng = np.random.default_rng(4)
    x = orc.bf16_round(rng.standard_normal((64, 512)).astype(np.float32))
    x[:, ::37] *= 20
    x = orc.bf16_round(x)
    _, _, xr = orc.rotquant(x, want_xrot=True)
    dense = (x.astype(np.float64) @ R_block(512)) / math.sqrt(128)
    ref_bits = orc.bf16_bits(dense.astype(np.float32)).astype(np.int32)
    got_bits = xr.astype(np.int32)
    sign_ok = (np.sign(dense) == np.sign(orc.bf16_to_f32(xr))) | (np.abs(dense) < 1e-30)
    assert sign_ok.all()
    assert np.abs(got_bits - ref_bits).max() <= 2


# ---------------------------------------------------------------------------------------------- quantizer
def test_rotquant_recovers_exact_codes_from_a_rotated_integer_row():
    """x = q0 R / 128 with row absmax 127 -> rotquant returns q0 and scale 1.0 exactly."""
    rng = np.random.default_rng(5)
    q0 = rng.integers(-127, 128, size=(6, 384))
    q0[:, 7] = 127                      # absmax exactly 127 in every row
    x = (q0 @ R_block(384) / 128.0).astype(np.float32)   # exact in f32 (integers/128 below 2^15)
    q, s, _ = orc.rotquant(x)
    assert np.array_equal(q.astype(np.int64), q0)
    assert np.array_equal(s, np.ones(6, np.float32))


def test_rotquant_round_half_to_even_known_answer():
    """Rotated row v = [254, 1, 3, 5, -1, -3, 7, 0...]: absmax 254 -> inv 0.5 -> v*inv hits .5 exactly."""
    v = np.zeros(128)
    v[:7] = [254, 1, 3, 5, -1, -3, 7]
    x = (v @ H128 / 128.0).astype(np.float32)[None]
    q, s, _ = orc.rotquant(x)
    assert list(q[0, :7]) == [127, 0, 2, 2, 0, -2, 4]
    assert s[0] == np.float32(2.0)


def test_rotquant_zero_row_and_absmax_element():
    rng = np.random.default_rng(6)
    x = orc.bf16_round(rng.standard_normal((4, 256)).astype(np.float32))
    x[1] = 0
    q, s, _ = orc.rotquant(x)
    assert np.all(q[1] == 0) and s[1] == np.float32(1e-8) / np.float32(127)
    v = orc.fwht_blocks(x)
    for m in (0, 2, 3):
        j = np.argmax(np.abs(v[m]))
        assert abs(int(q[m, j])) == 127 and np.sign(q[m, j]) == np.sign(v[m, j])
        assert np.abs(q[m]).max() == 127


def test_rotquant_brute_force_tiny():
    """Pure-Python float32 restatement on a 2 x 128 input, element by element."""
    rng = np.random.default_rng(7)
    x = orc.bf16_round(rng.standard_normal((2, 128)).astype(np.float32) * 3)
    q, s, _ = orc.rotquant(x)
    v = orc.fwht_blocks(x)
    for m in range(2):
        amax = max(np.float32(abs(t)) for t in v[m])
        inv = np.float32(np.float32(127) / np.float32(amax))
        for k in range(128):
            p = np.float32(v[m, k] * inv)
            fl = math.floor(p)
            d = float(p) - fl
            r = fl + (1 if d > 0.5 or (d == 0.5 and fl % 2 == 1) else 0)
            assert q[m, k] == r
        assert s[m] == np.float32(np.float32(amax) / np.float32(127))


# ---------------------------------------------------------------------------------------------- int4
def test_int4_pack_known_answer_and_roundtrip():
    q = np.zeros((1, 16), np.int8)
    q[0, 0], q[0, 8] = 1, -1          # byte 0 = 0x1 | 0xF << 4
    q[0, 1], q[0, 9] = -7, 7          # byte 1 = 0x9 | 0x7 << 4
    p = orc.pack_i4(q)
    assert p[0, 0] == 0xF1 and p[0, 1] == 0x79 and np.all(p[0, 2:] == 0)
    rng = np.random.default_rng(8)
    q = rng.integers(-7, 8, size=(5, 256)).astype(np.int8)
    assert np.array_equal(orc.unpack_i4(orc.pack_i4(q)), q)


def test_int4_group_quant_known_answer():
    """A rotated group whose absmax is 7 * 2^-3 gets the exact bf16 scale 2^-3 and codes v / 2^-3."""
    v = np.zeros(128)
    v[:4] = [7 * 0.125, 0.125, -2.5 * 0.125, 3.5 * 0.125]    # group 0 (k < 64)
    v[64] = 7 * 4.0                                           # group 1 scale 4
    v[65] = -1.5 * 4.0
    x = (v @ H128 / 128.0).astype(np.float32)[None]
    q, s_bits = orc.quant_weight_i4(x)
    s = orc.bf16_to_f32(s_bits)
    assert s[0, 0] == np.float32(0.125) and s[0, 1] == np.float32(4.0)
    assert list(q[0, :4]) == [7, 1, -2, 4]            # -2.5 -> -2, 3.5 -> 4 (half to even)
    assert list(q[0, 64:66]) == [7, -2]
    assert np.abs(q).max() <= 7


# ---------------------------------------------------------------------------------------------- GEMM
def test_gemm_acc_brute_force_and_int_mm():
    rng = np.random.default_rng(9)
    qx = rng.integers(-127, 128, size=(3, 128)).astype(np.int8)
    qw = rng.integers(-127, 128, size=(4, 128)).astype(np.int8)
    acc = orc.gemm_acc(qx, qw)
    for m in range(3):
        for n in range(4):
            assert acc[m, n] == sum(int(qx[m, k]) * int(qw[n, k]) for k in range(128))
    qx = rng.integers(-127, 128, size=(64, 256)).astype(np.int8)
    qw = rng.integers(-127, 128, size=(48, 256)).astype(np.int8)
    ref = torch._int_mm(torch.from_numpy(qx), torch.from_numpy(qw).t().contiguous()).numpy()
    assert np.array_equal(orc.gemm_acc(qx, qw), ref)
    assert np.array_equal(orc.gemm_acc_fast(qx, qw), ref)


def test_gemm_groups_sum_to_full_acc():
    rng = np.random.default_rng(10)
    qx = rng.integers(-127, 128, size=(8, 256)).astype(np.int8)
    qw = rng.integers(-7, 8, size=(6, 256)).astype(np.int8)
    assert np.array_equal(orc.gemm_acc_groups(qx, qw).sum(-1), orc.gemm_acc(qx, qw).astype(np.int64))


# ---------------------------------------------------------------------------------------------- forward
def test_forward_closed_form_on_exactly_quantizable_inputs():
    """x = qx0 R/128, W = qw0 R/128 -> scales 1, and y = 2^-7 qx0 qw0^T = x W^T exactly (rotation
    invariance).  Pins the 2^-7, the orientation of the GEMM and the scale placement."""
    rng = np.random.default_rng(11)
    K = 256
    qx0 = rng.integers(-127, 128, size=(5, K))
    qx0[:, 3] = -127
    qw0 = rng.integers(-127, 128, size=(7, K))
    qw0[:, 9] = 127
    x = (qx0 @ R_block(K) / 128).astype(np.float32)
    W = (qw0 @ R_block(K) / 128).astype(np.float32)
    qw, sw = orc.quant_weight_i8(W)
    out = orc.forward(x, qw, sw)
    np.testing.assert_allclose(out["y64"], x.astype(np.float64) @ W.astype(np.float64).T, rtol=0, atol=1e-9)


def test_forward_w4_equal_group_scales_equals_w8():
    rng = np.random.default_rng(12)
    x = orc.bf16_round(rng.standard_normal((9, 256)).astype(np.float32))
    q = rng.integers(-7, 8, size=(5, 256)).astype(np.int8)
    s = np.full(5, 0.25, np.float32)
    s4 = orc.bf16_bits(np.full((5, 4), 0.25, np.float32))
    y8 = orc.forward(x, q, s)["y64"]
    y4 = orc.forward(x, q, s4, w4=True)["y64"]
    np.testing.assert_allclose(y4, y8, rtol=1e-14, atol=0)


def test_forward_tracks_the_unquantized_linear():
    """W8A8 with the rotation stays within a few percent of x W^T on outlier-laden activations."""
    g = torch.Generator().manual_seed(0)
    M, K, N = 64, 512, 96
    x = torch.randn(M, K, generator=g)
    idx = torch.randperm(K, generator=g)[: K // 100 + 1]
    x[:, idx] *= 20
    x = x.to(torch.bfloat16).float().numpy()
    W = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).float().numpy()
    qw, sw = orc.quant_weight_i8(W)
    y = orc.forward(x, qw, sw)["y64"]
    ref = x.astype(np.float64) @ W.astype(np.float64).T
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < 0.03


def test_lora_term_matches_reference_formula_and_is_linear():
    """lora.py:47-48: out + s * ((x.f32 @ A^T) @ B^T); s = 0 gives the base; the term is linear in s."""
    rng = np.random.default_rng(13)
    x = orc.bf16_round(rng.standard_normal((6, 128)).astype(np.float32))
    W = orc.bf16_round((rng.standard_normal((8, 128)) * 0.02).astype(np.float32))
    A = (rng.standard_normal((16, 128)) * 0.01).astype(np.float32)
    B = (rng.standard_normal((8, 16)) * 0.01).astype(np.float32)
    qw, sw = orc.quant_weight_i8(W)
    base = orc.forward(x, qw, sw)["y64"]
    assert np.array_equal(orc.forward(x, qw, sw, lora_A=A, lora_B=B, lora_scale=0.0)["y64"], base)
    y1 = orc.forward(x, qw, sw, lora_A=A, lora_B=B, lora_scale=1.5)["y64"]
    ym = orc.forward(x, qw, sw, lora_A=A, lora_B=B, lora_scale=-1.5)["y64"]
    ref = torch.from_numpy(x) @ torch.from_numpy(A).t() @ torch.from_numpy(B).t()
    np.testing.assert_allclose(y1 - base, 1.5 * ref.double().numpy(), rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(y1 - base, -(ym - base), rtol=1e-12, atol=1e-15)


# ---------------------------------------------------------------------------------------------- backward
@pytest.mark.parametrize("w4", [False, True])
def test_backward_matches_torch_autograd(w4):
    """dX, dA, dB of the oracle equal torch autograd (f64) of the dequantized straight-through forward
    y = 2^-7 (x R) W_hat^T + s (x A^T) B^T."""
    rng = np.random.default_rng(14)
    M, K, N, r = 5, 256, 6, 16
    x = rng.standard_normal((M, K))
    if w4:
        q = rng.integers(-7, 8, size=(N, K)).astype(np.int8)
        ws = orc.bf16_bits((rng.uniform(0.5, 2, size=(N, K // 64))).astype(np.float32))
    else:
        q = rng.integers(-127, 128, size=(N, K)).astype(np.int8)
        ws = rng.uniform(0.5, 2, size=N).astype(np.float32)
    A = rng.standard_normal((r, K)) * 0.1
    B = rng.standard_normal((N, r)) * 0.1
    dy = rng.standard_normal((M, N))
    s = 0.75
    out = orc.backward(dy, x, q, ws, w4=w4, lora_A=A, lora_B=B, lora_scale=s)

    Wh = torch.from_numpy(orc.dequant_weight(q, ws, w4=w4))
    R = torch.from_numpy(R_block(K))
    xt = torch.from_numpy(x).requires_grad_(True)
    At = torch.from_numpy(A).requires_grad_(True)
    Bt = torch.from_numpy(B).requires_grad_(True)
    y = (xt @ R) @ Wh.t() / 128 + s * (xt @ At.t()) @ Bt.t()
    y.backward(torch.from_numpy(dy))
    np.testing.assert_allclose(out["dx64"], xt.grad.numpy(), rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(out["dA"], At.grad.numpy(), rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(out["dB"], Bt.grad.numpy(), rtol=1e-10, atol=1e-10)


# ---------------------------------------------------------------------------------------------- fp8 base
def test_fp8_weight_quant_known_answer():
    """quantize.py:34-39 on a row with amax 448: scale 1 and e4m3 codes = RNE of the values."""
    w = np.array([[448.0, 1.0, -3.3, 0.1, 17.0, -448.0, 0.0, 2.6]], np.float32)
    q, s = orc.fp8_weight_quant(w)
    assert float(s[0, 0]) == 1.0
    assert q.float().tolist()[0] == [448.0, 1.0, -3.25, 0.1015625, 16.0, -448.0, 0.0, 2.5]


# ---------------------------------------------------------------------------------------------- producers
def _bf16(a):
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16)


def _ulp_diff(a, b):
    """Distance in bf16 steps between two float32 arrays holding bf16 values (same sign assumed near 0)."""
    ia = orc.bf16_bits(a).astype(np.int32)
    ib = orc.bf16_bits(b).astype(np.int32)
    ia = np.where(ia & 0x8000, 0x8000 - ia, ia)   # sign-magnitude -> ordered integers
    ib = np.where(ib & 0x8000, 0x8000 - ib, ib)
    return np.abs(ia - ib)


def test_swiglu_closed_forms():
    """silu(0) = 0; silu(g) rounds to g for g >= 16 (exp(-g) < 2^-23 of 1) and to -0 for g <= -104 (exp
    overflows); u = 0 gives 0; the product is rounded to bf16 once more (3 * 0.73046875 -> 2.1875)."""
    g = np.array([0.0, 16.0, 24.0, -120.0, 1.0, 1.0], np.float32)
    u = np.array([5.0, 3.0, -2.0, 7.0, 0.0, 3.0], np.float32)
    h = orc.swiglu(g, u)
    assert h.tolist()[:5] == [0.0, 48.0, -48.0, 0.0, 0.0]
    assert h[5] == orc.bf16_round(np.float32(3.0) * np.float32(0.73046875))  # bf16(silu(1)) = 0.73046875
    assert orc.swiglu(np.float32([1.0]), np.float32([1.0]))[0] == np.float32(0.73046875)


def test_swiglu_matches_torch_eager_bf16():
    """Against torch's CPU ``F.silu(g) * u`` on bf16 tensors (its own exp): within one bf16 step, and equal
    almost everywhere (a rounding-order mistake would move far more than 0.1% of the elements)."""
    rng = np.random.default_rng(21)
    g = orc.bf16_round(rng.standard_normal((64, 512)).astype(np.float32) * 3)
    u = orc.bf16_round(rng.standard_normal((64, 512)).astype(np.float32))
    ref = (torch.nn.functional.silu(_bf16(g)) * _bf16(u)).float().numpy()
    d = _ulp_diff(orc.swiglu(g, u), ref)
    assert d.max() <= 1 and (d == 0).mean() > 0.999


def test_swiglu_backward_matches_torch_autograd_bf16():
    rng = np.random.default_rng(22)
    g = orc.bf16_round(rng.standard_normal((32, 512)).astype(np.float32) * 3)
    u = orc.bf16_round(rng.standard_normal((32, 512)).astype(np.float32))
    dh = orc.bf16_round(rng.standard_normal((32, 512)).astype(np.float32) * 1e-3)
    gt, ut = _bf16(g).requires_grad_(True), _bf16(u).requires_grad_(True)
    (torch.nn.functional.silu(gt) * ut).backward(_bf16(dh))
    dg, du = orc.swiglu_backward(dh, g, u)
    d_u = _ulp_diff(du, ut.grad.float().numpy())
    d_g = _ulp_diff(dg, gt.grad.float().numpy())
    assert d_u.max() <= 1 and (d_u == 0).mean() > 0.999
    assert d_g.max() <= 2 and (d_g == 0).mean() > 0.99


def test_rmsmod_closed_forms():
    """A row of +-c with c a power of two has rms c, so n = sign * (scale + 1) exactly (eps = 0); p = -1
    zeroes the modulated norm and leaves the shift; p = b = 0 gives n; the batch entry of row m is m // L."""
    K = 256
    x = np.full((2, K), 4.0, np.float32)
    x[:, ::2] = -4.0
    ns = np.zeros(K, np.float32)
    ns[:4] = [0.5, -0.25, 1.0, 0.0]
    zero = np.zeros((1, K), np.float32)
    n = orc.rmsmod(x, ns, 0.0, zero, zero, 2)
    assert np.array_equal(n, np.sign(x) * (ns + 1.0)[None, :])
    b = orc.bf16_round(np.linspace(-2, 2, K, dtype=np.float32))[None, :]
    assert np.array_equal(orc.rmsmod(x, ns, 0.0, -np.ones((1, K), np.float32), b, 2), np.repeat(b, 2, 0))
    ms = np.stack([np.zeros(K, np.float32), np.ones(K, np.float32)])       # batch 1 doubles its rows
    h = orc.rmsmod(np.tile(x, (2, 1)), ns, 0.0, ms, np.zeros((2, K), np.float32), 2)
    assert np.array_equal(h[2:], orc.bf16_round(2 * h[:2]))


def test_rmsmod_matches_torch_eager_bf16():
    """Against torch's CPU ``(1 + p) * F.rms_norm(x.float(), eps, weight=scale + 1).to(bf16) + b`` on bf16
    tensors shaped as in the block (x (B,L,K), p / b (B,1,K)): within one bf16 step, almost all equal."""
    rng = np.random.default_rng(23)
    B, L, K, eps = 2, 48, 768, 1e-5
    x = orc.bf16_round(rng.standard_normal((B * L, K)).astype(np.float32) * 2)
    ns = (rng.standard_normal(K) * 0.1).astype(np.float32)
    p = orc.bf16_round(rng.standard_normal((B, K)).astype(np.float32) * 0.3)
    b = orc.bf16_round(rng.standard_normal((B, K)).astype(np.float32) * 0.3)
    xt = _bf16(x).reshape(B, L, K)
    n = torch.nn.functional.rms_norm(xt.float(), (K,), eps=eps, weight=torch.from_numpy(ns) + 1.0)
    ref = ((1 + _bf16(p)[:, None, :]) * n.to(torch.bfloat16) + _bf16(b)[:, None, :]).float().reshape(B * L, K)
    d = _ulp_diff(orc.rmsmod(x, ns, eps, p, b, L), ref.numpy())
    assert d.max() <= 1 and (d == 0).mean() > 0.999


def test_rmsmod_backward_x_matches_torch_autograd():
    """Against torch's CPU autograd of the reference formula (bf16 tensors, ``F.rms_norm`` on float32):
    close in relative Frobenius norm and equal in most elements; a dropped bf16 rounding of ``dn`` or a
    missing ``+1`` on the norm weight fails it."""
    rng = np.random.default_rng(24)
    B, L, K, eps = 2, 32, 512, 1e-5
    x = orc.bf16_round(rng.standard_normal((B * L, K)).astype(np.float32) * 2)
    ns = (rng.standard_normal(K) * 0.1).astype(np.float32)
    p = orc.bf16_round(rng.standard_normal((B, K)).astype(np.float32) * 0.3)
    b = orc.bf16_round(rng.standard_normal((B, K)).astype(np.float32) * 0.3)
    dh = orc.bf16_round(rng.standard_normal((B * L, K)).astype(np.float32) * 1e-2)
    xt = _bf16(x).reshape(B, L, K).requires_grad_(True)
    n = torch.nn.functional.rms_norm(xt.float(), (K,), eps=eps, weight=torch.from_numpy(ns) + 1.0)
    h = (1 + _bf16(p)[:, None, :]) * n.to(torch.bfloat16) + _bf16(b)[:, None, :]
    h.backward(_bf16(dh).reshape(B, L, K))
    ref = xt.grad.float().reshape(B * L, K).numpy()
    dx = orc.rmsmod_backward_x(dh, x, ns, eps, p, L)
    assert np.linalg.norm(dx - ref) / np.linalg.norm(ref) < 1e-3     # unrounded dn: 2.8e-3
    assert (_ulp_diff(dx, ref) == 0).mean() > 0.99                    # unrounded dn: 73% equal
