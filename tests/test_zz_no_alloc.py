"""GPU test of ``k2q_lora_grads_noalloc`` (the LoRA gradients with the workspace in the library's own device
scratch) against ``k2q_lora_grads`` (caller workspace): bit-identical outputs on two calls in a row, the second
with a smaller input (the scratch keeps the first call's contents), called through the C ABI; nothing allocated
by torch during the calls; a shape beyond the scratch is refused with K2Q_ESCRATCH before any launch."""
import ctypes
import gc

import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(M, N, K, r, seed, dev):
    g = torch.Generator().manual_seed(seed)
    dy = (torch.randn(M, N, generator=g) * 1e-3).to(torch.bfloat16).to(dev)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    u = torch.randn(M, r, generator=g).to(dev)
    B = (torch.randn(N, r, generator=g) * 0.01).to(dev)
    return dy, x, u, B


def _noalloc(lib, dy, x, u, B, s, dev):
    M, N = dy.shape
    K, r = x.shape[1], B.shape[1]
    g = torch.empty(M, r, device=dev)
    dA = torch.empty(r, K, device=dev)
    dB = torch.empty(N, r, device=dev)
    # earlier tests' reference cycles (modules with patched bound methods) are collected now, and the collector
    # stays off during the call, so that only the call itself can move torch's count
    gc.collect()
    torch.cuda.synchronize()
    gc.disable()
    try:
        before = torch.cuda.memory_allocated(dev)
        rc = lib.k2q_lora_grads_noalloc(dy.data_ptr(), x.data_ptr(), u.data_ptr(), B.data_ptr(), r, s, M, N, K,
                                        g.data_ptr(), dA.data_ptr(), dB.data_ptr(),
                                        torch.cuda.current_stream(dev).cuda_stream)
        torch.cuda.synchronize()
        after = torch.cuda.memory_allocated(dev)
    finally:
        gc.enable()
    assert rc == 0
    assert after == before
    return g, dA, dB


def test_noalloc_lora_grads_match_workspace_entry(k2, dev):
    lib = k2._lib.load()
    for (M, N, K, r), seed in (((4608, 3072, 12288, 64), 1), ((777, 640, 1280, 48), 2)):   # large, then smaller
        dy, x, u, B = _inputs(M, N, K, r, seed, dev)
        g0, dA0, dB0 = k2._lib.lora_grads(dy, x, u, B, 0.75)
        g1, dA1, dB1 = _noalloc(lib, dy, x, u, B, 0.75, dev)
        assert torch.equal(g1, g0) and torch.equal(dA1, dA0) and torch.equal(dB1, dB0), (M, N, K, r)
        # the Python wrapper: same entry, caller-provided outputs
        g2, dA2, dB2 = torch.empty_like(g0), torch.empty_like(dA0), torch.empty_like(dB0)
        k2._lib.lora_grads_noalloc(dy, x, u, B, 0.75, g2, dA2, dB2)
        assert torch.equal(g2, g0) and torch.equal(dA2, dA0) and torch.equal(dB2, dB0)


def test_noalloc_refuses_shapes_beyond_its_scratch(k2, dev):
    lib = k2._lib.load()
    M, N, K, r = 16896, 12288, 3072, 128
    assert lib.k2q_lora_grads_ws_bytes(M, N, K, r) > k2._lib.SCRATCH_BYTES
    buf = torch.zeros(64, device=dev)
    p = buf.data_ptr()
    assert lib.k2q_lora_grads_noalloc(p, p, p, p, r, 1.0, M, N, K, p, p, p,
                                      torch.cuda.current_stream(dev).cuda_stream) == -5
    dy = torch.zeros(M, N, dtype=torch.bfloat16, device=dev)
    B = torch.zeros(N, r, device=dev)
    with pytest.raises(ValueError, match="scratch"):
        k2._lib.lora_grads_noalloc(dy, None, None, B, 1.0, torch.empty(M, r, device=dev))
