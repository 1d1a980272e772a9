"""Benchmark of the ConvRot QuantLinear + LoRA forward on one MI355X (BASELINE.json metric and configs).

A step is one QuantLinear+LoRA forward over one batch of synthetic input resident in HBM, as the module
runs it: one library call (k2q_linear_fwd) issuing rotate+quantize (kernel 1), the LoRA down-projection and
the int8 MFMA GEMM with the fused dequant/bias/LoRA epilogue (kernels 2+3).  The default workload is
BASELINE.json configs[2] (M=16384+512, K=3072, N=12288, r=32), the configuration the north_star's targets are
stated on.  ``value`` is the forward's throughput in TOPS (2*M*N*K per step time).  Times are the GPU's: the
events bracketing each timed region are preceded by untimed device copies long enough for the host to enqueue
the whole region first (``queue_head``), so the GPU never waits for a launch; the host's issue time per call
is reported beside (``host_us_per_step``).  Rank 0 prints one JSON line; ``roofline`` covers the dominant
kernel (the GEMM, int8-MFMA bound) with its average duration measured by HIP events around it in K steps
that launch the three kernels one by one, on the stream the kernels run on; ``cpu_baseline`` times the CPU
oracle (a port of the same arithmetic) on a bounded sample of rows.
Before the W warmup steps, ``--settle`` seconds of untimed steps let the GPU clocks leave their ramp-up
state (``extra.settle_s`` reports it).

Every BASELINE.json configuration gets its own record in ``extra`` (``cfg0`` .. ``cfg4``): GPU ms and TOPS,
the roofline fraction of its dominant kernel against the peak that bounds it (int8 MFMA for the forward GEMMs,
bf16 MFMA for the input-gradient GEMM, HBM for rotate/quant and the M=2 GEMV), and two CPU paths timed in the
same process on the host's cores: the oracle (this build's arithmetic restated on the CPU) and the reference's
own ``Fp8Linear`` + ``LoRALinear`` maths restated with torch CPU ops.

    python bench.py [--steps K] [--warmup W] [--settle S] [--config 2] [--no-cpu]
    python bench.py --profile-pass          # fixed launches for rocprofv3 counter passes
    python bench.py --pmc-summary DIR       # traffic table from two rocprofv3 --pmc runs over --profile-pass
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import platform
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

INT8_PEAK_TOPS = 5000.0     # MI355X dense int8 MFMA (5.0 POP/s)
BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
METRIC = "QuantLinear+LoRA fwd TOPS & % int8 MFMA peak; rotate/quant GB/s; block fwd ms"

# BASELINE.json configs -> shapes
CONFIGS = {
    0: dict(M=4096, K=3072, N=3072, r=16, w4=False, bias=True,
            name="cfg0: ConvRot W8A8 QuantLinear+LoRA fwd, M=4096 K=3072 N=3072 r=16, fp32 bias"),
    1: dict(M=4096, K=3072, N=3072, r=16, w4=True, bias=True,
            name="cfg1: ConvRot W4A8 (g64) QuantLinear+LoRA fwd, M=4096 K=3072 N=3072 r=16"),
    2: dict(M=16896, K=3072, N=12288, r=32, w4=False, bias=False,
            name="cfg2: ConvRot W8A8 QuantLinear+LoRA fwd (MLP up @2048^2), M=16384+512 K=3072 N=12288 r=32"),
}


CFG3 = dict(M=4608, K=12288, N=3072, r=64,
            name="cfg3: LoRA training step through the frozen W8A8 base (MLP down), M=4608 K=12288 N=3072 r=64")
# cfg4: one double-stream block's quantized linears at 1024^2, CFG batch 2, r=16 on every linear
CFG4_LINEARS = (("qkv", 3072, 9216), ("out", 3072, 3072), ("up", 3072, 12288), ("down", 12288, 3072))
CFG4_STREAMS = (("image", 8192), ("text", 1024))
CFG4_ADALN = (3072, 18432, 2)


def synth(M, K, N, r, bias, seed=0):
    """BASELINE.json inputs, generated on the CPU in the fixed order x -> outlier idx -> W -> bias -> A -> B."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g)
    idx = torch.randperm(K, generator=g)[: K // 100]
    x[:, idx] *= 20
    x = x.to(torch.bfloat16)
    W = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(N, generator=g) * 0.02 if bias else None
    A = torch.randn(r, K, generator=g) * 0.01
    B = torch.randn(N, r, generator=g) * 0.01
    return x, W, b, A, B


def settle(fn, seconds):
    """Runs ``fn`` untimed for ``seconds`` of wall time.  The MI355X's clock governor takes about a second
    of sustained load to leave its ramp-up state (measured: ~1.5 GHz for the first ~1-1.5 s of a GEMM loop,
    then ~1.9 GHz at the 1.4 kW board limit), so a timed region that starts on a cold GPU measures the ramp,
    not the kernels."""
    if seconds <= 0:
        return
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(4):
            fn()
        torch.cuda.synchronize()


_HEAD = {}
HOST_US = {}   # host issue time per call of the last fn timed by time_loop, keyed by fn's qualified name


def queue_head(dev, ms):
    """Enqueues about ``ms`` of untimed device copies (256 MB each, ~0.1 ms) and returns without waiting, so
    the host can enqueue a whole timed region before the GPU reaches it: the events around that region then
    measure the GPU's time per step, with no gaps where the GPU waited for the host to launch the next kernel
    (as in a training loop, where the host runs ahead during the large GEMMs, or a replayed HIP graph)."""
    if dev not in _HEAD:
        src = torch.empty(1 << 28, dtype=torch.uint8, device=dev)
        _HEAD[dev] = (src, torch.empty_like(src))
    src, dst = _HEAD[dev]
    for _ in range(max(1, min(int(ms / 0.1) + 1, 500))):
        dst.copy_(src)


def time_loop(fn, iters, warm=3, dev=None):
    """GPU ms per call of ``fn`` over ``iters`` calls between two events.  The warm calls also measure the host's
    issue time per call (``HOST_US``); a queue head of 1.5x the timed region's host time lets the host run ahead
    (``queue_head``).  ``dev`` None: no head (the host's launch cost is then part of the time when it exceeds
    the GPU's)."""
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(warm):
        fn()
    host_ms = (time.perf_counter() - t0) * 1e3 / warm
    HOST_US[getattr(fn, "__qualname__", "fn")] = host_ms * 1e3
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    if dev is not None:
        queue_head(dev, 1.5 * host_ms * iters + 0.3)
    s.record()
    for _ in range(iters):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / iters   # ms


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(cfg, x, W, b, A, B, budget_s=12.0, rows=2048):
    """The CPU oracle's forward (numpy FWHT + quant, exact int32 GEMM via torch._int_mm, f64 epilogue) on a
    bounded sample: the first ``rows`` rows, repeated until ``budget_s`` of work; returns TOPS."""
    import numpy as np
    from oracle import convrot as orc

    torch.set_num_threads(os.cpu_count() or 1)
    K, N = cfg["K"], cfg["N"]
    if cfg["w4"]:
        qw, sw = orc.quant_weight_i4(W.float().numpy())
    else:
        qw, sw = orc.quant_weight_i8(W.float().numpy())
    xs = x[:rows].float().numpy()
    bn = None if b is None else b.numpy()
    An, Bn = A.numpy(), B.numpy()
    times = []
    t_end = time.perf_counter() + budget_s
    while not times or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        orc.forward(xs, qw, sw, w4=cfg["w4"], bias=bn, lora_A=An, lora_B=Bn, lora_scale=1.0, fast=True)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    return {"value": 2.0 * rows * N * K / t / 1e12, "unit": "TOPS", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{rows} of {cfg['M']} rows of {cfg['name'].split(':')[0]}, median of {len(times)} runs "
                      f"({t * 1e3:.0f} ms each) on {cpu_model()}"}


def cpu_reference_path(cfg, x, W, b, A, B, budget_s=6.0, rows=2048):
    """The reference's own quantized linear + adapter on the CPU, restated (oracle.convrot.fp8_linear is
    Fp8Linear.forward, quantize.py:48-51: bf16 dequant then F.linear; the adapter is lora.py:47-48 in fp32):
    the same bounded sample as the ConvRot CPU baseline, for comparison.  Returns TOPS (2*rows*N*K/time)."""
    import numpy as np
    from oracle import convrot as orc

    torch.set_num_threads(os.cpu_count() or 1)
    K, N = cfg["K"], cfg["N"]
    wq, sc = orc.fp8_weight_quant(W.float().numpy())
    xs = x[:rows].contiguous()
    bb = None if b is None else b.to(torch.bfloat16)

    def run():
        out = orc.fp8_linear(xs, wq, sc, bb)
        delta = (xs.float() @ A.t()) @ B.t()
        return out + delta.to(out.dtype)

    times = []
    t_end = time.perf_counter() + budget_s
    while not times or (time.perf_counter() < t_end and len(times) < 30):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    return {"value": round(2.0 * rows * N * K / t / 1e12, 4), "unit": "TOPS", "cores": torch.get_num_threads(),
            "kind": "port", "path": "Fp8Linear + LoRALinear forward (bf16 F.linear, fp32 adapter)",
            "sample": f"{rows} of {cfg['M']} rows, median of {len(times)} runs ({t * 1e3:.0f} ms each)"}


PROBE_LIB = ROOT / "krea-2_amd" / "libk2q_probe.so"
_probe = {}


def mfma_probe_i8(iters: int, workgroups: int, dev) -> int:
    """Launches the register-only int8 MFMA loop of ``libk2q_probe.so`` (krea-2_amd/csrc/probe.hip, a measurement
    aid built beside the product library) on the current stream; returns the int8 operations it performs."""
    import ctypes
    if "lib" not in _probe:
        lib = ctypes.CDLL(str(PROBE_LIB))
        lib.k2q_mfma_probe_i8_ops.argtypes, lib.k2q_mfma_probe_i8_ops.restype = [ctypes.c_int64] * 2, ctypes.c_int64
        lib.k2q_mfma_probe_i8.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
        lib.k2q_mfma_probe_i8.restype = ctypes.c_int
        _probe["lib"] = lib
    lib = _probe["lib"]
    out = _probe.get(dev)
    if out is None or out.numel() < workgroups * 512:
        out = _probe[dev] = torch.empty(workgroups * 512, dtype=torch.int32, device=dev)
    rc = lib.k2q_mfma_probe_i8(iters, workgroups, out.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
    if rc != 0:
        raise RuntimeError(f"k2q_mfma_probe_i8 failed with status {rc}")
    return lib.k2q_mfma_probe_i8_ops(iters, workgroups)


def mfma_probe(k2, dev, seconds=1.0):
    """Sustained int8 MFMA rate of this board in this run (register-only v_mfma_i32_32x32x32_i8 loop, two
    waves per SIMD on every CU, pseudo-random operands): the same-run ceiling the GEMM is compared with."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    iters = 2000
    settle(lambda: mfma_probe_i8(iters, cus, dev), 0.5)
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ops, n, t_end = 0, 0, time.perf_counter() + seconds
    s_ev.record()
    while time.perf_counter() < t_end:
        for _ in range(4):
            ops += mfma_probe_i8(iters, cus, dev)
        n += 4
        torch.cuda.synchronize()
    e_ev.record()
    torch.cuda.synchronize()
    ms = s_ev.elapsed_time(e_ev)
    return ops / (ms * 1e-3) / 1e12


def run_config(k2, cfg, steps, warmup, dev, settle_s=0.0):
    L = k2._lib
    M, K, N, r = cfg["M"], cfg["K"], cfg["N"], cfg["r"]
    x, W, b, A, B = synth(M, K, N, r, cfg["bias"])
    xd, Ad, Bd = x.to(dev), A.to(dev), B.to(dev)
    bd = None if b is None else b.to(dev)
    w4 = cfg["w4"]
    if w4:
        qw, sw = L.quant_weight_i4(W.to(dev))
        gemm = L.gemm_w4a8
    else:
        qw, sw = L.quant_weight_i8(W.to(dev))
        gemm = L.gemm_w8a8
    qx = torch.empty((M, K), dtype=torch.int8, device=dev)
    sx = torch.empty((M,), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    def step():
        """The module's inference path: one library call (k2q_linear_fwd) issues rotate/quant, the LoRA
        down-projection and the GEMM with its fused epilogue (which adds the down-projection's K-slices)."""
        return L.linear_fwd(xd, qx, sx, False, Ad, Bd, 1.0, qw, sw, bd, w4, need_u=False)[0]

    settle(step, settle_s)
    for _ in range(warmup):
        step()
    # Timed region: K steps between two events on the stream the kernels run on (the GPU's time per step).
    ms_step = time_loop(step, steps, dev=dev)
    host_us = HOST_US[step.__qualname__]

    # Per-kernel breakdown over K more steps: the same three launches issued one by one, events between them
    # on that stream, so the GEMM's average launch duration comes from timed steps.
    fused_down = L.linear_fwd_fuses_down(M, K, r)

    def step_events(ev):
        ev[0].record()
        if fused_down:     # the one-call forward's route: u from the rotate/quant pass
            q_, s_, u = L.rotquant_lora(xd, Ad)
            ev[1].record()
        else:
            q_, s_, _ = L.rotquant(xd)
            ev[1].record()
            u = L.lora_down(xd, Ad)
        ev[2].record()
        gemm(q_, s_, qw, sw, bd, u, Bd, 1.0)
        ev[3].record()

    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    for _ in range(3):
        step_events(evs[0])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    queue_head(dev, 0.3 + 1.5 * 0.06 * steps)   # ~60 us of host time per instrumented step
    for i in range(steps):
        step_events(evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_rot = sum(ev[0].elapsed_time(ev[1]) for ev in evs) / steps
    ms_lora = sum(ev[1].elapsed_time(ev[2]) for ev in evs) / steps
    ms_gemm = sum(ev[2].elapsed_time(ev[3]) for ev in evs) / steps
    # Rotate/quant as a stream: back to back over 4 distinct inputs (4 x 2MK bytes, beyond the 256 MB
    # last-level cache for cfg2), so every call reads its input from HBM.  (Inside the step, the interval
    # before rotate/quant also absorbs the write-back of the previous GEMM's output.)
    xs = [xd] + [xd.roll(i, 0).contiguous() for i in range(1, 4)]

    def rot4():
        for xi in xs:
            L.rotquant(xi)

    # Median of 7 timed batches of 40 passes (~35 ms of streaming at cfg2): one short batch right after the
    # GEMM loop has read anywhere from 5.0 to 5.9 TB/s on the same build.
    batches = sorted(time_loop(rot4, 40, dev=dev) for _ in range(7))
    ms_rot_stream = batches[len(batches) // 2] / len(xs)
    del xs
    ops = 2.0 * M * N * K
    rot_bytes = 2 * M * K + M * K + 4 * M
    return dict(ms_step=ms_step, wall=wall, host_us=host_us, ms_rot=ms_rot, ms_rot_stream=ms_rot_stream,
                ms_lora=ms_lora, ms_gemm=ms_gemm, ops=ops, fused_down=fused_down,
                rot_bytes=rot_bytes, tops=ops / (ms_step * 1e-3) / 1e12, x=x, W=W, b=b, A=A, B=B)


def make_layer(k2, K, N, r, dev, seed=0, bias=False):
    """A LoRALinear over a ConvRotLinear W8A8 base with BASELINE.json weight/LoRA distributions."""
    g = torch.Generator().manual_seed(seed)
    lin = torch.nn.Linear(K, N, bias=bias, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_((torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16))
    base = k2.ConvRotLinear(lin.to(dev), "w8a8")
    layer = k2.LoRALinear(base, r, float(r))
    with torch.no_grad():
        layer.lora_A.copy_(torch.randn(r, K, generator=g) * 0.01)
        layer.lora_B.copy_(torch.randn(N, r, generator=g) * 0.01)
    return layer


def _no_input_reuse(k2):
    """Switches off the reuse of the last input's int8 codes (``quantize.shared_input_quant``) while a leg
    times the same input tensor over and over: in training every step brings a new activation, so each
    timed call must rotate and quantize its input.  Returns the previous setting."""
    prev = k2.quantize.shared_input_quant.enabled
    k2.quantize.shared_input_quant.enabled = False
    return prev


def run_cfg3(k2, steps, dev, settle_s=0.0, cpu=False):
    """Forward + backward (dX through the frozen base with the inverse rotation, dA, dB) of one layer; with
    ``cpu``, the CPU paths of the same step (:func:`cpu_cfg3`)."""
    c = CFG3
    layer = make_layer(k2, c["K"], c["N"], c["r"], dev, seed=3)
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(c["M"], c["K"], generator=g)).to(torch.bfloat16).to(dev).requires_grad_(True)
    dy = (torch.randn(c["M"], c["N"], generator=g) * 1e-3).to(torch.bfloat16).to(dev)

    def step():
        x.grad = None
        layer.lora_A.grad = None
        layer.lora_B.grad = None
        layer(x).backward(dy)

    prev = _no_input_reuse(k2)
    try:
        settle(step, settle_s)
        ms = time_loop(step, steps, dev=dev)    # every backward builds its effective weight (the default)
        with torch.no_grad():
            ms_fwd = time_loop(lambda: layer(x), steps, dev=dev)
        k2.set_dx_weight_cache(layer, True)     # the effective weight kept resident (2 more bytes per weight)
        ms_kept = time_loop(step, steps, dev=dev)
        k2.set_dx_weight_cache(layer, False)
    finally:
        k2.quantize.shared_input_quant.enabled = prev

    # The reference's step on the same GPU: Fp8Linear.forward (quantize.py:48-51) + LoRALinear.forward
    # (lora.py:47-48) restated with torch ops, its autograd through the dequantized bf16 weight.
    F_ = torch.nn.functional
    w = (torch.randn(c["N"], c["K"], generator=torch.Generator().manual_seed(3)) * 0.02).to(dev)
    scale = w.abs().amax(dim=1, keepdim=True).clamp(min=1e-8) / 448.0
    wq, sc = (w / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn), scale.to(torch.bfloat16)
    A = layer.lora_A.detach().clone().requires_grad_(True)
    B = layer.lora_B.detach().clone().requires_grad_(True)
    del w

    def ref_step():
        x.grad = A.grad = B.grad = None
        out = F_.linear(x, wq.to(torch.bfloat16) * sc)
        out = out + ((x.to(A.dtype) @ A.t()) @ B.t()).to(out.dtype)
        out.backward(dy)

    ms_ref = time_loop(ref_step, steps, dev=dev)
    # The backward's kernels alone: the input-gradient GEMM (bf16 MFMA, with its LoRA term) on the layer's
    # effective weight, and the per-call pass that builds that weight (HBM: N K int8 in, 2 N K bf16 out).
    L = k2._lib
    base = layer.base
    wt = L.dx_weight(base.qweight, base.weight_scale)
    gg = (torch.randn(c["M"], c["r"], generator=g) * 1e-3).to(dev)
    A_ = layer.lora_A.detach()
    ms_dx = sorted(time_loop(lambda: L.gemm_dx(dy, base.qweight, base.weight_scale, g=gg, lora_a=A_, wt=wt), steps, dev=dev)
                   for _ in range(3))[1]
    ms_prep = sorted(time_loop(lambda: L.dx_weight(base.qweight, base.weight_scale), steps, dev=dev) for _ in range(3))[1]
    del wt
    ops_fwd = 2.0 * c["M"] * c["N"] * c["K"]
    dx_tflops = ops_fwd / (ms_dx * 1e-3) / 1e12
    prep_gbs = 3.0 * c["N"] * c["K"] / (ms_prep * 1e-3) / 1e9
    fwd_tops = ops_fwd / (ms_fwd * 1e-3) / 1e12
    return {"workload": c["name"], "ms": round(ms, 4), "step_ms": round(ms, 4), "fwd_ms": round(ms_fwd, 4),
            "bwd_ms": round(ms - ms_fwd, 4), "fwd_tops": round(fwd_tops, 1),
            "tops": round(2 * ops_fwd / (ms * 1e-3) / 1e12, 1),
            "dx_gemm_ms": round(ms_dx, 4), "dx_gemm_tflops": round(dx_tflops, 1),
            "dx_weight_pass_ms": round(ms_prep, 4),
            "roofline": roofline_entry("gemm_nt_kernel<EPI_DXLIN> (input gradient)", "mfma", dx_tflops,
                                       BF16_PEAK_TFLOPS, "TFLOP/s"),
            "fwd_roofline": roofline_entry("forward (rotate/quant + LoRA down + W8A8 GEMM)", "mfma", fwd_tops,
                                           INT8_PEAK_TOPS, "TOPS"),
            "dx_weight_roofline": roofline_entry("rot_dequant_t_kernel (effective weight)", "hbm", prep_gbs,
                                                 HBM_PEAK_GBS, "GB/s"),
            "step_ms_dx_weight_kept": round(ms_kept, 4),
            "reference_fp8_step_ms_gpu": round(ms_ref, 4),
            **({"cpu": cpu_cfg3(*_layer_tensors(layer, 3, c["K"], c["N"]))} if cpu else {})}


def run_producers(k2, steps, dev):
    """The two producer-fused rotate/quant kernels at cfg4's image-stream shapes (M = 2 x 4096 tokens): the
    modulated RMSNorm of the block input (K = 3072, per-batch modulation) and the SwiGLU product that feeds
    the down projection (K = 12288).  Each is timed fused (one kernel: h and its codes) and as the reference
    computes it (torch's eager ops, mmdit.py:156-161,177-178,314-317) followed by rotate/quant of h.  Inputs
    rotate over 4 tensors so that every call reads them from HBM; bytes are the fused kernel's algorithmic
    traffic: RMSNorm 2MK in + 2MK h + MK codes + 4M scales, SwiGLU 4MK in + 2MK h + MK codes + 4M."""
    L = k2._lib
    F_ = torch.nn.functional
    B, Lt, K, KH = 2, 4096, 3072, 12288
    M = B * Lt
    g = torch.Generator().manual_seed(11)
    xs = [torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev) for _ in range(4)]
    ns = (torch.randn(K, generator=g) * 0.1).to(dev)
    vec = (torch.randn(B, 1, 6 * K, generator=g) * 0.3).to(torch.bfloat16).to(dev)
    ps, sh = vec[..., :K], vec[..., K:2 * K]
    gus = [(torch.randn(M, KH, generator=g) * 3).to(torch.bfloat16).to(dev) for _ in range(2)] + \
          [torch.randn(M, KH, generator=g).to(torch.bfloat16).to(dev) for _ in range(2)]
    pairs = [(gus[0], gus[2]), (gus[1], gus[3]), (gus[2], gus[0]), (gus[3], gus[1])]

    def rms_fused():
        for x in xs:
            L.rmsmod_rotquant(x, ns, 1e-5, ps.reshape(B, K), sh.reshape(B, K), Lt)

    def rms_ref():
        for x in xs:
            n = F_.rms_norm(x.view(B, Lt, K).float(), (K,), eps=1e-5, weight=ns + 1.0).to(torch.bfloat16)
            L.rotquant(((1 + ps) * n + sh).view(M, K))

    def swi_fused():
        for gt, ut in pairs:
            L.swiglu_rotquant(gt, ut)

    def swi_ref():
        for gt, ut in pairs:
            L.rotquant(F_.silu(gt) * ut)

    out = {}
    for name, fused, ref, nbytes in (("rmsnorm_mod", rms_fused, rms_ref, 5 * M * K + 4 * M),
                                     ("swiglu", swi_fused, swi_ref, 7 * M * KH + 4 * M)):
        tf = sorted(time_loop(fused, steps, dev=dev) for _ in range(5))[2] / 4
        tr = sorted(time_loop(ref, steps, dev=dev) for _ in range(5))[2] / 4
        gbs = nbytes / (tf * 1e-3) / 1e9
        out[name] = {"M": M, "K": K if name == "rmsnorm_mod" else KH, "fused_ms": round(tf, 4),
                     "unfused_ms": round(tr, 4), "fused_GBps": round(gbs, 1),
                     "fused_pct_hbm": round(100 * gbs / HBM_PEAK_GBS, 2)}
    return out


def run_grouped(k2, steps, dev):
    """The attention inputs of a Krea 2 block (wq 6144->6144, wk / wv 6144->1536, gate 6144->6144, all reading
    one tensor, mmdit.py:199), each a LoRALinear (r=16) over a W8A8 ConvRot base, at M = 4608 (1024^2) and
    16896 (2048^2): the four layers called one after another (the shared input quantized once) against the
    same four after group_siblings (one grouped GEMM and one stacked LoRA down-projection)."""
    import types

    from krea2_amd import fused

    out = {}
    Ns = (6144, 1536, 1536, 6144)
    K = 6144
    for M in (4608, 16896):
        attn = types.SimpleNamespace(**{n: make_layer(k2, K, N, 16, dev, seed=N + i)
                                        for i, (n, N) in enumerate(zip(("wq", "wk", "wv", "gate"), Ns))})
        mods = [attn.wq, attn.wk, attn.wv, attn.gate]
        x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16).to(dev)

        def calls():
            for m in mods:
                m(x)

        with torch.no_grad():
            t_sep = sorted(time_loop(calls, steps, dev=dev) for _ in range(5))[2]
            assert fused.group_siblings(types.SimpleNamespace(blocks=[types.SimpleNamespace(attn=attn)])) == 1
            t_grp = sorted(time_loop(calls, steps, dev=dev) for _ in range(5))[2]
        ops = 2.0 * M * K * sum(Ns)
        out[f"M{M}"] = {"separate_ms": round(t_sep, 4), "grouped_ms": round(t_grp, 4),
                        "separate_tops": round(ops / (t_sep * 1e-3) / 1e12, 1),
                        "grouped_tops": round(ops / (t_grp * 1e-3) / 1e12, 1)}
    return out


def run_krea_block(k2, steps, dev):
    """The quantized-linear work of one Krea 2 single-stream block at 1024^2 (M = 4608, width 6144, 48 heads
    of 128 with 12 KV heads, SwiGLU 16384; mmdit.py:164-212,294-319), LoRA r=16 on all eight linears: the
    modulated RMSNorm, wq/wk/wv/gate, wo, the second modulated RMSNorm, mlp.gate/up, the SwiGLU product and
    mlp.down, with the residual adds and gates.  Attention itself is left out: each KV head's `k * v` added to
    its four query heads, times `sigmoid(gate)`, stands in for `attention(q, k, v) * sigmoid(gate)` (same
    shapes into wo, and gradients reach wq, wk, wv and gate as attention's do), so the time is the linears,
    their producers and the elementwise glue.  Timed forward (no_grad) and forward + backward, as the reference
    computes the producers (torch eager ops, every linear quantizing its own input or hitting the
    shared-input cache) against fuse_producers' kernels plus group_siblings' groups (attention inputs and
    SwiGLU gate / up: one grouped forward launch and one input-gradient GEMM each)."""
    block, fwd_bwd, group, x0, shape = _krea_block(k2, dev)
    out = {}
    for fuse in (False, True):
        if fuse:
            group()
        with torch.no_grad():
            t_f = sorted(time_loop(lambda: block(x0, fuse), steps, dev=dev) for _ in range(3))[1]
        t_fb = sorted(time_loop(lambda: fwd_bwd(fuse), max(3, steps // 2), dev=dev) for _ in range(3))[1]
        out["fused" if fuse else "reference_ops"] = {"fwd_ms": round(t_f, 4), "fwd_bwd_ms": round(t_fb, 4)}
    out["shape"] = shape
    return out


def krea_block_pass(k2, dev, iters):
    """Fixed launches for a kernel trace of the Krea 2 block leg: ``iters`` fused forward + backward passes
    (producers fused, both sibling groups), after 3 untimed ones that build the resident effective weights."""
    block, fwd_bwd, group, _, shape = _krea_block(k2, dev)
    group()
    for _ in range(3):
        fwd_bwd(True)
    torch.cuda.synchronize()
    progress("krea block pass: warm")
    for _ in range(iters):
        fwd_bwd(True)
    torch.cuda.synchronize()
    print(json.dumps({"krea_block_pass": shape, "fused_fwd_bwd_iterations": iters}), flush=True)


def cfg3_pass(k2, dev, iters):
    """Fixed launches for a kernel trace of the cfg3 leg: ``iters`` training steps (forward, then dX, dA, dB
    through autograd) of the cfg3 layer, after 5 untimed ones, every call rotating and quantizing its input."""
    c = CFG3
    layer = make_layer(k2, c["K"], c["N"], c["r"], dev, seed=3)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(c["M"], c["K"], generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    dy = (torch.randn(c["M"], c["N"], generator=g) * 1e-3).to(torch.bfloat16).to(dev)

    def step():
        x.grad = None
        layer.lora_A.grad = None
        layer.lora_B.grad = None
        layer(x).backward(dy)

    prev = _no_input_reuse(k2)
    try:
        for _ in range(5):
            step()
        torch.cuda.synchronize()
        progress("cfg3 pass: warm")
        for _ in range(iters):
            step()
        torch.cuda.synchronize()
    finally:
        k2.quantize.shared_input_quant.enabled = prev
    print(json.dumps({"cfg3_pass": c["name"], "training_steps": iters}), flush=True)


def _krea_block(k2, dev):
    """The Krea 2 block leg's layers, inputs and callables: ``block(x, fuse)``, ``fwd_bwd(fuse)``, ``group()``
    (group_siblings on both groups), the input and a shape string."""
    import types

    from krea2_amd import fused

    F_ = torch.nn.functional
    M, D, KV, HID, r = 4608, 6144, 1536, 16384, 16
    g = torch.Generator().manual_seed(21)

    def norm():
        return types.SimpleNamespace(scale=(torch.randn(D, generator=g) * 0.1).to(torch.bfloat16).to(dev), eps=1e-5)

    attn = types.SimpleNamespace(wq=make_layer(k2, D, D, r, dev, 1), wk=make_layer(k2, D, KV, r, dev, 2),
                                 wv=make_layer(k2, D, KV, r, dev, 3), gate=make_layer(k2, D, D, r, dev, 4),
                                 wo=make_layer(k2, D, D, r, dev, 5))
    mlp = types.SimpleNamespace(gate=make_layer(k2, D, HID, r, dev, 6), up=make_layer(k2, D, HID, r, dev, 7),
                                down=make_layer(k2, HID, D, r, dev, 8))
    pre, post = norm(), norm()
    lin = (torch.randn(6 * D, generator=g) * 0.1).to(torch.bfloat16).to(dev)
    vec = (torch.randn(1, 1, 6 * D, generator=g) * 0.3).to(torch.bfloat16).to(dev)
    x0 = torch.randn(1, M, D, generator=g).to(torch.bfloat16).to(dev)
    dy = (torch.randn(1, M, D, generator=g) * 1e-2).to(torch.bfloat16).to(dev)

    def rms(nm, x):
        return F_.rms_norm(x.float(), (D,), eps=nm.eps, weight=nm.scale.float() + 1.0).to(x.dtype)

    def block(x, fuse):
        ps, sh, pg, qs, qsh, qg = (vec + lin).chunk(6, dim=-1)
        h = fused.modulated_rmsnorm(pre, x, ps, sh) if fuse else (1 + ps) * rms(pre, x) + sh
        q, k, v, gt = attn.wq(h), attn.wk(h), attn.wv(h), attn.gate(h)
        # attention stand-in: every KV head's k * v added to its 4 query heads (GQA 48 / 12 of 128)
        o = (q.unflatten(-1, (KV // 128, -1, 128)) + (k * v).unflatten(-1, (KV // 128, 1, 128))).flatten(-3)
        x = x + pg * attn.wo(o * torch.sigmoid(gt))
        h = fused.modulated_rmsnorm(post, x, qs, qsh) if fuse else (1 + qs) * rms(post, x) + qsh
        a, b = mlp.gate(h), mlp.up(h)
        return x + qg * mlp.down(fused.swiglu(a, b) if fuse else F_.silu(a) * b)

    def fwd_bwd(fuse):
        x = x0.clone().requires_grad_(True)
        block(x, fuse).backward(dy)

    def group():
        fused.group_siblings(types.SimpleNamespace(blocks=[types.SimpleNamespace(attn=attn, mlp=mlp)]))

    return block, fwd_bwd, group, x0, f"M={M} width={D} kv={KV} hidden={HID} r={r}; attention excluded"


def run_vram(k2, dev):
    """Device memory of one Krea 2 single-stream block's eight linears (width 6144, 48 heads of 128 with 12 KV
    heads, SwiGLU 16384; mmdit.py:170-175,188-194) under a LoRA step at 1024^2 (M = 4608, r = 16 on every
    linear), for each frozen base: bf16 ``nn.Linear`` (the reference without quantization), fp8 (the
    reference's ``Fp8Linear`` storage, quantize.py:33-42, this package's kernels), ConvRot w8a8, and ConvRot
    w8a8 with the effective input-gradient weight kept.  ``base_GB``: the layers' resident bytes (base
    parameters + adapters + any kept weight); ``peak_GB``: the most allocated during two gradient-checkpointed
    forward + backward passes (torch.utils.checkpoint, non-reentrant, as mmdit.py:479-481), measured from the
    empty state before the layers were built; ``paged_GB``: the bytes block swap moves per page-out (every
    frozen parameter, mmdit.py:409-414).  The reference's published figures for the whole trainer at 768^2
    (docs/TRAINING.md:101-107) are 28.8 GB bf16 and 17.5 GB fp8."""
    import gc

    F_ = torch.nn.functional
    M, D, KV, HID, r = 4608, 6144, 1536, 16384, 16
    shapes = {"wq": (D, D), "wk": (D, KV), "wv": (D, KV), "gate": (D, D), "wo": (D, D), "mlp_gate": (D, HID),
              "mlp_up": (D, HID), "mlp_down": (HID, D)}
    gen = torch.Generator(device=dev).manual_seed(31)

    def build(kind):
        layers = {}
        for name, (K, N) in shapes.items():
            lin = torch.nn.Linear(K, N, bias=False, dtype=torch.bfloat16, device=dev)
            with torch.no_grad():
                lin.weight.normal_(0.0, 0.02, generator=gen)
            base = lin if kind == "bf16" else k2.Fp8Linear(lin) if kind == "fp8" else k2.ConvRotLinear(lin, "w8a8")
            del lin
            layer = k2.LoRALinear(base, r, float(r))
            with torch.no_grad():
                layer.lora_B.normal_(0.0, 0.01, generator=gen)
            if kind == "convrot_w8a8_kept":
                k2.set_dx_weight_cache(layer, True)
            layers[name] = layer
        return layers

    def block(L, x):
        # the quantized linears of SingleStreamBlock.forward (mmdit.py:310-319) with RMSNorm / modulation /
        # attention reduced to the ops that keep the linears' shapes (attention: k * v added to the query heads)
        h = F_.rms_norm(x.float(), (D,), eps=1e-5).to(x.dtype)
        q, k, v, g = L["wq"](h), L["wk"](h), L["wv"](h), L["gate"](h)
        o = (q.unflatten(-1, (KV // 128, -1, 128)) + (k * v).unflatten(-1, (KV // 128, 1, 128))).flatten(-3)
        x = x + L["wo"](o * torch.sigmoid(g))
        h = F_.rms_norm(x.float(), (D,), eps=1e-5).to(x.dtype)
        return x + L["mlp_down"](F_.silu(L["mlp_gate"](h)) * L["mlp_up"](h))

    def gb(b):
        return round(b / 1e9, 3)

    out = {"shape": f"one block, M={M} width={D} kv={KV} hidden={HID} r={r}; checkpointed fwd+bwd"}
    xg = torch.Generator().manual_seed(32)
    x0 = torch.randn(1, M, D, generator=xg).to(torch.bfloat16)
    dy0 = (torch.randn(1, M, D, generator=xg) * 1e-2).to(torch.bfloat16)
    for kind in ("bf16", "fp8", "convrot_w8a8", "convrot_w8a8_kept"):
        k2.quantize.shared_input_quant.clear()     # codes kept from an earlier leg would leave the baseline
        gc.collect()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        m0 = torch.cuda.memory_allocated(dev)
        L = build(kind)
        x, dy = x0.to(dev), dy0.to(dev)
        torch.cuda.synchronize()
        resident = torch.cuda.memory_allocated(dev) - m0 - x.nbytes - dy.nbytes
        paged = sum(p.nbytes for m in L.values() for p in m.parameters() if not p.requires_grad)
        torch.cuda.reset_peak_memory_stats(dev)
        for _ in range(2):
            xi = x.clone().requires_grad_(True)
            torch.utils.checkpoint.checkpoint(block, L, xi, use_reentrant=False).backward(dy)
            del xi
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated(dev) - m0
        kept = torch.cuda.memory_allocated(dev) - m0 - x.nbytes - dy.nbytes \
            - sum(p.grad.nbytes for m in L.values() for p in m.parameters() if p.grad is not None)
        out[kind] = {"base_GB": gb(resident), "base_GB_after_step": gb(kept), "peak_GB": gb(peak),
                     "paged_GB": gb(paged), "base_GB_28_blocks": gb(28 * kept)}
        del L, x, dy
    gc.collect()
    torch.cuda.empty_cache()
    return out


def run_reference_gpu(k2, res, steps, dev):
    """The reference's own quantized linear + adapter (``Fp8Linear.forward``, quantize.py:48-51: a bf16
    dequantization of the fp8 weight on every call, then ``F.linear``; ``LoRALinear.forward``, lora.py:47-48:
    two fp32 products and a bf16 add) restated with torch ops and run on this GPU at cfg2 (torch's own
    kernels, hipBLASLt for the products), beside this package's fp8 base (``Fp8Linear`` on the gfx950 kernels:
    dequantization kernel and bf16 MFMA GEMM with the fused adapter).  Same inputs as the headline step."""
    F_ = torch.nn.functional
    x, W, A, B = res["x"].to(dev), res["W"].to(dev), res["A"].to(dev), res["B"].to(dev)
    M, K, N = x.shape[0], x.shape[1], W.shape[0]
    w = W.float()
    scale = w.abs().amax(dim=1, keepdim=True).clamp(min=1e-8) / 448.0          # quantize.py:36
    wq = (w / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)             # quantize.py:37
    sc = scale.to(torch.bfloat16)
    del w

    def ref():
        wd = wq.to(torch.bfloat16) * sc.to(torch.bfloat16)                     # quantize.py:49
        out = F_.linear(x, wd, None)                                           # quantize.py:51
        delta = (x.to(A.dtype) @ A.t()) @ B.t()                                 # lora.py:47
        return out + 1.0 * delta.to(out.dtype)                                 # lora.py:48

    lin = torch.nn.Linear(K, N, bias=False, dtype=torch.bfloat16, device=dev)
    with torch.no_grad():
        lin.weight.copy_(W)
    fp8 = k2.LoRALinear(k2.Fp8Linear(lin), A.shape[0], float(A.shape[0]))
    del lin
    with torch.no_grad():
        fp8.lora_A.copy_(A)
        fp8.lora_B.copy_(B)
        t_ref = sorted(time_loop(ref, steps, dev=dev) for _ in range(3))[1]
        t_fp8 = sorted(time_loop(lambda: fp8(x), steps, dev=dev) for _ in range(3))[1]
    ops = 2.0 * M * N * K
    return {"reference_fp8_path": {"ms": round(t_ref, 4), "tops": round(ops / (t_ref * 1e-3) / 1e12, 1),
                                   "path": "Fp8Linear.forward + LoRALinear.forward restated with torch ops on the GPU"},
            "k2q_fp8_path": {"ms": round(t_fp8, 4), "tops": round(ops / (t_fp8 * 1e-3) / 1e12, 1),
                             "path": "krea2_amd Fp8Linear + LoRALinear (same numerics, gfx950 kernels)"},
            "convrot_speedup_vs_reference": round(t_ref / res["ms_step"], 2)}


def run_cfg4(k2, steps, dev, settle_s=0.0, cpu=False):
    """Summed forward time of one double-stream block's quantized linears (image + text stream, plus the
    per-stream adaLN modulation at M=2), each a LoRALinear (r=16) over a W8A8 ConvRot base; with ``cpu``, the
    CPU paths of the same ten linears (:func:`cpu_cfg4`)."""
    total_ops = 0.0
    layers, seeds = [], []
    for sname, M in CFG4_STREAMS:
        for lname, K, N in CFG4_LINEARS:
            layers.append((f"{sname}.{lname}", make_layer(k2, K, N, 16, dev, seed=K + N + M), M, K, N))
            seeds.append(K + N + M)
        K, N, Ma = CFG4_ADALN
        layers.append((f"{sname}.adaln", make_layer(k2, K, N, 16, dev, seed=7 + M), Ma, K, N))
        seeds.append(7 + M)
    # One input tensor per linear: in the block each linear reads a different activation, so nothing here
    # may reuse another linear's quantized input.
    xs = {}
    for i, (name, layer, M, K, N) in enumerate(layers):
        xs[name] = torch.randn(M, K, generator=torch.Generator().manual_seed(M + K + i)).to(torch.bfloat16).to(dev)
        total_ops += 2.0 * M * N * K

    def block():
        for name, layer, M, K, N in layers:
            layer(xs[name])

    prev = _no_input_reuse(k2)
    try:
        with torch.no_grad():
            settle(block, settle_s)
            ms = time_loop(block, steps, dev=dev)
            per, host = {}, {}
            for name, layer, M, K, N in layers:
                def call():
                    layer(xs[name])
                per[name] = round(time_loop(call, max(3, steps // 2), dev=dev), 4)
                host[name] = round(HOST_US[call.__qualname__], 1)   # the module call's host issue time
    finally:
        k2.quantize.shared_input_quant.enabled = prev
    tops = total_ops / (ms * 1e-3) / 1e12
    K, N, Ma = CFG4_ADALN
    adaln_ms = min(per[f"{sname}.adaln"] for sname, _ in CFG4_STREAMS)
    adaln_gbs = (N * K + 4 * N + 2 * Ma * K + 2 * Ma * N) / (adaln_ms * 1e-3) / 1e9
    return {"workload": "cfg4: one double-stream block's quantized linears at 1024^2, CFG batch 2 (image M=8192, "
                        "text M=1024; qkv, out, up, down + adaLN at M=2), W8A8, LoRA r=16 on each",
            "ms": round(ms, 4), "block_linears_ms": round(ms, 4), "tops": round(tops, 1),
            "roofline": roofline_entry("the ten linears' launches (W8A8 GEMMs, GEMV, rotate/quant, LoRA)", "mfma",
                                       tops, INT8_PEAK_TOPS, "TOPS"),
            "adaln_roofline": roofline_entry("adaLN linear at M=2 (rotate/quant, LoRA down, GEMV: weight read once)",
                                             "hbm", adaln_gbs,
                                             HBM_PEAK_GBS, "GB/s"),
            "per_linear_ms": per,
            "per_linear_host_us": host,
            **({"cpu": cpu_cfg4([(M, K, N, *_layer_tensors(layer, sd, K, N))
                                 for (_, layer, M, K, N), sd in zip(layers, seeds)])} if cpu else {})}


def profile_pass(k2, dev):
    """Fixed launches for rocprofv3 counter passes: cfg2 rotate/quant, LoRA down, GEMM, 3 times each; the W4A8
    GEMM at cfg1 and at the cfg2 shape, 3 times each; cfg0's rotate/quant with the LoRA down-projection in the
    same pass, 3 times; the cfg3
    input-gradient GEMM (with its LoRA term) and the cfg3 LoRA gradients 3 times each; the two producer kernels at cfg4's image-stream shapes
    and the grouped attention-input GEMM (M = 4608, 6144 -> 6144 | 1536 | 1536 | 6144, r = 16) 3 times each;
    then a plain 256 MiB device copy (Tensor.copy_) 3 times, the calibration point for FETCH/WRITE_SIZE."""
    L = k2._lib
    c = CONFIGS[2]
    x, W, b, A, B = synth(c["M"], c["K"], c["N"], c["r"], c["bias"])
    xd, Ad, Bd = x.to(dev), A.to(dev), B.to(dev)
    qw, sw = L.quant_weight_i8(W.to(dev))
    for _ in range(3):
        qx, sx, _ = L.rotquant(xd)
        u = L.lora_down(xd, Ad)
        L.gemm_w8a8(qx, sx, qw, sw, None, u, Bd, 1.0)
    # the W4A8 GEMM at cfg1 (LoRA r = 16, bias) and at the cfg2 shape with int4 weights (LoRA r = 32)
    c1 = CONFIGS[1]
    x1, W1, b1, A1, B1 = synth(c1["M"], c1["K"], c1["N"], c1["r"], c1["bias"])
    x1d = x1.to(dev)
    qw4, sw4 = L.quant_weight_i4(W1.to(dev))
    qx1, sx1, _ = L.rotquant(x1d)
    u1 = L.lora_down(x1d, A1.to(dev))
    b1d = None if b1 is None else b1.to(dev)
    qw4b, sw4b = L.quant_weight_i4(W.to(dev))
    for _ in range(3):
        L.gemm_w4a8(qx1, sx1, qw4, sw4, b1d, u1, B1.to(dev), 1.0)
    for _ in range(3):
        L.gemm_w4a8(qx, sx, qw4b, sw4b, None, u, Bd, 1.0)
    # cfg0: rotate/quant with the LoRA down-projection from the same pass (the one-call forward's route there)
    c0 = CONFIGS[0]
    x0, _, _, A0, _ = synth(c0["M"], c0["K"], c0["N"], c0["r"], c0["bias"])
    x0d, A0d = x0.to(dev), A0.to(dev)
    for _ in range(3):
        L.rotquant_lora(x0d, A0d)
    del x1d, qw4, sw4, qx1, sx1, u1, qw4b, sw4b, x0d, A0d
    c3 = CFG3
    g3 = torch.Generator().manual_seed(3)
    qw3, sw3 = L.quant_weight_i8((torch.randn(c3["N"], c3["K"], generator=g3) * 0.02).to(torch.bfloat16).to(dev))
    dy = (torch.randn(c3["M"], c3["N"], generator=g3) * 1e-3).to(torch.bfloat16).to(dev)
    A3 = (torch.randn(c3["r"], c3["K"], generator=g3) * 0.01).to(dev)
    g = (torch.randn(c3["M"], c3["r"], generator=g3) * 1e-3).to(dev)
    for _ in range(3):
        L.gemm_dx(dy, qw3, sw3, g=g, lora_a=A3)
    # cfg3's LoRA gradients: dA and dB in one wgrad launch
    x3 = torch.randn(c3["M"], c3["K"], generator=g3).to(torch.bfloat16).to(dev)
    u3 = torch.randn(c3["M"], c3["r"], generator=g3).to(dev)
    B3 = (torch.randn(c3["N"], c3["r"], generator=g3) * 0.01).to(dev)
    for _ in range(3):
        L.lora_grads(dy, x3, u3, B3, 0.5)
    del qw3, dy, A3, g, x3, u3, B3
    # the producer kernels at cfg4's image-stream shapes and the grouped attention-input GEMM at M = 4608
    Mi, Ki, Kh = 8192, 3072, 12288
    xi = torch.randn(Mi, Ki, generator=g3).to(torch.bfloat16).to(dev)
    ns = (torch.randn(Ki, generator=g3) * 0.1).to(dev)
    mod = (torch.randn(2, Ki, generator=g3) * 0.3).to(torch.bfloat16).to(dev)
    gt = (torch.randn(Mi, Kh, generator=g3) * 3).to(torch.bfloat16).to(dev)
    ut = torch.randn(Mi, Kh, generator=g3).to(torch.bfloat16).to(dev)
    for _ in range(3):
        L.rmsmod_rotquant(xi, ns, 1e-5, mod, mod, Mi // 2)
        L.swiglu_rotquant(gt, ut)
    del xi, gt, ut
    Mg, Kg, r = 4608, 6144, 16
    qg = torch.randint(-127, 128, (Mg, Kg), generator=g3, dtype=torch.int8).to(dev)
    sg = (torch.rand(Mg, generator=g3) * 0.05).to(dev)
    ug = torch.randn(Mg, 4 * r, generator=g3).to(dev)
    segs = []
    for i, Ng in enumerate((6144, 1536, 1536, 6144)):
        segs.append((torch.randint(-127, 128, (Ng, Kg), generator=g3, dtype=torch.int8).to(dev),
                     (torch.rand(Ng, generator=g3) * 0.01).to(dev), None,
                     (torch.randn(Ng, r, generator=g3) * 0.01).to(dev), i * r, 1.0))
    for _ in range(3):
        L.gemm_w8a8_grouped(qg, sg, segs, ug)
    del qg, segs, ug
    src = torch.ones(1 << 28, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("profile pass done", flush=True)


def _smi_sample():
    """(socket power W, GFX clock MHz) from amd-smi, run as a child process; None fields if unavailable."""
    import re
    import subprocess
    try:
        out = subprocess.run(["amd-smi", "metric", "-p", "-c", "-g", "0"], capture_output=True, text=True,
                             timeout=5).stdout
    except (OSError, subprocess.SubprocessError):
        return None, None
    p = re.search(r"SOCKET_POWER:\s*(\d+)", out)
    c = re.search(r"\bCLK:\s*(\d+)\s*MHz", out)
    return (int(p.group(1)) if p else None), (int(c.group(1)) if c else None)


def power_pass(k2, dev, seconds=4.0):
    """The cfg2 GEMM (this build's kernel, no LoRA) next to hipBLASLt's int8 GEMM (torch._int_mm, int32 out,
    no epilogue) and torch's bf16 GEMM at the same shape, each run back to back for ``seconds`` while
    amd-smi samples board power and GFX clock from a child process.  Prints one JSON line."""
    import threading
    L = k2._lib
    c = CONFIGS[2]
    M, K, N = c["M"], c["K"], c["N"]
    g = torch.Generator(device=dev).manual_seed(0)
    qx = torch.randint(-127, 128, (M, K), device=dev, dtype=torch.int8, generator=g)
    qw = torch.randint(-127, 128, (N, K), device=dev, dtype=torch.int8, generator=g)
    sx = torch.rand(M, device=dev) + 0.5
    sw = torch.rand(N, device=dev) * 0.01
    xb = torch.randn(M, K, device=dev, dtype=torch.bfloat16, generator=g)
    wb = torch.randn(N, K, device=dev, dtype=torch.bfloat16, generator=g)
    qwt = qw.t()
    ops = 2.0 * M * N * K
    res = {}
    for name, fn in (("k2q gemm_w8a8 (bf16 out, dequant epilogue)", lambda: L.gemm_w8a8(qx, sx, qw, sw, None)),
                     ("torch._int_mm / hipBLASLt (int32 out)", lambda: torch._int_mm(qx, qwt)),
                     ("torch.mm bf16", lambda: torch.mm(xb, wb.t()))):
        samples, stop = [], threading.Event()

        def sampler():
            while not stop.is_set():
                samples.append(_smi_sample())
                stop.wait(0.25)

        settle(fn, 1.0)
        th = threading.Thread(target=sampler)
        th.start()
        s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n, t_end = 0, time.perf_counter() + seconds
        s_ev.record()
        while time.perf_counter() < t_end:
            for _ in range(10):
                fn()
            n += 10
            torch.cuda.synchronize()
        e_ev.record()
        torch.cuda.synchronize()
        stop.set()
        th.join()
        ms = s_ev.elapsed_time(e_ev) / n
        pw = [p for p, _ in samples[2:] if p]      # the first samples lag the load
        ck = [ck for _, ck in samples[2:] if ck]
        res[name] = {"ms": round(ms, 4), "TOPS": round(ops / ms / 1e9, 1),
                     "power_W_median": sorted(pw)[len(pw) // 2] if pw else None,
                     "gfx_clock_MHz_median": sorted(ck)[len(ck) // 2] if ck else None, "samples": len(pw)}
    print(json.dumps({"power_pass": f"cfg2 GEMM shape M={M} K={K} N={N}, {seconds} s each", "results": res}),
          flush=True)


TRAFFIC_JSON = ROOT / "profiles" / "traffic_cfg2.json"


def kernel_sources_sha() -> str:
    """sha1 over the kernel sources (krea-2_amd/csrc): a traffic profile describes the kernels it was measured
    on, so it is used only while the sources are the same."""
    h = hashlib.sha1()
    for f in sorted((ROOT / "krea-2_amd" / "csrc").glob("*")):
        if f.suffix in (".hip", ".h"):
            h.update(f.name.encode())
            h.update(f.read_bytes())
    return h.hexdigest()[:16]


def measured_traffic(kernel_key: str):
    """HBM bytes per launch of a kernel from the committed rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE,
    copy-calibrated) and whether it applies: ``(bytes, True)`` when the summary was made from the current kernel
    sources, ``(None, False)`` when it is stale or missing."""
    try:
        data = json.loads(TRAFFIC_JSON.read_text())
        if data.get("kernel_sources_sha") != kernel_sources_sha():
            return None, False
        return data["kernels"][kernel_key]["traffic_bytes"], True
    except (OSError, KeyError, ValueError):
        return None, False


# Output tile shapes of the GEMM kernel: plan name -> the TileCfg<TA, TB, waves along A, workgroups per CU> text
# in the kernel's name, (TA, TB, workgroups per CU).
_TILE_CFG = {"256x256": ("TileCfg<256, 256, 2, 1>", (256, 256, 1)), "256x320": ("TileCfg<256, 320, 4, 1>", (256, 320, 1)),
             "192x256": ("TileCfg<192, 256, 2, 1>", (192, 256, 1)), "128x128": ("TileCfg<128, 128, 2, 2>", (128, 128, 2))}


def _gemm_kernel(L, epi, M, N, K, grouped=False, cus=256):
    """(kernel-name substrings, grid threads) of the one tile launch of a W8A8 GEMM (epi 0; K in int8 elements)
    or of the input-gradient GEMM on the effective weight (epi 4; K in bytes: 2 x the bf16 reduction length) on
    ``cus`` CUs, as the library schedules it: the shape the W8 plan picks for the same output and reduction bytes
    (the two epilogues share the chooser), a balanced persistent grid of ceil(tiles / rounds) workgroups of 512
    threads.  Split-K schedules are not profiled."""
    tile, pieces = L.gemm_w8a8_plan(M, N, K, cus, grouped)
    if pieces != 1:
        raise ValueError(f"profiled GEMM {M}x{N}x{K} takes a split-K schedule")
    name, (ta, tb, wpc) = _TILE_CFG[tile]
    tiles = -(-N // ta) * -(-M // tb)
    rounds = -(-tiles // (cus * wpc))
    return (f"gemm_nt_kernel<{epi}, 0,", name), -(-tiles // rounds) * 512


# Kernels of --profile-pass: (label, kernel-name substring(s), grid threads, algorithmic read, algorithmic write).
def _profiled_kernels(L):
    M2, K2, N2, r2 = 16896, 3072, 12288, 32
    M0, K0, r0 = 4096, 3072, 16
    M3, K3, N3, r3 = 4608, 12288, 3072, 64
    Mi, Ki, Kh = 8192, 3072, 12288
    Mg, Kg, Ng, rg = 4608, 6144, 15360, 16
    copy = 1 << 28
    return [
        ("gemm_nt_kernel<EPI_W8> cfg2", *_gemm_kernel(L, 0, M2, N2, K2),
         M2 * K2 + N2 * K2 + 4 * M2 + 4 * N2 + 4 * M2 * r2 + 4 * N2 * r2, 2 * M2 * N2),
        ("rotquant_kernel cfg2", "rotquant_kernel", 1081344, 2 * M2 * K2, M2 * K2 + 4 * M2),
        ("lora_down_as_kernel<2> cfg2", "lora_down_as_kernel<2>", None, 2 * M2 * K2 + 4 * r2 * K2, 3 * 4 * M2 * r2),
        ("lora_reduce_kernel cfg2", "lora_reduce_kernel", 135168, 3 * 4 * M2 * r2, 4 * M2 * r2),
        # x once and A once from HBM (each 16-row tile re-reads A, but from L2); codes, scales and u written
        ("rotquant_lora_kernel cfg0 (codes and u in one pass)", "rotquant_lora_kernel", 262144,
         2 * M0 * K0 + 4 * r0 * K0, M0 * K0 + 4 * M0 + 4 * M0 * r0),
        ("gemm_nt_kernel<EPI_DXLIN> cfg3 (input gradient)", *_gemm_kernel(L, 4, M3, K3, 2 * N3),
         2 * M3 * N3 + 2 * K3 * N3 + 4 * M3 * r3 + 4 * r3 * K3, 2 * M3 * K3),
        ("rot_dequant_t_kernel cfg3 (effective weight)", "rot_dequant_t_kernel<false>", 1179648, N3 * K3 + 4 * N3,
         2 * K3 * N3),
        # x and dY once, the hi/lo rows of g^T and u^T; writes: the two gradients (slice partials come on top)
        ("wgrad_kernel<4> cfg3 (LoRA dA and dB, one launch)", "wgrad_kernel<4>", None,
         2 * M3 * K3 + 2 * M3 * N3 + 8 * r3 * M3, 4 * r3 * (K3 + N3)),
        ("prodquant_kernel<RMSMOD> cfg4 image (M=8192, K=3072)", "prodquant_kernel<1, 1, 3, false>", 524288,
         2 * Mi * Ki, 2 * Mi * Ki + Mi * Ki + 4 * Mi),
        ("prodquant_kernel<SWIGLU> cfg4 image (M=8192, K=12288)", "prodquant_kernel<0, 4, 3, false>", 2097152,
         4 * Mi * Kh, 2 * Mi * Kh + Mi * Kh + 4 * Mi),
        ("gemm_nt_kernel<EPI_W8> grouped attention inputs (M=4608)", *_gemm_kernel(L, 0, Mg, Ng, Kg, grouped=True),
         Mg * Kg + Ng * Kg + 4 * Mg + 4 * Ng + 4 * Mg * 4 * rg + 4 * Ng * rg, 2 * Mg * Ng),
        ("copy 256 MiB (hipMemcpy device to device)", "copyBuffer", 131072, copy, copy),
    ]


def pmc_summary(k2, fetch_dir: str, write_dir: str) -> None:
    """Bytes per dispatch from two ``rocprofv3 --pmc FETCH_SIZE`` / ``--pmc WRITE_SIZE`` runs over
    ``--profile-pass`` (KiB counters, median over the dispatches), each scaled by what the counter reads for the
    pass's 256 MiB device copy; writes ``profiles/traffic_cfg2.json`` (stamped with the kernel sources' sha1)
    and prints the markdown table."""
    import csv
    import statistics

    def load(d):
        out = {}
        for f in Path(d).glob("**/*counter_collection.csv"):
            for row in csv.DictReader(open(f)):
                out.setdefault((row["Kernel_Name"], int(row["Grid_Size"])), []).append(float(row["Counter_Value"]))
        return out

    F_, W_ = load(fetch_dir), load(write_dir)

    def find(sub, grid, d):
        subs = (sub,) if isinstance(sub, str) else sub
        for (n, g), v in d.items():
            if all(x in n for x in subs) and (grid is None or g == grid):
                return v
        raise KeyError((sub, grid))

    copy = 1 << 28
    ff = copy / (statistics.median(find("copyBuffer", 131072, F_)) * 1024)
    wf = copy / (statistics.median(find("copyBuffer", 131072, W_)) * 1024)
    out = {"kernel_sources_sha": kernel_sources_sha(),
           "calibration": {"copy_bytes": copy, "fetch_factor": ff, "write_factor": wf}, "kernels": {}}
    lines = ["| kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM read bytes | HBM write bytes | "
             "algorithmic read / write bytes |", "|---|---|---|---|---|---|---|"]
    for label, sub, grid, ar, aw in _profiled_kernels(k2._lib):
        f, w = find(sub, grid, F_), find(sub, grid, W_)
        fk, wk = statistics.median(f), statistics.median(w)
        rb, wb = fk * 1024 * ff, wk * 1024 * wf
        out["kernels"][label] = {"dispatches": len(f), "fetch_kib": fk, "write_kib": wk, "read_bytes": rb,
                                 "write_bytes": wb, "traffic_bytes": rb + wb, "algorithmic_read": ar,
                                 "algorithmic_write": aw}
        lines.append(f"| {label} | {len(f)} | {fk:.0f} | {wk:.0f} | {rb / 1e6:.1f} MB | {wb / 1e6:.1f} MB | "
                     f"{ar / 1e6:.1f} MB / {aw / 1e6:.1f} MB |")
    TRAFFIC_JSON.write_text(json.dumps(out, indent=1) + "\n")
    print(f"fetch factor {ff:.4f}, write factor {wf:.4f}, kernel sources {out['kernel_sources_sha']}")
    print("\n".join(lines))


# ----------------------------------------------------------------------------------------------------------
# Per-config CPU paths (bounded samples, timed on this host's cores)
# ----------------------------------------------------------------------------------------------------------
def _median_time(fn, budget_s, min_runs=3, max_runs=30):
    import numpy as np
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_runs or (time.perf_counter() < t_end and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def _layer_tensors(layer, seed, K, N):
    """CPU copies of a bench layer's operands: the W8A8 codes and scales the GPU quantizer made (offline weight
    preparation; equal to the oracle's quant_weight_i8 bit for bit, which the GPU tests check), the bf16 weight
    (regenerated from the layer's seed, as make_layer drew it) and the LoRA factors."""
    g = torch.Generator().manual_seed(seed)
    W = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    return (layer.base.qweight.cpu().numpy(), layer.base.weight_scale.cpu().numpy(), W,
            layer.lora_A.detach().cpu(), layer.lora_B.detach().cpu())


def cpu_cfg3(qw, sw, W, A, B, rows=128, budget_s=2.0):
    """cfg3's training step on the CPU for ``rows`` of the 4608 tokens: the oracle's forward + backward (the
    ConvRot arithmetic) and the reference's own step restated (``Fp8Linear.forward`` + ``LoRALinear.forward``
    under torch autograd, quantize.py:48-51, lora.py:47-48).  ms are scaled to the full M."""
    from oracle import convrot as orc

    torch.set_num_threads(os.cpu_count() or 1)
    c = CFG3
    M, K, N = c["M"], c["K"], c["N"]
    g = torch.Generator().manual_seed(33)
    x = torch.randn(rows, K, generator=g).to(torch.bfloat16)
    dy = (torch.randn(rows, N, generator=g) * 1e-3).to(torch.bfloat16)
    xs, dys, An, Bn = x.float().numpy(), dy.float().numpy(), A.numpy(), B.numpy()

    def oracle_step():
        orc.forward(xs, qw, sw, lora_A=An, lora_B=Bn, lora_scale=1.0, fast=True)
        orc.backward(dys, xs, qw, sw, lora_A=An, lora_B=Bn, lora_scale=1.0)

    wq, sc = orc.fp8_weight_quant(W.float().numpy())
    Ar, Br = A.clone().requires_grad_(True), B.clone().requires_grad_(True)

    def ref_step():
        xr = x.clone().requires_grad_(True)
        out = torch.nn.functional.linear(xr, wq.to(torch.bfloat16) * sc.to(torch.bfloat16))
        out = out + ((xr.to(torch.float32) @ Ar.t()) @ Br.t()).to(out.dtype)
        out.backward(dy)

    ops = 2.0 * 2.0 * M * N * K      # forward GEMM + input-gradient GEMM
    res = {}
    for name, fn in (("oracle", oracle_step), ("reference_fp8", ref_step)):
        t, n = _median_time(fn, budget_s)
        ms = t * 1e3 * M / rows
        res[name] = {"ms": round(ms, 2), "tops": round(ops / (ms * 1e-3) / 1e12, 4), "cores": torch.get_num_threads(),
                     "kind": "port", "sample": f"{rows} of {M} rows, forward + backward, median of {n} runs, "
                                               "ms scaled to M"}
    return res


def cpu_cfg4(items, rows=128, budget_s=0.3):
    """cfg4's ten block linears on the CPU: each linear's forward (oracle ConvRot W8A8 + LoRA r=16, and the
    reference's Fp8Linear + LoRALinear restated) on up to ``rows`` tokens, scaled to the stream's M and summed.
    ``items``: (M, K, N, qw, sw, W, A, B) per linear, as :func:`_layer_tensors` gives them."""
    from oracle import convrot as orc

    torch.set_num_threads(os.cpu_count() or 1)
    tot = {"oracle": 0.0, "reference_fp8": 0.0}
    ops = 0.0
    for M, K, N, qw, sw, W, A, B in items:
        n = min(rows, M)
        x = torch.randn(n, K, generator=torch.Generator().manual_seed(M + K)).to(torch.bfloat16)
        xs, An, Bn = x.float().numpy(), A.numpy(), B.numpy()
        wq, sc = orc.fp8_weight_quant(W.float().numpy())
        t_o, _ = _median_time(lambda: orc.forward(xs, qw, sw, lora_A=An, lora_B=Bn, lora_scale=1.0, fast=True),
                              budget_s)

        def ref():
            out = orc.fp8_linear(x, wq, sc)
            return out + ((x.float() @ A.t()) @ B.t()).to(out.dtype)

        t_r, _ = _median_time(ref, budget_s)
        tot["oracle"] += t_o * M / n
        tot["reference_fp8"] += t_r * M / n
        ops += 2.0 * M * N * K
    return {name: {"ms": round(t * 1e3, 2), "tops": round(ops / t / 1e12, 4), "cores": torch.get_num_threads(),
                   "kind": "port",
                   "sample": f"each linear on up to {rows} of its M rows (adaLN: both), median of >= 3 runs, "
                             "ms scaled to M and summed"} for name, t in tot.items()}


def roofline_entry(kernel, bound, achieved, peak, unit):
    return {"kernel": kernel, "bound": bound, "achieved": round(achieved, 1), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4)}


def forward_record(cfg, res, cpu=None, cpu_ref=None):
    """One BASELINE forward config (rotate/quant + LoRA down-projection + GEMM with the fused epilogue)."""
    gemm_tops = res["ops"] / (res["ms_gemm"] * 1e-3) / 1e12
    rot_gbs = res["rot_bytes"] / (res["ms_rot_stream"] * 1e-3) / 1e9
    rec = {"workload": cfg["name"], "ms": round(res["ms_step"], 4), "tops": round(res["tops"], 1),
           "pct_int8_peak": round(100 * res["tops"] / INT8_PEAK_TOPS, 2),
           "host_us_per_step": round(res["host_us"], 1),
           "gemm_ms": round(res["ms_gemm"], 4), "lora_down_ms": round(res["ms_lora"], 4),
           "rotquant_ms_in_step": round(res["ms_rot"], 4),
           "lora_down_in_rotquant_pass": bool(res["fused_down"]),
           "roofline": roofline_entry("gemm_w4_kernel" if cfg["w4"] else "gemm_nt_kernel<EPI_W8>", "mfma", gemm_tops,
                                      INT8_PEAK_TOPS, "TOPS"),
           "rotquant_roofline": roofline_entry("rotquant_kernel (4 inputs streamed from HBM)", "hbm", rot_gbs,
                                               HBM_PEAK_GBS, "GB/s")}
    rec["rotquant_roofline"]["ms"] = round(res["ms_rot_stream"], 4)
    if cpu is not None:
        rec["cpu"] = {"oracle": cpu, "reference_fp8": cpu_ref}
    return rec


_T0 = time.perf_counter()


def progress(what: str) -> None:
    """One line per finished leg on stderr (stdout carries only the JSON line)."""
    print(f"[bench {time.perf_counter() - _T0:6.1f} s] {what}", file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--settle", type=float, default=2.0,
                    help="seconds of untimed steps before the warmup steps, so the clocks leave their ramp-up "
                         "state (0 disables)")
    ap.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--profile-pass", action="store_true", help="fixed launches for rocprofv3 counter runs")
    ap.add_argument("--power", action="store_true",
                    help="GEMM vs hipBLASLt int8 vs bf16 at the cfg2 shape with board power / clock samples")
    ap.add_argument("--krea-block-pass", type=int, default=0, metavar="N",
                    help="N fused forward + backward passes of the Krea 2 block leg (for kernel traces)")
    ap.add_argument("--cfg3-pass", type=int, default=0, metavar="N",
                    help="N cfg3 training steps of one layer (for kernel traces)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="write profiles/traffic_cfg2.json from two rocprofv3 --pmc runs over --profile-pass")
    a = ap.parse_args()
    if a.pmc_summary:
        import __graft_entry__ as ge
        pmc_summary(ge.load_package(), *a.pmc_summary)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus > 1 or world > 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (the per-token rows of the path "
              "shard over GPUs with no communication). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)

    import __graft_entry__ as ge
    k2 = ge.load_package()
    dev = torch.device("cuda:0")
    if a.profile_pass:
        profile_pass(k2, dev)
        return
    if a.power:
        power_pass(k2, dev)
        return
    if a.krea_block_pass:
        krea_block_pass(k2, dev, a.krea_block_pass)
        return
    if a.cfg3_pass:
        cfg3_pass(k2, dev, a.cfg3_pass)
        return
    cfg = CONFIGS[a.config]
    res = run_config(k2, cfg, a.steps, a.warmup, dev, a.settle)
    progress(f"cfg{a.config} forward timed")

    gemm_tops = res["ops"] / (res["ms_gemm"] * 1e-3) / 1e12
    rot_gbs = res["rot_bytes"] / (res["ms_rot_stream"] * 1e-3) / 1e9
    extra = {
        "fwd_tops": round(res["tops"], 1),
        "fwd_pct_int8_peak": round(100 * res["tops"] / INT8_PEAK_TOPS, 2),
        "gemm_ms": round(res["ms_gemm"], 4), "gemm_tops": round(gemm_tops, 1),
        "gemm_pct_int8_peak": round(100 * gemm_tops / INT8_PEAK_TOPS, 2),
        "rotquant_ms": round(res["ms_rot_stream"], 4), "rotquant_GBps": round(rot_gbs, 1),
        "rotquant_ms_in_step": round(res["ms_rot"], 4),
        "rotquant_pct_hbm": round(100 * rot_gbs / HBM_PEAK_GBS, 2),
        "lora_down_ms": round(res["ms_lora"], 4),
        "lora_ops": 2.0 * cfg["M"] * cfg["r"] * (cfg["K"] + cfg["N"]),
    }
    extra["settle_s"] = a.settle
    probe = mfma_probe(k2, dev)
    extra["mfma_probe_int8_tops"] = round(probe, 1)
    extra["gemm_pct_of_mfma_probe"] = round(100 * gemm_tops / probe, 2)
    extra["reference_path_gpu_cfg2"] = run_reference_gpu(k2, res, max(5, a.steps // 2), dev)
    progress("MFMA probe and the reference's GPU path timed")
    cpu = cpu_ref = None
    if not a.no_cpu:
        cpu = cpu_baseline(cfg, res["x"], res["W"], res["b"], res["A"], res["B"])
        cpu_ref = cpu_reference_path(cfg, res["x"], res["W"], res["b"], res["A"], res["B"])
        extra["cpu_reference_fp8_path"] = cpu_ref
        progress("CPU paths of the headline config timed")
    # every BASELINE.json configuration: GPU time, roofline fraction, CPU paths
    extra[f"cfg{a.config}"] = forward_record(cfg, res, cpu, cpu_ref)
    for c in sorted(CONFIGS):
        if c == a.config:
            continue
        rc = run_config(k2, CONFIGS[c], a.steps, a.warmup, dev, a.settle / 2)
        cc = ccr = None
        if not a.no_cpu:
            cc = cpu_baseline(CONFIGS[c], rc["x"], rc["W"], rc["b"], rc["A"], rc["B"], budget_s=3.0, rows=512)
            ccr = cpu_reference_path(CONFIGS[c], rc["x"], rc["W"], rc["b"], rc["A"], rc["B"], budget_s=2.0, rows=512)
        extra[f"cfg{c}"] = forward_record(CONFIGS[c], rc, cc, ccr)
        del rc
        progress(f"cfg{c} timed")
    # the W4A8 base at the headline shape (not a BASELINE config: cfg2's M, K, N and r with cfg1's int4 weights)
    w4c = dict(CONFIGS[2], w4=True, name="cfg2 shape with W4A8 (g64) weights, M=16896 K=3072 N=12288 r=32")
    rw = run_config(k2, w4c, max(5, a.steps // 2), a.warmup, dev, a.settle / 2)
    extra["cfg2_shape_w4a8"] = forward_record(w4c, rw)
    del rw
    progress("cfg2 shape with W4A8 weights timed")
    extra["cfg3"] = run_cfg3(k2, max(5, a.steps // 2), dev, a.settle / 2, cpu=not a.no_cpu)
    progress("cfg3 timed")
    extra["cfg4"] = run_cfg4(k2, max(5, a.steps // 2), dev, a.settle / 2, cpu=not a.no_cpu)
    progress("cfg4 timed")
    extra["producers_cfg4_image"] = run_producers(k2, max(5, a.steps // 2), dev)
    extra["grouped_attn_inputs"] = run_grouped(k2, max(5, a.steps // 2), dev)
    extra["krea_block_linears"] = run_krea_block(k2, max(5, a.steps // 2), dev)
    progress("producers, grouped attention inputs and the Krea 2 block timed")
    extra["vram_krea_block"] = run_vram(k2, dev)
    progress("device memory of the Krea 2 block's linears measured")
    traffic, fresh = measured_traffic("gemm_nt_kernel<EPI_W8> cfg2") if a.config == 2 and not cfg["w4"] else (None, False)
    extra["traffic_profile"] = ("profiles/traffic_cfg2.json, measured on these kernel sources" if fresh else
                                "no PMC profile of these kernel sources: traffic omitted")
    line = {
        "metric": METRIC,
        "value": round(res["tops"], 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(res["ms_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: BASELINE.json distributions (x~N(0,1) bf16 with 1% outlier channels x20, "
                "W~N(0,0.02), LoRA A,B~N(0,0.01)), seed 0",
        "config": {"workload": cfg["name"], "M": cfg["M"], "K": cfg["K"], "N": cfg["N"], "rank": cfg["r"],
                   "weights": "int4 g64" if cfg["w4"] else "int8 per-channel", "hadamard_block": 128},
        "roofline": {"bound": "mfma", "kernel": "gemm_nt_kernel<EPI_W8>" if not cfg["w4"] else "gemm_w4_kernel",
                     "achieved": round(gemm_tops, 1), "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                     "frac": round(gemm_tops / INT8_PEAK_TOPS, 4), "traffic": traffic},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
