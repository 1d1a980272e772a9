"""ctypes binding of ``libk2q.so`` (declared in ``include/k2q.h``) plus host-side argument checks.

Every wrapper validates shapes, dtypes, devices and contiguity on the host and raises ``ValueError`` /
``RuntimeError`` before any launch; a nonzero status from the library becomes ``RuntimeError``.  Kernels
run on ``torch.cuda.current_stream()`` of the tensors' device.  Outputs are allocated with ``torch.empty``
(PyTorch's caching allocator owns all memory).  There is no fallback: if the library or a gfx950 GPU is
missing, the call raises.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libk2q.so"

K2Q_OK = 0
_STATUS = {-1: "K2Q_EINVAL (bad shape, null or misaligned pointer)", -2: "K2Q_EARCH (device is not gfx950)",
           -3: "K2Q_ELAUNCH (kernel launch failed)", -4: "K2Q_EUNSUPPORTED (shape outside the kernels)",
           -5: "K2Q_ESCRATCH (the shape needs more device scratch than the library holds)"}
DTYPE_BF16 = 0
DTYPE_F32 = 1
HADAMARD_BLOCK = 128
INT4_GROUP = 64
MAX_RANK = 4096        # K2Q_MAX_RANK: ranks run in chunks of 128 inside the library
RANK_ALIGN = 16        # the kernels take ranks in multiples of 16 (callers pad with zero factor rows)

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float


class DxSegment(ctypes.Structure):
    """``k2q_dx_segment`` of ``include/k2q.h``: one linear of a grouped input gradient."""
    _fields_ = [("dy", ctypes.c_void_p), ("ldy", ctypes.c_int64), ("wt", ctypes.c_void_p), ("N", ctypes.c_int64)]


class LoraMember(ctypes.Structure):
    """``k2q_lora_member`` of ``include/k2q.h``: one linear of a grouped LoRA-gradient call."""
    _fields_ = [("dy", ctypes.c_void_p), ("ldy", ctypes.c_int64), ("N", ctypes.c_int64), ("lora_b", ctypes.c_void_p),
                ("scale", ctypes.c_float), ("dB", ctypes.c_void_p)]


class W8A8Segment(ctypes.Structure):
    """``k2q_w8a8_segment`` of ``include/k2q.h``: one linear of a grouped forward."""
    _fields_ = [("qw", ctypes.c_void_p), ("sw", ctypes.c_void_p), ("bias", ctypes.c_void_p),
                ("lora_b", ctypes.c_void_p), ("y", ctypes.c_void_p), ("N", ctypes.c_int64),
                ("u_col", ctypes.c_int64), ("lora_scale", ctypes.c_float)]


GROUP_MAX = 4          # segments per grouped launch
GROUP_ALIGN = 256      # each segment's out_features: a multiple of the GEMM tile

_SIGNATURES = {
    "k2q_version": ([], ctypes.c_char_p),
    "k2q_check_device": ([], _int),
    "k2q_rotquant": ([_p, _int, _i64, _i64, _i64, _p, _p, _p, _p], _int),
    "k2q_rotquant_lora": ([_p, _i64, _i64, _i64, _p, _p, _p, _i64, _p, _i64, _p], _int),
    "k2q_quant_weight_i4": ([_p, _int, _i64, _i64, _p, _p, _p], _int),
    "k2q_swiglu_rotquant": ([_p, _i64, _p, _i64, _i64, _i64, _p, _p, _p, _p], _int),
    "k2q_rmsmod_rotquant": ([_p, _i64, _i64, _i64, _p, _f32, _p, _p, _i64, _i64, _p, _p, _p, _p], _int),
    "k2q_swiglu_bwd": ([_p, _p, _p, _i64, _p, _p, _p], _int),
    "k2q_rmsmod_bwd": ([_p, _p, _i64, _i64, _p, _f32, _p, _i64, _i64, _p, _p], _int),
    "k2q_lora_down_ws_bytes": ([_i64, _i64, _i64], _i64),
    "k2q_lora_down": ([_p, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _p], _int),
    "k2q_lora_grads_ws_bytes": ([_i64, _i64, _i64, _i64], _i64),
    "k2q_lora_grads": ([_p, _p, _p, _p, _i64, _f32, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _p], _int),
    "k2q_lora_grads_grouped_ws_bytes": ([_p, _i64, _i64, _i64, _i64], _i64),
    "k2q_lora_grads_grouped": ([_p, _i64, _p, _p, _i64, _i64, _i64, _p, _p, _p, _i64, _p], _int),
    "k2q_lora_grads_noalloc": ([_p, _p, _p, _p, _i64, _f32, _i64, _i64, _i64, _p, _p, _p, _p], _int),
    "k2q_gemm_w8a8_ws_bytes": ([_i64, _i64, _i64], _i64),
    "k2q_gemm_w8a8": ([_p, _p, _p, _p, _p, _p, _p, _i64, _f32, _i64, _i64, _i64, _p, _p, _i64, _p], _int),
    "k2q_gemm_w8a8_grouped": ([_p, _p, _i64, _i64, _p, _i64, _p, _i64, _i64, _p, _i64, _p], _int),
    "k2q_gemm_w4a8": ([_p, _p, _p, _p, _p, _p, _p, _i64, _f32, _i64, _i64, _i64, _p, _p], _int),
    "k2q_linear_fwd_ws_bytes": ([_int, _i64, _i64, _i64, _i64], _i64),
    "k2q_linear_fwd_fuses_down": ([_i64, _i64, _i64], _int),
    "k2q_linear_fwd": ([_p, _i64, _i64, _i64, _p, _p, _int, _p, _p, _i64, _f32, _p, _int, _p, _p, _p, _i64, _p, _p,
                        _i64, _p], _int),
    "k2q_gemm_w8a8_acc": ([_p, _p, _i64, _i64, _i64, _p, _p, _i64, _int, _p], _int),
    "k2q_gemm_w8a8_tile": ([_p, _p, _p, _p, _p, _p, _p, _i64, _f32, _i64, _i64, _i64, _p, _p, _i64, _int, _p], _int),
    "k2q_gemm_w8a8_plan": ([_i64, _i64, _i64, _int, _int, ctypes.POINTER(_int)], _int),
    "k2q_gemm_w4a8_f32": ([_p, _p, _p, _i64, _i64, _i64, _p, _p], _int),
    "k2q_quant_weight_fp8": ([_p, _int, _i64, _i64, _p, _p, _p], _int),
    "k2q_dequant_fp8": ([_p, _p, _i64, _i64, _int, _p, _p], _int),
    "k2q_gemm_bf16_ws_bytes": ([_i64, _i64, _i64], _i64),
    "k2q_gemm_bf16": ([_p, _p, _p, _p, _p, _i64, _f32, _i64, _i64, _i64, _p, _p, _i64, _p], _int),
    "k2q_gemm_dx_lin": ([_p, _p, _i64, _i64, _i64, _p, _p, _i64, _p, _p, _i64, _p], _int),
    "k2q_dx_prep": ([_p, _p, _p, _p, _i64, _i64, _p, _p], _int),
    "k2q_dx_prep_eff": ([_p, _p, _p, _p, _i64, _i64, _p, _p], _int),
    "k2q_gemm_dx_ws_bytes": ([_i64, _i64, _i64], _i64),
    "k2q_gemm_dx": ([_p, _p, _i64, _i64, _i64, _p, _p, _i64, _p, _p, _i64, _p], _int),
    "k2q_gemm_dx_grouped": ([_p, _i64, _i64, _i64, _p, _i64, _p, _i64, _p, _p], _int),
}
EXPORTS = tuple(_SIGNATURES)

_lib = None
_lock = threading.Lock()
_device_ok: dict[int, bool] = {}


def load() -> ctypes.CDLL:
    """Load ``libk2q.so`` once and bind every entry point's signature.  Raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(f"{LIB_PATH} is not built; run krea-2_amd/build.py (hipcc, gfx950)")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (args, res) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = res
            _lib = lib
    return _lib


def version() -> str:
    return load().k2q_version().decode()


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _check(rc: int, name: str) -> None:
    if rc != K2Q_OK:
        raise RuntimeError(f"{name} failed: {_STATUS.get(rc, rc)}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(dev: torch.device) -> int:
    """The raw ``hipStream_t`` of the current stream of ``dev`` (torch's own getter when it has one: a tenth of
    the host time of building a ``torch.cuda.Stream`` object per call)."""
    if _raw_stream is not None:
        return _raw_stream(dev.index if dev.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(dev).cuda_stream


def _device_check(dev: torch.device) -> None:
    if dev.type != "cuda":
        raise RuntimeError(f"k2q kernels need a gfx950 GPU tensor, got device {dev}")
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in _device_ok:
        with torch.cuda.device(idx):
            _device_ok[idx] = load().k2q_check_device() == K2Q_OK
    if not _device_ok[idx]:
        raise RuntimeError(f"device cuda:{idx} is not gfx950 (MI355X); the k2q kernels are built for gfx950 only")


def _need(t: torch.Tensor, name: str, dtype, ndim: int | None = None, dev: torch.device | None = None):
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must be {ndim}-D, got shape {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if dev is not None and t.device != dev:
        raise ValueError(f"{name} is on {t.device}, expected {dev}")
    if t.data_ptr() % 16:
        raise ValueError(f"{name} must be 16-byte aligned")


def _workspace(nbytes: int, dev: torch.device):
    """Scratch device memory for a kernel's split pieces (from PyTorch's caching allocator), or none."""
    if nbytes <= 0:
        return None, 0
    return torch.empty((nbytes,), dtype=torch.uint8, device=dev), nbytes


def _check_k(K: int) -> None:
    if K < HADAMARD_BLOCK or K % HADAMARD_BLOCK:
        raise ValueError(f"in_features={K} must be a positive multiple of the Hadamard block {HADAMARD_BLOCK}")
    if K > 16384:
        raise ValueError(f"in_features={K} exceeds the rotate/quant kernel's 16384 limit")


def _check_rank(r: int) -> None:
    if r < RANK_ALIGN or r > MAX_RANK or r % RANK_ALIGN:
        raise ValueError(f"LoRA rank {r} must be a multiple of {RANK_ALIGN} in [{RANK_ALIGN}, {MAX_RANK}] "
                         "(pad the factors with zero ranks)")


# ----------------------------------------------------------------------------------------------------------
# (1) rotate + quantize
# ----------------------------------------------------------------------------------------------------------
def rotquant(x: torch.Tensor, want_xrot: bool = False):
    """Per-row FWHT-128 rotation + int8 quantization.  ``x`` (M,K) bf16 or f32, contiguous.
    Returns ``(q int8 (M,K), s f32 (M,), xrot bf16 (M,K) | None)``."""
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"x must be bf16 or f32, got {x.dtype}")
    _need(x, "x", x.dtype, 2)
    M, K = x.shape
    _check_k(K)
    if M < 1:
        raise ValueError("x has no rows")
    _device_check(x.device)
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    s = torch.empty((M,), dtype=torch.float32, device=x.device)
    xr = torch.empty((M, K), dtype=torch.bfloat16, device=x.device) if want_xrot else None
    dt = DTYPE_BF16 if x.dtype == torch.bfloat16 else DTYPE_F32
    _check(load().k2q_rotquant(_ptr(x), dt, M, K, K, _ptr(q), _ptr(s), _ptr(xr), _stream(x.device)),
           "k2q_rotquant")
    return q, s, xr


def rotquant_lora_fits(K: int, r: int) -> bool:
    """Whether :func:`rotquant_lora` takes the shape (one row per wave: K <= 3072, K % 512 == 0; r 16-64)."""
    return 512 <= K <= 3072 and K % 512 == 0 and r in (16, 32, 48, 64) and 16 * (r // 16) * 1024 <= 16 * (K + 8) * 2


def rotquant_lora(x: torch.Tensor, A: torch.Tensor):
    """Rotate/quant of ``x`` (M,K) bf16 with the LoRA down-projection ``u = x A^T`` from the same pass
    (``k2q_rotquant_lora``; ``A`` (r,K) f32).  Returns ``(q int8 (M,K), s f32 (M,), u f32 (M,r))``; the codes
    equal :func:`rotquant`'s bit for bit."""
    _need(x, "x", torch.bfloat16, 2)
    M, K = x.shape
    _check_k(K)
    if M < 1:
        raise ValueError("x has no rows")
    _need(A, "lora_a", torch.float32, 2, x.device)
    r = A.shape[0]
    if A.shape[1] != K:
        raise ValueError(f"lora_a {tuple(A.shape)} does not match K={K}")
    if not rotquant_lora_fits(K, r):
        raise ValueError(f"rotquant_lora takes K <= 3072 with K % 512 == 0 and r in 16..64 by 16, got K={K} r={r}")
    _device_check(x.device)
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    s = torch.empty((M,), dtype=torch.float32, device=x.device)
    u = torch.empty((M, r), dtype=torch.float32, device=x.device)
    _check(load().k2q_rotquant_lora(_ptr(x), M, K, K, _ptr(q), _ptr(s), _ptr(A), r, _ptr(u), r, _stream(x.device)),
           "k2q_rotquant_lora")
    return q, s, u


def _need_rows(t: torch.Tensor, name: str, dev: torch.device | None = None) -> None:
    """A 2-D bf16 tensor whose rows are contiguous and 16-byte aligned (the row stride may exceed K)."""
    if not isinstance(t, torch.Tensor) or t.dtype != torch.bfloat16 or t.dim() != 2:
        raise ValueError(f"{name} must be a 2-D bf16 tensor")
    if t.stride(1) != 1 or t.stride(0) < t.shape[1] or t.stride(0) % 8 or t.data_ptr() % 16:
        raise ValueError(f"{name} needs contiguous 16-byte aligned rows (strides {t.stride()})")
    if dev is not None and t.device != dev:
        raise ValueError(f"{name} is on {t.device}, expected {dev}")


def swiglu_rotquant(g: torch.Tensor, u: torch.Tensor):
    """``h = bf16(bf16(silu(g)) * u)`` with the codes of ``rotquant(h)`` from the same pass.
    ``g``, ``u`` (M,K) bf16 with contiguous rows.  Returns ``(h bf16 (M,K), q int8 (M,K), s f32 (M,))``."""
    _need_rows(g, "gate")
    _need_rows(u, "up", g.device)
    if g.shape != u.shape:
        raise ValueError(f"gate {tuple(g.shape)} and up {tuple(u.shape)} differ in shape")
    M, K = g.shape
    _check_k(K)
    if M < 1:
        raise ValueError("no rows")
    _device_check(g.device)
    h = torch.empty((M, K), dtype=torch.bfloat16, device=g.device)
    q = torch.empty((M, K), dtype=torch.int8, device=g.device)
    s = torch.empty((M,), dtype=torch.float32, device=g.device)
    _check(load().k2q_swiglu_rotquant(_ptr(g), g.stride(0), _ptr(u), u.stride(0), M, K, _ptr(h), _ptr(q), _ptr(s),
                                      _stream(g.device)), "k2q_swiglu_rotquant")
    return h, q, s


def rmsmod_rotquant(x: torch.Tensor, norm_scale: torch.Tensor, eps: float, mod_scale: torch.Tensor,
                    mod_shift: torch.Tensor, rows_per_batch: int):
    """Modulated RMSNorm ``h = bf16(bf16(bf16(1 + p) * n) + b)``, ``n = bf16(rms_norm(x) * (norm_scale + 1))``,
    with the codes of ``rotquant(h)`` from the same pass.  ``x`` (M,K) bf16 rows; ``norm_scale`` (K,) f32;
    ``mod_scale`` / ``mod_shift`` (B,K) bf16 with contiguous rows and one common row stride, row ``m`` using
    entry ``m // rows_per_batch`` (B == 1: every row uses entry 0).  Returns ``(h, q, s)``."""
    _need_rows(x, "x")
    dev = x.device
    M, K = x.shape
    _check_k(K)
    if M < 1:
        raise ValueError("no rows")
    _need(norm_scale, "norm_scale", torch.float32, 1, dev)
    if norm_scale.shape[0] != K:
        raise ValueError(f"norm_scale has {norm_scale.shape[0]} entries, x has {K} features")
    for t, nm in ((mod_scale, "mod_scale"), (mod_shift, "mod_shift")):
        if not isinstance(t, torch.Tensor) or t.dtype != torch.bfloat16 or t.dim() != 2 or t.shape[1] != K:
            raise ValueError(f"{nm} must be a (B, {K}) bf16 tensor")
        if t.stride(1) != 1 or t.data_ptr() % 16 or t.device != dev:
            raise ValueError(f"{nm} needs contiguous 16-byte aligned rows on {dev}")
    if mod_scale.shape != mod_shift.shape:
        raise ValueError("mod_scale and mod_shift differ in shape")
    B = mod_scale.shape[0]
    ldm = 0 if B == 1 else mod_scale.stride(0)
    if B > 1 and (mod_shift.stride(0) != ldm or ldm % 8):
        raise ValueError("mod_scale and mod_shift need one common row stride, a multiple of 8")
    rows_per_batch = int(rows_per_batch)
    if rows_per_batch < 1 or (B > 1 and rows_per_batch * B != M):
        raise ValueError(f"rows_per_batch={rows_per_batch} does not split {M} rows into {B} entries")
    _device_check(dev)
    h = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    q = torch.empty((M, K), dtype=torch.int8, device=dev)
    s = torch.empty((M,), dtype=torch.float32, device=dev)
    _check(load().k2q_rmsmod_rotquant(_ptr(x), x.stride(0), M, K, _ptr(norm_scale), float(eps), _ptr(mod_scale),
                                      _ptr(mod_shift), ldm, rows_per_batch if B > 1 else M, _ptr(h), _ptr(q),
                                      _ptr(s), _stream(dev)), "k2q_rmsmod_rotquant")
    return h, q, s


def rmsmod_bwd(dh: torch.Tensor, x: torch.Tensor, norm_scale: torch.Tensor, eps: float, mod_scale: torch.Tensor,
               rows_per_batch: int) -> torch.Tensor:
    """Input gradient of :func:`rmsmod_rotquant`'s ``h`` for ``x``: ``dx`` (M,K) bf16.  ``dh``, ``x`` (M,K) bf16
    contiguous; ``norm_scale`` (K,) f32; ``mod_scale`` (B,K) bf16 rows indexed as in the forward."""
    _need(dh, "dh", torch.bfloat16, 2)
    dev = dh.device
    _need(x, "x", torch.bfloat16, 2, dev)
    if dh.shape != x.shape:
        raise ValueError("dh and x differ in shape")
    M, K = x.shape
    if M < 1 or K % 8 or K > 16384:
        raise ValueError(f"x {tuple(x.shape)}: K must be a multiple of 8 up to 16384")
    _need(norm_scale, "norm_scale", torch.float32, 1, dev)
    if norm_scale.shape[0] != K:
        raise ValueError("norm_scale length != K")
    if mod_scale.dtype != torch.bfloat16 or mod_scale.dim() != 2 or mod_scale.shape[1] != K or \
            mod_scale.stride(1) != 1 or mod_scale.data_ptr() % 16 or mod_scale.device != dev:
        raise ValueError(f"mod_scale must be a (B, {K}) bf16 tensor with contiguous 16-byte aligned rows")
    B = mod_scale.shape[0]
    ldm = 0 if B == 1 else mod_scale.stride(0)
    rows_per_batch = int(rows_per_batch)
    if B > 1 and (ldm % 8 or rows_per_batch * B != M):
        raise ValueError(f"rows_per_batch={rows_per_batch} does not split {M} rows into {B} entries")
    _device_check(dev)
    dx = torch.empty_like(x)
    _check(load().k2q_rmsmod_bwd(_ptr(dh), _ptr(x), M, K, _ptr(norm_scale), float(eps), _ptr(mod_scale), ldm,
                                 rows_per_batch if B > 1 else M, _ptr(dx), _stream(dev)), "k2q_rmsmod_bwd")
    return dx


def swiglu_bwd(dh: torch.Tensor, g: torch.Tensor, u: torch.Tensor):
    """Autograd of ``bf16(bf16(silu(g)) * u)``: ``(dg, du)``, bf16, shapes of ``g``; all contiguous."""
    _need(dh, "dh", torch.bfloat16)
    _need(g, "gate", torch.bfloat16, dev=dh.device)
    _need(u, "up", torch.bfloat16, dev=dh.device)
    if not (dh.shape == g.shape == u.shape):
        raise ValueError("dh, gate and up differ in shape")
    n = dh.numel()
    if n < 1 or n % 8:
        raise ValueError(f"element count {n} must be a positive multiple of 8")
    _device_check(dh.device)
    dg = torch.empty_like(g)
    du = torch.empty_like(u)
    _check(load().k2q_swiglu_bwd(_ptr(dh), _ptr(g), _ptr(u), n, _ptr(dg), _ptr(du), _stream(dh.device)),
           "k2q_swiglu_bwd")
    return dg, du


def quant_weight_i8(w: torch.Tensor):
    """int8 per-output-channel quantization of ``W R``: ``(q int8 (N,K), s f32 (N,))``."""
    q, s, _ = rotquant(w)
    return q, s


def quant_weight_i4(w: torch.Tensor):
    """int4 group-64 quantization of ``W R``: ``(q4 uint8 (N,K/2) packed, s4 bf16 (K/64,N) group-major)``."""
    if w.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"w must be bf16 or f32, got {w.dtype}")
    _need(w, "w", w.dtype, 2)
    N, K = w.shape
    _check_k(K)
    _device_check(w.device)
    q4 = torch.empty((N, K // 2), dtype=torch.uint8, device=w.device)
    s4 = torch.empty((K // INT4_GROUP, N), dtype=torch.bfloat16, device=w.device)
    dt = DTYPE_BF16 if w.dtype == torch.bfloat16 else DTYPE_F32
    _check(load().k2q_quant_weight_i4(_ptr(w), dt, N, K, _ptr(q4), _ptr(s4), _stream(w.device)),
           "k2q_quant_weight_i4")
    return q4, s4


# ----------------------------------------------------------------------------------------------------------
# LoRA down-projection
# ----------------------------------------------------------------------------------------------------------
def lora_down(x: torch.Tensor, A: torch.Tensor) -> torch.Tensor:
    """``u = x.f32 @ A^T`` (M, r) f32; ``x`` (M,K) bf16, ``A`` (r,K) f32."""
    _need(x, "x", torch.bfloat16, 2)
    dev = x.device
    _need(A, "lora_A", torch.float32, 2, dev)
    M, K = x.shape
    r = A.shape[0]
    if A.shape[1] != K:
        raise ValueError(f"lora_A has in_features {A.shape[1]}, x has {K}")
    _check_rank(r)
    _device_check(dev)
    lib = load()
    nws = lib.k2q_lora_down_ws_bytes(M, K, r)
    ws = torch.empty((nws // 4,), dtype=torch.float32, device=dev) if nws else None
    u = torch.empty((M, r), dtype=torch.float32, device=dev)
    _check(lib.k2q_lora_down(_ptr(x), M, K, K, _ptr(A), r, _ptr(ws), nws, _ptr(u), _stream(dev)), "k2q_lora_down")
    return u


def lora_grads(dy, x, u, lora_b, lora_scale: float):
    """LoRA gradients (the autograd of ``lora.py:47-48``): ``g = s dy B`` (M,r), ``dA = g^T x`` (r,K) when
    ``x`` is given, ``dB = s dy^T u`` (N,r) when ``u`` is given; all f32.  ``dy`` (M,N) and ``x`` (M,K) bf16,
    ``u`` (M,r) and ``lora_b`` (N,r) f32.  Returns ``(g, dA | None, dB | None)``."""
    _need(dy, "dy", torch.bfloat16, 2)
    dev = dy.device
    M, N = dy.shape
    _need(lora_b, "lora_B", torch.float32, 2, dev)
    r = lora_b.shape[1]
    if lora_b.shape[0] != N:
        raise ValueError(f"lora_B has {lora_b.shape[0]} rows, dy has {N} columns")
    _check_rank(r)
    if N % HADAMARD_BLOCK:
        raise ValueError(f"out_features={N} must be a multiple of {HADAMARD_BLOCK} for the LoRA gradients")
    K = HADAMARD_BLOCK
    if x is not None:
        _need(x, "x", torch.bfloat16, 2, dev)
        if x.shape[0] != M:
            raise ValueError("x rows != dy rows")
        K = x.shape[1]
        _check_k(K)
    if u is not None:
        _need(u, "u", torch.float32, 2, dev)
        if u.shape != (M, r):
            raise ValueError(f"u must be {(M, r)}, got {tuple(u.shape)}")
    _device_check(dev)
    lib = load()
    nws = lib.k2q_lora_grads_ws_bytes(M, N, K, r)
    ws = torch.empty((nws,), dtype=torch.uint8, device=dev)
    g = torch.empty((M, r), dtype=torch.float32, device=dev)
    dA = torch.empty((r, K), dtype=torch.float32, device=dev) if x is not None else None
    dB = torch.empty((N, r), dtype=torch.float32, device=dev) if u is not None else None
    _check(lib.k2q_lora_grads(_ptr(dy), _ptr(x), _ptr(u), _ptr(lora_b), r, float(lora_scale), M, N, K, _ptr(g),
                              _ptr(dA), _ptr(dB), _ptr(ws), nws, _stream(dev)), "k2q_lora_grads")
    return g, dA, dB


LORA_GROUP_MAX = 8     # members per k2q_lora_grads_grouped call


def lora_grads_grouped(dys, x, u, lora_bs, scales, want_db=None):
    """LoRA gradients of linears that read one input (``k2q_lora_grads_grouped``; the autograd of ``lora.py:47-48``
    for every member of a grouped node).  Member i: output gradient ``dys[i]`` (M,N_i) bf16, ``lora_bs[i]``
    (N_i,r) f32 (one rank r <= 128 for all), scale ``scales[i]``.  ``x`` (M,K) bf16 or None (no dA); ``u`` (M, n r)
    f32, the grouped forward's stacked factors (needed when any dB is wanted).  Returns ``(g, dA | None, dBs)``:
    ``g`` (M, n r) f32 with member i's ``s_i dy_i B_i`` in columns ``[i r, (i+1) r)``; ``dA`` (n r, K) f32, member
    i's rows ``[i r, (i+1) r)``; ``dBs[i]`` (N_i, r) f32 where ``want_db[i]`` (default: every member), else None."""
    n = len(dys)
    if n < 1 or n > LORA_GROUP_MAX or len(lora_bs) != n or len(scales) != n:
        raise ValueError(f"lora_grads_grouped takes 1..{LORA_GROUP_MAX} members with one B and scale each")
    want_db = [True] * n if want_db is None else list(want_db)
    dev = dys[0].device
    M = dys[0].shape[0]
    r = lora_bs[0].shape[1]
    _check_rank(r)
    if r > 128:
        raise ValueError(f"lora_grads_grouped: rank {r} above 128 (use lora_grads per member)")
    arr = (LoraMember * n)()
    dBs = []
    for i, (dy, B) in enumerate(zip(dys, lora_bs)):
        if dy.dtype != torch.bfloat16 or dy.dim() != 2 or dy.device != dev or dy.shape[0] != M or dy.stride(1) != 1 \
                or dy.stride(0) % 8 or dy.data_ptr() % 16:
            raise ValueError(f"dy[{i}] must be ({M}, N) bf16 on {dev} with unit column stride and 16-byte rows")
        N = dy.shape[1]
        if N % HADAMARD_BLOCK:
            raise ValueError(f"member {i}: out_features={N} must be a multiple of {HADAMARD_BLOCK}")
        _need(B, f"lora_B[{i}]", torch.float32, 2, dev)
        if B.shape != (N, r):
            raise ValueError(f"member {i}: lora_B must be {(N, r)}, got {tuple(B.shape)}")
        dB = torch.empty((N, r), dtype=torch.float32, device=dev) if want_db[i] else None
        dBs.append(dB)
        arr[i] = LoraMember(dy.data_ptr(), dy.stride(0), N, B.data_ptr(), float(scales[i]), _ptr(dB))
    K = HADAMARD_BLOCK
    if x is not None:
        _need(x, "x", torch.bfloat16, 2, dev)
        if x.shape[0] != M:
            raise ValueError("x rows != dy rows")
        K = x.shape[1]
        _check_k(K)
    if any(want_db):
        _need(u, "u", torch.float32, 2, dev)
        if u.shape != (M, n * r):
            raise ValueError(f"u must be {(M, n * r)} (the stacked factors), got {tuple(u.shape)}")
    _device_check(dev)
    lib = load()
    nws = lib.k2q_lora_grads_grouped_ws_bytes(ctypes.addressof(arr), n, M, K, r)
    ws = torch.empty((nws,), dtype=torch.uint8, device=dev)
    g = torch.empty((M, n * r), dtype=torch.float32, device=dev)
    dA = torch.empty((n * r, K), dtype=torch.float32, device=dev) if x is not None else None
    _check(lib.k2q_lora_grads_grouped(ctypes.addressof(arr), n, _ptr(x), _ptr(u) if any(want_db) else None, r, M, K,
                                      g.data_ptr(), _ptr(dA), ws.data_ptr(), nws, _stream(dev)),
           "k2q_lora_grads_grouped")
    return g, dA, dBs


SCRATCH_BYTES = 64 << 20     # K2Q_SCRATCH_BYTES: the library's own device scratch per GPU


def lora_grads_noalloc(dy, x, u, lora_b, lora_scale: float, g, dA=None, dB=None) -> None:
    """:func:`lora_grads` into caller-provided outputs with nothing allocated, by the library or here: the
    workspace is the library's device scratch (``SCRATCH_BYTES`` per GPU, shared by every call on that GPU, so
    calls that overlap on one GPU race).  ``g`` (M,r), ``dA`` (r,K) and ``dB`` (N,r) f32 contiguous, the last two
    optional (with ``x`` / ``u``).  Raises before any launch when the shape needs more scratch than that."""
    _need(dy, "dy", torch.bfloat16, 2)
    dev = dy.device
    M, N = dy.shape
    _need(lora_b, "lora_B", torch.float32, 2, dev)
    r = lora_b.shape[1]
    if lora_b.shape[0] != N:
        raise ValueError(f"lora_B has {lora_b.shape[0]} rows, dy has {N} columns")
    _check_rank(r)
    if N % HADAMARD_BLOCK:
        raise ValueError(f"out_features={N} must be a multiple of {HADAMARD_BLOCK} for the LoRA gradients")
    _need(g, "g", torch.float32, 2, dev)
    if g.shape != (M, r):
        raise ValueError(f"g must be {(M, r)}, got {tuple(g.shape)}")
    K = HADAMARD_BLOCK
    if (x is None) != (dA is None):
        raise ValueError("x and dA go together")
    if (u is None) != (dB is None):
        raise ValueError("u and dB go together")
    if x is not None:
        _need(x, "x", torch.bfloat16, 2, dev)
        K = x.shape[1]
        _check_k(K)
        _need(dA, "dA", torch.float32, 2, dev)
        if x.shape[0] != M or dA.shape != (r, K):
            raise ValueError("x / dA shapes do not match dy and the rank")
    if u is not None:
        _need(u, "u", torch.float32, 2, dev)
        _need(dB, "dB", torch.float32, 2, dev)
        if u.shape != (M, r) or dB.shape != (N, r):
            raise ValueError("u / dB shapes do not match dy and the rank")
    need = load().k2q_lora_grads_ws_bytes(M, N, K, r)
    if need > SCRATCH_BYTES:
        raise ValueError(f"the LoRA gradients of M={M}, N={N}, K={K}, r={r} need {need} bytes of workspace, more than "
                         f"the library's {SCRATCH_BYTES}-byte scratch: use lora_grads")
    _device_check(dev)
    _check(load().k2q_lora_grads_noalloc(_ptr(dy), _ptr(x), _ptr(u), _ptr(lora_b), r, float(lora_scale), M, N, K,
                                         _ptr(g), _ptr(dA), _ptr(dB), _stream(dev)), "k2q_lora_grads_noalloc")


# ----------------------------------------------------------------------------------------------------------
# (2)+(3) GEMMs with fused epilogue
# ----------------------------------------------------------------------------------------------------------
def _gemm_common(qx, sx, N, bias, u, lora_b):
    _need(qx, "q_x", torch.int8, 2)
    dev = qx.device
    M, K = qx.shape
    _need(sx, "s_x", torch.float32, 1, dev)
    if sx.shape[0] != M:
        raise ValueError("s_x length != rows of q_x")
    if N % 4:
        raise ValueError(f"out_features={N} must be a multiple of 4")
    if bias is not None:
        _need(bias, "bias", torch.float32, 1, dev)
        if bias.shape[0] != N:
            raise ValueError("bias length != out_features")
    r = 0
    if u is not None:
        _need(u, "u", torch.float32, 2, dev)
        if lora_b is None:
            raise ValueError("u given without lora_B")
        _need(lora_b, "lora_B", torch.float32, 2, dev)
        r = u.shape[1]
        if u.shape[0] != M or lora_b.shape != (N, r):
            raise ValueError(f"LoRA shapes u{tuple(u.shape)} lora_B{tuple(lora_b.shape)} do not match M={M}, N={N}")
        _check_rank(r)
    return dev, M, K, r


TILES = {"auto": -1, "256x256": 0, "256x320": 1, "192x256": 2, "128x128": 3}   # K2Q_TILE_*
_TILE_NAMES = {v: k for k, v in TILES.items()} | {4: "gemv"}


def gemm_w8a8_plan(M: int, N: int, K: int, cus: int = 256, grouped: bool = False) -> tuple[str, int]:
    """The schedule ``k2q_gemm_w8a8`` (``grouped``: ``k2q_gemm_w8a8_grouped``, N = the segments' total) takes for
    an M x N x K problem on a GPU with ``cus`` compute units: (tile shape or "gemv", K-pieces of the last round
    of 256x256 tiles).  Host only."""
    pieces = _int(0)
    rc = load().k2q_gemm_w8a8_plan(M, N, K, cus, int(grouped), ctypes.byref(pieces))
    if rc < 0:
        _check(rc, "k2q_gemm_w8a8_plan")
    return _TILE_NAMES[rc], pieces.value


def gemm_w8a8(qx, sx, qw, sw, bias=None, u=None, lora_b=None, lora_scale: float = 1.0, *,
              split: bool = True, tile: str = "auto") -> torch.Tensor:
    """``y = bf16(2^-7 s_x s_w acc + bias + lora_scale u lora_B^T)`` (M,N).  ``split=False`` runs every tile
    over the full K (the result is the same; the split schedule only fills the GPU's last round); ``tile`` forces
    an output tile shape (``TILES``; the result is the same)."""
    _need(qw, "q_w", torch.int8, 2)
    N = qw.shape[0]
    dev, M, K, r = _gemm_common(qx, sx, N, bias, u, lora_b)
    if qw.shape[1] != K or qw.device != dev:
        raise ValueError("q_w shape/device mismatch")
    _need(sw, "s_w", torch.float32, 1, dev)
    if sw.shape[0] != N:
        raise ValueError("s_w length != out_features")
    _check_k(K)
    _device_check(dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    lib = load()
    ws, nws = _workspace(lib.k2q_gemm_w8a8_ws_bytes(M, N, K) if split else 0, dev)
    _check(lib.k2q_gemm_w8a8_tile(_ptr(qx), _ptr(sx), _ptr(qw), _ptr(sw), _ptr(bias), _ptr(u), _ptr(lora_b), r,
                                  float(lora_scale), M, N, K, _ptr(y), _ptr(ws), nws, TILES[tile], _stream(dev)),
           "k2q_gemm_w8a8")
    return y


WMODE_W8, WMODE_W4 = 0, 1


# workspace bytes of k2q_linear_fwd per (wmode, M, N, K, r), as (any call, a call with u given and codes not
# given): pure functions of the shape and the device's CU count (one GPU model per process here), asked once per shape
_FWD_WS: dict = {}


def linear_fwd_fuses_down(M: int, K: int, r: int) -> bool:
    """Whether :func:`linear_fwd` (codes not given, rank ``r`` factors) takes u from the rotate/quant pass."""
    return bool(load().k2q_linear_fwd_fuses_down(M, K, r))


def linear_fwd(x2, qx, sx, codes_ready: bool, A, B, lora_scale: float, qw, sw, bias, w4: bool,
               need_u: bool = True):
    """One quantized linear + LoRA forward in one library call (``k2q_linear_fwd``): rotate/quant of ``x2`` into
    ``qx`` / ``sx`` (unless ``codes_ready``), ``u = x2 A^T`` (when ``A``), the GEMM with the fused epilogue.
    Returns ``(y, u | None)``; ``need_u=False`` (inference: no backward will read the factors) lets the library
    keep u internal (for M > 8 the GEMM epilogue then adds the down-projection's slices itself) and returns
    ``(y, None)``.  The module's per-call entry: the weights and factors come from the module (their shapes
    fixed when it was built), so only the relations a foreign call needs are checked here, cheaply; the library
    checks pointers and alignment again.  ``x2`` (M,K) bf16 rows of stride ``x2.stride(0)``."""
    M, K = x2.shape
    N = qw.shape[0]
    dev = x2.device
    if x2.dtype != torch.bfloat16 or x2.stride(1) != 1 or qw.device != dev or qx.shape != (M, K) or sx.shape != (M,):
        raise ValueError("linear_fwd: x / code buffers do not match the layer")
    r = 0
    if A is not None:
        r = A.shape[0]
        if A.shape != (r, K) or B.shape != (N, r) or A.dtype != torch.float32 or B.dtype != torch.float32 \
                or A.device != dev or not (A.is_contiguous() and B.is_contiguous()):
            raise ValueError("linear_fwd: LoRA factors do not match the layer")
        _check_rank(r)
    if bias is not None and (bias.shape != (N,) or bias.dtype != torch.float32 or bias.device != dev):
        raise ValueError("linear_fwd: bias does not match the layer")
    _device_check(dev)
    lib = load()
    wmode = WMODE_W4 if w4 else WMODE_W8
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    u = torch.empty((M, r), dtype=torch.float32, device=dev) if r and (need_u or M <= 8) else None
    key = (wmode, M, N, K, r)
    plan = _FWD_WS.get(key)
    if plan is None:
        nws = lib.k2q_linear_fwd_ws_bytes(wmode, M, N, K, r)
        # with u given, a call that takes u from the rotate/quant pass and whose GEMM does not split uses no ws
        unused = r and M > 8 and lib.k2q_linear_fwd_fuses_down(M, K, r) and \
            (w4 or lib.k2q_gemm_w8a8_ws_bytes(M, N, K) == 0)
        plan = _FWD_WS.setdefault(key, (nws, 0 if unused else nws))
    nws = plan[1] if u is not None and not codes_ready else plan[0]
    ws = torch.empty((nws,), dtype=torch.uint8, device=dev) if nws > 0 else None
    _check(lib.k2q_linear_fwd(x2.data_ptr(), x2.stride(0), M, K, qx.data_ptr(), sx.data_ptr(), int(codes_ready),
                              _ptr(A), _ptr(B), r, float(lora_scale), _ptr(u), wmode, qw.data_ptr(), sw.data_ptr(),
                              _ptr(bias), N, y.data_ptr(), _ptr(ws), nws, _stream(dev)), "k2q_linear_fwd")
    return y, (u if need_u else None)


def gemm_w8a8_grouped(qx, sx, segments, u=None):
    """Several W8A8 linears that read the same codes in one launch.  ``segments``: sequence of
    ``(q_w, s_w, bias, lora_b, u_col, lora_scale)`` (bias, lora_b nullable; a segment with ``lora_b`` uses
    columns ``u_col .. u_col + r`` of ``u``, (M, ldu) f32 with r = ``lora_b.shape[1]``).  Returns one bf16
    (M, N_i) output per segment, each equal to :func:`gemm_w8a8` of that segment."""
    _need(qx, "q_x", torch.int8, 2)
    dev = qx.device
    M, K = qx.shape
    _need(sx, "s_x", torch.float32, 1, dev)
    if sx.shape[0] != M:
        raise ValueError("s_x length != rows of q_x")
    _check_k(K)
    if not 1 <= len(segments) <= GROUP_MAX:
        raise ValueError(f"a grouped launch takes 1..{GROUP_MAX} segments, got {len(segments)}")
    if M <= 8:
        raise ValueError("grouped launches need M > 8 (skinny M runs the per-linear GEMV)")
    r, ldu = 0, 0
    if u is not None:
        if u.dtype != torch.float32 or u.dim() != 2 or u.shape[0] != M or u.stride(1) != 1 or u.data_ptr() % 16 \
                or u.stride(0) % 4 or u.device != dev:
            raise ValueError("u must be (M, ldu) f32 with contiguous 16-byte aligned rows")
        ldu = u.stride(0)
    arr = (W8A8Segment * len(segments))()
    outs, keep = [], []
    for i, (qw, sw, bias, lb, u_col, scale) in enumerate(segments):
        _need(qw, f"q_w[{i}]", torch.int8, 2, dev)
        N = qw.shape[0]
        if qw.shape[1] != K or N % GROUP_ALIGN:
            raise ValueError(f"segment {i}: q_w {tuple(qw.shape)} needs K={K} and N a multiple of {GROUP_ALIGN}")
        _need(sw, f"s_w[{i}]", torch.float32, 1, dev)
        if sw.shape[0] != N:
            raise ValueError(f"segment {i}: s_w length != N")
        if bias is not None:
            _need(bias, f"bias[{i}]", torch.float32, 1, dev)
            if bias.shape[0] != N:
                raise ValueError(f"segment {i}: bias length != N")
        if lb is not None:
            _need(lb, f"lora_b[{i}]", torch.float32, 2, dev)
            if u is None or lb.shape[0] != N:
                raise ValueError(f"segment {i}: lora_b needs u and N rows")
            if r and lb.shape[1] != r:
                raise ValueError("every segment's adapter must have the same rank")
            r = lb.shape[1]
            _check_rank(r)
            if u_col < 0 or u_col + r > ldu or u_col % 4:
                raise ValueError(f"segment {i}: factor columns {u_col}..{u_col + r} outside u")
        y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
        outs.append(y)
        keep.extend([qw, sw, bias, lb])
        arr[i] = W8A8Segment(_ptr(qw), _ptr(sw), _ptr(bias), _ptr(lb), _ptr(y), N, int(u_col or 0), float(scale))
    _device_check(dev)
    _check(load().k2q_gemm_w8a8_grouped(_ptr(qx), _ptr(sx), M, K, ctypes.cast(arr, ctypes.c_void_p), len(segments),
                                        _ptr(u), r, ldu, None, 0, _stream(dev)), "k2q_gemm_w8a8_grouped")
    return outs


def gemm_w4a8(qx, sx, q4, s4, bias=None, u=None, lora_b=None, lora_scale: float = 1.0) -> torch.Tensor:
    """W4A8 variant of :func:`gemm_w8a8` (packed int4 codes, group-major bf16 group scales)."""
    _need(q4, "q_w4", torch.uint8, 2)
    N = q4.shape[0]
    dev, M, K, r = _gemm_common(qx, sx, N, bias, u, lora_b)
    if q4.shape[1] * 2 != K or q4.device != dev:
        raise ValueError("q_w4 shape/device mismatch")
    _need(s4, "s_w4", torch.bfloat16, 2, dev)
    if s4.shape != (K // INT4_GROUP, N):
        raise ValueError(f"s_w4 must be (K/64, N) = {(K // INT4_GROUP, N)}, got {tuple(s4.shape)}")
    _check_k(K)
    _device_check(dev)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    _check(load().k2q_gemm_w4a8(_ptr(qx), _ptr(sx), _ptr(q4), _ptr(s4), _ptr(bias), _ptr(u), _ptr(lora_b), r,
                                float(lora_scale), M, N, K, _ptr(y), _stream(dev)), "k2q_gemm_w4a8")
    return y


def gemm_w8a8_acc(qx, qw, *, split: bool = True, tile: str = "auto") -> torch.Tensor:
    """Debug: raw int32 accumulators ``qx @ qw^T`` (M,N), optionally with a forced tile shape (``TILES``)."""
    _need(qx, "q_x", torch.int8, 2)
    dev = qx.device
    _need(qw, "q_w", torch.int8, 2, dev)
    M, K = qx.shape
    N = qw.shape[0]
    if qw.shape[1] != K or N % 4:
        raise ValueError("shape mismatch")
    _check_k(K)
    _device_check(dev)
    acc = torch.empty((M, N), dtype=torch.int32, device=dev)
    lib = load()
    ws, nws = _workspace(lib.k2q_gemm_w8a8_ws_bytes(M, N, K) if split else 0, dev)
    _check(lib.k2q_gemm_w8a8_acc(_ptr(qx), _ptr(qw), M, N, K, _ptr(acc), _ptr(ws), nws, TILES[tile], _stream(dev)),
           "k2q_gemm_w8a8_acc")
    return acc


def gemm_w4a8_f32(qx, q4, s4) -> torch.Tensor:
    """Debug: ``sum_g s4[g,n] * acc_g[m,n]`` in f32 (M,N), no s_x / 2^-7 / bias / LoRA."""
    _need(qx, "q_x", torch.int8, 2)
    dev = qx.device
    _need(q4, "q_w4", torch.uint8, 2, dev)
    _need(s4, "s_w4", torch.bfloat16, 2, dev)
    M, K = qx.shape
    N = q4.shape[0]
    if q4.shape[1] * 2 != K or s4.shape != (K // INT4_GROUP, N) or N % 4:
        raise ValueError("shape mismatch")
    _check_k(K)
    _device_check(dev)
    out = torch.empty((M, N), dtype=torch.float32, device=dev)
    _check(load().k2q_gemm_w4a8_f32(_ptr(qx), _ptr(q4), _ptr(s4), M, N, K, _ptr(out), _stream(dev)),
           "k2q_gemm_w4a8_f32")
    return out


# ----------------------------------------------------------------------------------------------------------
# (4) input gradient
# ----------------------------------------------------------------------------------------------------------
def dx_weight(qw, sw, *, w4: bool = False) -> torch.Tensor:
    """The effective weight of the straight-through forward, ``bf16(2^-7 W_hat R)^T`` (K,N): what
    :func:`gemm_dx` builds on every call unless it is handed one (``wt=``)."""
    dev = qw.device
    if w4:
        _need(qw, "q_w4", torch.uint8, 2, dev)
        N, K = qw.shape[0], qw.shape[1] * 2
        _need(sw, "s_w4", torch.bfloat16, 2, dev)
        if sw.shape != (K // INT4_GROUP, N):
            raise ValueError("s_w4 shape mismatch")
    else:
        _need(qw, "q_w", torch.int8, 2, dev)
        N, K = qw.shape
        _need(sw, "s_w", torch.float32, 1, dev)
        if sw.shape[0] != N:
            raise ValueError("s_w length mismatch")
    _check_k(K)
    if N % 64:
        raise ValueError(f"out_features={N} must be a multiple of 64 for the input-gradient GEMM")
    _device_check(dev)
    wt = torch.empty((K, N), dtype=torch.bfloat16, device=dev)
    _check(load().k2q_dx_prep_eff(None if w4 else _ptr(qw), None if w4 else _ptr(sw), _ptr(qw) if w4 else None,
                                  _ptr(sw) if w4 else None, N, K, _ptr(wt), _stream(dev)), "k2q_dx_prep_eff")
    return wt


def gemm_dx(dy, qw, sw, *, w4: bool = False, g=None, lora_a=None, split: bool = True,
            fold_rotation: bool = True, wt=None) -> torch.Tensor:
    """``dx = bf16(2^-7 (dy W_hat) R + g lora_A)`` (M,K); ``dy`` (M,N) bf16, ``g`` (M,r) f32 already
    scaled (``lora_scale * dy @ lora_B``), ``lora_a`` (r,K) f32.  ``fold_rotation`` (default) builds the
    effective weight ``bf16(2^-7 W_hat R)^T`` (or takes it as ``wt``, from :func:`dx_weight`) and runs the
    plain GEMM; otherwise ``bf16(W_hat)^T`` and the GEMM with the inverse rotation in its epilogue."""
    _need(dy, "dy", torch.bfloat16, 2)
    dev = dy.device
    M, N = dy.shape
    if w4:
        _need(qw, "q_w4", torch.uint8, 2, dev)
        K = qw.shape[1] * 2
        _need(sw, "s_w4", torch.bfloat16, 2, dev)
        if sw.shape != (K // INT4_GROUP, N):
            raise ValueError("s_w4 shape mismatch")
    else:
        _need(qw, "q_w", torch.int8, 2, dev)
        K = qw.shape[1]
        _need(sw, "s_w", torch.float32, 1, dev)
        if sw.shape[0] != N:
            raise ValueError("s_w length mismatch")
    if qw.shape[0] != N:
        raise ValueError(f"dy has {N} columns, weight has {qw.shape[0]} rows")
    _check_k(K)
    if N % 64:
        raise ValueError(f"out_features={N} must be a multiple of 64 for the input-gradient GEMM")
    r = 0
    if g is not None:
        _need(g, "g", torch.float32, 2, dev)
        _need(lora_a, "lora_A", torch.float32, 2, dev)
        r = g.shape[1]
        if g.shape[0] != M or lora_a.shape != (r, K):
            raise ValueError("LoRA gradient shapes mismatch")
        _check_rank(r)
    _device_check(dev)
    st = _stream(dev)
    lib = load()
    if wt is not None:
        if not fold_rotation:
            raise ValueError("a prebuilt effective weight needs fold_rotation=True")
        _need(wt, "wt", torch.bfloat16, 2, dev)
        if wt.shape != (K, N):
            raise ValueError(f"wt must be (K, N) = {(K, N)}, got {tuple(wt.shape)}")
    else:
        wt = torch.empty((K, N), dtype=torch.bfloat16, device=dev)
        prep = lib.k2q_dx_prep_eff if fold_rotation else lib.k2q_dx_prep
        _check(prep(None if w4 else _ptr(qw), None if w4 else _ptr(sw), _ptr(qw) if w4 else None,
                    _ptr(sw) if w4 else None, N, K, _ptr(wt), st), "k2q_dx_prep")
    dx = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    ws, nws = _workspace(lib.k2q_gemm_dx_ws_bytes(M, N, K) if split else 0, dev)
    gemm = lib.k2q_gemm_dx_lin if fold_rotation else lib.k2q_gemm_dx
    _check(gemm(_ptr(dy), _ptr(wt), M, N, K, _ptr(g), _ptr(lora_a) if r else None, r, _ptr(dx),
                _ptr(ws), nws, st), "k2q_gemm_dx")
    return dx


def gemm_dx_grouped(segments, g=None, lora_a=None) -> torch.Tensor:
    """Input gradient of linears that share their input, in one GEMM: ``dx = bf16(sum_i dy_i wt_i^T + g A)``.
    ``segments``: ``(dy_i, wt_i)`` with ``dy_i`` (M, N_i) bf16 (row stride a multiple of 8, unit column
    stride) and ``wt_i`` (K, N_i) bf16 from :func:`dx_weight`; ``g`` (M, r) f32 (row stride a multiple of 4)
    and ``lora_a`` (r, K) f32 the members' LoRA terms stacked along the rank, or None."""
    if not 1 <= len(segments) <= GROUP_MAX:
        raise ValueError(f"a grouped input gradient takes 1..{GROUP_MAX} segments, got {len(segments)}")
    dy0, wt0 = segments[0]
    if not isinstance(dy0, torch.Tensor) or dy0.dim() != 2 or not isinstance(wt0, torch.Tensor) or wt0.dim() != 2:
        raise ValueError("segments must be (dy (M, N_i), wt (K, N_i)) tensor pairs")
    dev = dy0.device
    M = dy0.shape[0]
    K = wt0.shape[0]
    arr = (DxSegment * len(segments))()
    for i, (dy, wt) in enumerate(segments):
        if dy.dtype != torch.bfloat16 or dy.dim() != 2 or dy.device != dev or dy.stride(1) != 1 \
                or dy.stride(0) % 8 or dy.data_ptr() % 16:
            raise ValueError(f"dy[{i}] must be (M, N) bf16 on {dev} with unit column stride and 16-byte rows")
        _need(wt, f"wt[{i}]", torch.bfloat16, 2, dev)
        N = dy.shape[1]
        if dy.shape[0] != M or wt.shape != (K, N):
            raise ValueError(f"segment {i}: dy {tuple(dy.shape)} / wt {tuple(wt.shape)} do not match M={M}, K={K}")
        if N % 64:
            raise ValueError(f"segment {i}: out_features={N} must be a multiple of 64")
        arr[i] = DxSegment(dy.data_ptr(), dy.stride(0), wt.data_ptr(), N)
    _check_k(K)
    r, ldg = 0, 0
    if g is not None:
        if g.dtype != torch.float32 or g.dim() != 2 or g.device != dev or g.shape[0] != M or g.stride(1) != 1 \
                or g.stride(0) % 4 or g.data_ptr() % 16:
            raise ValueError("g must be (M, r) f32 with unit column stride and 16-byte rows")
        _need(lora_a, "lora_A", torch.float32, 2, dev)
        r, ldg = g.shape[1], g.stride(0)
        if lora_a.shape != (r, K):
            raise ValueError("lora_A must be (r, K) for g of r columns")
        _check_rank(r)
    _device_check(dev)
    dx = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    _check(load().k2q_gemm_dx_grouped(ctypes.addressof(arr), len(segments), M, K, _ptr(g), ldg,
                                      _ptr(lora_a) if r else None, r, _ptr(dx), _stream(dev)),
           "k2q_gemm_dx_grouped")
    return dx


# ----------------------------------------------------------------------------------------------------------
# fp8-e4m3 weight-only base (the reference's Fp8Linear, quantize.py:23-51)
# ----------------------------------------------------------------------------------------------------------
def quant_weight_fp8(w: torch.Tensor):
    """``Fp8Linear.__init__`` (``quantize.py:34-37``) on the GPU: ``(q float8_e4m3fn (N,K), scale bf16 (N,1))``."""
    if w.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError(f"w must be bf16 or f32, got {w.dtype}")
    _need(w, "w", w.dtype, 2)
    N, K = w.shape
    _device_check(w.device)
    q = torch.empty((N, K), dtype=torch.uint8, device=w.device)
    s = torch.empty((N, 1), dtype=torch.bfloat16, device=w.device)
    dt = DTYPE_BF16 if w.dtype == torch.bfloat16 else DTYPE_F32
    _check(load().k2q_quant_weight_fp8(_ptr(w), dt, N, K, _ptr(q), _ptr(s), _stream(w.device)), "k2q_quant_weight_fp8")
    return q.view(torch.float8_e4m3fn), s


def _fp8_operands(q, s):
    if q.dtype != torch.float8_e4m3fn:
        raise ValueError(f"fp8 weight must be float8_e4m3fn, got {q.dtype}")
    _need(q, "weight_fp8", q.dtype, 2)
    N, K = q.shape
    if s.dtype != torch.bfloat16 or s.numel() != N or not s.is_contiguous() or s.device != q.device:
        raise ValueError("scale must be a contiguous bf16 tensor with one value per output row")
    if K % 64:
        raise ValueError(f"in_features={K} must be a multiple of 64 for the fp8 base")
    return N, K


def dequant_fp8(q, s, transpose: bool = False) -> torch.Tensor:
    """``bf16(q * s)`` per element (``quantize.py:49``): (N,K), or (K,N) with ``transpose``."""
    N, K = _fp8_operands(q, s)
    if transpose and N % 8:
        raise ValueError("the transposed dequantization needs out_features % 8 == 0")
    _device_check(q.device)
    out = torch.empty((K, N) if transpose else (N, K), dtype=torch.bfloat16, device=q.device)
    _check(load().k2q_dequant_fp8(_ptr(q), _ptr(s), N, K, int(transpose), _ptr(out), _stream(q.device)),
           "k2q_dequant_fp8")
    return out


def gemm_bf16(x, w, bias=None, u=None, lora_b=None, lora_scale: float = 1.0, *, split: bool = True) -> torch.Tensor:
    """``y = bf16(x w^T + bias) + LoRA`` (``quantize.py:51`` + ``lora.py:47-48``); x (M,K), w (N,K) bf16."""
    _need(x, "x", torch.bfloat16, 2)
    dev = x.device
    _need(w, "w", torch.bfloat16, 2, dev)
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K or K % 64 or N % 4:
        raise ValueError(f"shapes x{tuple(x.shape)} w{tuple(w.shape)}: need matching K % 64 == 0 and N % 4 == 0")
    r = 0
    if bias is not None:
        _need(bias, "bias", torch.float32, 1, dev)
        if bias.shape[0] != N:
            raise ValueError("bias length != out_features")
    if u is not None:
        _need(u, "u", torch.float32, 2, dev)
        _need(lora_b, "lora_B", torch.float32, 2, dev)
        r = u.shape[1]
        if u.shape[0] != M or lora_b.shape != (N, r):
            raise ValueError("LoRA shapes do not match")
        _check_rank(r)
    _device_check(dev)
    lib = load()
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    ws, nws = _workspace(lib.k2q_gemm_bf16_ws_bytes(M, N, K) if split else 0, dev)
    _check(lib.k2q_gemm_bf16(_ptr(x), _ptr(w), _ptr(bias), _ptr(u), _ptr(lora_b), r, float(lora_scale), M, N, K,
                             _ptr(y), _ptr(ws), nws, _stream(dev)), "k2q_gemm_bf16")
    return y


def gemm_dx_fp8(dy, q, s, *, g=None, lora_a=None, split: bool = True) -> torch.Tensor:
    """``dx = bf16(dy W_deq + g lora_A)`` for the fp8 base (``W_deq = bf16(q s)``)."""
    _need(dy, "dy", torch.bfloat16, 2)
    dev = dy.device
    N, K = _fp8_operands(q, s)
    M = dy.shape[0]
    if dy.shape[1] != N or N % 64:
        raise ValueError(f"dy has {dy.shape[1]} columns; need out_features = {N} and a multiple of 64")
    r = 0
    if g is not None:
        _need(g, "g", torch.float32, 2, dev)
        _need(lora_a, "lora_A", torch.float32, 2, dev)
        r = g.shape[1]
        if g.shape[0] != M or lora_a.shape != (r, K):
            raise ValueError("LoRA gradient shapes mismatch")
        _check_rank(r)
    _device_check(dev)
    lib = load()
    st = _stream(dev)
    wt = dequant_fp8(q, s, transpose=True)
    dx = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    ws, nws = _workspace(lib.k2q_gemm_dx_ws_bytes(M, N, K) if split else 0, dev)
    _check(lib.k2q_gemm_dx_lin(_ptr(dy), _ptr(wt), M, N, K, _ptr(g), _ptr(lora_a) if r else None, r, _ptr(dx),
                               _ptr(ws), nws, st), "k2q_gemm_dx_lin")
    return dx
