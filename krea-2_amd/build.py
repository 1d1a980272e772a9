"""Build ``libk2q.so`` (the gfx950 HIP kernels behind the C ABI of ``include/k2q.h``) in-tree.

``python krea-2_amd/build.py`` or ``build()`` from Python.  hipcc cross-compiles for gfx950 without a GPU,
so this runs in the CPU container; the resulting ``.so`` sits next to this file and travels with the tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
LIB = HERE / "libk2q.so"
SOURCES = ("api.hip", "rotquant.hip", "producers.hip", "gemm.hip", "gemv.hip", "lora.hip", "lora_grad.hip", "fp8.hip",
           "linear.hip")
# bench.py's same-run MFMA ceiling: a measurement aid, built into its own library, not into the product's
PROBE_SOURCES = ("probe.hip",)
PROBE_LIB = HERE / "libk2q_probe.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# -ffp-contract=off: the rotation/quantization arithmetic is specified op by op (bit-exact int8 codes);
# deliberate fused multiply-adds are written as __builtin_fmaf.  packed-fp32-ops is disabled on purpose.
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}", "-Wall", "-Wno-unused-function",
]


def _compile(src: Path, obj: Path) -> None:
    cmd = [HIPCC, *CFLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr}")


def _link(objs, lib: Path) -> None:
    tmp = lib.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of {lib.name} failed:\n{r.stderr}")
    os.replace(tmp, lib)


def build(verbose: bool = False) -> Path:
    """Compile every kernel source for gfx950 and link ``libk2q.so`` (and bench.py's ``libk2q_probe.so``).
    Always recompiles."""
    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)
    srcs = SOURCES + PROBE_SOURCES
    objs = {s: objdir / (Path(s).stem + ".o") for s in srcs}
    with cf.ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 1)) as ex:
        list(ex.map(lambda s: _compile(CSRC / s, objs[s]), srcs))
    _link([objs[s] for s in SOURCES], LIB)
    _link([objs[s] for s in PROBE_SOURCES], PROBE_LIB)
    if verbose:
        print(f"built {LIB} ({LIB.stat().st_size} bytes) and {PROBE_LIB.name}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
