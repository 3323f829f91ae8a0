"""Builds the gfx950 HIP library ``rusty_amd/librusty_hip.so``.

Each ``csrc/*.hip`` translation unit is compiled to an object in parallel with
``hipcc --offload-arch=gfx950``, then linked into one shared library that
exports the C ABI of ``include/rusty_hip.h``.  Packed-FP32 instruction
selection is disabled for device code (``-packed-fp32-ops``): the kernels
are written against scalar f32 arithmetic.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
OBJ_DIR = PKG / "_build"
LIB = PKG / "librusty_hip.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


# Per-file flags.  gemm.hip flushes f32 denormals: that lets the compiler
# select v_fma_mix{lo,hi}_f16 for the affine weight expansion (fma of an fp16
# and two f32 operands, rounded once to fp16).  The file's other f32 VALU math,
# all under the same flag:
#  * epilogues: per-feature scale and per-token power-of-two factor times O(1)
#    sums; the RoPE rotation of q/k (cos, sin in [-1, 1]); silu(g) * u, whose
#    results below 2^-126 would round to zero in the fp16 h anyway; the
#    matrix-core input gradient's rows (backward.hip), sums of values scaled
#    to [2^14, 2^15) times their row's 2^e: only results below 2^-126, far
#    under the row's own resolution, flush;
#  * k_affine_prep: b - 1024 s per group (a group whose s or b is an f32
#    denormal dequantizes to 0 instead of ~1e-38);
#  * k_cast_f16_rows: the row maximum and the x * 2^-e scaling.  An f32
#    denormal element reads as 0; where the row maximum is normal such an
#    element is below the fp16 result's resolution (2^-24 of the maximum) in
#    any case, so only rows made entirely of denormals change (to zero).
FILE_FLAGS = {"gemm.hip": ["-fgpu-flush-denormals-to-zero"]}


def _compile(src: Path, verbose: bool) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
    # The host pass does not know the device-only target feature; that warning is expected.
    noise = ("packed-fp32-ops", "warning: unknown target feature")
    for line in (r.stderr or "").splitlines():
        if line.strip() and not any(n in line for n in noise) and verbose:
            print(line, file=sys.stderr)
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compiles every HIP source and links ``librusty_hip.so``; returns its path."""
    OBJ_DIR.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 16)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
