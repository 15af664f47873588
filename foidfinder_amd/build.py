"""Builds the gfx950 kernel library `libfoidfinder_rocm.so` in-tree with hipcc (no torch involved).

    python -m foidfinder_amd.build           # or: __graft_entry__.build()

Replaces the reference's nvcc JIT / `build-kernels` step (foidfinder/backends/cuda/kernels.py:22-35).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
LIB = PKG / "libfoidfinder_rocm.so"
SOURCES = ["capi.hip", "rotq8.hip", "gemm_s8.hip", "attention.hip", "resample.hip", "pool.hip"]
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Quantization and epilogue arithmetic is specified without fused multiply-add and with IEEE division and sqrt.
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # No packed-fp32 instructions (v_pk_{add,mul,fma}_f32) in any kernel.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = shutil.which("hipcc") or os.path.join(rocm, "bin", "hipcc")
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return path


def build(verbose: bool = False) -> Path:
    """Compiles every source (in parallel) and links the shared library; always rebuilds."""
    obj_dir = PKG / "_build"
    obj_dir.mkdir(exist_ok=True)
    cc = hipcc()

    def compile_one(src: str) -> Path:
        obj = obj_dir / (Path(src).stem + ".o")
        cmd = [cc, *FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr}")
        return obj

    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
