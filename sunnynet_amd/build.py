"""Build recipe for the HIP backend library (libsnhip.so, gfx950).

Compiles every ``csrc/*.hip`` (in parallel, one hipcc per translation unit)
and links them into an in-tree shared library. Runs on a machine without a
GPU (hipcc cross-compiles).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIB = PKG / "libsnhip.so"
ARCH = os.environ.get("SNHIP_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC",
    f"--offload-arch={ARCH}",
    # Packed-FP32 VALU forms are kept out of generated code on this target.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-rdc",
    # No implicit contraction: kernels write fmaf() exactly where the
    # reference fuses, and keep a*b + c as two roundings elsewhere.
    "-ffp-contract=off",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if c and Path(c).exists():
            return c
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def sources() -> list:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False, extra: list | None = None) -> Path:
    """Compile libsnhip.so (always rebuilds): every translation unit in
    parallel into a private object directory, then one link."""
    import concurrent.futures as cf
    import tempfile
    base = [hipcc()] + HIPCC_FLAGS + (extra or []) + [f"-I{INCLUDE}", f"-I{CSRC}"]
    srcs = sources()
    with tempfile.TemporaryDirectory(prefix="snhip_obj_") as od:
        def compile_one(src):
            obj = Path(od) / (src.stem + ".o")
            cmd = base + ["-c", str(src), "-o", str(obj)]
            if verbose:
                print(" ".join(cmd), flush=True)
            r = subprocess.run(cmd, capture_output=True, text=True)
            if r.returncode != 0:
                raise RuntimeError(f"hipcc failed on {src.name} ({r.returncode}):\n{r.stderr[-6000:]}")
            return obj
        jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
        with cf.ThreadPoolExecutor(jobs) as ex:
            objs = list(ex.map(compile_one, srcs))
        tmp = LIB.with_suffix(".so.tmp")
        cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-fno-gpu-rdc"]
        cmd += [str(o) for o in objs] + ["-o", str(tmp)]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc link failed ({r.returncode}):\n{r.stderr[-6000:]}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    p = build(verbose="-v" in sys.argv)
    print(p)
