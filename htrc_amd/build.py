"""In-tree build of libhtrc_flat.so with hipcc for gfx950 (no torch C++ involved).

The library is a plain C-ABI shared object (include/htrc_flat.h) loaded with ctypes;
it links the HIP runtime by soname, so inside a process that imported torch first
it binds to torch's own HIP runtime.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
SRC = HERE / "csrc" / "htrc_flat.hip"
LIB = HERE / "libhtrc_flat.so"

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-shared",
    "-fPIC",
    "-ffp-contract=off",                 # no FMA contraction: pack/select are bit-exact restatements
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",   # MFMA results in VGPRs: no accumulator-register copies
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libhtrc_flat.so)")


def build(verbose: bool = False) -> Path:
    """Compile csrc/htrc_flat.hip into htrc_amd/libhtrc_flat.so (always rebuilds)."""
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{ROOT / 'include'}", f"-I{HERE / 'csrc'}", str(SRC), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-4000:]}")
    if verbose:
        print(" ".join(cmd))
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
