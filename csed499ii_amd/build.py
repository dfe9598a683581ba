"""Build ``libmarlin_hip.so`` (the C-ABI library) in-tree with hipcc for gfx950.

    python -m csed499ii_amd.build          # or __graft_entry__.build()

Every HIP source under ``csrc/`` is compiled for ``--offload-arch=gfx950`` only.
Packed-FP32 instruction selection is disabled (``-packed-fp32-ops``): the kernels
use packed FP16 arithmetic, never packed FP32.
"""
from __future__ import annotations

import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libmarlin_hip.so"
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm under /opt/rocm)")


def sources() -> list[pathlib.Path]:
    return sorted(CSRC.glob("*.hip"))


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-command-line-argument",
    ]


def build(verbose: bool = False) -> pathlib.Path:
    """Compile all sources into ``csed499ii_amd/libmarlin_hip.so`` (always rebuilds)."""
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *compile_flags(), "-shared", "-o", str(tmp), *map(str, srcs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 target feature: drop that noise.
    noise = ("packed-fp32-ops", "is not a recognized feature")
    msgs = [ln for ln in (proc.stdout + proc.stderr).splitlines() if not any(n in ln for n in noise)]
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs), flush=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(f"built {path}")
