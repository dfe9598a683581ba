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
PROBE_LIB = PKG / "libmarlin_probe.so"
#: The same library with the decode kernel's per-wave phase timestamps compiled in
#: (SM24_SPANS=1): a measurement build for ``bench.py --workload spans`` only.
SPANS_LIB = PKG / "libmarlin_hip_spans.so"
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


# The translation units of the decode-sized kernels (sm24_decode_*, the lane-native
# decode kernel in sm24_gemm.hip, the dense Marlin kernel): their leading scalar
# arguments (up to 14 dwords) are preloaded into SGPRs by the dispatcher, so their
# prologue waits for no kernel-argument load.  Kernels whose first argument is a
# struct are not affected.
_PRELOAD = ["-mllvm", "-amdgpu-kernarg-preload-count=14"]
EXTRA_FLAGS: dict[str, list[str]] = {
    name: _PRELOAD for name in ("sm24_decode_16.hip", "sm24_decode_32.hip", "sm24_decode_64.hip", "sm24_gemm.hip",
                                "marlin_dense.hip")}

# hipcc's host pass does not know the packed-fp32 target feature: drop that noise.
_NOISE = ("packed-fp32-ops", "is not a recognized feature")


def _run(cmd: list[str], verbose: bool) -> subprocess.Popen:
    if verbose:
        print(" ".join(cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)


def _finish(proc: subprocess.Popen, what: str, verbose: bool) -> None:
    out, _ = proc.communicate()
    msgs = [ln for ln in out.splitlines() if not any(n in ln for n in _NOISE)]
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {what}:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs), flush=True)


def build(verbose: bool = False) -> pathlib.Path:
    """Compile every source to an object (in parallel), then link
    ``csed499ii_amd/libmarlin_hip.so`` (the GEMM library, from ``csrc/*.hip``),
    ``csed499ii_amd/libmarlin_hip_spans.so`` (the same sources with SM24_SPANS=1: the
    measurement build whose decode kernel records per-wave phase timestamps) and
    ``csed499ii_amd/libmarlin_probe.so`` (bench.py's measurement aids, from
    ``csrc/probe/*.hip``); always rebuilds all three."""
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    probe_srcs = sorted((CSRC / "probe").glob("*.hip"))
    variants = [(LIB, srcs, PKG / "_build", []), (SPANS_LIB, srcs, PKG / "_build_spans", ["-DSM24_SPANS=1"]),
                (PROBE_LIB, probe_srcs, PKG / "_build", [])]
    links, procs = [], []
    for lib, lib_srcs, obj_dir, defs in variants:
        obj_dir.mkdir(exist_ok=True)
        objs = []
        for src in lib_srcs:
            obj = obj_dir / (src.stem + ".o")
            objs.append(obj)
            cmd = [hipcc(), *compile_flags(), *defs, *EXTRA_FLAGS.get(src.name, []), "-c", "-o", str(obj), str(src)]
            procs.append((_run(cmd, verbose), src.name))
        links.append((lib, objs))
    for proc, name in procs:
        _finish(proc, name, verbose)
    for lib, lib_objs in links:
        if not lib_objs:
            continue
        tmp = lib.with_suffix(".so.tmp")
        link = _run([hipcc(), f"--offload-arch={ARCH}", "-fPIC", "-shared", "-o", str(tmp), *map(str, lib_objs)],
                    verbose)
        _finish(link, f"link of {lib.name}", verbose)
        os.replace(tmp, lib)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(f"built {path}")
