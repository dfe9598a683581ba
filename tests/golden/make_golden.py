"""Write golden vectors for the 2:4 metadata converter from the reference itself.

The metadata reorder of ``sparse_semi_structured_from_dense_cutlass``
(kernel_experiments/sparse_marlin/src/marlin/_semi_structured_conversions.py:21-48,
54-179) is a layout, not a formula that any closed form, truth table or invariant
fixes, so it is pinned by vectors produced by the reference's own code.  The module
imports only torch and runs on the CPU; it is loaded by file path so that the
package ``marlin/__init__.py`` (which needs the CUDA extension) is never imported.

Run from the repository root, in the container where ``/root/reference`` exists:

    python tests/golden/make_golden.py

Output: ``tests/golden/semi_structured.npz`` (plain arrays, no pickles).
"""
from __future__ import annotations

import hashlib
import importlib.util
import pathlib

import numpy as np
import torch

REF = pathlib.Path("/root/reference/kernel_experiments/sparse_marlin/src/marlin/_semi_structured_conversions.py")
OUT = pathlib.Path(__file__).resolve().parent / "semi_structured.npz"


def _load_reference():
    spec = importlib.util.spec_from_file_location("ref_semi_structured", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _all_patterns_dense(rows: int, k: int, gen: torch.Generator) -> torch.Tensor:
    """Dense int32 matrix whose groups of 4 cycle through all 16 nonzero-flag
    patterns, with random nonzero values (1..15) where the flag is set."""
    ngroups = rows * k // 4
    pat = torch.arange(ngroups) % 16
    pat = pat[torch.randperm(ngroups, generator=gen)]
    flags = torch.stack([(pat >> b) & 1 for b in range(4)], dim=-1)
    vals = torch.randint(1, 16, (ngroups, 4), generator=gen, dtype=torch.int32)
    return (flags * vals).to(torch.int32).reshape(rows, k)


def main() -> None:
    ref = _load_reference()
    gen = torch.Generator().manual_seed(20261019)
    out: dict[str, np.ndarray] = {}
    # 1) converter on all 16 flag patterns, int32 and fp16 inputs
    for tag, (rows, k) in {"a": (64, 32), "b": (64, 64), "c": (128, 96), "d": (256, 256)}.items():
        dense = _all_patterns_dense(rows, k, gen)
        sparse, meta = ref.sparse_semi_structured_from_dense_cutlass(dense)
        back = ref.sparse_semi_structured_to_dense_cutlass(sparse, meta)
        out[f"conv_{tag}_dense"] = dense.numpy()
        out[f"conv_{tag}_sparse"] = sparse.numpy()
        out[f"conv_{tag}_meta"] = meta.numpy()
        out[f"conv_{tag}_back"] = back.numpy()
    dense_h = torch.randn(64, 128, generator=gen).to(torch.float16)
    dense_h = dense_h * (torch.rand(64, 128, generator=gen) > 0.5)
    sparse, meta = ref.sparse_semi_structured_from_dense_cutlass(dense_h)
    out["conv_h_dense"] = dense_h.numpy()
    out["conv_h_sparse"] = sparse.numpy()
    out["conv_h_meta"] = meta.numpy()
    # 2) raw scatter offsets for int16 metadata
    for rows, ncols in [(64, 2), (64, 4), (192, 6), (256, 16)]:
        off = ref._calculate_meta_reordering_scatter_offsets(rows, ncols, torch.int16, "cpu")
        out[f"offsets_{rows}x{ncols}"] = off.numpy()
    # 3) mask_creator on tie-free inputs (ties are not pinned: unstable argsort)
    x = torch.randn(96, 64, generator=gen)
    out["mask_x"] = x.numpy()
    out["mask_ref"] = ref.mask_creator(x).numpy()
    out["source_sha256"] = np.frombuffer(hashlib.sha256(REF.read_bytes()).digest(), dtype=np.uint8)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
