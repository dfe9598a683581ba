"""2:4 semi-structured conversions in the CUTLASS metadata layout (torch, any device).

Drop-in for ``kernel_experiments/sparse_marlin/src/marlin/_semi_structured_conversions.py``:
same function names, arguments, outputs, and error behaviour for the 16-bit and
int32 element types used by the 2:4 INT4 path.

Metadata layout (what the GEMM kernels read): each group of 4 dense elements gets a
nibble ``idx0 | idx1 << 2`` with ``idx0 < idx1`` the kept positions; four nibbles form
an int16 (16 dense elements).  The int16 matrix ``[rows, k/16]`` is then stored in
CUTLASS ``ColumnMajorInterleaved<2>`` order with a row swizzle inside every 64 rows
and a transpose of every 2x2 block (reference lines 21-48).
"""
from __future__ import annotations

import torch

__all__ = [
    "sparse_semi_structured_from_dense_cutlass",
    "sparse_semi_structured_to_dense_cutlass",
    "mask_creator",
]


def _meta_scatter_offsets(rows: int, ncols: int, device) -> torch.Tensor:
    """Flat position of logical ``meta[r, c]`` (int16 metadata), reference lines 21-48.

    Write ``r = 64*R + 8a + 4b + 2c + d``; the swizzled row is
    ``64*R + 4a + 32c + 2d + b``; then elements (even row, odd col) and
    (odd row, even col) of every 2x2 block swap; finally column-major with an
    interleave of 2 columns.
    """
    r = torch.arange(rows, device=device, dtype=torch.int64)[:, None]
    c = torch.arange(ncols, device=device, dtype=torch.int64)[None, :]
    lr = r % 64
    sr = (r - lr) + 4 * (lr // 8) + 32 * ((lr // 2) % 2) + 2 * (lr % 2) + (lr // 4) % 2
    sr = sr.expand(rows, ncols)
    cc = c.expand(rows, ncols)
    odd_r = sr % 2
    odd_c = cc % 2
    swap = odd_r ^ odd_c  # off-diagonal of the 2x2 block
    # (even r, odd c) -> (r+1, c-1); (odd r, even c) -> (r-1, c+1)
    delta = swap * (1 - 2 * odd_r)
    sr2 = sr + delta
    cc2 = cc - delta
    return ((cc2 // 2) * rows * 2 + sr2 * 2 + cc2 % 2).reshape(-1)


def _encode_groups(m0, m1, m2, m3):
    """Nonzero flags of a group of 4 -> (idx0, idx1), the Espresso-minimised
    boolean functions of the reference (lines 133-141): exactly two flags set gives
    their positions; fewer or more flags give the fixed encodings listed there."""
    expr0 = m0 & m1
    expr1 = ~m0 & m1
    expr2 = ~m0 & ~m1
    bit0 = expr1
    bit1 = expr2
    bit2 = expr0 | expr2 | m3
    bit3 = expr1 | ~m1
    idx0 = bit0.to(torch.int64) | (bit1.to(torch.int64) << 1)
    idx1 = bit2.to(torch.int64) | (bit3.to(torch.int64) << 1)
    return idx0, idx1


def _meta_dtype_for(dtype: torch.dtype) -> torch.dtype:
    if dtype in (torch.half, torch.bfloat16, torch.int32, torch.int16):
        return torch.int16
    raise RuntimeError(f"Invalid datatype {dtype} of dense matrix")


def sparse_semi_structured_from_dense_cutlass(dense: torch.Tensor, mask: torch.Tensor | None = None):
    """Compress ``dense [m, k]`` (2:4 along k) into ``(sparse [m, k/2], meta [m, k/16] int16)``.

    Kept positions are the nonzero entries (reference line 92).  ``mask`` (an
    extension for pre-pruned weights) selects them explicitly instead, so that kept
    zero values are still encoded where they are.
    """
    if dense.dim() != 2:
        raise RuntimeError(f"Expected 2-dimensional dense tensor, got {dense.dim()}-dimensional tensor")
    m, k = dense.shape
    meta_dtype = _meta_dtype_for(dense.dtype)
    if m % 32 != 0:
        raise RuntimeError(f"Number of rows of dense matrix {m} must be divisible by 32")
    if k % 16 != 0:
        raise RuntimeError(f"Number of columns of dense matrix {k} must be divisible by 16")
    if m % 64 != 0 or k % 32 != 0:
        # The reorder scatter (reference lines 29-48) leaves its bounds otherwise.
        raise RuntimeError(f"dense matrix {m}x{k}: rows must be a multiple of 64 and columns of 32")
    device = dense.device
    d4 = dense.reshape(m, k // 4, 4)
    flags = (d4 != 0) if mask is None else mask.reshape(m, k // 4, 4).to(torch.bool)
    m0, m1, m2, m3 = flags.unbind(-1)
    idx0, idx1 = _encode_groups(m0, m1, m2, m3)
    s0 = d4.gather(-1, idx0.unsqueeze(-1))
    s1 = d4.gather(-1, idx1.unsqueeze(-1))
    sparse = torch.stack((s0, s1), dim=-1).reshape(m, k // 2)
    nib = (idx0 | (idx1 << 2)).reshape(m, k // 16, 4)
    meta = nib[..., 0] | (nib[..., 1] << 4) | (nib[..., 2] << 8) | (nib[..., 3] << 12)
    meta = torch.where(meta >= 1 << 15, meta - (1 << 16), meta).to(meta_dtype)
    out = torch.empty(m * (k // 16), dtype=meta_dtype, device=device)
    out.scatter_(0, _meta_scatter_offsets(m, k // 16, device), meta.reshape(-1))
    return sparse, out.view(m, k // 16)


def sparse_semi_structured_to_dense_cutlass(sparse: torch.Tensor, meta_reordered: torch.Tensor):
    """Inverse of :func:`sparse_semi_structured_from_dense_cutlass` (reference 186-283)."""
    if sparse.dim() != 2:
        raise RuntimeError(f"Expected 2-dimensional sparse tensor, got {sparse.dim()}-dimensional tensor")
    m, k = sparse.shape
    device = sparse.device
    if meta_reordered.dim() != 2:
        raise RuntimeError(f"Expected 2-dimensional meta tensor, got {meta_reordered.dim()}-dimensional tensor")
    if meta_reordered.device != device:
        raise RuntimeError(f"Expected meta matrix to be on {device} device, got matrix on {meta_reordered.device} device")
    if meta_reordered.dtype != torch.int16:
        raise RuntimeError(f"Invalid datatype {meta_reordered.dtype} of meta matrix")
    meta_nrows, meta_ncols = meta_reordered.shape
    if meta_nrows != m:
        raise RuntimeError(
            f"Number of rows of meta matrix {meta_nrows} must be equal to number of columns of spase matrix {m}")
    if meta_ncols * 16 != 2 * k:
        raise RuntimeError(
            f"Number of columns of sparse matrix {k} different from the {meta_ncols * 8}, "
            "expected according to the number of columns of meta matrix")
    off = _meta_scatter_offsets(m, meta_ncols, device)
    meta = meta_reordered.reshape(-1).gather(0, off).to(torch.int64) & 0xFFFF
    shifts = torch.arange(0, 16, 2, device=device, dtype=torch.int64)
    idx = ((meta.view(m, meta_ncols, 1) >> shifts) & 3).reshape(m, k)  # one 2-bit index per value
    base = torch.arange(k, device=device, dtype=torch.int64).reshape(1, k) // 2 * 4
    dense = torch.zeros((m, 2 * k), dtype=sparse.dtype, device=device)
    dense.scatter_(1, base + idx, sparse)
    return dense


def mask_creator(tensor: torch.Tensor) -> torch.Tensor:
    """2:4 mask keeping the two largest ``|x|`` of every 4 consecutive elements
    (reference lines 286-314).  Returns float ones/zeros of ``tensor``'s shape.

    Ties keep the lower index (a stable descending sort); the reference's unstable
    argsort leaves tie order unspecified.
    """
    n, m_ = 2, 4
    if tensor.numel() % m_ != 0:
        raise ValueError(f"Tensor of size {tensor.shape} can't be evenly divided into {m_} groups")
    groups = tensor.detach().abs().reshape(-1, m_)
    keep = torch.argsort(groups, dim=1, descending=True, stable=True)[:, :n]
    mask = torch.zeros(groups.shape, device=groups.device)
    mask.scatter_(1, keep, 1.0)
    return mask.reshape(tensor.shape)
