"""Sparse-Marlin 2:4 INT4 x FP16 GEMM for MI355X (gfx950): the Python surface.

Drop-in for ``kernel_experiments/sparse_marlin/src/marlin/__init__.py`` on the 2:4
path: ``mul_2_4``, ``Layer_2_4`` (with its ``pack()`` layout), ``replace_linear`` and
the permutation tables.  The arithmetic runs in the hand-written HIP kernels of
``libmarlin_hip.so`` through its C ABI; there is no CPU fallback.

Extensions that the reference keeps in side experiments:

* ``mul_2_4_meta3`` / ``pack_meta3`` / ``unpack_meta3``: 3-bit 2:4 metadata
  (kernel_experiments/sparse_marlin/metadata_decode).
* ``expand3``: 3-bit code stream -> nibbles (kernel_experiments/3bit_encoding).
* ``mul_2_4_w3`` / ``pack_w3``: 3-bit nonzero values (no reference implementation).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch
import torch.nn as nn

from .. import _lib
from ._semi_structured_conversions import (
    mask_creator,
    sparse_semi_structured_from_dense_cutlass,
    sparse_semi_structured_to_dense_cutlass,
)

__all__ = [
    "mul_2_4",
    "mul_2_4_noalloc",
    "plan_2_4",
    "mul_2_4_meta3",
    "mul_2_4_w3",
    "Layer_2_4",
    "replace_linear",
    "mask_creator",
    "sparse_semi_structured_from_dense_cutlass",
    "sparse_semi_structured_to_dense_cutlass",
    "pack_2_4",
    "pack_w3",
    "pack_meta3",
    "unpack_meta3",
    "expand3",
    "pack_native",
    "unpack_native",
    "mul_2_4_native",
    "mul",
    "Layer",
    "pack_dense",
]


# ---------------------------------------------------------------------------
# The GEMM entry points
# ---------------------------------------------------------------------------


def _ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _check_operands(A, B, meta, C, s, workspace, b_elems: int, b_dtype: torch.dtype, meta_elems: int,
                    meta_dtype: torch.dtype):
    """Device, dtype, contiguity and size checks (``meta`` and ``workspace`` may be
    None: the dense op has no metadata, the no-allocation op no workspace).  The
    reference binding checks none of these (it hands raw pointers to the kernel);
    here a mismatch raises instead of reading or writing out of bounds on the GPU."""
    tensors = {"A": A, "B": B, "C": C, "s": s}
    if meta is not None:
        tensors["meta"] = meta
    if workspace is not None:
        tensors["workspace"] = workspace
    for name, t in tensors.items():
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if not t.is_cuda:
            raise RuntimeError(f"{name} must be a GPU tensor (there is no CPU implementation)")
        if t.device != A.device:
            raise RuntimeError(f"{name} is on {t.device}, expected {A.device}")
        if not t.is_contiguous():
            raise RuntimeError(f"{name} must be contiguous")
    for name, t, dt in (("A", A, torch.half), ("C", C, torch.half), ("s", s, torch.half),
                        ("B", B, b_dtype), ("meta", meta, meta_dtype)):
        if t is not None and t.dtype != dt:
            raise RuntimeError(f"{name} must be {dt}, got {t.dtype}")
    if A.dim() != 2 or C.dim() != 2 or s.dim() != 2:
        raise RuntimeError("A, C and s must be 2-dimensional")
    M, K = A.shape
    N = C.shape[1]
    if C.shape[0] != M:
        raise RuntimeError(f"C has {C.shape[0]} rows, A has {M}")
    if s.shape[1] != N:
        raise RuntimeError(f"s has {s.shape[1]} columns, C has {N}")
    if B.numel() != b_elems:
        raise RuntimeError(f"B has {B.numel()} elements, expected {b_elems} for K={K}, N={N}")
    if meta is not None and meta.numel() != meta_elems:
        raise RuntimeError(f"meta has {meta.numel()} elements, expected {meta_elems} for K={K}, N={N}")
    for name, t in tensors.items():
        if t.numel() and t.data_ptr() % 16:
            raise RuntimeError(f"{name} must be 16-byte aligned")


def _groupsize_and_checks(A, C, s, workspace, max_par):
    """Shape inference and checks of the reference binding (marlin_cuda.cpp:66-80)."""
    prob_n = A.size(0)
    prob_m = C.size(1)
    prob_k = A.size(1)
    groupsize = -1 if s.size(0) == 1 else prob_k // 2 // s.size(0)
    if groupsize != -1 and groupsize * s.size(0) != prob_k // 2:
        raise RuntimeError(f"k={prob_k} not compatible with {s.size(0)} groups.")
    if workspace is not None and workspace.numel() < prob_m // 128 * max_par:
        raise RuntimeError(f"workspace must be of size at least {prob_m // 128 * max_par}.")
    return prob_m, prob_n, prob_k, groupsize


def _raise_for(err: int, prob_m, prob_n, prob_k, thread_k, thread_m, groupsize):
    """Error mapping of the reference binding (marlin_cuda.cpp:86-93)."""
    if err == _lib.OK:
        return
    if err == _lib.ERR_PROB_SHAPE:
        raise RuntimeError(f"Problem (m={prob_m}, n={prob_n}, k={prob_k}) not compatible with "
                           f"thread_k={thread_k}, thread_m={thread_m}.")
    if err == _lib.ERR_KERN_SHAPE:
        raise RuntimeError(f"No kernel implementation for thread_k={thread_k}, thread_m={thread_m}, "
                           f"groupsize={groupsize}.")
    raise RuntimeError(_lib.last_error() or f"marlin_hip error {err}")


def _call(fn_name, A, B, meta, C, s, workspace, thread_k, thread_m, sms, max_par, b_elems_fn, b_dtype,
          meta_elems_fn, meta_dtype):
    lib = _lib.load()
    prob_m, prob_n, prob_k, groupsize = _groupsize_and_checks(A, C, s, workspace, max_par)
    _check_operands(A, B, meta, C, s, workspace, b_elems_fn(prob_k, prob_m), b_dtype,
                    meta_elems_fn(prob_k, prob_m), meta_dtype)
    dev = A.get_device()
    stream = torch.cuda.current_stream(A.device).cuda_stream
    err = getattr(lib, fn_name)(_ptr(A), _ptr(B), _ptr(meta), _ptr(C), _ptr(s), prob_m, prob_n, prob_k,
                                _ptr(workspace), groupsize, dev, ctypes.c_void_p(stream), thread_k, thread_m,
                                sms, max_par)
    _raise_for(err, prob_m, prob_n, prob_k, thread_k, thread_m, groupsize)


def mul_2_4(A, B, meta, C, s, workspace, thread_k=-1, thread_m=-1, sms=-1, max_par=16):
    """Marlin FP16 x (INT4 + 2:4 sparsity) multiply: ``C = A @ W``.

    Mirrors ``marlin.mul_2_4`` (reference __init__.py:45-58; binding
    marlin_cuda.cpp:66-94): ``A`` fp16 ``[M, K]``; ``B`` int32 packed weights
    (``K*N/16`` elements, ``Layer_2_4.pack`` layout); ``meta`` int16 2:4 metadata
    (``K*N/16`` elements); ``C`` fp16 ``[M, N]``, overwritten; ``s`` fp16 scales
    ``[K/128, N]`` or ``[1, N]``; ``workspace`` int32 with at least ``N/128*max_par``
    elements (kept for compatibility; it is neither read nor written: the library
    keeps its split-K scratch per device and stream, so calls on different streams
    may overlap).
    ``thread_k``/``thread_m`` are validated like the reference's tile choices;
    ``sms`` is the number of compute units to plan for (-1: all).  Asynchronous on
    the current stream of ``A``'s device.
    """
    _call("marlin_hip_mul_2_4", A, B, meta, C, s, workspace, thread_k, thread_m, sms, max_par,
          lambda k, n: k * n // 16, torch.int32, lambda k, n: k * n // 16, torch.int16)


def mul(A, B, C, s, workspace, thread_k=-1, thread_n=-1, sms=-1, max_par=16):
    """Dense Marlin FP16 x INT4 multiply: ``C = A @ W``.

    Mirrors ``marlin.mul`` (reference __init__.py:61-75; binding marlin_cuda.cpp:38-64):
    ``A`` fp16 ``[M, K]``; ``B`` int32 weights in the dense ``Layer.pack`` layout
    (``K*N/8`` elements); ``C`` fp16 ``[M, N]``, overwritten; ``s`` fp16 scales
    ``[K/128, N]`` or ``[1, N]``; ``workspace`` int32 with at least ``N/128*max_par``
    elements (neither read nor written).  Unlike ``mul_2_4`` the binding names the
    batch ``m`` and the output features ``n``, and the group size is in dense K."""
    lib = _lib.load()
    prob_m, prob_n, prob_k = A.size(0), C.size(1), A.size(1)
    groupsize = -1 if s.size(0) == 1 else prob_k // s.size(0)
    if groupsize != -1 and groupsize * s.size(0) != prob_k:
        raise RuntimeError(f"k={prob_k} not compatible with {s.size(0)} groups.")
    if workspace.numel() < prob_n // 128 * max_par:
        raise RuntimeError(f"workspace must be of size at least {prob_n // 128 * max_par}.")
    _check_operands(A, B, None, C, s, workspace, prob_k * prob_n // 8, torch.int32, 0, torch.int16)
    stream = torch.cuda.current_stream(A.device).cuda_stream
    err = lib.marlin_hip_mul(_ptr(A), _ptr(B), _ptr(C), _ptr(s), prob_m, prob_n, prob_k, _ptr(workspace),
                             groupsize, A.get_device(), ctypes.c_void_p(stream), thread_k, thread_n, sms, max_par)
    if err == _lib.OK:
        return
    if err == _lib.ERR_PROB_SHAPE:
        raise RuntimeError(f"Problem (m={prob_m}, n={prob_n}, k={prob_k}) not compatible with "
                           f"thread_k={thread_k}, thread_n={thread_n}.")
    if err == _lib.ERR_KERN_SHAPE:
        raise RuntimeError(f"No kernel implementation for thread_k={thread_k}, thread_n={thread_n}, "
                           f"groupsize={groupsize}.")
    raise RuntimeError(_lib.last_error() or f"marlin_hip error {err}")


_KERNELS = {-1: None, 0: "decode", 1: "large_m", 2: "general", 3: "decode_dma"}


def plan_2_4(M: int, K: int, N: int, groupsize: int = 128, thread_k: int = -1, thread_m: int = -1, sms: int = -1,
             noalloc: bool = False) -> dict:
    """The launch plan of a ``mul_2_4`` call on ``A [M, K]`` and an ``N``-column weight
    (``noalloc=True``: of ``mul_2_4_noalloc``), computed on the host without a GPU
    (``marlin_hip_plan``): kernel, workgroups and K splits of the first launch,
    threads per workgroup and launches.  ``splits > 1`` means the call uses its
    stream's split-K scratch.  Raises like ``mul_2_4`` for shapes it refuses."""
    out = (ctypes.c_int * 5)()
    g = groupsize // 2 if groupsize != -1 else -1
    err = _lib.load().marlin_hip_plan(N, M, K, g, thread_k, thread_m, sms, int(noalloc), out)
    _raise_for(err, N, M, K, thread_k, thread_m, g)
    return {"kernel": _KERNELS[out[0]], "workgroups": out[1], "threads": out[2], "splits": out[3],
            "launches": out[4]}


def mul_2_4_noalloc(A, B, meta, C, s, thread_k=-1, thread_m=-1, sms=-1):
    """``mul_2_4`` through ``marlin_hip_mul_2_4_noalloc``: the same product without any
    device allocation (it never splits K, so it needs no split-K scratch; safe to
    capture on a stream that has never run a call).  No reference counterpart."""
    lib = _lib.load()
    prob_m, prob_n, prob_k, groupsize = _groupsize_and_checks(A, C, s, None, 0)
    _check_operands(A, B, meta, C, s, None, prob_k * prob_m // 16, torch.int32, prob_k * prob_m // 16, torch.int16)
    stream = torch.cuda.current_stream(A.device).cuda_stream
    err = lib.marlin_hip_mul_2_4_noalloc(_ptr(A), _ptr(B), _ptr(meta), _ptr(C), _ptr(s), prob_m, prob_n, prob_k,
                                         groupsize, A.get_device(), ctypes.c_void_p(stream), thread_k, thread_m,
                                         sms)
    _raise_for(err, prob_m, prob_n, prob_k, thread_k, thread_m, groupsize)


def mul_2_4_meta3(A, B, meta3, C, s, workspace, thread_k=-1, thread_m=-1, sms=-1, max_par=16):
    """``mul_2_4`` with 3-bit-compressed metadata (``pack_meta3`` output, int32,
    ``K*N*3/128`` words).  Mirrors the ``fetch``/``matmul`` bindings of the reference's
    metadata_decode experiment (setup.py:36-44)."""
    _call("marlin_hip_mul_2_4_meta3", A, B, meta3, C, s, workspace, thread_k, thread_m, sms, max_par,
          lambda k, n: k * n // 16, torch.int32, lambda k, n: k * n * 3 // 128, torch.int32)


def mul_2_4_w3(A, B3, meta, C, s, workspace, thread_k=-1, thread_m=-1, sms=-1, max_par=16):
    """``mul_2_4`` with 3-bit nonzero values (``pack_w3`` output: uint8 stream of
    ``K*N*3/16`` bytes), codes offset by 4."""
    _call("marlin_hip_mul_2_4_w3", A, B3, meta, C, s, workspace, thread_k, thread_m, sms, max_par,
          lambda k, n: k * n * 3 // 16, torch.uint8, lambda k, n: k * n // 16, torch.int16)


# ---------------------------------------------------------------------------
# Codecs
# ---------------------------------------------------------------------------


# ---------------------------------------------------------------------------
# Lane-native decode layout (this library's own repack; no reference counterpart)
# ---------------------------------------------------------------------------


def _check_gpu(name: str, t: torch.Tensor, dtype: torch.dtype, numel: int, device):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda or t.device != device:
        raise RuntimeError(f"{name} must be a GPU tensor on {device}")
    if not t.is_contiguous() or t.dtype != dtype:
        raise RuntimeError(f"{name} must be a contiguous {dtype} tensor")
    if t.numel() != numel:
        raise RuntimeError(f"{name} has {t.numel()} elements, expected {numel}")
    if t.numel() and t.data_ptr() % 16:
        raise RuntimeError(f"{name} must be 16-byte aligned")


def pack_native(B: torch.Tensor, meta: torch.Tensor, s: torch.Tensor):
    """Repack a ``Layer_2_4.pack`` weight (``B``, ``meta``, ``s``) into the lane-native
    decode layout (each smfmac lane's operand words contiguous; same bytes).
    Returns ``(Bn int32 [N/16, K/256, 64, 4], metan int16 [N/16, K/256, 64, 4], sn)``
    with ``sn`` fp16 ``[N/16, K/256, 16, 2]`` (group size 128) or ``[1, N]``
    (per-column scales).  Needs ``N % 64 == 0`` and ``K % 256 == 0``.  Exact inverse:
    :func:`unpack_native`."""
    if not (isinstance(s, torch.Tensor) and s.dim() == 2):
        raise RuntimeError("s must be a 2-dimensional fp16 tensor")
    N = s.shape[1]
    if N == 0 or B.numel() * 16 % N:
        raise RuntimeError("B does not match the scales' column count")
    K = B.numel() * 16 // N
    grouped = s.shape[0] != 1
    if N % 64 or K % 256 or (grouped and s.shape[0] * 128 != K):
        raise RuntimeError(f"the native layout needs N % 64 == 0, K % 256 == 0 and group size 128 or -1 "
                           f"(K={K}, N={N}, {s.shape[0]} scale rows)")
    dev = B.device
    _check_gpu("B", B, torch.int32, K * N // 16, dev)
    _check_gpu("meta", meta, torch.int16, K * N // 16, dev)
    _check_gpu("s", s, torch.half, s.numel(), dev)
    Bn = torch.empty((N // 16, K // 256, 64, 4), dtype=torch.int32, device=dev)
    Mn = torch.empty((N // 16, K // 256, 64, 4), dtype=torch.int16, device=dev)
    Sn = torch.empty((N // 16, K // 256, 16, 2) if grouped else (1, N), dtype=torch.half, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    err = _lib.load().marlin_hip_native_pack(_ptr(B), _ptr(meta), _ptr(s), _ptr(Bn), _ptr(Mn), _ptr(Sn), N, K,
                                             64 if grouped else -1, B.get_device(), ctypes.c_void_p(stream))
    if err != _lib.OK:
        raise RuntimeError(_lib.last_error() or f"marlin_hip_native_pack error {err}")
    return Bn, Mn, Sn


def unpack_native(Bn: torch.Tensor, metan: torch.Tensor, sn: torch.Tensor):
    """Inverse of :func:`pack_native`: returns the reference layout ``(B int32
    [K/32, 2N], meta int16 [N, K/16], s fp16 [K/128 or 1, N])``."""
    if not (isinstance(Bn, torch.Tensor) and Bn.dim() == 4 and tuple(Bn.shape[2:]) == (64, 4)):
        raise RuntimeError("Bn must be the [N/16, K/256, 64, 4] tensor of pack_native")
    N, K = 16 * Bn.shape[0], 256 * Bn.shape[1]
    grouped = sn.numel() != N
    dev = Bn.device
    _check_gpu("Bn", Bn, torch.int32, K * N // 16, dev)
    _check_gpu("metan", metan, torch.int16, K * N // 16, dev)
    _check_gpu("sn", sn, torch.half, K * N // 128 if grouped else N, dev)
    B = torch.empty((K // 32, 2 * N), dtype=torch.int32, device=dev)
    meta = torch.empty((N, K // 16), dtype=torch.int16, device=dev)
    s = torch.empty((K // 128 if grouped else 1, N), dtype=torch.half, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    err = _lib.load().marlin_hip_native_unpack(_ptr(Bn), _ptr(metan), _ptr(sn), _ptr(B), _ptr(meta), _ptr(s), N,
                                               K, 64 if grouped else -1, Bn.get_device(), ctypes.c_void_p(stream))
    if err != _lib.OK:
        raise RuntimeError(_lib.last_error() or f"marlin_hip_native_unpack error {err}")
    return B, meta, s


def mul_2_4_native(A: torch.Tensor, Bn: torch.Tensor, metan: torch.Tensor, C: torch.Tensor, sn: torch.Tensor,
                   sms: int = -1) -> None:
    """``C = A @ W`` with ``W`` in the lane-native layout of :func:`pack_native`.  The
    same product as :func:`mul_2_4` on the original weight (fp16 operands, fp32
    accumulation; only the summation order differs).  Batches above 16 rows run the
    reference-layout kernels on an unpacked copy, under :func:`mul_2_4`'s shape rules
    (N a multiple of 128, or of 256 above 16 rows)."""
    for name, t in (("A", A), ("C", C)):
        if not isinstance(t, torch.Tensor) or t.dim() != 2:
            raise RuntimeError(f"{name} must be a 2-dimensional tensor")
    M, K = A.shape
    N = C.shape[1]
    if C.shape[0] != M:
        raise RuntimeError(f"C has {C.shape[0]} rows, A has {M}")
    if N % 64 or K % 256:
        raise RuntimeError(f"the native layout needs N % 64 == 0 and K % 256 == 0 (K={K}, N={N})")
    grouped = sn.numel() != N
    dev = A.device
    _check_gpu("A", A, torch.half, M * K, dev)
    _check_gpu("C", C, torch.half, M * N, dev)
    _check_gpu("Bn", Bn, torch.int32, K * N // 16, dev)
    _check_gpu("metan", metan, torch.int16, K * N // 16, dev)
    _check_gpu("sn", sn, torch.half, K * N // 128 if grouped else N, dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    err = _lib.load().marlin_hip_mul_2_4_native(_ptr(A), _ptr(Bn), _ptr(metan), _ptr(C), _ptr(sn), N, M, K,
                                                64 if grouped else -1, A.get_device(), ctypes.c_void_p(stream),
                                                sms)
    _raise_for(err, N, M, K, -1, -1, 64 if grouped else -1)


def pack_meta3(meta: torch.Tensor) -> torch.Tensor:
    """4-bit 2:4 metadata (int16, multiple of 128 elements) -> 3-bit codes (int32,
    ``numel*3/8``).  Raises if a nibble is not a valid 2:4 pattern
    (reference metadata_decode/codec.cu:30-35)."""
    if not (meta.is_cuda and meta.is_contiguous() and meta.dtype == torch.int16 and meta.numel() % 128 == 0):
        raise RuntimeError("expected CUDA contiguous int16 metadata, multiple of 256 bytes")
    lib = _lib.load()
    out = torch.empty(meta.numel() * 3 // 8, dtype=torch.int32, device=meta.device)
    errors = torch.zeros(1, dtype=torch.int32, device=meta.device)
    stream = torch.cuda.current_stream(meta.device).cuda_stream
    err = lib.marlin_hip_meta3_pack(_ptr(meta), _ptr(out), meta.numel(), _ptr(errors), meta.get_device(),
                                    ctypes.c_void_p(stream))
    if err != _lib.OK:
        raise RuntimeError(_lib.last_error() or f"marlin_hip_meta3_pack error {err}")
    if int(errors.item()) != 0:
        raise RuntimeError("metadata contains unsupported 2:4 nibbles")
    return out


def unpack_meta3(packed: torch.Tensor) -> torch.Tensor:
    """Inverse of :func:`pack_meta3` (reference codec.cu:36-41)."""
    if not (packed.is_cuda and packed.is_contiguous() and packed.dtype == torch.int32 and packed.numel() % 48 == 0):
        raise RuntimeError("expected compressed metadata")
    lib = _lib.load()
    out = torch.empty(packed.numel() * 8 // 3, dtype=torch.int16, device=packed.device)
    stream = torch.cuda.current_stream(packed.device).cuda_stream
    err = lib.marlin_hip_meta3_unpack(_ptr(packed), _ptr(out), packed.numel(), packed.get_device(),
                                      ctypes.c_void_p(stream))
    if err != _lib.OK:
        raise RuntimeError(_lib.last_error() or f"marlin_hip_meta3_unpack error {err}")
    return out


def expand3(stream_bytes: torch.Tensor) -> torch.Tensor:
    """3-bit code stream (uint8, 48 bytes per 128 codes) -> nibbles (int32, 16 words
    per 128 codes) with ``{0..7} -> {4,4,9,8,E,E,D,C}`` (reference
    3bit_encoding/experiment.cu:12-40)."""
    if not (stream_bytes.is_cuda and stream_bytes.is_contiguous() and stream_bytes.dtype == torch.uint8
            and stream_bytes.numel() % 48 == 0):
        raise RuntimeError("expected CUDA contiguous uint8 stream, multiple of 48 bytes")
    if stream_bytes.numel() and stream_bytes.data_ptr() % 4:
        raise RuntimeError("stream must be 4-byte aligned")
    lib = _lib.load()
    groups = stream_bytes.numel() // 48
    out = torch.empty(groups * 16, dtype=torch.int32, device=stream_bytes.device)
    stream = torch.cuda.current_stream(stream_bytes.device).cuda_stream
    err = lib.marlin_hip_expand3(_ptr(stream_bytes), _ptr(out), groups, stream_bytes.get_device(),
                                 ctypes.c_void_p(stream))
    if err != _lib.OK:
        raise RuntimeError(_lib.last_error() or f"marlin_hip_expand3 error {err}")
    return out


# ---------------------------------------------------------------------------
# Weight / scale permutations and packing
# ---------------------------------------------------------------------------


def _get_perms_2_4():
    """Weight and scale permutations of the 2:4 layout (reference __init__.py:242-268).

    ``perm`` reorders each 1024-entry block (64 output columns x 16 compressed-K rows,
    tiled as (n//16 % 4, kc % 16, n % 16)) so that word ``4*i + j`` of the block holds,
    in nibbles 0..7, the codes of compressed rows {2t, 2t+8, 2t, 2t+8, 2t+1, 2t+9,
    2t+1, 2t+9} (t = i % 4) of columns 8*(i//4) + j (nibbles 0,1,4,5) and
    8*(i//4) + 4 + j (nibbles 2,3,6,7).
    """
    rows_of = np.array([0, 8, 0, 8, 1, 9, 1, 9])
    blk_of = np.array([0, 0, 1, 1, 0, 0, 1, 1])
    w = np.arange(128)[:, None]
    p = np.arange(8)[None, :]
    i, j = w // 4, w % 4
    g, t = i // 4, i % 4
    kc = 2 * t + rows_of[p]
    n = 8 * g + 4 * blk_of[p] + j
    perm = (n // 16) * 256 + kc * 16 + n % 16
    perm = torch.from_numpy(perm.reshape(-1).astype(np.int64))
    scale_perm = [8 * i + j for i in range(8) for j in (0, 4, 1, 5, 2, 6, 3, 7)]
    scale_perm_single = list(range(64))
    return perm, scale_perm, scale_perm_single


_perm_2_4, _scale_perm_2_4, _scale_perm_single_2_4 = _get_perms_2_4()


def _quant_codes(w: torch.Tensor, s: torch.Tensor, k: int, n: int, groupsize: int, maxq: int) -> torch.Tensor:
    """``clamp(round(w / s) + (maxq+1)/2, 0, maxq)`` in the group-major order of the
    reference pack (__init__.py:350-362); ``w`` is K x N."""
    if groupsize != k:
        wg = w.reshape((-1, groupsize, n)).permute(1, 0, 2).reshape((groupsize, -1))
        sg = s.reshape((1, -1))
    else:
        wg, sg = w, s
    q = torch.round(wg / sg).int()
    q += (maxq + 1) // 2
    q = torch.clamp(q, 0, maxq)
    if groupsize != k:
        q = q.reshape((groupsize, -1, n)).permute(1, 0, 2).reshape((k, n)).contiguous()
    return q


def _pack_scales(s: torch.Tensor, k: int, n: int, groupsize: int) -> torch.Tensor:
    if groupsize != k:
        s = s.reshape((-1, len(_scale_perm_2_4)))[:, _scale_perm_2_4]
    else:
        s = s.reshape((-1, len(_scale_perm_single_2_4)))[:, _scale_perm_single_2_4]
    return s.reshape((-1, n)).contiguous()


def _sparse_codes(q: torch.Tensor, mask: torch.Tensor | None):
    """Prune the K x N codes to 2:4 along K and compress: returns the compressed
    ``[K/2, N]`` codes and the metadata.  Without ``mask`` the reference rule applies
    (two largest codes per group, then the ``!= 0`` compression, __init__.py:367-370)."""
    if mask is None:
        keep = mask_creator(q.T).to(q.device).bool()
        sparse, meta = sparse_semi_structured_from_dense_cutlass(keep * q.T)
    else:
        keep = mask.T.to(q.device).bool()
        sparse, meta = sparse_semi_structured_from_dense_cutlass(keep * q.T, mask=keep)
    return sparse.t(), meta


def _tile_and_permute(w: torch.Tensor, k2: int, n: int) -> torch.Tensor:
    """Compressed ``[K/2, N]`` codes -> ``[K/32, 16N]`` nibble stream in pack order
    (reference __init__.py:374-379)."""
    tile = 16
    w = w.reshape((k2 // tile, tile, n // tile, tile)).permute((0, 2, 1, 3)).reshape((k2 // tile, n * tile))
    perm = _perm_2_4.to(w.device)
    return w.reshape((-1, perm.numel()))[:, perm].reshape(w.shape)


def _nibbles_to_int32(res: torch.Tensor) -> torch.Tensor:
    """Pack 8 consecutive nibbles into one int32, nibble i at bits 4i (on device)."""
    r = res.to(torch.int64).reshape(res.shape[0], -1, 8)
    q = torch.zeros(r.shape[:2], dtype=torch.int64, device=res.device)
    for i in range(8):
        q |= (r[..., i] & 15) << (4 * i)
    q = torch.where(q >= 1 << 31, q - (1 << 32), q)
    return q.to(torch.int32)


def pack_2_4(w: torch.Tensor, scales: torch.Tensor, groupsize: int = -1, mask: torch.Tensor | None = None):
    """Pack a K x N fp16 weight into ``(B [K/32, 2N] int32, s, meta [N, K/16] int16)``
    (reference ``Layer_2_4.pack(..., trans=True)``, __init__.py:331-388).

    ``scales`` is ``[K/groupsize, N]`` (or ``[1, N]`` for ``groupsize=-1``).  ``mask``
    (K x N bool, 2:4 along K) marks the kept weights of a pre-pruned matrix; without
    it the reference rule keeps the two largest codes of every group of 4.
    """
    if w.dtype != torch.half:
        raise ValueError("Only `torch.half` weights are supported.")
    k, n = w.shape
    g = k if groupsize == -1 else groupsize
    q = _quant_codes(w, scales, k, n, g, 15)
    s = _pack_scales(scales, k, n, g)
    sparse, meta = _sparse_codes(q, mask)
    res = _tile_and_permute(sparse, k // 2, n)
    return _nibbles_to_int32(res), s, meta


def pack_w3(w: torch.Tensor, scales: torch.Tensor, groupsize: int, mask: torch.Tensor):
    """3-bit-value packing: codes ``clamp(round(w/s) + 4, 0, 7)`` in the 4-bit word
    order, stored as a 3-bit stream (code of nibble p of word u at bit 3*(8u + p)).
    Returns ``(B3 uint8 [K*N*3/16], s, meta)``.  No reference implementation exists."""
    if w.dtype != torch.half:
        raise ValueError("Only `torch.half` weights are supported.")
    k, n = w.shape
    g = k if groupsize == -1 else groupsize
    q = _quant_codes(w, scales, k, n, g, 7)
    s = _pack_scales(scales, k, n, g)
    sparse, meta = _sparse_codes(q, mask)
    res = _tile_and_permute(sparse, k // 2, n).to(torch.int64).reshape(-1, 8)
    x = torch.zeros(res.shape[0], dtype=torch.int64, device=res.device)
    for i in range(8):
        x |= (res[:, i] & 7) << (3 * i)
    b3 = torch.stack([x & 255, (x >> 8) & 255, (x >> 16) & 255], dim=-1).to(torch.uint8).reshape(-1)
    return b3, s, meta


# ---------------------------------------------------------------------------
# Module API
# ---------------------------------------------------------------------------


class Layer_2_4(nn.Module):
    """PyTorch Marlin 2:4 layer; 4-bit (symmetric grouped) linear layer without bias
    (reference __init__.py:274-388).

    Differences from the reference, all fixes of its quirks: ``B`` is allocated with
    the shape ``pack`` produces (``[K/32, 2N]``); ``pack`` leaves ``k`` and
    ``groupsize`` unchanged (so it can run twice); the workspace follows the module's
    device instead of being pinned to ``cuda:0``; ``pack`` accepts an explicit 2:4
    ``mask``; and ``trans=False`` (the dense-Marlin permutation, which the 2:4 kernel
    cannot read) raises instead of producing an unusable layout.
    """

    def __init__(self, infeatures, outfeatures, groupsize=-1):
        super().__init__()
        if groupsize not in [-1, 128]:
            raise ValueError("Only groupsize -1 and 128 are supported.")
        if infeatures % 128 != 0 or outfeatures % 64 != 0:
            raise ValueError("`infeatures` must be divisible by 128 and `outfeatures` by 64.")
        if groupsize == -1:
            groupsize = infeatures
        if infeatures % groupsize != 0:
            raise ValueError("`infeatures` must be divisible by `groupsize`.")
        self.k = infeatures
        self.n = outfeatures
        self.groupsize = groupsize
        self.register_buffer("B", torch.empty((self.k // 32, self.n * 2), dtype=torch.int))
        self.register_buffer("meta", torch.empty((self.n, self.k // 16), dtype=torch.int16))
        self.register_buffer("s", torch.empty((self.k // groupsize, self.n), dtype=torch.half))
        # 128 is the reference's minimum tile_n and 16 its default max_par.
        self.register_buffer("workspace", torch.zeros(self.n // 128 * 16, dtype=torch.int32), persistent=False)
        self.register_load_state_dict_post_hook(Layer_2_4._refresh_native)

    @staticmethod
    def _refresh_native(module, incompatible_keys):
        """After ``load_state_dict`` (in place or with ``assign=True``) a lane-native copy
        made by :meth:`to_native` holds the old weight: rebuild it from the loaded
        buffers."""
        if getattr(module, "Bn", None) is not None:
            module.to_native()

    def forward(self, A):
        C = torch.empty(A.shape[:-1] + (self.s.shape[1],), dtype=A.dtype, device=A.device)
        A2, C2 = A.view((-1, A.shape[-1])), C.view((-1, C.shape[-1]))
        if getattr(self, "Bn", None) is not None and A2.shape[0] <= self.NATIVE_MAX_ROWS and self.Bn.device == A.device:
            mul_2_4_native(A2, self.Bn, self.metan, C2, self.sn)
            return C
        ws = self.workspace
        if ws.device != A.device:
            ws = self.workspace = ws.to(A.device)
        mul_2_4(A2, self.B, self.meta, C2, self.s, ws)
        return C

    #: Largest batch that ``forward`` runs on the lane-native copy made by
    #: :meth:`to_native`.  Same box, per call over the decode sweeps: the native kernel
    #: is faster at 1 row (Llama-2-7B shapes -6.9 %, 70B -5.9 %), level at 2-4 rows,
    #: and slower from 8 rows (7B at 8 rows +5.0 %, at 16 rows +22.5 % against the
    #: pack() layout's 16-row kernel).
    NATIVE_MAX_ROWS = 4

    def to_native(self):
        """Keep a lane-native copy of the packed weight (:func:`pack_native`) for
        batches of at most ``NATIVE_MAX_ROWS`` rows, which ``forward`` then runs on
        :func:`mul_2_4_native`; larger batches keep using the pack() buffers, which
        stay the module's ``state_dict``.  Needs ``infeatures % 256 == 0``; the copy
        is as large as the packed weight.  ``pack`` and ``load_state_dict`` rebuild
        the copy; after an in-place edit of ``B``, ``meta`` or ``s`` call
        ``to_native()`` again.  Returns the module."""
        Bn, metan, sn = pack_native(self.B, self.meta, self.s)
        self.register_buffer("Bn", Bn, persistent=False)
        self.register_buffer("metan", metan, persistent=False)
        self.register_buffer("sn", sn, persistent=False)
        return self

    def pack(self, linear, scales, trans=False, mask=None):
        """Pack a fake-quantized linear layer into the 2:4 representation.

        ``linear.weight`` is read as K x N (``infeatures x outfeatures``), as the
        reference does (__init__.py:349); ``scales`` is ``[K/groupsize, N]``.
        """
        if linear.weight.dtype != torch.half:
            raise ValueError("Only `torch.half` weights are supported.")
        if not trans:
            raise ValueError("trans=False selects the dense Marlin permutation, which the 2:4 kernel "
                             "cannot read; call pack(linear, scales, True).")
        w = linear.weight.data
        if tuple(w.shape) != (self.k, self.n):
            raise ValueError(f"weight shape {tuple(w.shape)} != (k, n) = {(self.k, self.n)}")
        gs = -1 if self.groupsize == self.k else self.groupsize
        B, s, meta = pack_2_4(w, scales.to(w.device), gs, mask=mask)
        self.B = B.to(self.B.device)
        self.s = s.to(self.s.device)
        self.meta = meta.to(self.meta.device)
        if getattr(self, "Bn", None) is not None:  # a native copy of the old weight is stale
            self.to_native()


# ---------------------------------------------------------------------------
# Dense Marlin layout and module (reference __init__.py:78-99, 134-226)
# ---------------------------------------------------------------------------


def _dense_block_index() -> torch.Tensor:
    """Flat index (16 k x 64 n block, row-major) of nibble t of word w of one dense
    Marlin block (a 16-deep k-tile of a 64-column chunk): word w = 16 ci + 4 rq + jt
    holds columns 16 jt + ci (nibbles 0, 1, 4, 5) and 16 jt + ci + 8 (nibbles 2, 3, 6,
    7) at k = 2 rq + {0, 8, 0, 8, 1, 9, 1, 9}[t].  The same placement as the reference
    pack's tile permutation (__init__.py:78-99, 214-219), written as a closed form."""
    w = torch.arange(128)[:, None]
    t = torch.arange(8)[None, :]
    jt, rq, ci = w % 4, (w // 4) % 4, w // 16
    koff = torch.tensor([0, 8, 0, 8, 1, 9, 1, 9])[t]
    blk = torch.tensor([0, 0, 1, 1, 0, 0, 1, 1])[t]
    return ((2 * rq + koff) * 64 + 16 * jt + ci + 8 * blk).reshape(-1)


def _pack_dense_scales(s: torch.Tensor, n: int, grouped: bool) -> torch.Tensor:
    """Grouped: within 64 columns slot 8i + j holds column i + 8j (an 8 x 8
    transpose); per column: within 32 columns slot 8i + t holds column
    2i + {0, 1, 8, 9, 16, 17, 24, 25}[t] (reference __init__.py:93-98)."""
    if grouped:
        return s.reshape(-1, 8, 8).transpose(1, 2).reshape(-1, n).contiguous()
    return s.reshape(-1, 4, 4, 2).permute(0, 2, 1, 3).reshape(-1, n).contiguous()


def pack_dense(w: torch.Tensor, scales: torch.Tensor, groupsize: int = -1):
    """Pack a K x N fp16 weight into the dense Marlin layout: ``(B [K/16, 2N] int32,
    s)`` (reference ``Layer.pack(linear, scales)``, __init__.py:177-226): codes
    ``clamp(round(w / s) + 8, 0, 15)``, eight per int32."""
    if w.dtype != torch.half:
        raise ValueError("Only `torch.half` weights are supported.")
    k, n = w.shape
    if k % 16 or n % 64:
        raise ValueError("the dense layout needs K % 16 == 0 and N % 64 == 0")
    g = k if groupsize == -1 else groupsize
    q = _quant_codes(w, scales, k, n, g, 15)
    s = _pack_dense_scales(scales, n, g != k)
    blocks = q.reshape(k // 16, 16, n // 64, 64).permute(0, 2, 1, 3).reshape(k // 16, n // 64, 1024)
    codes = blocks[..., _dense_block_index().to(q.device)].reshape(k // 16, n // 64 * 128, 8)
    return _nibbles_to_int32(codes.reshape(k // 16, -1)), s


class Layer(nn.Module):
    """PyTorch dense Marlin layer; 4-bit (symmetric grouped) linear layer without bias
    (reference __init__.py:134-226), computed by :func:`mul`.

    Differences from the reference: the out-features check is the intended one
    (``outfeatures % 256``; the reference's chained comparison checks nothing,
    __init__.py:145), the workspace follows the module's device, and
    ``pack(..., trans=True)`` (the transposed permutation, which this kernel does
    not read) raises.
    """

    def __init__(self, infeatures, outfeatures, groupsize=-1):
        super().__init__()
        if groupsize not in [-1, 128]:
            raise ValueError("Only groupsize -1 and 128 are supported.")
        if infeatures % 128 != 0 or outfeatures % 256 != 0:
            raise ValueError("`infeatures` must be divisible by 128 and `outfeatures` by 256.")
        if groupsize == -1:
            groupsize = infeatures
        if infeatures % groupsize != 0:
            raise ValueError("`infeatures` must be divisible by `groupsize`.")
        self.k = infeatures
        self.n = outfeatures
        self.groupsize = groupsize
        self.register_buffer("B", torch.empty((self.k // 16, self.n * 16 // 8), dtype=torch.int))
        self.register_buffer("s", torch.empty((self.k // groupsize, self.n), dtype=torch.half))
        self.register_buffer("workspace", torch.zeros(self.n // 128 * 16, dtype=torch.int), persistent=False)

    def forward(self, A):
        C = torch.empty(A.shape[:-1] + (self.s.shape[1],), dtype=A.dtype, device=A.device)
        ws = self.workspace
        if ws.device != A.device:
            ws = self.workspace = ws.to(A.device)
        mul(A.view((-1, A.shape[-1])), self.B, C.view((-1, C.shape[-1])), self.s, ws)
        return C

    def pack(self, linear, scales, trans=False):
        """Pack a fake-quantized linear layer (``linear.weight`` read as K x N, as the
        reference does, __init__.py:193) with ``scales`` ``[K/groupsize, N]``."""
        if linear.weight.dtype != torch.half:
            raise ValueError("Only `torch.half` weights are supported.")
        if trans:
            raise ValueError("trans=True selects the transposed Marlin permutation, which the dense kernel "
                             "does not read; call pack(linear, scales).")
        w = linear.weight.data
        if tuple(w.shape) != (self.k, self.n):
            raise ValueError(f"weight shape {tuple(w.shape)} != (k, n) = {(self.k, self.n)}")
        gs = -1 if self.groupsize == self.k else self.groupsize
        B, s = pack_dense(w, scales.to(w.device), gs)
        self.B[:, :] = B.to(self.B.device)
        self.s[:, :] = s.to(self.s.device)


def replace_linear(module, name_filter=lambda n: True, groupsize=-1, name=""):
    """Recursively replace all ``torch.nn.Linear`` layers by empty Marlin 2:4 layers
    (reference __init__.py:391-415)."""
    if isinstance(module, Layer_2_4):
        return
    for attr in dir(module):
        tmp = getattr(module, attr)
        name1 = name + "." + attr if name != "" else attr
        if isinstance(tmp, nn.Linear) and name_filter(name1):
            setattr(module, attr, Layer_2_4(tmp.in_features, tmp.out_features, groupsize=groupsize))
    for name1, child in module.named_children():
        replace_linear(child, name_filter, groupsize=groupsize, name=name + "." + name1 if name != "" else name1)
