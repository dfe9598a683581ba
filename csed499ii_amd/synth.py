"""Seeded synthetic problems for the 2:4 INT4 GEMM (benchmarks and GPU tests).

Inputs follow the measurement recipe of the benchmark configs: ``A ~ N(0,1)`` fp16,
``W ~ N(0, 0.02)`` pruned to 2:4 along K (two largest ``|w|`` of each 4, ties to the
lower index), quantized symmetric with group size 128 along K and fp16 scales (the
quantizer of the reference's ``gen_quant4_NT``, test_2_4.py:22-37, with ``maxq`` 15
or 7), and packed through the explicit-mask ``pack_2_4`` / ``pack_w3``.

Random draws use a CPU ``torch.Generator`` so the data is device-independent; the
packing runs on ``device``.
"""
from __future__ import annotations

import torch

from .marlin import pack_2_4, pack_w3

SEED_BASE = 20261019


def prune_2_4(w: torch.Tensor) -> torch.Tensor:
    """K x N bool mask keeping the two largest ``|w|`` of every 4 consecutive rows of a
    column (ties keep the lower index)."""
    k, n = w.shape
    g = w.abs().float().t().reshape(n, k // 4, 4)
    keep = torch.argsort(g, dim=-1, descending=True, stable=True)[..., :2]
    mask = torch.zeros_like(g, dtype=torch.bool)
    mask.scatter_(-1, keep, True)
    return mask.reshape(n, k).t()


def quantize(w: torch.Tensor, groupsize: int, maxq: int = 15):
    """Symmetric grouped quantizer (reference test_2_4.py:22-37) on a K x N fp16
    weight.  Returns ``(q int32 [K,N], s fp16 [K/g or 1, N], ref fp16 [K,N])``."""
    k, n = w.shape
    g = k if groupsize == -1 else groupsize
    wg = w.reshape((-1, g, n)).permute(1, 0, 2).reshape((g, -1))
    s = torch.max(torch.abs(wg), 0, keepdim=True)[0]
    s *= 2 / maxq
    q = torch.round(wg / s).int()
    zero = (maxq + 1) // 2
    q += zero
    q = torch.clamp(q, 0, maxq)
    ref = (q - zero).half() * s
    q = q.reshape((g, -1, n)).permute(1, 0, 2).reshape((k, n)).contiguous()
    ref = ref.reshape((g, -1, n)).permute(1, 0, 2).reshape((k, n)).contiguous()
    return q, s.reshape((-1, n)).contiguous(), ref


def make_weight(K: int, N: int, seed: int, groupsize: int = 128, bits: int = 4, device="cuda",
                std: float = 0.02):
    """Packed 2:4 weight of one linear layer.

    Returns a dict with ``B`` (int32 ``[K/32, 2N]``; uint8 3-bit stream when
    ``bits == 3``), ``meta`` (int16 ``[N, K/16]``), ``s`` (fp16) and ``groupsize``.
    """
    gen = torch.Generator().manual_seed(seed)
    w = (torch.randn((K, N), generator=gen) * std).to(torch.float16).to(device)
    mask = prune_2_4(w)
    w = w * mask
    maxq = 15 if bits == 4 else 7
    _, s, _ = quantize(w, groupsize, maxq)
    if bits == 4:
        B, sp, meta = pack_2_4(w, s, groupsize, mask=mask)
    elif bits == 3:
        B, sp, meta = pack_w3(w, s, groupsize, mask=mask)
    else:
        raise ValueError("bits must be 4 or 3")
    return {"B": B, "meta": meta, "s": sp, "groupsize": groupsize, "bits": bits, "K": K, "N": N}


def make_activation(M: int, K: int, seed: int, device="cuda") -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed + 7919)
    return torch.randn((M, K), generator=gen).to(torch.float16).to(device)


def weight_bytes(K: int, N: int, bits: int = 4, groupsize: int = 128) -> int:
    """Algorithmic compressed-weight bytes: values K*N/2*bits/8 + metadata K*N/8 +
    fp16 scales (K/128)*N*2 (25/64*K*N for 4-bit values and group 128)."""
    g = K if groupsize == -1 else groupsize
    return K * N // 2 * bits // 8 + K * N // 8 + (K // g) * N * 2


def make_dense_weight(K: int, N: int, seed: int, groupsize: int = 128, device="cuda", std: float = 0.02):
    """Packed dense INT4 weight (no pruning) in the dense Marlin layout:
    ``{"B": int32 [K/16, 2N], "s": fp16, "bits": "dense", ...}``."""
    from .marlin import pack_dense

    gen = torch.Generator().manual_seed(seed)
    w = (torch.randn((K, N), generator=gen) * std).to(torch.float16).to(device)
    _, s, _ = quantize(w, groupsize, 15)
    B, sp = pack_dense(w, s, groupsize)
    return {"B": B, "meta": B, "s": sp, "groupsize": groupsize, "bits": "dense", "K": K, "N": N}


def dense_weight_bytes(K: int, N: int, groupsize: int = 128) -> int:
    """Algorithmic bytes of a dense INT4 weight: codes K*N/2 + fp16 scales."""
    g = K if groupsize == -1 else groupsize
    return K * N // 2 + (K // g) * N * 2
