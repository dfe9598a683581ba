"""Seeded random shapes through every GEMM entry point (4-bit, 3-bit metadata, 3-bit
values, lane-native, dense) against the CPU oracle: ragged batches across the decode,
chunked-decode, general and large-M paths, both scale modes."""
import random

import pytest
import torch

from csed499ii_amd import marlin, synth
from oracle import sm24_oracle as o
from tests.gpu_util import assert_close, oracle_gemm, to_cpu

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _cases(seed, n):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        kind = rng.choice(["mul", "mul", "meta3", "w3", "native"])
        g = rng.choice([128, -1])
        if kind == "native":
            M = rng.choice([1, 2, 3, 4, 5, 9, 16])
            N = rng.choice([256, 512, 1024])
            K = 256 * rng.choice([1, 2, 3, 6])
        else:
            M = rng.choice([1, 3, 8, 16, 17, 33, 65, 97, 100, 130, 160, 200])
            N = rng.choice([256, 512, 1024, 1536, 2048])
            K = 128 * (rng.choice([1, 2, 5, 8, 16, 33]) if g == 128 else rng.choice([1, 2, 4, 9]))
        out.append((kind, M, N, K, g))
    return out


@pytest.mark.parametrize("kind,M,N,K,g", _cases(20261019, 30))
def test_random_shapes_against_oracle(kind, M, N, K, g):
    wt = synth.make_weight(K, N, M * 7 + K + N, g, bits=3 if kind == "w3" else 4, device=DEV)
    A = synth.make_activation(M, K, M + N, device=DEV)
    C = torch.full((M, N), float("nan"), dtype=torch.half, device=DEV)
    ws = torch.zeros(max(N // 128 * 16, 16), dtype=torch.int32, device=DEV)
    if kind == "mul":
        marlin.mul_2_4(A, wt["B"], wt["meta"], C, wt["s"], ws)
    elif kind == "meta3":
        marlin.mul_2_4_meta3(A, wt["B"], marlin.pack_meta3(wt["meta"].reshape(-1)), C, wt["s"], ws)
    elif kind == "w3":
        marlin.mul_2_4_w3(A, wt["B"], wt["meta"], C, wt["s"], ws)
    else:
        Bn, Mn, Sn = marlin.pack_native(wt["B"], wt["meta"], wt["s"])
        marlin.mul_2_4_native(A, Bn, Mn, C, Sn)
    torch.cuda.synchronize()
    assert_close(C.cpu().numpy(), oracle_gemm(A.cpu().numpy(), to_cpu(wt)), f"{kind} M={M} N={N} K={K} g={g}")


def _dense_cases(seed, n):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        g = rng.choice([128, -1])
        M = rng.choice([1, 2, 7, 16, 31, 48, 65, 100, 129, 200, 333])
        N = rng.choice([256, 512, 768, 1024, 1536, 2048])
        K = 128 * (rng.choice([1, 2, 3, 8, 17, 40]) if g == 128 else rng.choice([1, 2, 4, 9]))
        out.append((M, N, K, g))
    return out


@pytest.mark.parametrize("M,N,K,g", _dense_cases(20261202, 20))
def test_random_dense_shapes_against_oracle(M, N, K, g):
    """The dense op (reference marlin/__init__.py:61-75) on seeded shapes that cross
    its small-batch and large-M kernels, with and without split-K."""
    wt = synth.make_dense_weight(K, N, M * 5 + K + N, g, device=DEV)
    A = synth.make_activation(M, K, M + N + 3, device=DEV)
    C = torch.full((M, N), float("nan"), dtype=torch.half, device=DEV)
    ws = torch.zeros(max(N // 128 * 16, 16), dtype=torch.int32, device=DEV)
    marlin.mul(A, wt["B"], C, wt["s"], ws)
    torch.cuda.synchronize()
    W = o.dense_dequant(wt["B"].cpu().numpy(), wt["s"].cpu().numpy(), K, N, g)
    assert_close(C.cpu().numpy(), o.gemm(A.cpu().numpy(), W), f"dense M={M} N={N} K={K} g={g}")
