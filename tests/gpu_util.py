"""Helpers of the GPU parity tests: oracle references for packed operands and
column slices of the packed layouts."""
import numpy as np
import torch

from oracle import sm24_oracle as o

REL_MAE = 1e-3   # mean|C - ref| / mean|ref|
MAX_REL = 2e-2   # max|C - ref| / max|ref|


def slice_cols(t: dict, c0: int, nc: int) -> dict:
    """Columns [64*c0, 64*(c0+nc)) of a packed weight (dict of CPU numpy arrays).

    Every packed operand is self-contained per 64-column chunk: B holds 128 words,
    the metadata 128 int16 and the scales 64 halves per chunk and k-block row."""
    K, N = t["K"], t["N"]
    rows = K // 32
    out = dict(t)
    if t["bits"] == 4:
        out["B"] = np.ascontiguousarray(t["B"].reshape(rows, 2 * N)[:, 128 * c0:128 * (c0 + nc)])
    else:
        out["B"] = np.ascontiguousarray(t["B"].reshape(rows, 6 * N)[:, 384 * c0:384 * (c0 + nc)]).ravel()
    out["meta"] = np.ascontiguousarray(t["meta"].reshape(-1).reshape(rows, 2 * N)[:, 128 * c0:128 * (c0 + nc)])
    out["s"] = np.ascontiguousarray(t["s"][:, 64 * c0:64 * (c0 + nc)])
    out["N"] = 64 * nc
    return out


def to_cpu(wt: dict) -> dict:
    return {k: (v.cpu().numpy() if isinstance(v, torch.Tensor) else v) for k, v in wt.items()}


def oracle_weight(t: dict) -> np.ndarray:
    K, N, g = t["K"], t["N"], t["groupsize"]
    if t["bits"] == 4:
        return o.dequant(t["B"], t["meta"], t["s"], K, N, g)
    return o.dequant_w3(t["B"], t["meta"], t["s"], K, N, g)


def oracle_gemm(A: np.ndarray, t: dict) -> np.ndarray:
    return o.gemm(A, oracle_weight(t))


def assert_close(C: np.ndarray, ref: np.ndarray, what: str = ""):
    C = C.astype(np.float64)
    ref = ref.astype(np.float64)
    assert np.isfinite(C).all(), f"{what}: non-finite output"
    err = np.abs(C - ref)
    rel = err.mean() / max(np.abs(ref).mean(), 1e-30)
    mx = err.max() / max(np.abs(ref).max(), 1e-30)
    assert rel <= REL_MAE, f"{what}: relative MAE {rel:.3e} > {REL_MAE}"
    assert mx <= MAX_REL, f"{what}: max error {mx:.3e} of max|ref| > {MAX_REL}"
    return rel, mx


_WEIGHTS = {}


def cached_weight(K: int, N: int, seed: int, device: str = "cuda:0"):
    """One large packed weight at a time (device copy and host copy), kept between the
    tests that use the same (K, N, seed) so that a Llama-2-70B weight is built once."""
    from csed499ii_amd import synth

    key = (K, N, seed)
    if key not in _WEIGHTS:
        _WEIGHTS.clear()
        wt = synth.make_weight(K, N, seed, 128, device=device)
        _WEIGHTS[key] = (wt, to_cpu(wt))
    return _WEIGHTS[key]


def check_slices(C, A_np: np.ndarray, t: dict, starts, nc: int, what: str):
    """Compare columns [64*c0, 64*(c0+nc)) of the GPU output C (all rows) with the
    oracle on the same column slice of the packed weight, for every c0 in starts."""
    for c0 in starts:
        ref = oracle_gemm(A_np, slice_cols(t, c0, nc))
        assert_close(C[:, 64 * c0:64 * (c0 + nc)].cpu().numpy(), ref, f"{what} slice {c0}")
